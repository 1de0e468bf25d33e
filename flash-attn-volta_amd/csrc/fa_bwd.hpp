// fa_bwd.hpp -- backward FlashAttention kernels for gfx950.
//
// FlashAttention backward (Dao et al. 2022, Algorithm 4).  The reference
// (flash_attn_volta/triton_fa_bwd.py:636-700) runs a delta op and two
// kernels.  The work is split the same way, into two kinds of workgroup
// ("blocks"):
//   dQ block   (dq_block)  : one query block, sweeping key tiles; dQ =
//                            scale * dS K (reference: _fa_bwd_dq_kernel_*,
//                            :73-307)
//   dK/dV block (dkdv_block): one key block, sweeping query tiles; dV =
//                            P^T dO, dK = scale * dS^T Q (reference:
//                            _fa_bwd_dkdv_kernel_*, :319-580)
// and delta = rowsum(dO * O) in fp32 (the torch op at :650).  fa_bwd runs
// them as
//   causal, D <= 64, and causal D = 128 on grids of at most four rounds
//   without the dQ split:
//                    fa_bwd_preprocess_kernel (delta), then ONE launch of
//                    fa_bwd_fused_kernel, every dK/dV block and then every
//                    dQ block in one grid: the dQ blocks fill the slots the
//                    causal sweeps of unequal length leave idle;
//   otherwise:       fa_bwd_dq_kernel, whose blocks also compute delta from
//                    the rows their lanes hold and write it, then
//                    fa_bwd_dkdv_kernel.
// Both ways compute delta with the same fp32 operations in the same order,
// so the gradients are the same bits.  The standalone entry points
// fa_bwd_preprocess / fa_bwd_dq / fa_bwd_dkdv run fa_bwd_preprocess_kernel
// and each block kernel by itself.
// P = exp(scale * Q K^T - LSE) is recomputed from the forward LSE and
// dS = P * (dO V^T - delta).  No floating-point atomics and no S x S
// buffer: every output element is written once by one lane, so results are
// bit-reproducible and a causal query row's dQ never reads a key block it
// cannot see.  (The one integer atomic, in the causal key-block split --
// of the eight-wave D = 128 dK/dV layout and of the D = 64 query-split
// layout, DkdvTile::KEY_SPLIT -- only decides which of two workgroups adds
// their two fp32 partials; the sum is the same either way.)
//
// Fragment layouts follow fa_common.hpp.  The dK/dV kernel computes S = Q K^T
// with queries as the (kperm-ordered) A rows, so a lane owns one key and its
// P / dS values are directly the B operand of dV^T = dO^T P and
// dK^T = Q^T dS.  The dQ kernel computes S^T = K Q^T like the forward, so a
// lane owns one query and its dS^T values feed dQ^T = K^T dS^T.  Every tile
// is staged row-major (kperm row order) with 16-byte buffer loads; the
// transposed operands (Q^T, dO^T, K^T) come from ds_read_b64_tr_b16.
//
// dS scaling.  dS is rounded to the element type (fp16 or bf16) for the
// MFMAs.  Its magnitude follows the upstream gradient and can sit far below
// the fp16 normal range (a loss averaged over thousands of tokens gives
// |dS| ~ 1e-9 deep in a network), where fp16 would flush it to zero.  Each
// lane therefore scales its output row's dS by a power of two 2^e and
// divides the result by 2^e at the end.  In dK (lane = key, summing over
// queries) e is settled per query tile, before the tile's MFMAs, from a
// bound on the lane's |dS| over the tile: |dS| = P |dO . V_k - delta| <=
// max|dO| ||V_k||_1 + max|delta| (P <= 1), with max|dO| and max|delta| over
// the tile's rows from the row-group maxima (BwdArgs::rmax) that the delta
// pass writes; e keeps the scaled bound in [2^8, 2^15] (re-settled to
// [2^14, 2^15) when it leaves), so no scaled dS passes fp16's 65504, with
// the fp32 accumulator rescaled exactly whenever e changes.  The maxima
// come in through the scalar cache with the tile's loads, and the check for
// tile t + 1 runs at the end of tile t, under its last MFMAs.  (Settling
// from the bound replaced a per-32x32-block maximum of the computed |dS| on
// the MFMAs' path: the backward -1.2 to -4.3 % at (1,4096,16,64),
// (1,4096,8,128), (1,4096,16,128), (2,2048,16,64), (1,8192,16,64) and
// (4,4096,16,64), causal and not; +-0.5 % at (2,1024,8,64) and
// (1,2048,16,64); +6.5 % at (4,512,4,32), whose sweeps of at most four
// tiles pay the per-block set-up -- ||V_k||_1, the first settle -- and a
// pre-pass that also writes the maxima.)  In dQ (lane = query) e
// is fixed per query before the sweep, from the query's dO row: dO and
// delta are scaled so that the row's largest |dO| lies in [2^-4, 2^-3),
// which bounds |dS * 2^e| by 2^-2 D max|V| and needs no per-tile checks.
// Scaling by powers of two changes no rounding in the normal range and
// depends only on the lane's own data, so results stay deterministic
// (bf16, with fp32's exponent range, does not need it but loses nothing by
// it).
#pragma once

#include "fa_common.hpp"

namespace fa {

// Swizzle of the dK/dV kernel's query tiles (read both ways): the padded
// SW_PD (fa_common.hpp) at D = 128, SW_AT at D = 64 and 32 (conflict-free
// both ways; its offsets fit since they are byte offsets hidden from
// loop-invariant code motion at each tile step).  At D = 32 (4 chunks a
// row) any chunk permutation serves the transposed reads; the row reads
// need rows r, r + 4, r + 8, r + 12 permuted apart, which SW_P8's period
// of 8 cannot do (12 % of the D = 32 fused launch's LDS cycles
// conflicted).
// Measured at D = 128: LDS bank conflicts 45 % of LDS-active cycles with
// SW_P8, 0 with SW_PD; the backward -3.2 to -3.8 % at (1,4096,8,128) and
// (1,4096,16,128).  At D = 64 SW_AT took the conflicts from 0.03-0.08 to
// 0.
template <int D>
constexpr int kDkdvSwizzle = D >= 128 ? SW_PD : SW_AT;

// 32-row groups of S rows (the row-group maxima's second-to-last extent)
__host__ __device__ __forceinline__ int row_groups(int S) { return (S + 31) >> 5; }

struct BwdArgs {
  TensorDesc q, k, v, dout;   // q, dout: (B, Sq, H, D); k, v: (B, Sk, Hk, D)
  const float *lse;     // (B, H, Sq) natural log
  const float *delta;   // (B, H, Sq)
  // dQ kernel only: when non-NULL, delta is not read but computed from O
  // and dO and written here (the pre-pass folded into the dQ kernel)
  float *delta_out;
  TensorDesc o;         // (B, Sq, H, D), read when delta_out is set
  // Row-group maxima: for every 32-query-row group of each (b, h), the
  // largest max_d |dO| and the largest |delta| over its rows, (B, H,
  // row_groups(Sq), 2) fp32.  The dK/dV blocks read them (rmax: the bound
  // that fixes their dS scale per query tile); the dQ kernel writes them
  // beside delta_out when rmax_out is set.
  const float *rmax;
  float *rmax_out;
  f16 *dq, *dk, *dv;    // dq: (B, Sq, H, D); dk, dv: (B, Sk, Hk, D)
  int64_t dq_sb, dq_ss, dq_sh;
  int64_t dk_sb, dk_ss, dk_sh;
  int64_t dv_sb, dv_ss, dv_sh;
  int B, Sq, Sk, H, Hk;
  int grp;              // query heads per key/value head (H / Hk)
  int off;              // causal: query i sees keys j <= i + off (off = Sk - Sq)
  int n_blocks;         // query blocks (dQ) or key blocks (dK/dV)
  float c;              // |sm_scale| * log2(e), clamped away from 0
  // dK/dV blocks: the LSE seed factor -log2(e) / cr, cr = c / ck (ck =
  // min(c, 1) for fp16, 1 for bf16), from the host: a uniform value that
  // a VGPR would hold for the whole sweep
  float lse_mul;
  float sm_scale;       // signed scale applied to dQ and dK
  int neg;              // 1 when sm_scale < 0 (K or Q negated in S recompute)
  int zigzag;           // causal block order: 1 zigzag heavy / light, 0 heaviest first
  // Causal key-block split (dK/dV layouts with KEY_SPLIT): key blocks
  // [0, split_kt) of every (b, key/value head) are each swept by two
  // workgroups, one per half of their query tiles.  Each writes its fp32
  // dK / dV partial to part[slot][segment] and counts itself in cnt[slot]
  // (slot = bhk * split_kt + kt); the second to finish adds the two and
  // writes dK / dV.  split_kt = 0: no split.
  int split_kt;
  unsigned *cnt;
  float *part;
  // dQ kernel: when non-NULL, workgroup 0 zeroes cnt_zero[0 .. n_cnt_zero)
  // (the split counters of the dK/dV launch that follows on the stream)
  unsigned *cnt_zero;
  int n_cnt_zero;
  // Causal query-block split of the dQ kernel: the last dq_split query
  // blocks (dq_bm rows each, dq_nblocks per (b, h)) are each swept by two
  // workgroups, one per half of the block's key tiles, which write their
  // fp32 dQ rows (already scaled) to dq_part[slot][segment] (row-major
  // dq_bm x D; slot = bh * dq_split + block - (dq_nblocks - dq_split)).
  // The dK/dV kernel that follows on the stream adds the two halves and
  // writes dq (the kernel boundary orders the accesses).  0: no split.
  int dq_split, dq_bm, dq_nblocks;
  float *dq_part;
};

struct PreArgs {
  TensorDesc o, dout;
  float *delta;
  float *rmax;   // row-group maxima (BwdArgs::rmax), (B, H, G, 2); NULL: not written
  int B, S, H;
  // when non-NULL, workgroup 0 zeroes cnt_zero[0 .. n_cnt_zero) (the
  // key-block split counters of the fused backward launch that follows)
  unsigned *cnt_zero;
  int n_cnt_zero;
};

// ---------------------------------------------------------------------------
// delta[b,h,s] = sum_d O * dO.  Two lanes per row; a workgroup covers 128
// rows of one (b, h), a wave 32 of them (delta writes contiguous).  Lane g
// of a pair sums its half of the row in the dQ kernel's fragment order --
// chunks 16c + 8g .. +7, c ascending, one fp32 FMA per element -- then the
// pair adds its two sums: the same fp32 operations, in the same order, as
// the dQ kernel's own delta (BwdArgs::delta_out), so every backward path
// sees bit-identical delta.  (dP - delta cancels exactly in exact
// arithmetic for a query with one visible key; in fp32 it leaves a few
// ulps of delta in dS, and which few depends on this order.)  With rmax
// set, each wave also writes its 32 rows' group maxima (max |dO|, max
// |delta|: BwdArgs::rmax), which maxima alone make exact whatever the order.
template <typename E, int D>
__global__ __launch_bounds__(256) void fa_bwd_preprocess_kernel(PreArgs a) {
  constexpr int RPB = 128;   // rows per block, all of one (b, h)
  const int tid = threadIdx.x;
  if (a.cnt_zero != nullptr && blockIdx.x == 0) {
    for (int i = tid; i < a.n_cnt_zero; i += 256) a.cnt_zero[i] = 0u;
  }
  const int nchunk = (a.S + RPB - 1) / RPB;
  const int64_t bh = blockIdx.x / nchunk;
  const int s0 = (int)(blockIdx.x % nchunk) * RPB;
  const int s = s0 + (tid >> 1);
  const int g = tid & 1;
  const bool valid = s < a.S;
  float acc = 0.0f, om = 0.0f;
  if (valid) {
    const int h = (int)(bh % a.H), b = (int)(bh / a.H);
    const f16 *po = a.o.head(b, h) + (int64_t)s * a.o.ss + 8 * g;
    const f16 *pg = a.dout.head(b, h) + (int64_t)s * a.dout.ss + 8 * g;
    vec8<E> ov[D / 16], gv[D / 16];
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      ov[c] = ld8<E>(po + 16 * c);
      gv[c] = ld8<E>(pg + 16 * c);
    }
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc = __builtin_fmaf((float)ov[c][j], (float)gv[c][j], acc);
        om = fmaxf(om, fabsf((float)gv[c][j]));
      }
  }
  acc += xor1(acc);   // the row's other half
  if (valid && g == 0) a.delta[bh * a.S + s] = acc;
  if (a.rmax != nullptr) {
    // the wave's 32 rows (64 lanes, rows past S contribute 0), maxima in
    // lane 63
    const unsigned dm = max_wave_nonneg(om);
    const unsigned am = max_wave_nonneg(valid ? fabsf(acc) : 0.0f);
    const int sw = s0 + 32 * (tid >> 6);   // the wave's first row
    if ((tid & 63) == 63 && sw < a.S) {
      float *p = a.rmax + (bh * row_groups(a.S) + sw / 32) * 2;
      p[0] = __uint_as_float(dm);
      p[1] = __uint_as_float(am);
    }
  }
}

// ---------------------------------------------------------------------------
// Power-of-two scale of one dK lane's dS column (see the header), settled
// per query tile from a bound on the lane's |dS| over that tile.
struct DsScale {
  float mul = 1.0f;   // 2^e, |e| <= 100 (a normal float)

  // e, from mul alone (one register per lane for the state)
  __device__ __forceinline__ int exp() const { return __builtin_amdgcn_frexp_expf(mul) - 1; }

  // Whether settle(bnd) would change the scale: bnd > 0 and bnd * 2^e
  // outside [2^8, 2^15].  When it is false in every lane, settle() would
  // return 1 everywhere and leave the state as it is.
  __device__ __forceinline__ bool stale(float bnd) const {
    const float sb = bnd * mul;
    // bitwise, not short-circuit: && / || would become branches
    return (bnd > 0.0f) & ((sb > 32768.0f) | (sb < 256.0f));
  }
  // New scale for a tile whose dS obey |dS| <= bnd: when stale, e := 15 -
  // exponent(bnd), so bnd * 2^e lies in [2^14, 2^15) (bnd = f * 2^x, f in
  // [0.5, 1)) and no scaled dS can pass fp16's 65504.  Returns the factor
  // by which the lane's accumulator must be multiplied (1 when e is
  // unchanged).  Straight-line selects, no per-lane branch.
  __device__ __forceinline__ float settle(float bnd) {
    const int e = exp();
    int en = 15 - __builtin_amdgcn_frexp_expf(bnd);
    en = en > 100 ? 100 : (en < -100 ? -100 : en);
    en = stale(bnd) ? en : e;
    const float f = __builtin_amdgcn_ldexpf(1.0f, en - e);
    mul = __builtin_amdgcn_ldexpf(1.0f, en);
    return f;
  }
};

// Store a D^T x 32 accumulator set (lane = row `row`, slots = columns) as
// row `row` of a (.., D) tensor of element type E, scaled by `mul`.
template <typename E, int D>
__device__ __forceinline__ void store_row(f16 *dst, const floatx16 (&acc)[D / 32], float mul, int g) {
#pragma unroll
  for (int d = 0; d < D / 32; ++d) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      vec4<E> v4;
#pragma unroll
      for (int j = 0; j < 4; ++j) v4[j] = (E)(acc[d][4 * r + j] * mul);
      *(vec4<E> *)(dst + 32 * d + c_row(4 * r, g)) = v4;
    }
  }
}

// The same rows as store_row, as fp32 (split partials).
template <int D>
__device__ __forceinline__ void store_row_f32(float *dst, const floatx16 (&acc)[D / 32], float mul,
                                              int g) {
#pragma unroll
  for (int d = 0; d < D / 32; ++d) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      floatx4 v4;
#pragma unroll
      for (int j = 0; j < 4; ++j) v4[j] = acc[d][4 * r + j] * mul;
      *(floatx4 *)(dst + 32 * d + c_row(4 * r, g)) = v4;
    }
  }
}

// dQ rows of split query blocks (BwdArgs::dq_split): dq = part[.][0] +
// part[.][1] (fp32 addition commutes, so the sum does not depend on which
// half is which), converted to E.  Every workgroup of the calling grid
// takes an equal share of the 4-element groups, `nt` threads each.
template <typename E, int D>
__device__ __forceinline__ void dq_split_combine(const BwdArgs &a, int nt) {
  const int64_t per_slot = (int64_t)a.dq_bm * (D / 4);
  const int64_t total = (int64_t)a.B * a.H * a.dq_split * per_slot;
  const int64_t grid = gridDim.x;
  const int64_t lo = total * blockIdx.x / grid, hi = total * (blockIdx.x + 1) / grid;
  for (int64_t gi = lo + threadIdx.x; gi < hi; gi += nt) {
    const int64_t slot = gi / per_slot;
    const int rem = (int)(gi - slot * per_slot);
    const int r = rem / (D / 4), c4 = rem % (D / 4);
    const int bh = (int)(slot / a.dq_split);
    const int qt = a.dq_nblocks - a.dq_split + (int)(slot - (int64_t)bh * a.dq_split);
    const int q = qt * a.dq_bm + r;
    if (q >= a.Sq) continue;
    const float *p0 = a.dq_part + (slot * 2 * a.dq_bm + r) * D + 4 * c4;
    const floatx4 x = *(const floatx4 *)p0;
    const floatx4 y = *(const floatx4 *)(p0 + (int64_t)a.dq_bm * D);
    vec4<E> v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (E)(x[j] + y[j]);
    const int b = bh / a.H, h = bh % a.H;
    *(vec4<E> *)(a.dq + b * a.dq_sb + h * a.dq_sh + (int64_t)q * a.dq_ss + 4 * c4) = v;
  }
}

// Load a lane's D/16 B-operand fragments of row `row` (clamped to S-1).
template <typename E, int D>
__device__ __forceinline__ void load_row_frags(vec8<E> (&f)[D / 16], const f16 *head, int64_t ss,
                                               int row, int S, int g) {
  const f16 *p = head + (int64_t)min(row, S - 1) * ss + 8 * g;
#pragma unroll
  for (int c = 0; c < D / 16; ++c) f[c] = ld8<E>(p + 16 * c);
}

// ---------------------------------------------------------------------------
// Partial-sum merge of two waves that own the same output rows (lane l of
// both waves holds the same row and the same D^T slots).  `buf` is LDS with
// room for 64 * (D/2 + 1) floats; every thread calls it (it has a barrier).
// The writer hands over acc * 2^-e (its power-of-two dS scale undone), the
// reader adds it to its own acc * 2^-e and returns the unscaled sum in acc.
template <int D>
__device__ __forceinline__ void merge_pair(float *buf, bool writer, floatx16 (&acc)[D / 32],
                                           const DsScale &sc, int lane) {
  const float inv = __builtin_amdgcn_ldexpf(1.0f, -sc.exp());
  if (writer) {
#pragma unroll
    for (int d = 0; d < D / 32; ++d)
#pragma unroll
      for (int i = 0; i < 16; ++i) buf[(16 * d + i) * 64 + lane] = acc[d][i] * inv;
  }
  __syncthreads();
  if (!writer) {
#pragma unroll
    for (int d = 0; d < D / 32; ++d)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[d][i] = acc[d][i] * inv + buf[(16 * d + i) * 64 + lane];
  }
}

// Agent-scope (device-wide) relaxed accesses for the split partials
// (global_store / global_load with sc1 on gfx950): they go to the point
// where all XCDs are coherent instead of a per-XCD L2 copy, so no L2
// write-back or invalidation is needed to exchange them.
__device__ __forceinline__ void store_agent(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// x * m + y with the product rounded before the sum (never one FMA): the
// two segments' partials are formed as x * m, so whichever of them adds
// the other's gets the same bits (fp32 addition commutes).
__device__ __forceinline__ float mul_then_add(float x, float m, float y) {
#pragma clang fp contract(off)
  const float p = x * m;
  return p + y;
}

// End of one segment of a split key block (see BwdArgs::split_kt): the
// merged dK (unscaled, times sm_scale here) and dV of the `holder` waves go
// to part[slot][seg] as fp32; thread 0 counts the segment in cnt[slot]
// once every wave's partial stores have completed, and the workgroup that
// counts second adds the other segment's partial to its own and stores
// dK / dV as E.  The first workgroup leaves: no workgroup ever waits for
// another.  Ordering: all partial accesses are agent-scope atomics, so the
// release / acquire that a device-scope fence would add reduce to waiting
// for the stores to complete (vmcnt(0)) before the barrier that precedes
// the counter update; the loads follow the counter's returned value.  A
// __threadfence() here would also write back and invalidate the XCD's
// whole L2 in every such workgroup, which costs more than the split gains.
//
// This is a hardware assumption, outside the HIP memory model's formal
// guarantees (which would need a release on the counter update and an
// acquire on its result): on gfx950, agent-scope relaxed stores and loads
// are issued with sc1 and bypass the non-coherent per-XCD L2, a store has
// reached the coherent level once vmcnt counts it complete, and the
// counter's atomicAdd is performed at that same level after the barrier.
// The library is built for gfx950 only (the #error below); another target
// must re-establish the ordering, e.g. with __hip_atomic_fetch_add(...,
// __ATOMIC_RELEASE / __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT).
// `pl` = the lane's index among the holders (key group * 64 + lane).
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "the split dK/dV exchange's ordering argument holds for gfx950 only"
#endif
template <typename E, int D, int NKG>
__device__ __forceinline__ void split_finish(const BwdArgs &a, floatx16 (&dk)[D / 32],
                                             floatx16 (&dv)[D / 32], int slot, int seg,
                                             bool holder, int pl, bool in_range, f16 *dk_row,
                                             f16 *dv_row, int g) {
  constexpr int HALF = (D / 32) * 16;   // floats per lane and tensor
  constexpr int LANES = 64 * NKG;
  __shared__ unsigned s_order;
  if (holder) {
    float *mine = a.part + ((size_t)slot * 2 + seg) * (2 * HALF * LANES) + pl;
#pragma unroll
    for (int d = 0; d < D / 32; ++d)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        store_agent(mine + (16 * d + i) * LANES, dk[d][i] * a.sm_scale);
        store_agent(mine + (HALF + 16 * d + i) * LANES, dv[d][i]);
      }
  }
  __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's partial stored
  __syncthreads();
  if (threadIdx.x == 0) s_order = atomicAdd(a.cnt + slot, 1u);
  __syncthreads();
  if (s_order == 0) return;   // the other segment finishes this block
  if (holder && in_range) {
    // dK added and stored before dV's partial is loaded: both partials in
    // flight beside dK and dV would pass 256 VGPRs at D = 128 (spills)
    float *other = a.part + ((size_t)slot * 2 + (seg ^ 1)) * (2 * HALF * LANES) + pl;
#pragma unroll
    for (int d = 0; d < D / 32; ++d)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        dk[d][i] = mul_then_add(dk[d][i], a.sm_scale, load_agent(other + (16 * d + i) * LANES));
    store_row<E, D>(dk_row, dk, 1.0f, g);
#pragma unroll
    for (int d = 0; d < D / 32; ++d)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        dv[d][i] = mul_then_add(dv[d][i], 1.0f, load_agent(other + (HALF + 16 * d + i) * LANES));
    store_row<E, D>(dv_row, dv, 1.0f, g);
  }
}

// ---------------------------------------------------------------------------
// dK / dV: a workgroup's waves own key groups of 32 keys; with NQH = 2 the
// two waves of a group take the two query halves of every tile and merge
// their dK / dV partial sums through LDS at the end (doubling the waves in
// flight for grids too small to fill the GPU; the launcher decides the
// split).  Query tiles of BQ rows stream through double-buffered LDS as Q
// and dO (kperm row order) plus LSE and delta.  Layouts:
//   * SPLIT = 1, D <= 64: 4 waves, one key group each (BK = 128), both
//     32-query sub-blocks of every 64-query tile;
//   * SPLIT = 2, D = 64 (KV_LDS): 4 waves = 2 key groups x 2 query halves
//     (BK = 64), and the keys' K and V rows in LDS rather than in per-lane
//     registers, which brings the kernel under 168 VGPRs: three waves per
//     SIMD instead of two (C4a-shaped causal dK/dV -11 %; kernel latency,
//     not MFMA or LDS throughput, bounds it, so more waves in flight pay);
//   * SPLIT = 2, D = 32 (EARLY_S): as above with K / V in registers and
//     128-query tiles, two 32-query sub-blocks per wave whose S and dP
//     MFMAs are all issued before the first sub-block's softmax;
//   * SPLIT = 2, D = 128: 2 key groups x 2 query halves, K / V in registers
//     (one wave per SIMD);
//   * SPLIT = 1, D = 128 (WIDE): 8 waves = 4 key groups x 2 query halves
//     (BK = 128) with K and V in LDS (129 KiB: one workgroup per CU), so
//     each SIMD runs two waves under 256 VGPRs where the 4-wave layout ran
//     one wave with the K / V fragments spilling.
template <int D, int SPLIT>
struct DkdvTile {
  static_assert(SPLIT == 1 || SPLIT == 2, "split is 1 or 2");
  static constexpr bool WIDE = D == 128 && SPLIT == 1;
  static constexpr int NW = WIDE ? 8 : 4;                       // waves per workgroup
  static constexpr int NQH = (SPLIT == 2 || WIDE) ? 2 : 1;      // query halves
  static constexpr int NKG = NW / NQH;                          // key groups of 32
  static constexpr bool KV_LDS = (D == 64 && SPLIT == 2) || WIDE;
  // issue all S / dP MFMAs of a tile first (measured: helps the split
  // variant, costs ~1 % unsplit, where two waves per SIMD already overlap)
  static constexpr bool EARLY_S = D <= 64 && SPLIT == 2 && !KV_LDS;
  // 32-query sub-blocks per wave per tile (64-query tiles unless EARLY_S)
  static constexpr int NSUB = EARLY_S ? 2 : 2 / NQH;
  static constexpr int BK = 32 * NKG;
  static constexpr int BQ = 32 * NSUB * NQH;   // queries per tile
  static constexpr int NT = 64 * NW;
  // waves per SIMD the register allocation is held to
  static constexpr int WAVES_PER_EU = (D == 64 && KV_LDS) ? 3 : (WIDE ? 2 : 1);
  // K and V staged in LDS are read only as B operands, row by row like an
  // A operand: at D = 64 they take SW_A (conflict-free for those reads,
  // with offsets of their own), at D = 128 the query tiles' SW_PD
  // (conflict-free both ways, 4 offset registers where SW_A takes 8)
  static constexpr int QSW = kDkdvSwizzle<D>;
  static constexpr int KVSW = (KV_LDS && D == 64) ? SW_A : QSW;
  static constexpr int LDS_TILE = lds_row<D, QSW>(BQ);   // one stage (fa_common.hpp)
  static constexpr int LDS_KV = KV_LDS ? lds_row<D, KVSW>(BK) : 8;   // K (or V), kperm rows
  // operand reads of sdp_grad's MFMAs this many MFMAs ahead (0: each just
  // before its MFMA), for the S / dP MFMAs, and with PF_ALL for the dV / dK
  // MFMAs too.  At D = 128 (two waves per SIMD) every MFMA otherwise waits
  // on its own LDS reads: the backward -1 to -2.4 % with the S / dP
  // operands ahead, and another -1 to -2.4 % with all of them (measured at
  // (1,4096,8,128), (1,4096,16,128), (1,8192,8,128) causal and non-causal;
  // two MFMAs ahead: +-0.8 %).  At D = 64 (three waves per SIMD, 168 VGPRs)
  // the dV / dK operands ahead would spill.
  static constexpr int PF_OPS = KV_LDS ? 1 : 0;
  static constexpr bool PF_ALL = WIDE || (D == 64 && KV_LDS);
  // layouts that implement the causal key-block split (BwdArgs::split_kt)
  static constexpr bool KEY_SPLIT = WIDE || (D == 64 && SPLIT == 2);
  static_assert(64 * (D / 2) * 4 <= LDS_TILE * 2, "a merge buffer must fit in one stage");
};

// The LDS arrays of one dK/dV workgroup.  One LDS object per stage: the
// compiler then sees that the DMA into one stage cannot alias reads of the
// other and does not wait for it early.  Declared by the kernel that runs
// the block (the dK/dV kernel, or the fused backward kernel, whose dQ
// blocks reuse the four tile stages) and passed in by pointer: the block
// functions are inlined, so every access still names its own object.
#define FA_DKDV_LDS(T)                                                                 \
  __shared__ __attribute__((aligned(16))) f16 s_q0[T::LDS_TILE], s_q1[T::LDS_TILE];   \
  __shared__ __attribute__((aligned(16))) f16 s_do0[T::LDS_TILE], s_do1[T::LDS_TILE]; \
  __shared__ __attribute__((aligned(16))) float s_lse[2][T::BQ];                     \
  __shared__ __attribute__((aligned(16))) float s_dl[2][T::BQ];                      \
  __shared__ __attribute__((aligned(16))) f16 s_k[T::LDS_KV], s_v[T::LDS_KV]

// One dK/dV block (workgroup `bid` of the dK/dV grid).
template <typename E, int D, bool CAUSAL, int SPLIT>
__device__ __forceinline__ void dkdv_block(const BwdArgs &a, const int bid, f16 *s_q0, f16 *s_q1,
                                           f16 *s_do0, f16 *s_do1,
                                           float (*s_lse)[DkdvTile<D, SPLIT>::BQ],
                                           float (*s_dl)[DkdvTile<D, SPLIT>::BQ], f16 *s_k,
                                           f16 *s_v) {
  using T = DkdvTile<D, SPLIT>;
  constexpr int BK = T::BK, BQ = T::BQ, NSUB = T::NSUB;
  auto q_st = [&](auto stc) -> f16 * { return decltype(stc)::value ? s_q1 : s_q0; };
  auto do_st = [&](auto stc) -> f16 * { return decltype(stc)::value ? s_do1 : s_do0; };

  // first the dQ rows of the preceding dQ launch's split query blocks
  if (CAUSAL && a.dq_split > 0) dq_split_combine<E, D>(a, T::NT);

  const int Sq = a.Sq, Sk = a.Sk, off = a.off;
  const int BHk = a.B * a.Hk;
  const int bhk = bid % BHk;
  const int rank = bid / BHk;
  // Causal: low key blocks see the most queries.  Blocks go heaviest
  // first (each slot that frees up takes the heaviest block left), or
  // zigzag heavy / light where the launcher measured that better (long
  // sweeps on grids of at most 1.5 rounds: a.zigzag).  With the key-block
  // split, ranks 2kt and 2kt + 1 are the two halves of block kt < split_kt,
  // then the unsplit blocks follow, heaviest first.
  const int nsplit = (T::KEY_SPLIT && CAUSAL) ? a.split_kt : 0;
  const bool split = rank < 2 * nsplit;
  const int seg = split ? (rank & 1) : 0;
  const int kt = split ? (rank >> 1)
                       : (nsplit > 0 ? rank - nsplit
                                     : ((CAUSAL && a.zigzag) ? zigzag_rank(rank, a.n_blocks)
                                                             : rank));
  const int b = bhk / a.Hk, hk = bhk % a.Hk;
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int kg = w / T::NQH;
  const int qh = w % T::NQH;
  const int g = lane >> 5, l32 = lane & 31;
  const int k0 = kt * BK;
  const int wk0 = k0 + 32 * kg;
  // this lane's key: K / V rows staged in LDS come in kperm order (the
  // tile loader's), so lane l32 then reads key wk0 + kperm(l32)
  const int key = wk0 + (T::KV_LDS ? kperm(l32) : l32);

  // K^T and V^T fragments (B operands): K[key][16c + 8g .. +7].  For fp16,
  // K is pre-multiplied by +-ck = +-min(c, 1) and rounded to fp16 (as the
  // reference pre-scales K^T, triton_fa_bwd.py:355), so the S MFMAs produce
  // ck * s directly; ck <= 1 keeps the product inside the fp16 range.  The
  // rest of c, cr = c / ck, is 1 unless |sm_scale| > ln 2.  bf16 keeps K
  // unscaled (ck = 1: a second bf16 rounding would cost 8-bit accuracy),
  // only its sign follows sm_scale.
  constexpr int NKF = T::KV_LDS ? 1 : D / 16;
  constexpr int QSW = T::QSW, KVSW = T::KVSW;
  // Element offset of A-operand row l32, chunk 2cc + g, of a tile laid out
  // with swizzle SW.  SW_PD (D = 128) permutes a chunk index's bits 2-3
  // only, so chunk 2cc + 2 + g sits 16 elements after chunk 2cc + g (cc
  // even): an immediate, not a register.
  // Offsets are in bytes and carry the wave's first row in the tile
  // (`base`, elements: a multiple of 32 rows); tile_step hides them from
  // loop-invariant code motion (opaque()), so each read is one offset
  // register plus an immediate (array, stage, sub-block).  Under SW_PD only
  // the even chunks' offsets are kept (odd = even + 32 bytes).
  auto row_offsets = [&](auto swc, int (&off)[D / 16], int base) {
    constexpr int SW = decltype(swc)::value;
    const int s = swz<D, SW>(l32);
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc)
      off[cc] = 2 * (base + lds_row<D, SW>(l32) + (((2 * cc + g) ^ s) << 3));
  };
  auto row_off = [&](auto swc, const int (&off)[D / 16], int cc) -> int {
    constexpr int SW = decltype(swc)::value;
    return (SW == SW_PD && (cc & 1)) ? off[cc - 1] + 32 : off[cc];
  };
  auto hide_offsets = [&](auto swc, int (&off)[D / 16]) {
    constexpr int SW = decltype(swc)::value;
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc)
      if (!(SW == SW_PD && (cc & 1))) opaque<16>(off[cc]);
  };
  // The eight-wave D = 128 layout keeps the wave's rows out of the offsets
  // and unhidden (FOLD false: the wave part is added to the array address,
  // as a scalar): folded and hidden there, the backward measured 1-1.5 %
  // slower at every D = 128 shape, with the same instruction counts.
  constexpr bool FOLD = !T::WIDE;
  const int kw = FOLD ? 0 : lds_row<D, KVSW>(32 * kg);   // elements
  int kv_off[T::KV_LDS ? D / 16 : 1];
  if constexpr (T::KV_LDS)
    row_offsets(std::integral_constant<int, KVSW>{}, kv_off, FOLD ? lds_row<D, KVSW>(32 * kg) : 0);
  vec8<E> kf[NKF], vf[NKF];
  const float ck = std::is_same<E, f16>::value ? fminf(a.c, 1.0f) : 1.0f;
  const float cr = a.c / ck;
  const float kmul = a.neg ? -ck : ck;
  // K and V loads are issued here and scaled once they land, after the
  // first query tile's loads are issued too (one memory latency for both)
  if constexpr (T::KV_LDS) {
    // the workgroup's BK keys into LDS (zeros past Sk)
    DmaStager<D, KVSW, BK, T::NW> stk, stv;
    stk.init(w, lane, a.k.ss);
    stv.init(w, lane, a.v.ss);
    stk.load(s_k, a.k.head(b, hk), a.k.ss, k0, Sk, w);
    stv.load(s_v, a.v.head(b, hk), a.v.ss, k0, Sk, w);
  } else {
    load_row_frags<E, D>(kf, a.k.head(b, hk), a.k.ss, key, Sk, g);
    load_row_frags<E, D>(vf, a.v.head(b, hk), a.v.ss, key, Sk, g);
  }
  // B operands of S and dP: K^T / V^T fragments K[key][16cc + 8g .. +7]
  // (registers, or LDS rows 32kg + l32 read like the query tiles' A rows)
  auto k_frag = [&](int cc) -> vec8<E> {
    if constexpr (T::KV_LDS) return ld8_b<E>(s_k + kw, row_off(std::integral_constant<int, KVSW>{}, kv_off, cc));
    else return kf[cc];
  };
  auto v_frag = [&](int cc) -> vec8<E> {
    if constexpr (T::KV_LDS) return ld8_b<E>(s_v + kw, row_off(std::integral_constant<int, KVSW>{}, kv_off, cc));
    else return vf[cc];
  };

  floatx16 dk[D / 32], dv[D / 32];
#pragma unroll
  for (int d = 0; d < D / 32; ++d) {
    dk[d] = floatx16{};
    dv[d] = floatx16{};
  }
  DsScale sc;

  // Query tiles: for each of the grp query heads sharing this key/value
  // head (their dK, dV contributions add up), the tiles from the first one
  // that can see key k0 (query k0 - off, causal) to the end.  Flattened:
  // tile t is tile t % nt_h of query head hk * grp + t / nt_h.
  const int m_first = CAUSAL ? max(0, k0 - off) : 0;
  const int m_begin = (m_first / BQ) * BQ;
  const int nt_h = (Sq > m_begin) ? (Sq - m_begin + BQ - 1) / BQ : 0;
  // A split block's segment 0 takes the first half of these tiles,
  // segment 1 the rest.
  const int n_all = nt_h * a.grp;
  const int t_begin = seg ? n_all / 2 : 0;
  const int n_tiles = split ? (seg ? n_all - n_all / 2 : n_all / 2) : n_all;

  // Per-query rows staged beside each tile, laid out as MFMA accumulator
  // seeds: s_lse = -LSE * log2(e) / cr (-inf past S, so P = 0 there) and
  // s_dl = -delta.  Seeding the S and dP MFMAs with them yields
  // ck * s - LSE' and dP - delta with no per-score VALU work.
  DmaStager<D, QSW, BQ, T::NW> stq, stg;
  stq.init(w, lane, a.q.ss);
  stg.init(w, lane, a.dout.ss);
  const float lse_mul = a.lse_mul;
  float lse_r = 0.0f, dl_r = 0.0f;   // raw LSE / delta of row m0 + tid
  // Q and dO go straight to LDS stage `st`; LSE / delta through VGPRs.
  // (cur_h, cur_m0) is tile t's query head and first row; advance()
  // steps to tile t + 1 incrementally (no per-tile scalar division by nt_h:
  // dK/dV -1 to -5 %).
  const int m_end = m_begin + nt_h * BQ;
  int cur_h = hk * a.grp + (t_begin > 0 ? t_begin / nt_h : 0);
  int cur_m0 = m_begin + (t_begin > 0 ? (t_begin % nt_h) * BQ : 0);
  auto advance = [&](int &h, int &m0) {
    m0 += BQ;
    if (m0 >= m_end) {
      m0 = m_begin;
      ++h;
    }
  };
  // Q / dO descriptors of the tile to load, walked by cursors: re-aimed at
  // a new query head, advanced by BQ rows otherwise; likewise the head's
  // row-group maxima (below).
  typedef const __attribute__((address_space(4))) float kfloat;
  const int ng = row_groups(Sq);
  RowCursor cq, cg;
  kfloat *rm_h;
  auto aim = [&](int h, int m0) {
    cq.init(a.q.head(b, h), a.q.ss, m0, Sq, D, BQ);
    cg.init(a.dout.head(b, h), a.dout.ss, m0, Sq, D, BQ);
    rm_h = (kfloat *)(a.rmax + ((int64_t)b * a.H + h) * ng * 2);
  };
  aim(cur_h, cur_m0);
  // The tile's row-group maxima (BwdArgs::rmax: max |dO| and max |delta|
  // of each 32 rows), for the bound |dS| <= P (|dO . V_k| + |delta|) <=
  // max|dO| ||V_k||_1 + max|delta| (P <= 1) that settles each lane's dS
  // scale before the tile's MFMAs: uniform loads through the scalar cache
  // (constant address space; no launch writes the maxima while this one
  // reads them), issued with the tile's other loads and held in SGPRs, so
  // that the settle at the tile's start waits on nothing.
  float nx_rm[2 * (BQ / 32)];
  auto load_tile = [&](int h, int m0, auto stc) {
    stq.load(q_st(stc), cq.rsrc(), w);
    stg.load(do_st(stc), cg.rsrc(), w);
    if (tid < BQ) {
      const int m = m0 + tid;
      const int64_t row = ((int64_t)b * a.H + h) * Sq + m;
      // rows past Sq: +inf LSE, so the seed below is -inf and P = 0
      lse_r = (m < Sq) ? a.lse[row] : kPosInf;
      dl_r = (m < Sq) ? a.delta[row] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < BQ / 32; ++i) {
      // a ragged last tile's groups past Sq read the head's last group
      // again, which the tile holds (tiles start below Sq): same bound
      const int gi = min((m0 >> 5) + i, ng - 1);
      nx_rm[2 * i] = rm_h[2 * gi];
      nx_rm[2 * i + 1] = rm_h[2 * gi + 1];
    }
  };
  // Publishing a stage: its LSE / delta rows go to LDS, then every DMA of
  // this wave is waited for (vmcnt(0)); the barrier after it makes the
  // whole tile visible.
  auto store_tile = [&](auto stc) {
    constexpr int st = decltype(stc)::value;
    if (tid < BQ) {
      s_lse[st][tid] = lse_r * lse_mul;
      s_dl[st][tid] = -dl_r;
    }
    __builtin_amdgcn_s_waitcnt(0x0f70);
  };

  // Per-lane LDS element offsets inside a stage (fa_common.hpp swizzle).
  // A-operand rows (Q, dO of this wave's 32-query sub-block): row l32, chunk
  // 2cc + g; transposed reads: rows 4g + (l16 >> 2), column chunk
  // 4d + 2((lane >> 4) & 1) + ((l16 >> 1) & 1), half 4 * (l16 & 1).
  // All in bytes, carrying the wave's first query row in the tile
  // (32 * NSUB * qh), as does the LSE / delta seed offset `s_row` (row
  // 32 * NSUB * qh + 8g of s_lse / s_dl).
  // (FOLD false: on the array addresses instead, qw and sw.)
  const int qbase = lds_row<D, QSW>(32 * NSUB * qh);
  const int qw = FOLD ? 0 : qbase, sw = FOLD ? 0 : 32 * NSUB * qh;
  int a_off[D / 16];
  TrOffsetsB<D, QSW> t_off;
  row_offsets(std::integral_constant<int, QSW>{}, a_off, FOLD ? qbase : 0);
  t_off.init(lane, FOLD ? qbase : 0);
  int s_row = 4 * (8 * g + (FOLD ? 32 * NSUB * qh : 0));
  auto a_at = [&](int cc) { return row_off(std::integral_constant<int, QSW>{}, a_off, cc); };
  // seed rows r .. r + 3 (r a compile-time multiple of 4) of a stage
  auto seed4 = [&](const float *arr, int r) {
    return *reinterpret_cast<const floatx4 *>(reinterpret_cast<const char *>(arr + sw) + s_row + 4 * r);
  };

  if (n_tiles > 0) load_tile(cur_h, cur_m0, std::integral_constant<int, 0>{});
  __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): K, V and the first tile resident
  if constexpr (T::KV_LDS) {
    // K scaled in place once every wave's part of it has landed, each
    // thread its 16-byte chunks; the barrier below publishes the result
    __syncthreads();
    if (kmul != 1.0f) {
#pragma unroll
      for (int ch = tid; ch < T::LDS_KV / 8; ch += T::NT) {   // padding too
        vec8<E> x = ld8<E>(s_k + 8 * ch);
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = (E)((float)x[j] * kmul);
        *reinterpret_cast<vec8<E> *>(s_k + 8 * ch) = x;
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) kf[c][j] = (E)((float)kf[c][j] * kmul);
  }
  if (n_tiles > 0) store_tile(std::integral_constant<int, 0>{});
  __syncthreads();

  // ||V_k||_1 of this lane's key (its half row and lane ^ 32's): sign bits
  // cleared two values at a time, pairs summed by v_dot2 against (1, 1)
  float nv = 0.0f;
#pragma unroll
  for (int cc = 0; cc < D / 16; ++cc) {
    const u32x4 x = __builtin_bit_cast(u32x4, v_frag(cc)) & 0x7fff7fffu;
#pragma unroll
    for (int j = 0; j < 4; ++j) nv = dot2_acc(__builtin_bit_cast(vec2<E>, x[j]), nv);
  }
  nv += xor32(nv);
  // A query tile's dS scale from the bound on its |dS| (the maxima loaded
  // with the tile): settled (and the dK accumulators rescaled by the
  // factor) only when some lane's scale must change -- a wave-uniform
  // branch, rarely taken once the sweep has found its range.  The first
  // tile's in the prologue, every later one's at the end of the tile
  // before it, where the check issues under that tile's last MFMAs.
  auto settle_scale = [&]() {
    // (non-negative: unsigned maxima of the bit patterns, scalar ops)
    unsigned mdo = __float_as_uint(nx_rm[0]), mdl = __float_as_uint(nx_rm[1]);
#pragma unroll
    for (int i = 1; i < BQ / 32; ++i) {
      mdo = max(mdo, __float_as_uint(nx_rm[2 * i]));
      mdl = max(mdl, __float_as_uint(nx_rm[2 * i + 1]));
    }
    const float bnd = __builtin_fmaf(__uint_as_float(mdo), nv, __uint_as_float(mdl));
    if (__any(sc.stale(bnd))) {
      const float f = sc.settle(bnd);
      if (__any(f != 1.0f)) {
#pragma unroll
        for (int d = 0; d < D / 32; ++d)
#pragma unroll
          for (int i = 0; i < 16; ++i) dk[d][i] *= f;
      }
    }
  };
  if (n_tiles > 0) settle_scale();   // the first tile's scale

  // One query tile; the LDS stage is a compile-time constant (the loop below
  // is unrolled by two) so every LDS address is a base plus an immediate.
  auto tile_step = [&](auto stc, int t) {
    constexpr int st = decltype(stc)::value;
    if constexpr (FOLD) {
      hide_offsets(std::integral_constant<int, QSW>{}, a_off);
      if constexpr (T::KV_LDS) hide_offsets(std::integral_constant<int, KVSW>{}, kv_off);
      t_off.hide();
      opaque<32>(s_row);
    }
    const int m0 = cur_m0;
    const bool more = t + 1 < n_tiles;
    int nxt_h = cur_h, nxt_m0 = cur_m0;
    advance(nxt_h, nxt_m0);
    if (more) {
      if (nxt_h != cur_h) {
        aim(nxt_h, nxt_m0);
      } else {
        cq.advance();
        cg.advance();
      }
      load_tile(nxt_h, nxt_m0, std::integral_constant<int, st ^ 1>{});
    }

    // 32-query sub-block sb of this wave: queries m0 + 32 * (NSUB*qh + sb)
    auto sub_m = [&](int sb) { return m0 + 32 * (NSUB * qh + sb); };
    // live: not entirely above this wave's keys' diagonal, not past Sq
    auto live = [&](int sb) {
      const int ms = sub_m(sb);
      return !(CAUSAL && ms + 31 + off < wk0) && ms < Sq;
    };
    // S = c_k Q K^T - LSE' and dP = dO V^T - delta for sub-block sb: the
    // accumulators start from the LDS seeds (slots 8hh + j hold rows
    // 32qs + 16hh + 8g + j; slot i <-> query ms + slot_row(i, g), lane <->
    // key).
    auto s_dp = [&](int sb, floatx16 &sacc, floatx16 &dpacc) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int r = 32 * sb + 16 * hh;
        const floatx4 l_lo = seed4(s_lse[st], r);
        const floatx4 l_hi = seed4(s_lse[st], r + 4);
        const floatx4 d_lo = seed4(s_dl[st], r);
        const floatx4 d_hi = seed4(s_dl[st], r + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          sacc[8 * hh + j] = l_lo[j];
          sacc[8 * hh + 4 + j] = l_hi[j];
          dpacc[8 * hh + j] = d_lo[j];
          dpacc[8 * hh + 4 + j] = d_hi[j];
        }
      }
      const f16 *qr = q_st(stc) + qw + lds_row<D, QSW>(32 * sb);
      const f16 *gr = do_st(stc) + qw + lds_row<D, QSW>(32 * sb);
#pragma unroll
      for (int cc = 0; cc < D / 16; ++cc) {
        sacc = mfma32(ld8_b<E>(qr, a_at(cc)), k_frag(cc), sacc);
        dpacc = mfma32(ld8_b<E>(gr, a_at(cc)), v_frag(cc), dpacc);
      }
    };
    // Softmax-gradient of sub-block sb and its dV / dK MFMAs.
    auto grad = [&](int sb, floatx16 &sacc, const floatx16 &dpacc) {
      const int ms = sub_m(sb);
      // Invisible scores become -inf (P = 0) in one pass, taken only by
      // diagonal and ragged sub-blocks, so the softmax below is branch-free.
      if ((CAUSAL && ms + off < wk0 + 31) || (ms + 31 >= Sq) || (wk0 + 31 >= Sk)) {
        // query ms + slot_row(i, g) sees this lane's key iff
        // lo <= slot_row(i, 0) < hi (nothing when the key is past Sk)
        const int base = ms + 8 * g;
        const int hi = key < Sk ? Sq - base : -(1 << 30);
        const int lo = CAUSAL ? key - off - base : -(1 << 30);
#pragma unroll
        for (int i = 0; i < 16; ++i)
          sacc[i] = (slot_row(i, 0) >= lo && slot_row(i, 0) < hi) ? sacc[i] : kNegInf;
      }
      if (cr != 1.0f) {
#pragma unroll
        for (int i = 0; i < 16; ++i) sacc[i] *= cr;
      }
      floatx16 p, ds;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        p[i] = fast_exp2(sacc[i]);
        ds[i] = p[i] * dpacc[i];
      }
      // dS in E at the tile's power-of-two scale
      vec8<E> pf[2], dsf[2];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        pf[i >> 3][i & 7] = (E)p[i];
        dsf[i >> 3][i & 7] = (E)(ds[i] * sc.mul);
      }
      // dV^T += dO^T P ; dK^T += Q^T dS   (k = queries ms + 16hh + 8g ..)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        // kperm rows 32qs + 16hh + 4g + (0..3) and +8: this 8-query slice
        const int rb = qw + lds_row<D, QSW>(32 * sb + 16 * hh);
#pragma unroll
        for (int d = 0; d < D / 32; ++d) {
          dv[d] = mfma32(load_tr_pair_b<E>(do_st(stc) + rb, t_off.lo(d), t_off.hi(d)), pf[hh], dv[d]);
          dk[d] = mfma32(load_tr_pair_b<E>(q_st(stc) + rb, t_off.lo(d), t_off.hi(d)), dsf[hh], dk[d]);
        }
      }
    };

    // One sub-block's S, dP, softmax gradient and dV / dK MFMAs as one block
    // in program order, so the VALU work issues under MFMAs it does not
    // depend on --
    //   S MFMAs;  dP MFMAs, with exp2 of S (P, rounded to E) between them;
    //   dV MFMAs (they need only P), with dS = P (dP - delta) between
    //   them;  dK MFMAs, with dS's scaled conversion between.
    // A MFMA runs ~32 cycles in the matrix pipe while the wave issues the
    // VALU slice after it; sched_barrier(0) keeps the compiler from
    // regrouping the slices.  Invisible scores (diagonal and ragged
    // sub-blocks only) get a -inf seed, so S is -inf and P = 0 there, as in
    // grad(); |sm_scale| > ln 2 scales S by cr before the exp2, as grad()
    // does.  Same operations on the same values as s_dp() + grad().
    auto sdp_grad = [&](int sb) {
      constexpr int NC = D / 16;          // S / dP MFMAs (K-dim chunks of 16)
      constexpr int NO = 2 * (D / 32);    // dV / dK MFMAs (2 query halves x D / 32)
      // operand reads this many MFMAs ahead (the non-causal D = 64 variant
      // would spill)
      constexpr int PFD = T::PF_OPS;
      constexpr int NM = 2 * NC + 2 * NO;
      floatx16 sacc, dpacc;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int r = 32 * sb + 16 * hh;
        const floatx4 l_lo = seed4(s_lse[st], r);
        const floatx4 l_hi = seed4(s_lse[st], r + 4);
        const floatx4 d_lo = seed4(s_dl[st], r);
        const floatx4 d_hi = seed4(s_dl[st], r + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          sacc[8 * hh + j] = l_lo[j];
          sacc[8 * hh + 4 + j] = l_hi[j];
          dpacc[8 * hh + j] = d_lo[j];
          dpacc[8 * hh + 4 + j] = d_hi[j];
        }
      }
      const int ms = sub_m(sb);
      if ((CAUSAL && ms + off < wk0 + 31) || (ms + 31 >= Sq) || (wk0 + 31 >= Sk)) {
        // query ms + slot_row(i, g) sees this lane's key iff
        // lo <= slot_row(i, 0) < hi (nothing when the key is past Sk)
        const int base = ms + 8 * g;
        const int hi = key < Sk ? Sq - base : -(1 << 30);
        const int lo = CAUSAL ? key - off - base : -(1 << 30);
#pragma unroll
        for (int i = 0; i < 16; ++i)
          sacc[i] = (slot_row(i, 0) >= lo && slot_row(i, 0) < hi) ? sacc[i] : kNegInf;
      }
      const f16 *qr = q_st(stc) + qw + lds_row<D, QSW>(32 * sb);
      const f16 *gr = do_st(stc) + qw + lds_row<D, QSW>(32 * sb);
      const int rb0 = qw + lds_row<D, QSW>(32 * sb);
      // LDS operands of MFMA i of the block (S: Q and K^T; dP: dO and V^T;
      // dV: dO^T; dK: Q^T), in ring slot i % (PFD + 1)
      vec8<E> opa[PFD + 1], opb[PFD + 1];
      auto fetch = [&](auto ic) {
        constexpr int i = decltype(ic)::value;
        constexpr int sl = i % (PFD + 1);
        if constexpr (i < NC) {
          opa[sl] = ld8_b<E>(qr, a_at(i));
          opb[sl] = k_frag(i);
        } else if constexpr (i < 2 * NC) {
          opa[sl] = ld8_b<E>(gr, a_at(i - NC));
          opb[sl] = v_frag(i - NC);
        } else if constexpr (i < 2 * NC + NO) {
          constexpr int o = i - 2 * NC, hh = o / (D / 32), d = o % (D / 32);
          opa[sl] = load_tr_pair_b<E>(do_st(stc) + rb0 + lds_row<D, QSW>(16 * hh), t_off.lo(d),
                                    t_off.hi(d));
        } else {
          constexpr int o = i - 2 * NC - NO, hh = o / (D / 32), d = o % (D / 32);
          opa[sl] = load_tr_pair_b<E>(q_st(stc) + rb0 + lds_row<D, QSW>(16 * hh), t_off.lo(d),
                                    t_off.hi(d));
        }
      };
      // before MFMA i: the operands of MFMA i + PFD (PFD = 0: its own); at
      // D = 64 the dV / dK operand of MFMA i itself (reading those ahead
      // too spills a register there)
      auto ahead = [&](auto ic) {
        constexpr int i = decltype(ic)::value;
        if constexpr (T::PF_ALL) {
          if constexpr (i + PFD < NM) fetch(std::integral_constant<int, i + PFD>{});
        } else if constexpr (i < 2 * NC) {
          if constexpr (i + PFD < 2 * NC) fetch(std::integral_constant<int, i + PFD>{});
        } else {
          fetch(ic);
        }
      };
      static_for<PFD>([&](auto ic) { fetch(ic); });
      static_for<NC>([&](auto ic) {
        constexpr int cc = decltype(ic)::value;
        ahead(ic);
        sacc = mfma32(opa[cc % (PFD + 1)], opb[cc % (PFD + 1)], sacc);
      });
      if (cr != 1.0f) {
#pragma unroll
        for (int i = 0; i < 16; ++i) sacc[i] *= cr;
      }
      __builtin_amdgcn_sched_barrier(0);
      // dP MFMAs; exp2 of S in NC - 1 slices after the second one onwards
      // (S's last MFMA has finished by then)
      floatx16 p;
      vec8<E> pf[2];
      static_for<NC>([&](auto ic) {
        constexpr int cc = decltype(ic)::value, i = NC + cc;
        ahead(std::integral_constant<int, i>{});
        dpacc = mfma32(opa[i % (PFD + 1)], opb[i % (PFD + 1)], dpacc);
        if constexpr (cc >= 1) {
          constexpr int i0 = (cc - 1) * 16 / (NC - 1), i1 = cc * 16 / (NC - 1);
          static_for<i1 - i0>([&](auto kc) {
            constexpr int e = i0 + decltype(kc)::value;
            p[e] = fast_exp2(sacc[e]);
            pf[e >> 3][e & 7] = (E)p[e];
          });
        }
        __builtin_amdgcn_sched_barrier(0);
      });
      // dV^T += dO^T P, with dS = P dP (into p: P is needed as E only from
      // here on) in NO - 1 slices
      floatx16 &ds = p;
      static_for<NO>([&](auto io) {
        constexpr int o = decltype(io)::value, i = 2 * NC + o;
        constexpr int hh = o / (D / 32), d = o % (D / 32);
        ahead(std::integral_constant<int, i>{});
        dv[d] = mfma32(opa[i % (PFD + 1)], pf[hh], dv[d]);

        if constexpr (o >= 1) {
          constexpr int i0 = (o - 1) * 16 / (NO - 1), i1 = o * 16 / (NO - 1);
          static_for<i1 - i0>([&](auto kc) {
            constexpr int e = i0 + decltype(kc)::value;
            ds[e] *= dpacc[e];
          });
        }
        __builtin_amdgcn_sched_barrier(0);
      });
      // dK^T += Q^T dS, dS in E at the tile's power-of-two scale: each query half's 8 conversions before its MFMAs
      vec8<E> dsf[2];
      static_for<2>([&](auto ih) {
        constexpr int hh = decltype(ih)::value;
#pragma unroll
        for (int j = 0; j < 8; ++j) dsf[hh][j] = (E)(ds[8 * hh + j] * sc.mul);
        static_for<D / 32>([&](auto id) {
          constexpr int d = decltype(id)::value, i = 2 * NC + NO + hh * (D / 32) + d;
          ahead(std::integral_constant<int, i>{});
          dk[d] = mfma32(opa[i % (PFD + 1)], dsf[hh], dk[d]);
        });
        __builtin_amdgcn_sched_barrier(0);
      });
    };
    if constexpr (T::EARLY_S) {
      floatx16 sacc[NSUB], dpacc[NSUB];
#pragma unroll
      for (int sb = 0; sb < NSUB; ++sb)
        if (live(sb)) s_dp(sb, sacc[sb], dpacc[sb]);
#pragma unroll
      for (int sb = 0; sb < NSUB; ++sb)
        if (live(sb)) grad(sb, sacc[sb], dpacc[sb]);
    } else {
#pragma unroll
      for (int sb = 0; sb < NSUB; ++sb) {
        if (live(sb)) sdp_grad(sb);
      }
    }

    if (more) {
      settle_scale();   // tile t + 1's scale, under this tile's last MFMAs
      store_tile(std::integral_constant<int, st ^ 1>{});
    }
    cur_h = nxt_h;
    cur_m0 = nxt_m0;
    __syncthreads();
  };

  for (int t = 0; t < n_tiles; t += 2) {
    tile_step(std::integral_constant<int, 0>{}, t);
    if (t + 1 < n_tiles) tile_step(std::integral_constant<int, 1>{}, t + 1);
  }

  float dk_mul = a.sm_scale / sc.mul;
  if (T::NQH == 2) {
    // the loop's last barrier ordered every tile read before these writes
    const DsScale unit;
    if constexpr (T::NKG == 2) {
      merge_pair<D>(reinterpret_cast<float *>(kg ? s_q1 : s_q0), qh == 1, dk, sc, lane);
      merge_pair<D>(reinterpret_cast<float *>(kg ? s_do1 : s_do0), qh == 1, dv, unit, lane);
    } else {
      // four key groups: one stage buffer each, dK then (once every reader
      // is done) dV
      f16 *buf = kg == 0 ? s_q0 : (kg == 1 ? s_q1 : (kg == 2 ? s_do0 : s_do1));
      merge_pair<D>(reinterpret_cast<float *>(buf), qh == 1, dk, sc, lane);
      __syncthreads();
      merge_pair<D>(reinterpret_cast<float *>(buf), qh == 1, dv, unit, lane);
    }
    if constexpr (T::KEY_SPLIT && CAUSAL) {
      if (split) {
        split_finish<E, D, T::NKG>(a, dk, dv, bhk * nsplit + kt, seg, qh == 0, kg * 64 + lane,
                                  key < Sk,
                                  a.dk + b * a.dk_sb + hk * a.dk_sh + (int64_t)key * a.dk_ss,
                                  a.dv + b * a.dv_sb + hk * a.dv_sh + (int64_t)key * a.dv_ss, g);
        return;
      }
    }
    if (qh == 1) return;
    dk_mul = a.sm_scale;
  }
  if (key < Sk) {
    store_row<E, D>(a.dk + b * a.dk_sb + hk * a.dk_sh + (int64_t)key * a.dk_ss, dk, dk_mul, g);
    store_row<E, D>(a.dv + b * a.dv_sb + hk * a.dv_sh + (int64_t)key * a.dv_ss, dv, 1.0f, g);
  }
}

template <typename E, int D, bool CAUSAL, int SPLIT>
__global__ __launch_bounds__((DkdvTile<D, SPLIT>::NT))
__attribute__((amdgpu_waves_per_eu(DkdvTile<D, SPLIT>::WAVES_PER_EU))) void fa_bwd_dkdv_kernel(
    BwdArgs a) {
  using T = DkdvTile<D, SPLIT>;
  FA_DKDV_LDS(T);
  dkdv_block<E, D, CAUSAL, SPLIT>(a, blockIdx.x, s_q0, s_q1, s_do0, s_do1, s_lse, s_dl, s_k, s_v);
}

// ---------------------------------------------------------------------------
// dQ: workgroup = 4 waves.  SPLIT = 1: wave w owns 32 queries (BM = 128)
// and both 32-key sub-blocks of every 64-key tile.  SPLIT = 2: wave w owns
// query group qg = w / 2 (BM = 64) and key half kh = w % 2 of every tile;
// the two key halves of a query group merge their dQ partial sums through
// LDS at the end.  Key tiles of BN = 64 rows stream through double-buffered
// LDS as K and V (kperm row order).  (The dK/dV kernel's 128-row tiles with
// early S/dP issue measured 12 % slower here: the second score set costs
// the third wave per SIMD.)
template <int D, int SPLIT, int NW = 4>
struct DqTile {
  static_assert(SPLIT == 1 || SPLIT == 2, "split is 1 or 2");
  static_assert(NW == 4 || (NW == 8 && D >= 64), "eight waves need D >= 64");
  static constexpr int NQG = NW / SPLIT;   // query groups of 32
  static constexpr int NSUB = 2 / SPLIT;
  static constexpr int BM = 32 * NQG;
  static constexpr int BN = 64;
  static constexpr int NT = 64 * NW;
  static constexpr int LDS_TILE = BN * D;   // swizzled, unpadded (fa_common.hpp)
  static_assert(64 * (D / 2) * 4 <= LDS_TILE * 2, "a merge buffer must fit in one K stage");
};

// PRE (fp16 with c <= 1, chosen by the launcher): Q is scaled by c once and
// rounded to fp16, as in the forward's pre-scaled mode, and the S^T MFMAs
// start from -LSE * log2(e), so they produce c s - LSE' and P is one exp2
// per score, no FMA.
// NW = 8 (non-causal grids, chosen by the launcher): twice the query groups
// share each K / V tile.
// One dQ block (workgroup `bid` of the dQ grid) on four LDS stages of at
// least DqTile::LDS_TILE elements each: K and V, double-buffered (one LDS
// object per stage, as in the dK/dV block).
template <typename E, int D, bool CAUSAL, int SPLIT, bool PRE, int NW>
__device__ __forceinline__ void dq_block(const BwdArgs &a, const int bid, f16 *s_k0, f16 *s_k1,
                                         f16 *s_v0, f16 *s_v1) {
  static_assert(!PRE || std::is_same<E, f16>::value, "the pre-scaled mode is fp16 only");
  using T = DqTile<D, SPLIT, NW>;
  constexpr int BM = T::BM, BN = T::BN, NSUB = T::NSUB;
  auto k_st = [&](auto stc) -> f16 * { return decltype(stc)::value ? s_k1 : s_k0; };
  auto v_st = [&](auto stc) -> f16 * { return decltype(stc)::value ? s_v1 : s_v0; };

  const int Sq = a.Sq, Sk = a.Sk, off = a.off;
  const int BH = a.B * a.H;
  // zero the split counters of the dK/dV launch that follows on the stream
  if (a.cnt_zero != nullptr && bid == 0) {
    for (int i = threadIdx.x; i < a.n_cnt_zero; i += T::NT) a.cnt_zero[i] = 0u;
  }
  const int bh = bid % BH;
  const int rank = bid / BH;
  // Causal: late query blocks are the heavy ones; order chosen by the
  // launcher as in the forward kernel.  With the query-block split, ranks
  // 2j and 2j + 1 are the two halves of the j-th heaviest block, then the
  // unsplit blocks follow, heaviest first.
  const int nsplit = CAUSAL ? a.dq_split : 0;
  const bool split = rank < 2 * nsplit;
  const int seg = split ? (rank & 1) : 0;
  const int qt = !CAUSAL ? rank
                 : a.n_blocks - 1 -
                       (split ? (rank >> 1)
                              : (nsplit > 0 ? rank - nsplit
                                            : (a.zigzag ? zigzag_rank(rank, a.n_blocks) : rank)));
  const int b = bh / a.H, h = bh % a.H;
  const int hk = h / a.grp;
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int qg = SPLIT == 2 ? (w >> 1) : w;
  const int kh = SPLIT == 2 ? (w & 1) : 0;
  const int g = lane >> 5, l32 = lane & 31;
  const int q0 = qt * BM;
  const int wq0 = q0 + 32 * qg;
  const int qrow = wq0 + l32;

  const f16 *kb = a.k.head(b, hk);
  const f16 *vb = a.v.head(b, hk);

  vec8<E> qf[D / 16], gf[D / 16];
  load_row_frags<E, D>(qf, a.q.head(b, h), a.q.ss, qrow, Sq, g);
  load_row_frags<E, D>(gf, a.dout.head(b, h), a.dout.ss, qrow, Sq, g);

  int kv_end = Sk;
  if (CAUSAL) kv_end = min(Sk, q0 + BM + off);
  // 0 when every query of the block precedes every key (causal, Sq > Sk)
  const int n_tiles = kv_end > 0 ? (kv_end + BN - 1) / BN : 0;
  // key tiles [t_lo, t_hi) of this workgroup: a split block's segment 0
  // takes the first half, segment 1 the rest
  const int t_lo = seg ? n_tiles / 2 : 0;
  const int t_hi = (split && seg == 0) ? n_tiles / 2 : n_tiles;
  const float c = a.c;

  // K and V tiles go straight to LDS (fa_common.hpp DmaStager).
  DmaStager<D, SW_AT, BN, NW> stk, stv;
  stk.init(w, lane, a.k.ss);
  stv.init(w, lane, a.v.ss);
  auto load_tile = [&](int n0, auto stc) {
    stk.load(k_st(stc), kb, a.k.ss, n0, Sk, w);
    stv.load(v_st(stc), vb, a.v.ss, n0, Sk, w);
  };
  // the loop loads tile t + 1 during tile t: cursors from tile t_lo + 1,
  // advanced by a tile per load
  RowCursor ck, cv;
  ck.init(kb, a.k.ss, (t_lo + 1) * BN, Sk, D, BN);
  cv.init(vb, a.v.ss, (t_lo + 1) * BN, Sk, D, BN);
  auto load_next = [&](auto stc) {
    stk.load(k_st(stc), ck.rsrc(), w);
    stv.load(v_st(stc), cv.rsrc(), w);
    ck.advance();
    cv.advance();
  };

  // the first key tile's DMA overlaps the row loads and the work below
  if (t_hi > t_lo) load_tile(t_lo * BN, std::integral_constant<int, 0>{});

  if (a.neg) {
#pragma unroll
    for (int c = 0; c < D / 16; ++c) qf[c] = neg8(qf[c]);
  }
  if constexpr (PRE) {
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) qf[c][j] = (E)((float)qf[c][j] * a.c);
  }
  const int qc = min(qrow, Sq - 1);
  const float l2 = qrow < Sq ? a.lse[(int64_t)bh * Sq + qc] * kLog2e : kPosInf;
  float dl;
  if (a.delta_out != nullptr) {
    // delta = rowsum(O * dO) from the lane's half row and its lane ^ 32
    // partner's (the pre-pass, folded in); the dK/dV kernel reads it later
    vec8<E> of[D / 16];
    load_row_frags<E, D>(of, a.o.head(b, h), a.o.ss, qrow, Sq, g);
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc = __builtin_fmaf((float)of[c][j], (float)gf[c][j], acc);
    acc += xor32(acc);
    dl = qrow < Sq ? acc : 0.0f;
    if (qrow < Sq && g == 0 && kh == 0 && seg == 0) a.delta_out[(int64_t)bh * Sq + qrow] = dl;
  } else {
    dl = qrow < Sq ? a.delta[(int64_t)bh * Sq + qc] : 0.0f;
  }

  // Power-of-two scale 2^e of this query's dS, fixed for the whole sweep:
  // the lane's dO row is scaled so that its largest |value| lies in
  // [2^-4, 2^-3) (exact: a power of two that cannot overflow), and delta
  // with it, so the MFMAs below produce dS * 2^e directly.  Then
  // |dS * 2^e| <= P (|dO' . V| + |delta'|) <= 2^-2 D max|V|, far inside
  // fp16 for any sane V, while dO ~ 1e-6 (fp16 subnormals) still yields dS
  // well above fp16's subnormal range.  dQ is unscaled at the store.
  float gm = 0.0f;
#pragma unroll
  for (int c = 0; c < D / 16; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) gm = fmaxf(gm, fabsf((float)gf[c][j]));
  gm = max_xor32(gm);   // the row's other half is in lane ^ 32
  if (a.rmax_out != nullptr && kh == 0 && seg == 0) {
    // the wave's 32 rows' group maxima, beside delta (BwdArgs::rmax); the
    // two lane halves hold the same rows (the low half's maxima end in
    // lane 31), rows past Sq contribute 0
    const unsigned dm = max_halves_nonneg(qrow < Sq ? gm : 0.0f);
    const unsigned am = max_halves_nonneg(fabsf(dl));
    if (lane == 31 && wq0 < Sq) {
      float *p = a.rmax_out + ((int64_t)bh * row_groups(a.Sq) + wq0 / 32) * 2;
      p[0] = __uint_as_float(dm);
      p[1] = __uint_as_float(am);
    }
  }
  int ge = 0;
  if (gm > 0.0f && gm < kPosInf) {
    ge = -3 - __builtin_amdgcn_frexp_expf(gm);
    ge = ge > 126 ? 126 : (ge < -126 ? -126 : ge);
  }
  const float gmul = __builtin_amdgcn_ldexpf(1.0f, ge);
#pragma unroll
  for (int c = 0; c < D / 16; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) gf[c][j] = (E)((float)gf[c][j] * gmul);

  floatx16 dq[D / 32];
#pragma unroll
  for (int d = 0; d < D / 32; ++d) dq[d] = floatx16{};
  const float shift = -l2;   // P = exp2(c s - LSE * log2(e))
  // dP^T MFMAs start from -delta (the lane's query), so they yield dP - delta
  floatx16 dl_seed, s_seed;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    dl_seed[i] = -dl * gmul;
    s_seed[i] = PRE ? shift : 0.0f;
  }

  // Per-lane LDS byte offsets inside a stage (as in the dK/dV kernel):
  // A-operand rows l32, chunk 2cc + g; transposed reads of K rows
  // 4g + (l16 >> 2); both carrying the wave's first key row in the tile
  // (32 * NSUB * kh) and hidden from loop-invariant code motion at every
  // step (fa_common.hpp opaque()).
  const int wrow = 32 * NSUB * kh * D;
  int a_off[D / 16];
  TrOffsetsB<D, SW_AT> t_off;
  {
    const int sa = swz<D, SW_AT>(l32);
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc)
      a_off[cc] = 2 * (wrow + l32 * D + (((2 * cc + g) ^ sa) << 3));
    t_off.init(lane, wrow);
  }

  __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): rows, LSE, delta and the first tile resident
  __syncthreads();

  auto tile_step = [&](auto stc, int t) {
    constexpr int st = decltype(stc)::value;
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc) opaque<16>(a_off[cc]);
    t_off.hide();
    const int n0 = t * BN;
    const bool more = t + 1 < t_hi;
    if (more) load_next(std::integral_constant<int, st ^ 1>{});   // tile t + 1

    // 32-key sub-block sb of this wave: keys n0 + 32 * (NSUB*kh + sb)
    auto sub_n = [&](int sb) { return n0 + 32 * (NSUB * kh + sb); };
    auto live = [&](int sb) {
      const int ns = sub_n(sb);
      return !(CAUSAL && ns > wq0 + 31 + off) && ns < Sk;
    };
    // S^T = K Q^T (PRE: c s - LSE') and dP^T = V dO^T for sub-block sb
    auto s_dp = [&](int sb, floatx16 &sacc, floatx16 &dpacc) {
      const f16 *kr = k_st(stc) + 32 * sb * D;
      const f16 *vr = v_st(stc) + 32 * sb * D;
      sacc = mfma32(ld8_b<E>(kr, a_off[0]), qf[0], s_seed);
      dpacc = mfma32(ld8_b<E>(vr, a_off[0]), gf[0], dl_seed);
#pragma unroll
      for (int cc = 1; cc < D / 16; ++cc) {
        sacc = mfma32(ld8_b<E>(kr, a_off[cc]), qf[cc], sacc);
        dpacc = mfma32(ld8_b<E>(vr, a_off[cc]), gf[cc], dpacc);
      }
    };
    auto grad = [&](int sb, floatx16 &sacc, const floatx16 &dpacc) {
      const int ns = sub_n(sb);
      // invisible scores -> -inf (P = 0), diagonal / ragged sub-blocks only
      if ((CAUSAL && ns + 31 > wq0 + off) || (ns + 31 >= Sk)) {
        // key ns + slot_row(i, g) is visible iff slot_row(i, 0) <= lim
        int lim = Sk - 1;
        if (CAUSAL) lim = min(lim, qrow + off);
        lim -= ns + 8 * g;
#pragma unroll
        for (int i = 0; i < 16; ++i) sacc[i] = slot_row(i, 0) <= lim ? sacc[i] : kNegInf;
      }
      // dpacc holds (dP - delta) * 2^e, so ds is dS * 2^e
      floatx16 ds;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float p = PRE ? fast_exp2(sacc[i]) : fast_exp2(__builtin_fmaf(sacc[i], c, shift));
        ds[i] = p * dpacc[i];
      }
      vec8<E> dsf[2];
#pragma unroll
      for (int i = 0; i < 16; ++i) dsf[i >> 3][i & 7] = (E)ds[i];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        // kperm rows 32(NSUB kh + sb) + 16hh + 4g + (0..3) and +8: this
        // 8-key slice
        const int rb = (32 * sb + 16 * hh) * D;
#pragma unroll
        for (int d = 0; d < D / 32; ++d)
          dq[d] = mfma32(load_tr_pair_b<E>(k_st(stc) + rb, t_off.lo(d), t_off.hi(d)), dsf[hh], dq[d]);
      }
    };

#pragma unroll
    for (int sb = 0; sb < NSUB; ++sb) {
      if (!live(sb)) continue;
      floatx16 sacc, dpacc;
      s_dp(sb, sacc, dpacc);
      grad(sb, sacc, dpacc);
    }

    if (more) __builtin_amdgcn_s_waitcnt(0x0f70);   // this wave's DMAs of the next stage
    __syncthreads();
  };

  for (int t = t_lo; t < t_hi; t += 2) {
    tile_step(std::integral_constant<int, 0>{}, t);
    if (t + 1 < t_hi) tile_step(std::integral_constant<int, 1>{}, t + 1);
  }

  const float dq_mul = a.sm_scale / gmul;
  if (SPLIT == 2) {
    // the loop's last barrier ordered every tile read before these writes;
    // both key halves of a query carry the same scale
    // one K / V stage buffer per query group (up to four)
    f16 *buf = qg == 0 ? s_k0 : (qg == 1 ? s_k1 : (qg == 2 ? s_v0 : s_v1));
    merge_pair<D>(reinterpret_cast<float *>(buf), kh == 1, dq, DsScale{}, lane);
    if (kh == 1) return;
  }
  if (split) {
    // this segment's scaled fp32 rows; the dK/dV kernel adds the halves
    const int slot = bh * nsplit + qt - (a.n_blocks - nsplit);
    store_row_f32<D>(a.dq_part + ((int64_t)(slot * 2 + seg) * BM + (qrow - q0)) * D, dq, dq_mul, g);
    return;
  }
  if (qrow < Sq)
    store_row<E, D>(a.dq + b * a.dq_sb + h * a.dq_sh + (int64_t)qrow * a.dq_ss, dq, dq_mul, g);
}

template <typename E, int D, bool CAUSAL, int SPLIT, bool PRE = false, int NW = 4>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(D <= 64 ? 3 : 1)))
void fa_bwd_dq_kernel(BwdArgs a) {
  using T = DqTile<D, SPLIT, NW>;
  __shared__ __attribute__((aligned(16))) f16 s_k0[T::LDS_TILE], s_k1[T::LDS_TILE];
  __shared__ __attribute__((aligned(16))) f16 s_v0[T::LDS_TILE], s_v1[T::LDS_TILE];
  dq_block<E, D, CAUSAL, SPLIT, PRE, NW>(a, blockIdx.x, s_k0, s_k1, s_v0, s_v1);
}

// ---------------------------------------------------------------------------
// Fused backward (causal; four-wave blocks at D <= 64, the eight-wave dK/dV
// layout with eight-wave dQ blocks at D = 128): the dK/dV blocks and the dQ blocks of
// one backward in one grid -- workgroups [0, n_kv) run dkdv_block with
// `akv`, the rest dq_block with `aq` -- so that the dQ blocks, dispatched
// after every dK/dV block, fill the slots the causal sweeps of unequal
// length leave idle, and no kernel boundary drains the GPU between the
// two.  Both read only the inputs, delta and the row-group maxima (the
// pre-pass computes them and zeroes the key-block split's counters first)
// and write disjoint outputs,
// so no workgroup waits for another.  The dQ blocks run in the dK/dV
// blocks' four tile stages.
template <typename E, int D, bool CAUSAL, int KVSPLIT, int QSPLIT, bool PRE>
__global__ __launch_bounds__((DkdvTile<D, KVSPLIT>::NT))
__attribute__((amdgpu_waves_per_eu(D <= 64 ? 3 : 2)))
void fa_bwd_fused_kernel(BwdArgs akv, BwdArgs aq, int n_kv) {
  using T = DkdvTile<D, KVSPLIT>;
  using Q = DqTile<D, QSPLIT, T::NW>;
  static_assert(T::NT == Q::NT, "both blocks take the same waves");
  static_assert(D <= 64 ? T::NW == 4 : T::WIDE, "four-wave blocks at D <= 64, eight at D = 128");
  static_assert(T::LDS_TILE >= Q::LDS_TILE, "a dQ stage fits in a dK/dV tile stage");
  FA_DKDV_LDS(T);
  const int bid = blockIdx.x;
  if (bid < n_kv)
    dkdv_block<E, D, CAUSAL, KVSPLIT>(akv, bid, s_q0, s_q1, s_do0, s_do1, s_lse, s_dl, s_k, s_v);
  else
    dq_block<E, D, CAUSAL, QSPLIT, PRE, T::NW>(aq, bid - n_kv, s_q0, s_q1, s_do0, s_do1);
}

}  // namespace fa
