// fa_fwd.hpp -- forward FlashAttention kernel for gfx950.
//
// Computes, for one (query tile, batch*head), O = softmax(c * Q K^T) V with an
// online (streaming) softmax over key tiles, fp16 or bf16 (E) MFMA with fp32
// accumulation, and the natural-log row LSE.  Behaviour follows the reference forward
// (flash_attn_volta/triton_fa.py:63-159): causal tiles above the diagonal are
// skipped (:110-117), masked scores are -inf (:123-126), O = acc / l
// (:146-150) and LSE = m + ln(l), +inf when a row saw no key (:152-159).
//
// MI355X layout of the work:
//   * workgroup = 4 waves over 64 queries of one (b, h): 2 query groups of
//     32 x 2 key halves of every tile, merged at the end (see the kernel);
//   * key/value tiles of BN = 64 rows stream through LDS.  K lives in a
//     2-slot ring one tile ahead of V (2-slot ring), so the S^T MFMAs of
//     tile t+1 are issued before the softmax of tile t and run under it;
//   * K and V tiles go from global memory straight into LDS (buffer loads
//     with the LDS-direct bit: no VGPRs hold tile data), 32-row blocks in
//     kperm order and 16-byte chunks XOR-swizzled per row, so every lane's
//     K A-operand read is a conflict-free 16-byte ds_read of LDS row
//     (lane % 32), and the V^T operand of O^T = V^T P^T is read with
//     ds_read_b64_tr_b16 (fa_common.hpp);
//   * the wave's Q fragment stays in registers for the whole sweep;
//   * a lane owns one query row: the running max / sum and the O^T
//     accumulator column live in that lane, the only cross-lane step is one
//     v_permlane32_swap per key half when a row max is taken;
//   * probabilities are rounded to E once and the row sum accumulates
//     those rounded values (v_dot2_f32_f16), so numerator and denominator
//     see the same weights;
//   * most tiles take no row max at all: probabilities are computed against
//     the running max, and the lane's sum of them (an upper bound of each,
//     since p >= 0) proves them inside fp16 when it is <= kFastSum; only
//     the first tile with a visible key and tiles whose scores outgrow the
//     running max by more than log2 kFastSum take the max, rescale and
//     recompute.  The final O and LSE use the same max, so the result is
//     exact either way;
//   * the tile loads use raw buffer descriptors whose extent ends at row
//     Sk-1, so rows past the end read as zeros without any branch (they only
//     ever meet -inf scores); the Q row index is clamped (never stored).
#pragma once

#include "fa_common.hpp"

namespace fa {

// Bound on a lane's per-tile sum of probabilities taken against a stale
// running max (so every probability is <= 2^15, inside fp16's range).
constexpr float kFastSum = 32768.0f;

struct FwdArgs {
  TensorDesc q, k, v;  // q: (B, Sq, H, D); k, v: (B, Sk, Hk, D)
  f16 *o;              // (B, Sq, H, D)
  int64_t o_sb, o_ss, o_sh;
  float *lse;          // (B, H, Sq) or nullptr
  int B, Sq, Sk, H;
  int grp;             // query heads per key/value head (H / Hk)
  int off;             // causal: query i sees keys j <= i + off (off = Sk - Sq)
  int n_qtiles;
  float c;             // |sm_scale| * log2(e), clamped away from 0
  int neg;             // 1 when sm_scale < 0: Q is negated on load
  int zigzag;          // causal tile order: 1 zigzag heavy / light, 0 heaviest first
  // split-KV mode only (fa_fwd_kernel<..., SPLITKV = true>):
  int kv_split;        // keys per split, a multiple of the 64-key tile
  float *part_o;       // (n_splits, B, H, Sq, D) fp32: each split's normalised O
  float *part_lse;     // (n_splits, B, H, Sq) fp32: each split's LSE in log2 units
  // The balanced causal mode (BAL = true) writes its split tiles' halves to
  // part_o / part_lse as (2, B, H, n_qtiles / 2, BM, D) and (2, B, H,
  // n_qtiles / 2, BM): half, (b, h), pair, row in the tile.
};

// Key tiles (BN keys each) that query tile qt of BM rows sees under the
// causal mask: keys up to the tile's last row + off, at most Sk.
__device__ __forceinline__ int causal_tiles_of(int Sk, int off, int qt, int BM, int BN) {
  const int e = min(Sk, qt * BM + BM + off);
  return e > 0 ? (e + BN - 1) / BN : 0;
}

// Balanced causal schedule (fa_fwd_kernel<..., BAL = true>), for square
// causal grids (Sq == Sk, 64-row tiles: query tile i sees n(i) = i + 1 key
// tiles).  Tiles pair up light with heavy -- i = p and j = nb - 1 - p for
// pair p -- and each pair's n(i) + n(j) = nb + 1 key tiles are cut in
// three work items of one segment each:
//   X: heavy tile j, key tiles [0, hx), hx = ceil((nb + 1) / 2);
//   Y: heavy tile j, key tiles [hx, n(j)) (empty, and X whole, when
//      n(j) <= hx);
//   Z: light tile i, all its key tiles.
// X and Y write tile j's two halves as partial results (slot (b, h, p),
// half 0 and 1) that fa_fwd_combine_kernel merges.  With nb odd, the middle
// tile (n = (nb + 1) / 2 key tiles) is one more item.  Items are ordered by
// size, largest first -- every X (hx), the middle tile, then Y and Z
// alternating as their sizes fall (Z of pair np - 1 - k, then Y of pair k)
// -- and the grid is rank-major (workgroup = rank * B * H + (b, h)), so
// each freed workgroup slot takes the largest item left: every slot ends
// within about one item of the average instead of on the heaviest tile.
struct BalItem {
  int qt, t0, t1, part;   // tile qt, key tiles [t0, t1), partial slot * 2 + half or -1
};

__device__ __forceinline__ bool bal_split(int ni, int nj, int &hx) {
  hx = min((ni + nj + 1) >> 1, nj);
  return hx > 0 && hx < nj;
}

__device__ __forceinline__ BalItem fa_fwd_bal_item(const FwdArgs &a, int u, int bh, int BM,
                                                   int BN) {
  const int nb = a.n_qtiles, np = nb >> 1, odd = nb & 1;
  BalItem it{0, 0, 0, -1};
  int p, kind;   // kind 0: X, 1: Y, 2: Z
  if (u < np) {
    p = u;
    kind = 0;
  } else if (odd && u == np) {
    it.qt = np;   // the middle tile, whole
    it.t1 = causal_tiles_of(a.Sk, a.off, np, BM, BN);
    return it;
  } else {
    const int r = u - np - odd, k = r >> 1;
    p = (r & 1) ? k : np - 1 - k;
    kind = (r & 1) ? 1 : 2;
  }
  const int i = p, j = nb - 1 - p;
  const int ni = causal_tiles_of(a.Sk, a.off, i, BM, BN);
  const int nj = causal_tiles_of(a.Sk, a.off, j, BM, BN);
  int hx;
  const bool split = bal_split(ni, nj, hx);
  const int slot = bh * np + p;
  if (kind == 0) {
    it.qt = j;
    it.t1 = split ? hx : nj;
    it.part = split ? 2 * slot : -1;
  } else if (kind == 1) {
    it.qt = split ? j : -1;   // -1: nothing to do
    it.t0 = hx;
    it.t1 = nj;
    it.part = 2 * slot + 1;
  } else {
    it.qt = i;
    it.t1 = ni;
  }
  return it;
}

// Work items per (b, h) of the balanced schedule: three per pair, one more
// for an odd middle tile.
__host__ __device__ constexpr int bal_items(int nb) { return 3 * (nb >> 1) + (nb & 1); }

template <int D, int KSPLIT, int NW = 4>
struct FwdTile {
  static_assert(KSPLIT == 1 || KSPLIT == 2 || KSPLIT == 4, "key split is 1, 2 or 4");
  static_assert(NW == 4 || (NW == 8 && D >= 64), "eight waves need D >= 64");
  static_assert(NW % KSPLIT == 0, "every query group takes all key parts");
  static constexpr int NQG = NW / KSPLIT;  // query groups of 32 per workgroup
  static constexpr int NSUB = KSPLIT == 1 ? 2 : 1;   // 32-key sub-blocks per wave per tile
  static constexpr int BM = 32 * NQG;      // queries per workgroup
  static constexpr int BN = 32 * NSUB * KSPLIT;   // keys per tile: 64, or 128 with four parts
  static constexpr int NT = 64 * NW;       // NW waves
  static constexpr int LDS_TILE = BN * D;  // swizzled, unpadded (fa_common.hpp)
  // O^T partial sums of a key-part wave handed over for the final merge:
  // one buffer per (query group, key part > 0), in the four K / V slots
  // (one per slot with two parts, two per slot with four)
  static constexpr int MERGE_FLOATS = 64 * (D / 2);
  static constexpr int MERGE_PER_SLOT = KSPLIT == 4 ? 2 : 1;
  static_assert(MERGE_FLOATS * 4 * MERGE_PER_SLOT <= LDS_TILE * 2, "merge buffers must fit a slot");
  static_assert(NQG * (KSPLIT - 1) <= 4 * MERGE_PER_SLOT, "the merge buffers must fit the slots");
};

// Workgroup = NW waves (4 or 8).  KSPLIT = 1: each wave owns 32 queries
// and both 32-key halves of every 64-key tile.  KSPLIT = 2: wave w owns
// query group qg = w / 2 and key half kh = w % 2 of every tile; each wave
// runs its own online softmax over its key half and the two halves of a
// query group merge through LDS at the end (lane l of both waves holds the
// same query and the same O^T rows, so the merge is element-wise).
// KSPLIT = 4: 128-key tiles, wave w owns query group w / 4 and the 32-key
// quarter w % 4 of every tile; the quarters merge the same way.  Splitting
// keys divides each wave's work per tile and multiplies the waves in
// flight: it pays when the grid is too small to fill the GPU, and for
// causal attention, whose last query tile walks every key tile.  The
// launcher picks KSPLIT from the grid size.
//
// SPLITKV (decode against a long cache): the rows of a tile are the
// (query position, query head) pairs of one key/value head's group, row
// r = position * grp + head-in-group, so the group's heads share each K/V
// tile; blockIdx.y selects a range of kv_split keys, and the workgroup
// writes its rows' normalised O and log2-domain LSE over that range to
// part_o / part_lse, which fa_fwd_combine_kernel merges.
template <typename E, int D, bool CAUSAL, int KSPLIT, bool SPLITKV = false, bool PRE = false,
          bool BAL = false, int NW = 4>
__global__ __launch_bounds__(64 * NW) void fa_fwd_kernel(FwdArgs a) {
  static_assert(!PRE || std::is_same<E, f16>::value, "the pre-scaled mode is fp16 only");
  static_assert(!BAL || (CAUSAL && !SPLITKV), "the balanced schedule is for causal grids");
  static_assert(KSPLIT <= 2 || (!BAL && !SPLITKV), "four key parts: the plain schedule only");
  using T = FwdTile<D, KSPLIT, NW>;
  constexpr int NSUB = T::NSUB;
  constexpr int BM = T::BM, BN = T::BN;
  // One LDS object per slot, so the compiler sees that a DMA into one slot
  // cannot alias reads of another and does not wait for it early.
  __shared__ __attribute__((aligned(16))) f16 sk0[T::LDS_TILE], sk1[T::LDS_TILE];
  __shared__ __attribute__((aligned(16))) f16 sv0[T::LDS_TILE], sv1[T::LDS_TILE];
  // merge: m, l per query group (key-split layouts)
  __shared__ __attribute__((aligned(16))) float s_ml[KSPLIT >= 2 ? T::NQG * (KSPLIT - 1) : 1][2][64];
  auto k_sl = [&](auto sc) -> f16 * { return decltype(sc)::value ? sk1 : sk0; };
  auto v_sl = [&](auto sc) -> f16 * { return decltype(sc)::value ? sv1 : sv0; };

  const int Sq = a.Sq;
  const int grp = a.grp;
  // (b, h) pairs, or (b, key/value head) pairs in split-KV mode
  const int BH = SPLITKV ? a.B * (a.H / grp) : a.B * a.H;
  const int bid = blockIdx.x;
  const int bh = bid % BH;
  // Causal: late query tiles are the heavy ones.  The launcher picks the
  // order: heaviest first when the grid takes several rounds of resident
  // workgroups (each freed slot then takes the heaviest tile left), zigzag
  // heavy / light when it fits one round (co-resident workgroups then share
  // a CU's time evenly).  Workgroups of one (b, h) are BH apart, so with
  // BH % 8 == 0 they land on one XCD and share its L2.
  //
  // BAL: the work item of rank bid / BH (fa_fwd_bal_item): query tile qt
  // against key tiles [t0, t1), into O or, part >= 0, into a partial.
  int qt, t0 = 0, t1 = 0, part = -1;
  if constexpr (BAL) {
    const BalItem it = fa_fwd_bal_item(a, bid / BH, bh, BM, BN);
    if (it.qt < 0) return;   // an empty half of a tile that runs whole
    qt = it.qt;
    t0 = it.t0;
    t1 = it.t1;
    part = it.part;
  } else {
    qt = (CAUSAL && !SPLITKV)
             ? a.n_qtiles - 1 - (a.zigzag ? zigzag_rank(bid / BH, a.n_qtiles) : bid / BH)
             : bid / BH;
  }
  const int hx = SPLITKV ? a.H / grp : a.H;
  const int b = bh / hx;
  const int h = SPLITKV ? 0 : bh % hx;               // SPLITKV: the head is per lane
  const int hk = SPLITKV ? bh % hx : h / grp;        // key/value head
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = wave_id();
  const int qg = w / KSPLIT;
  const int kh = w % KSPLIT;
  const int g = lane >> 5, l32 = lane & 31;
  const int q0 = qt * BM;
  const int wq0 = q0 + 32 * qg;   // first row of this wave
  const int qrow = wq0 + l32;     // row owned by this lane
  const int nrows = SPLITKV ? grp * Sq : Sq;
  // Query positions for the causal mask: the lane's, the wave's first and
  // last, the block's last (rows are positions, or position * grp + head).
  const int qpos = SPLITKV ? qrow / grp : qrow;
  const int wpos_lo = SPLITKV ? wq0 / grp : wq0;
  const int wpos_hi = SPLITKV ? (wq0 + 31) / grp : wq0 + 31;
  const int bpos_hi = SPLITKV ? min((q0 + BM - 1) / grp, Sq - 1) : q0 + BM - 1;

  // Key range of this workgroup: all keys, split blockIdx.y's, or (BAL)
  // key tiles [t0, t1)
  const int kbase = SPLITKV ? (int)blockIdx.y * a.kv_split : (BAL ? t0 * BN : 0);
  const int Sk = SPLITKV ? min(a.kv_split, a.Sk - kbase) : (BAL ? min(a.Sk, t1 * BN) - kbase : a.Sk);
  const int off = a.off - kbase;   // key j (relative) is visible to position i iff j <= i + off

  const f16 *kb = a.k.head(b, hk) + (int64_t)kbase * a.k.ss;
  const f16 *vb = a.v.head(b, hk) + (int64_t)kbase * a.v.ss;

  int kv_end = Sk;
  if (CAUSAL) kv_end = min(Sk, bpos_hi + 1 + off);
  // 0 when every query of the block precedes every key (causal, Sq > Sk)
  const int n_tiles = kv_end > 0 ? (kv_end + BN - 1) / BN : 0;

  // ---- K and V tiles go straight to LDS (fa_common.hpp DmaStager): both
  // in kperm row order, chunks swizzled; rows past Sk read as zeros.
  DmaStager<D, SW_A, BN, NW> stk;   // K: read only as A operands
  DmaStager<D, SW_T, BN, NW> stv;   // V: read only transposed
  stk.init(w, lane, a.k.ss);
  stv.init(w, lane, a.v.ss);
  auto load_k = [&](int n0, auto sc) { stk.load(k_sl(sc), kb, a.k.ss, n0, Sk, w); };
  // Iteration t loads K(t + 2) and V(t) (the prologue K(0), K(1) and, at
  // D = 128, V(0)):
  // cursors at those rows, each advanced by a tile per load (no per-tile
  // 64-bit multiplies).
  RowCursor ck, cv;
  ck.init(kb, a.k.ss, 2 * BN, Sk, D, BN);
  cv.init(vb, a.v.ss, 0, Sk, D, BN);
  auto load_k_next = [&](auto sc) {
    stk.load(k_sl(sc), ck.rsrc(), w);
    ck.advance();
  };
  auto load_v_next = [&](auto sc) {
    stv.load(v_sl(sc), cv.rsrc(), w);
    cv.advance();
  };

  // Per-lane LDS byte offsets inside a slot: K rows l32 (A operand of
  // S^T = K Q^T), chunk 2cc + g; V^T transpose reads of rows 4g + (l16 >> 2)
  // (and + 8), i.e. natural V rows 8g + (l16 >> 2) (and + 4).  Both carry
  // the wave's first key row in the tile (32 * NSUB * kh) and are hidden
  // from loop-invariant code motion at every step (fa_common.hpp opaque()),
  // so a read is one offset register plus an immediate (slot, sub-block).
  const int wrow = 32 * NSUB * kh * D;
  int a_off[D / 16];
  TrOffsetsB<D, SW_T> t_off;
  {
    const int sa = swz<D, SW_A>(l32);
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc)
      a_off[cc] = 2 * (wrow + l32 * D + (((2 * cc + g) ^ sa) << 3));
    t_off.init(lane, wrow);
  }
  auto hide_offsets = [&]() {
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc) opaque<16>(a_off[cc]);
    t_off.hide();
  };

  // Sub-block sb (32 keys) of this wave in the tile at n0 starts at key
  // n0 + 32 * (NSUB * kh + sb); it is dead when it lies entirely above the
  // wave's causal diagonal (the last key its last query sees is wq0+31+off).
  auto sub_key = [&](int n0, int sb) { return n0 + 32 * (NSUB * kh + sb); };
  auto dead = [&](int n0, int sb) { return CAUSAL && sub_key(n0, sb) > wpos_hi + off; };

  // Tiles that need no mask for this wave: every key of its part of the
  // tile (offsets up to kmax inside the tile) exists and, causal, is
  // visible to the wave's first query.  Such tiles form a prefix
  // [0, t_mask) of the sweep (masks only start at the diagonal or the
  // ragged end); the loop runs them through a branch-free body.
  int t_mask;
  {
    const int kmax = 32 * (NSUB * kh + NSUB) - 1;
    const int x = Sk - kmax;   // first tile t with t * BN + kmax >= Sk
    t_mask = x <= 0 ? 0 : (x + BN - 1) / BN;
    if (CAUSAL) {
      const int y = wpos_lo + off - kmax;   // first t with t * BN + kmax > wpos_lo + off
      t_mask = min(t_mask, y < 0 ? 0 : y / BN + 1);
    }
  }

  // ---- S^T = K Q^T for this wave's sub-blocks of a tile (dead sub-blocks
  // skipped when CHECK: the diagonal mask overwrites them)
  vec8<E> qf[D / 16];
  // PRE (fp16 with c <= 1, chosen by the launcher): Q is pre-scaled by c
  // once, rounded to fp16 as the reference's kernel pre-scales Q
  // (triton_fa.py:108; c <= 1 cannot overflow), and every S^T MFMA chain
  // starts from negm = -m instead of 0, so the MFMAs produce c*s - m
  // directly and the softmax is one v_exp_f32 per score.  Invariant: the
  // scores of a tile are relative to the running max m (or to 0 while m is
  // -inf).  Otherwise (bf16, whose 8-bit mantissa would make the extra
  // rounding visible, or c > 1) negm stays 0 and the softmax applies c in
  // an FMA.
  constexpr bool pre = PRE;
  floatx16 negm = {};
  auto qk = [&](auto sc, auto checkc, int n0, floatx16 (&s)[NSUB]) {
#pragma unroll
    for (int sb = 0; sb < NSUB; ++sb) {
      if (decltype(checkc)::value && dead(n0, sb)) continue;
      const f16 *kr = k_sl(sc) + 32 * sb * D;
      floatx16 acc = mfma32(ld8_b<E>(kr, a_off[0]), qf[0], negm);
#pragma unroll
      for (int cc = 1; cc < D / 16; ++cc) acc = mfma32(ld8_b<E>(kr, a_off[cc]), qf[cc], acc);
      s[sb] = acc;
    }
  };

  // ---- O^T += V^T P^T for the tile at n0, from V slot sc
  floatx16 oacc[D / 32];
#pragma unroll
  for (int d = 0; d < D / 32; ++d) oacc[d] = floatx16{};
  auto pv = [&](auto sc, auto checkc, int n0, vec8<E> (&pf)[NSUB][2]) {
#pragma unroll
    for (int sb = 0; sb < NSUB; ++sb) {
      if (decltype(checkc)::value && dead(n0, sb)) continue;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        // kperm rows 32 * (sub-block) + 16hh + 4g (+8): keys 16hh + 8g + 0..7
        const int rb = (32 * sb + 16 * hh) * D;
#pragma unroll
        for (int d = 0; d < D / 32; ++d)
          oacc[d] = mfma32(load_tr_pair_b<E>(v_sl(sc) + rb, t_off.lo(d), t_off.hi(d)), pf[sb][hh],
                           oacc[d]);
      }
    }
  };

  using C0 = std::integral_constant<int, 0>;
  using C1 = std::integral_constant<int, 1>;
  using Fast = std::false_type;    // no dead-sub-block checks
  using Check = std::true_type;
  // ---- prologue: K(0) -> K slot 0, K(1) -> K slot 1, (D = 128) V(0) ->
  // V slot 0, Q to registers, then the scores of tile 0
  if (n_tiles > 0) load_k(0, C0{});
  if (n_tiles > 1) load_k(BN, C1{});
  // D = 128: V(0) as well, so that its latency overlaps Q's and K's (one
  // memory round trip before the first tile instead of two; step 0 skips
  // it).  Measured: the C5 layer's forward -1.5 to -2.8 %; at D = 64 the
  // larger first burst costs more than it saves (+0.3 to +1.9 % at C4a).
  constexpr bool v0_early = D >= 128;
  if (v0_early && n_tiles > 0) load_v_next(C0{});
  {
    const int qr = min(qrow, nrows - 1);
    const f16 *qp = (SPLITKV ? a.q.head(b, hk * grp + qr % grp) + (int64_t)(qr / grp) * a.q.ss
                             : a.q.head(b, h) + (int64_t)qr * a.q.ss) + 8 * g;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) qf[c] = ld8<E>(qp + 16 * c);
    if (pre) {
#pragma unroll
      for (int c = 0; c < D / 16; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) qf[c][j] = (E)((float)qf[c][j] * a.c);
    }
    if (a.neg) {
#pragma unroll
      for (int c = 0; c < D / 16; ++c) qf[c] = neg8(qf[c]);
    }
  }
  // Q (and this wave's tile DMAs) must be complete before the loop:
  // otherwise the waitcnt pass cannot prove Q resident and stalls every
  // iteration's MFMAs on the prefetch loads.
  __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
  __syncthreads();

  // Scores and probabilities ping-pong between two register sets (tile t's
  // in the `a` sets when t is even, `b` when odd), so no copy waits for the
  // MFMAs that produce the next tile's scores.
  floatx16 s_a[NSUB], s_b[NSUB];
  vec8<E> p_a[NSUB][2], p_b[NSUB][2];
  if (n_tiles > 0) qk(C0{}, Check{}, 0, s_a);
  // K slot 0 is refilled with K(2) at the start of the first iteration
  __syncthreads();

  float m_run = kNegInf;   // running max of c*s (log2 units), stale by <= log2 kFastSum
  float l_run = 0.0f;      // this lane's share of the running sum
  const float c = a.c;

  // P = exp2(beta * s + neg_mu) rounded to E -- exp2(c*s - m) for the
  // stored scores s of either mode -- and the lane's sum of the rounded
  // values (two partial sums: shorter chains).
  const float beta = pre ? 1.0f : c;
  auto probs = [&](auto checkc, int n0, floatx16 (&s)[NSUB], vec8<E> (&pf)[NSUB][2],
                   float neg_m) -> float {
    float l0 = 0.0f, l1 = 0.0f;
#pragma unroll
    for (int sb = 0; sb < NSUB; ++sb) {
      if (decltype(checkc)::value && dead(n0, sb)) continue;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          vec2<E> pr = __builtin_convertvector(
              (floatx2){fast_exp2(__builtin_fmaf(s[sb][8 * hh + j], beta, neg_m)),
                        fast_exp2(__builtin_fmaf(s[sb][8 * hh + j + 1], beta, neg_m))},
              vec2<E>);
          if (hh == 0) l0 = dot2_acc(pr, l0);
          else l1 = dot2_acc(pr, l1);
          pf[sb][hh][j] = pr[0];
          pf[sb][hh][j + 1] = pr[1];
        }
      }
    }
    return l0 + l1;
  };

  // The softmax step of tile t (scores s, probabilities into pf): p >= 0,
  // so the lane's sum of its rounded p bounds each of them: a sum <=
  // kFastSum proves every p inside E's range and the tile needs no row
  // max.  Otherwise (the first tile with a visible key, or a score grown
  // past m by more than log2 kFastSum) the wave takes the row max,
  // rescales what has been accumulated (O includes tile t - 1's P V, issued
  // earlier in the same iteration) and recomputes.  In the pre mode the
  // next tile's scores s_nxt, already issued against the old m, move to the
  // new one (when `has_next`), and so does negm for the MFMAs to come.
  auto finish_softmax = [&](auto checkc, int n0, floatx16 (&s)[NSUB], vec8<E> (&pf)[NSUB][2],
                            float l_tile, floatx16 (&s_nxt)[NSUB], bool has_next) {
    const bool slow = m_run == kNegInf || !(l_tile <= kFastSum);
    if (__any(slow)) {
      float mx = kNegInf;
#pragma unroll
      for (int sb = 0; sb < NSUB; ++sb) {
        if (decltype(checkc)::value && dead(n0, sb)) continue;
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[sb][i]);
      }
      mx = max_xor32(mx);
      // reference of the stored scores: m (pre, finite m) or 0
      const float ref = pre && m_run != kNegInf ? m_run : 0.0f;
      const float m_new = fmaxf(m_run, pre ? mx + ref : mx * c);
      const bool grow = m_new > m_run;
      const float alpha = grow ? fast_exp2(m_run - m_new) : 1.0f;   // 0 from -inf
      m_run = grow ? m_new : m_run;
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < D / 32; ++d)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[d][i] *= alpha;
      // shift of the stored scores' reference: m - ref (0 while m is -inf)
      const float shift = m_run == kNegInf ? 0.0f : m_run - ref;
      l_tile = probs(checkc, n0, s, pf, pre ? -shift : (m_run == kNegInf ? 0.0f : -m_run));
      if (pre) {
        if (has_next) {
#pragma unroll
          for (int sb = 0; sb < NSUB; ++sb)
#pragma unroll
            for (int i = 0; i < 16; ++i) s_nxt[sb][i] -= shift;
        }
        const float nm = m_run == kNegInf ? 0.0f : -m_run;
#pragma unroll
        for (int i = 0; i < 16; ++i) negm[i] = nm;
      }
    }
    l_run += l_tile;
  };

  // One key tile.  Iteration t issues the MFMAs of two other tiles -- S^T
  // of tile t + 1 (K slot pc ^ 1) and P V of tile t - 1 (V slot pc ^ 1) --
  // alongside the softmax of tile t, whose scores came from the previous
  // iteration: none of the three depends on another, so the wave keeps the
  // matrix pipe busy while its VALU work runs.  The DMAs of K(t + 2) / V(t)
  // refill K slot pc / V slot pc, whose last readers (S^T of tile t, P V of
  // tile t - 2) finished before the previous barrier.  `pc` = t & 1 as a
  // compile-time constant (the loops are unrolled by two).
  //
  // General step: any tile (first, last, diagonal, ragged), with the
  // neighbours' existence, dead sub-blocks and the mask checked.
  auto step_general = [&](auto pcc, int t, floatx16 (&s_cur)[NSUB], floatx16 (&s_nxt)[NSUB],
                          vec8<E> (&p_prev)[NSUB][2], vec8<E> (&p_cur)[NSUB][2]) {
    constexpr int pc = decltype(pcc)::value;
    using CP = std::integral_constant<int, pc>;
    using CQ = std::integral_constant<int, pc ^ 1>;
    hide_offsets();
    const int n0 = t * BN;
    if (t + 2 < n_tiles) load_k_next(CP{});   // K(t + 2)
    if (!v0_early || t > 0) load_v_next(CP{});   // V(t) (V(0) at D = 128: the prologue)
    if (t + 1 < n_tiles) qk(CQ{}, Check{}, n0 + BN, s_nxt);
    if (t >= 1) pv(CQ{}, Check{}, n0 - BN, p_prev);
    if (!dead(n0, 0)) {
      // ---- masking (diagonal / ragged sub-blocks only)
#pragma unroll
      for (int sb = 0; sb < NSUB; ++sb) {
        const int ns = sub_key(n0, sb);
        if ((CAUSAL && ns + 31 > wpos_lo + off) || (ns + 31 >= Sk)) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = ns + slot_row(i, g);
            const bool vis = key < Sk && (!CAUSAL || key <= qpos + off);
            s_cur[sb][i] = vis ? s_cur[sb][i] : kNegInf;
          }
        }
      }
      const float l_tile = probs(Check{}, n0, s_cur, p_cur, pre ? 0.0f : -m_run);
      finish_softmax(Check{}, n0, s_cur, p_cur, l_tile, s_nxt, t + 1 < n_tiles);
    }
    __builtin_amdgcn_s_waitcnt(0x0f70);   // this wave's DMAs into the next slots
    __syncthreads();
  };

  // Interior step: 1 <= t, t + 1 < n_tiles and t < t_mask, so both
  // neighbours exist and every sub-block of tiles t - 1 and t is visible
  // with nothing to mask -- one straight-line block for the scheduler.
  // K(t + 2) past the last tile is a DMA of zeros (the cursor's extent is
  // 0 there) into a slot nobody reads again.
  auto step_interior = [&](auto pcc, int t, floatx16 (&s_cur)[NSUB], floatx16 (&s_nxt)[NSUB],
                           vec8<E> (&p_prev)[NSUB][2], vec8<E> (&p_cur)[NSUB][2]) {
    constexpr int pc = decltype(pcc)::value;
    using CP = std::integral_constant<int, pc>;
    using CQ = std::integral_constant<int, pc ^ 1>;
    hide_offsets();
    // The block in issue order: MQ S^T MFMAs (K slot pc ^ 1) and MP P V
    // MFMAs (V slot pc ^ 1), alternating while both remain, each followed
    // by its share of tile t's softmax (NPAIR pairs of scores: two FMAs, two
    // exp2, one conversion, one dot2).  A MFMA runs ~32 cycles in the
    // matrix pipe while the wave issues the VALU slice after it; its A
    // operand was read from LDS PF MFMAs earlier.  sched_barrier(0) keeps
    // the compiler from regrouping the slices.  The first operand reads go
    // out before this iteration's DMAs (K(t + 2), V(t)) and their scalar
    // address updates, so the first MFMA waits less after the barrier.
    constexpr int MQ = NSUB * (D / 16), MP = NSUB * 2 * (D / 32), M = MQ + MP;
    constexpr int NPAIR = NSUB * 8;
    const f16 *ks = k_sl(CQ{});
    const f16 *vs = v_sl(CQ{});
    // MFMA i of the block: S^T (sb, cc) or P V (sb, hh, d), ordered
    // Q0 P0 Q1 P1 ... while both kinds remain.
    auto kind_index = [](int i, bool &is_q, int &j) {
      const int lo = MQ < MP ? MQ : MP;
      if (i < 2 * lo) { is_q = (i & 1) == 0; j = i >> 1; }
      else { is_q = MQ > MP; j = i - lo; }
    };
    auto operand = [&](auto ic) -> vec8<E> {
      constexpr int i = decltype(ic)::value;
      bool is_q = false; int j = 0;
      kind_index(i, is_q, j);
      if (is_q) {
        const int sb = j / (D / 16), cc = j % (D / 16);
        return ld8_b<E>(ks + 32 * sb * D, a_off[cc]);
      }
      const int sb = j / (2 * (D / 32)), hh = (j / (D / 32)) % 2, d = j % (D / 32);
      return load_tr_pair_b<E>(vs + (32 * sb + 16 * hh) * D, t_off.lo(d), t_off.hi(d));
    };
    const float c_ = c, neg_m = -m_run;
    float l0 = 0.0f, l1 = 0.0f;
    // softmax pair q of tile t: scores 2 (q % 4) and + 1 of half (q / 4) % 2
    // of sub-block q / 8
    auto pair_exp = [&](auto qc) -> floatx2 {
      constexpr int q = decltype(qc)::value;
      constexpr int sb = q / 8, hh = (q / 4) % 2, jj = 2 * (q % 4);
      if constexpr (PRE) {
        return (floatx2){fast_exp2(s_cur[sb][8 * hh + jj]), fast_exp2(s_cur[sb][8 * hh + jj + 1])};
      } else {
        return (floatx2){fast_exp2(__builtin_fmaf(s_cur[sb][8 * hh + jj], c_, neg_m)),
                         fast_exp2(__builtin_fmaf(s_cur[sb][8 * hh + jj + 1], c_, neg_m))};
      }
    };
    auto pair_store = [&](auto qc, floatx2 e) -> vec2<E> {
      constexpr int q = decltype(qc)::value;
      constexpr int sb = q / 8, hh = (q / 4) % 2, jj = 2 * (q % 4);
      const vec2<E> pr = __builtin_convertvector(e, vec2<E>);
      p_cur[sb][hh][jj] = pr[0];
      p_cur[sb][hh][jj + 1] = pr[1];
      return pr;
    };
    auto pair_sum = [&](auto qc, vec2<E> pr) {
      if constexpr (decltype(qc)::value & 1) l1 = dot2_acc(pr, l1);
      else l0 = dot2_acc(pr, l0);
    };
    constexpr int MAXP = (NPAIR + M - 1) / M;   // pairs per slice, at most
    floatx2 eh[MAXP];                           // exp2s awaiting conversion
    // operands read this many MFMAs ahead (3 at D = 128: -1 to -2 % there;
    // at D = 64 it gains nothing)
    constexpr int PF = D >= 128 ? 3 : 2;
    vec8<E> op[PF + 1];
    static_for<PF>([&](auto ic) {
      if constexpr (decltype(ic)::value < M) op[decltype(ic)::value] = operand(ic);
    });
    __builtin_amdgcn_sched_barrier(0);
    load_k_next(CP{});   // K(t + 2)
    load_v_next(CP{});   // V(t)
    __builtin_amdgcn_sched_barrier(0);
    static_for<M>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      if constexpr (i + PF < M) op[(i + PF) % (PF + 1)] = operand(std::integral_constant<int, i + PF>{});
      bool is_q = false; int j = 0;
      kind_index(i, is_q, j);
      if (is_q) {
        const int sb = j / (D / 16), cc = j % (D / 16);
        s_nxt[sb] = mfma32(op[i % (PF + 1)], qf[cc], cc == 0 ? negm : s_nxt[sb]);
      } else {
        const int sb = j / (2 * (D / 32)), hh = (j / (D / 32)) % 2, d = j % (D / 32);
        oacc[d] = mfma32(op[i % (PF + 1)], p_prev[sb][hh], oacc[d]);
      }
      // softmax pairs [i * NPAIR / M, (i + 1) * NPAIR / M) of tile t: their
      // exp2s now, their conversion and sum in the next slice (the
      // previous slice's pairs are converted first and summed last), so no
      // instruction waits on the result of the one before it
      constexpr int b_cur = i * NPAIR / M, n_cur = (i + 1) * NPAIR / M - b_cur;
      constexpr int b_prv = i > 0 ? (i - 1) * NPAIR / M : 0, n_prv = i > 0 ? b_cur - b_prv : 0;
      vec2<E> pr[MAXP];
      static_for<n_prv>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        pr[k] = pair_store(std::integral_constant<int, b_prv + k>{}, eh[k]);
      });
      static_for<n_cur>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        eh[k] = pair_exp(std::integral_constant<int, b_cur + k>{});
      });
      static_for<n_prv>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        pair_sum(std::integral_constant<int, b_prv + k>{}, pr[k]);
      });
      __builtin_amdgcn_sched_barrier(0);
    });
    {
      constexpr int b_last = (M - 1) * NPAIR / M;
      static_for<NPAIR - b_last>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        pair_sum(std::integral_constant<int, b_last + k>{},
                 pair_store(std::integral_constant<int, b_last + k>{}, eh[k]));
      });
    }
    finish_softmax(Fast{}, t * BN, s_cur, p_cur, l0 + l1, s_nxt, true);
    __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();
  };

  // Tile 0, then the interior tiles two at a time, then the rest two at a
  // time.  Every loop starts at an odd tile, so tile t's register sets are
  // fixed by its parity in all three (tile t's scores in s_a when t is
  // even, s_b when odd; likewise its probabilities in p_a / p_b).
  if (n_tiles > 0) step_general(C0{}, 0, s_a, s_b, p_b, p_a);
  const int t_fast_end = min(t_mask, n_tiles - 1);
  int t = 1;
  for (; t + 1 < t_fast_end; t += 2) {
    step_interior(C1{}, t, s_b, s_a, p_a, p_b);
    step_interior(C0{}, t + 1, s_a, s_b, p_b, p_a);
  }
  for (; t < n_tiles; t += 2) {
    step_general(C1{}, t, s_b, s_a, p_a, p_b);
    if (t + 1 < n_tiles) step_general(C0{}, t + 1, s_a, s_b, p_b, p_a);
  }
  // P V of the last tile (V slot and probabilities of its parity)
  if (n_tiles > 0) {
    const int nl = (n_tiles - 1) * BN;
    if ((n_tiles - 1) & 1) pv(C1{}, Check{}, nl, p_b);
    else pv(C0{}, Check{}, nl, p_a);
  }

  // ---- merge the two key halves of each query group, through one LDS
  // slot per group: K slots (the loop's last barrier ordered every read of
  // them before these writes), and with four groups the V slots too, which
  // the last tile's P V above still reads until the barrier here
  if constexpr (KSPLIT == 4) {
    // key parts 1..3 of query group qg hand over (m, l, O^T) in buffer
    // qg * 3 + kh - 1 (two per LDS slot, the V slots too: the barrier
    // first ends the last tile's P V reads); part 0 merges them in order
    __syncthreads();
    auto mbuf_of = [&](int i) -> float * {
      const int sl = i >> 1;
      f16 *slot = sl == 0 ? sk0 : (sl == 1 ? sk1 : (sl == 2 ? sv0 : sv1));
      return reinterpret_cast<float *>(slot) + (i & 1) * T::MERGE_FLOATS;
    };
    if (kh > 0) {
      const int i = qg * 3 + kh - 1;
      float *mbuf = mbuf_of(i);
      s_ml[i][0][lane] = m_run;
      s_ml[i][1][lane] = l_run;
#pragma unroll
      for (int d = 0; d < D / 32; ++d)
#pragma unroll
        for (int j = 0; j < 16; ++j) mbuf[(16 * d + j) * 64 + lane] = oacc[d][j];
    }
    __syncthreads();
    if (kh > 0) return;
    float mp[3], m = m_run;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      mp[k] = s_ml[qg * 3 + k][0][lane];
      m = fmaxf(m, mp[k]);
    }
    const float f0 = (m == kNegInf) ? 0.0f : fast_exp2(m_run - m);
    l_run *= f0;
#pragma unroll
    for (int d = 0; d < D / 32; ++d)
#pragma unroll
      for (int j = 0; j < 16; ++j) oacc[d][j] *= f0;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const float fk = (m == kNegInf) ? 0.0f : fast_exp2(mp[k] - m);
      const float *mbuf = mbuf_of(qg * 3 + k);
      l_run += s_ml[qg * 3 + k][1][lane] * fk;
#pragma unroll
      for (int d = 0; d < D / 32; ++d)
#pragma unroll
        for (int j = 0; j < 16; ++j) oacc[d][j] += mbuf[(16 * d + j) * 64 + lane] * fk;
    }
    m_run = m;
  }
  if (KSPLIT == 2) {
    if constexpr (T::NQG > 2) __syncthreads();
    f16 *slot = qg == 0 ? sk0 : (qg == 1 ? sk1 : (qg == 2 ? sv0 : sv1));
    float *mbuf = reinterpret_cast<float *>(slot);
    if (kh == 1) {
      s_ml[qg][0][lane] = m_run;
      s_ml[qg][1][lane] = l_run;
#pragma unroll
      for (int d = 0; d < D / 32; ++d)
#pragma unroll
        for (int i = 0; i < 16; ++i) mbuf[(16 * d + i) * 64 + lane] = oacc[d][i];
    }
    __syncthreads();
    if (kh == 1) return;
    const float m_b = s_ml[qg][0][lane];
    const float l_b = s_ml[qg][1][lane];
    const float m = fmaxf(m_run, m_b);
    const float fa = (m == kNegInf) ? 0.0f : fast_exp2(m_run - m);
    const float fb = (m == kNegInf) ? 0.0f : fast_exp2(m_b - m);
    l_run = l_run * fa + l_b * fb;
#pragma unroll
    for (int d = 0; d < D / 32; ++d)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        oacc[d][i] = oacc[d][i] * fa + mbuf[(16 * d + i) * 64 + lane] * fb;
    m_run = m;
  }

  // ---- epilogue: O = acc / l, LSE = (m + log2 l) * ln2
  const float l_tot = l_run + xor32(l_run);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (SPLITKV || (BAL && part >= 0)) {
    // this split's normalised O and log2-domain LSE (-inf: no visible key)
    if (qrow < nrows) {
      int64_t prow;
      if (SPLITKV) {
        const int hq = hk * grp + qrow % grp;
        prow = (((int64_t)blockIdx.y * a.B + b) * a.H + hq) * Sq + qrow / grp;
      } else {
        // (half, slot (b, h, pair), row in the tile)
        const int64_t rows = (int64_t)BH * (a.n_qtiles >> 1) * BM;
        prow = (part & 1) * rows + (int64_t)(part >> 1) * BM + (qrow - q0);
      }
      float *po = a.part_o + prow * D;
#pragma unroll
      for (int d = 0; d < D / 32; ++d) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          floatx4 v4;
#pragma unroll
          for (int j = 0; j < 4; ++j) v4[j] = oacc[d][4 * r + j] * inv;
          *(floatx4 *)(po + 32 * d + c_row(4 * r, g)) = v4;
        }
      }
      if (g == 0) a.part_lse[prow] = l_tot > 0.0f ? m_run + fast_log2(l_tot) : kNegInf;
    }
    return;
  }
  if (qrow < Sq) {
    f16 *orow = a.o + b * a.o_sb + h * a.o_sh + (int64_t)qrow * a.o_ss;
#pragma unroll
    for (int d = 0; d < D / 32; ++d) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        vec4<E> v4;
#pragma unroll
        for (int j = 0; j < 4; ++j) v4[j] = (E)(oacc[d][4 * r + j] * inv);
        *(vec4<E> *)(orow + 32 * d + c_row(4 * r, g)) = v4;
      }
    }
    if (a.lse != nullptr && g == 0) {
      const float lse = l_tot > 0.0f ? (m_run + fast_log2(l_tot)) * kLn2 : kPosInf;
      a.lse[(int64_t)bh * Sq + qrow] = lse;
    }
  }
}

// ---- merge of the split-KV partials: per row (b, h, position)
//   m = max_z lse_z,  w_z = 2^(lse_z - m),  O = sum_z w_z O_z / sum_z w_z,
//   LSE = (m + log2 sum_z w_z) ln 2  (+inf and O = 0 when no split saw a key).
// A row's D values belong to D/8 lanes (8 fp32 each) and its splits to
// `zgroups` lane groups (split z to group z % zgroups), each merging its
// splits online with a running maximum; the groups then merge through LDS
// in group order.  Every sum has a fixed order (reproducible results).
//
// Pair mode (pair_bm > 0): the partials of the balanced causal schedule
// (fa_fwd_bal_item), two per row of a split heavy tile; rows of tiles that
// ran whole are skipped (the forward kernel wrote them).
struct CombineArgs {
  const float *part_o, *part_lse;   // as written by fa_fwd_kernel<..., SPLITKV or BAL>
  f16 *o;
  int64_t o_sb, o_ss, o_sh;
  float *lse;                       // (B, H, Sq) or nullptr
  int B, Sq, H, n_splits;
  int zgroups;                      // power of two, at most 256 / (D / 8)
  // pair mode: the forward's tile rows (0: split-KV layout), query tiles
  // per (b, h), key tile and causal offset
  int pair_bm, nb, bn, Sk, off;
};

template <typename E, int D>
__global__ __launch_bounds__(256) void fa_fwd_combine_kernel(CombineArgs a) {
  constexpr int LPR = D / 8;
  constexpr int SLOTS = 256 / LPR;   // (row, split group) pairs per workgroup
  __shared__ float s_m[SLOTS], s_sum[SLOTS];
  __shared__ __attribute__((aligned(16))) float s_acc[SLOTS][D];
  const int zn = a.zgroups;
  const int rpb = SLOTS / zn;
  const int slot = threadIdx.x / LPR, j = threadIdx.x % LPR;
  const int rloc = slot / zn, zg = slot % zn;
  const int64_t row = (int64_t)blockIdx.x * rpb + rloc;
  // the partials' row count, and this row's (b, h) and position
  int64_t rows, bh;
  int s;
  bool valid;
  if (a.pair_bm > 0) {
    const int np = a.nb >> 1;
    rows = (int64_t)a.B * a.H * np * a.pair_bm;
    const int64_t ps = row / a.pair_bm;   // slot (b, h, pair)
    const int p = (int)(ps % np), jt = a.nb - 1 - p;
    bh = ps / np;
    s = jt * a.pair_bm + (int)(row % a.pair_bm);
    int hx;
    valid = row < rows && s < a.Sq &&
            bal_split(causal_tiles_of(a.Sk, a.off, p, a.pair_bm, a.bn),
                      causal_tiles_of(a.Sk, a.off, jt, a.pair_bm, a.bn), hx);
  } else {
    rows = (int64_t)a.B * a.H * a.Sq;
    bh = row / a.Sq;
    s = (int)(row % a.Sq);
    valid = row < rows;
  }

  float m = kNegInf, sum = 0.0f;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (valid) {
#pragma unroll 4
    for (int z = zg; z < a.n_splits; z += zn) {
      const float lz = a.part_lse[z * rows + row];
      const floatx4 *src = (const floatx4 *)(a.part_o + (z * rows + row) * D + 8 * j);
      const floatx4 x0 = src[0], x1 = src[1];
      if (lz == kNegInf) continue;   // no visible key in this split
      if (lz > m) {
        const float sc = fast_exp2(m - lz);   // 0 while m is -inf
        sum *= sc;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] *= sc;
        m = lz;
      }
      const float wz = fast_exp2(lz - m);
      sum += wz;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[i] += wz * x0[i];
        acc[4 + i] += wz * x1[i];
      }
    }
  }
  if (j == 0) {
    s_m[slot] = m;
    s_sum[slot] = sum;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) s_acc[slot][8 * j + i] = acc[i];
  __syncthreads();
  if (zg != 0 || !valid) return;

  float mt = kNegInf;
  for (int k = 0; k < zn; ++k) mt = fmaxf(mt, s_m[slot + k]);
  float tot = 0.0f;
  float o8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (mt != kNegInf) {
    for (int k = 0; k < zn; ++k) {
      const float mk = s_m[slot + k];
      const float sc = mk == kNegInf ? 0.0f : fast_exp2(mk - mt);
      tot += sc * s_sum[slot + k];
#pragma unroll
      for (int i = 0; i < 8; ++i) o8[i] += sc * s_acc[slot + k][8 * j + i];
    }
  }
  const float inv = tot > 0.0f ? 1.0f / tot : 0.0f;
  const int hh = (int)(bh % a.H), b = (int)(bh / a.H);
  vec8<E> out;
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = (E)(o8[i] * inv);
  *(vec8<E> *)(a.o + b * a.o_sb + s * a.o_ss + hh * a.o_sh + 8 * j) = out;
  if (a.lse != nullptr && j == 0)
    a.lse[bh * a.Sq + s] = tot > 0.0f ? (mt + fast_log2(tot)) * kLn2 : kPosInf;
}

}  // namespace fa
