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
};

template <int D, int KSPLIT>
struct FwdTile {
  static_assert(KSPLIT == 1 || KSPLIT == 2, "key split is 1 or 2");
  static constexpr int NQG = 4 / KSPLIT;   // query groups of 32 per workgroup
  static constexpr int NSUB = 2 / KSPLIT;  // 32-key sub-blocks per wave per tile
  static constexpr int BM = 32 * NQG;      // queries per workgroup
  static constexpr int BN = 64;            // keys per tile
  static constexpr int NT = 256;           // 4 waves
  static constexpr int LDS_TILE = BN * D;  // swizzled, unpadded (fa_common.hpp)
  // O^T partial sums of a key-half wave handed over for the final merge
  static_assert(64 * (D / 2) * 4 <= LDS_TILE * 2, "a merge buffer must fit in one K slot");
};

// Workgroup = 4 waves.  KSPLIT = 1: each wave owns 32 queries (BM = 128)
// and both 32-key halves of every 64-key tile.  KSPLIT = 2: wave w owns
// query group qg = w / 2 (BM = 64) and key half kh = w % 2 of every tile;
// each wave runs its own online softmax over its key half and the two halves
// of a query group merge through LDS at the end (lane l of both waves holds
// the same query and the same O^T rows, so the merge is element-wise).
// Splitting keys halves each wave's work per tile and doubles the waves in
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
template <typename E, int D, bool CAUSAL, int KSPLIT, bool SPLITKV = false>
__global__ __launch_bounds__(256) void fa_fwd_kernel(FwdArgs a) {
  using T = FwdTile<D, KSPLIT>;
  constexpr int NSUB = T::NSUB;
  constexpr int BM = T::BM, BN = T::BN;
  // One LDS object per slot, so the compiler sees that a DMA into one slot
  // cannot alias reads of another and does not wait for it early.
  __shared__ __attribute__((aligned(16))) f16 sk0[T::LDS_TILE], sk1[T::LDS_TILE];
  __shared__ __attribute__((aligned(16))) f16 sv0[T::LDS_TILE], sv1[T::LDS_TILE];
  __shared__ __attribute__((aligned(16))) float s_ml[2][2][64];   // merge: m, l per query group
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
  const int qt = (CAUSAL && !SPLITKV)
                     ? a.n_qtiles - 1 - (a.zigzag ? zigzag_rank(bid / BH, a.n_qtiles) : bid / BH)
                     : bid / BH;
  const int hx = SPLITKV ? a.H / grp : a.H;
  const int b = bh / hx;
  const int h = SPLITKV ? 0 : bh % hx;               // SPLITKV: the head is per lane
  const int hk = SPLITKV ? bh % hx : h / grp;        // key/value head
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = wave_id();
  const int qg = KSPLIT == 2 ? (w >> 1) : w;
  const int kh = KSPLIT == 2 ? (w & 1) : 0;
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

  // Key range of this workgroup: all keys, or split blockIdx.y's
  const int kbase = SPLITKV ? (int)blockIdx.y * a.kv_split : 0;
  const int Sk = SPLITKV ? min(a.kv_split, a.Sk - kbase) : a.Sk;
  const int off = a.off - kbase;   // key j (relative) is visible to position i iff j <= i + off

  const f16 *kb = a.k.head(b, hk) + (int64_t)kbase * a.k.ss;
  const f16 *vb = a.v.head(b, hk) + (int64_t)kbase * a.v.ss;

  int kv_end = Sk;
  if (CAUSAL) kv_end = min(Sk, bpos_hi + 1 + off);
  // 0 when every query of the block precedes every key (causal, Sq > Sk)
  const int n_tiles = kv_end > 0 ? (kv_end + BN - 1) / BN : 0;

  // ---- K and V tiles go straight to LDS (fa_common.hpp DmaStager): both
  // in kperm row order, chunks swizzled; rows past Sk read as zeros.
  DmaStager<D> stk, stv;
  stk.init(w, lane, a.k.ss);
  stv.init(w, lane, a.v.ss);
  auto load_k = [&](int n0, auto sc) { stk.load(k_sl(sc), kb, a.k.ss, n0, Sk, w); };
  auto load_v = [&](int n0, auto sc) { stv.load(v_sl(sc), vb, a.v.ss, n0, Sk, w); };
  // In the loop K is loaded two tiles ahead and V one: cursors at those
  // rows, each advanced by a tile per load (no per-tile 64-bit multiplies).
  RowCursor ck, cv;
  ck.init(kb, a.k.ss, 2 * BN, Sk, D, BN);
  cv.init(vb, a.v.ss, BN, Sk, D, BN);
  auto load_k_next = [&](auto sc) {
    stk.load(k_sl(sc), ck.rsrc(), w);
    ck.advance();
  };
  auto load_v_next = [&](auto sc) {
    stv.load(v_sl(sc), cv.rsrc(), w);
    cv.advance();
  };

  // Per-lane LDS element offsets inside a slot: K rows l32 (A operand of
  // S^T = K Q^T), chunk 2cc + g; V^T transpose reads of rows 4g + (l16 >> 2)
  // (and + 8), i.e. natural V rows 8g + (l16 >> 2) (and + 4).
  int a_off[D / 16], t_off[D / 32];
  {
    const int sa = swz<D>(l32);
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc) a_off[cc] = l32 * D + (((2 * cc + g) ^ sa) << 3);
    const int l16 = lane & 15, tr = 4 * g + (l16 >> 2);
    const int st_ = swz<D>(tr);
#pragma unroll
    for (int d = 0; d < D / 32; ++d)
      t_off[d] = tr * D + (((4 * d + 2 * ((lane >> 4) & 1) + ((l16 >> 1) & 1)) ^ st_) << 3) +
                 4 * (l16 & 1);
  }

  // Sub-block sb (32 keys) of this wave in the tile at n0 starts at key
  // n0 + 32 * (NSUB * kh + sb); it is dead when it lies entirely above the
  // wave's causal diagonal (the last key its last query sees is wq0+31+off).
  auto sub_key = [&](int n0, int sb) { return n0 + 32 * (NSUB * kh + sb); };
  auto dead = [&](int n0, int sb) { return CAUSAL && sub_key(n0, sb) > wpos_hi + off; };

  // ---- S^T = K Q^T for this wave's sub-blocks of a tile
  vec8<E> qf[D / 16];
  auto qk = [&](auto sc, int n0, floatx16 (&s)[NSUB]) {
#pragma unroll
    for (int sb = 0; sb < NSUB; ++sb) {
      // dead sub-blocks are skipped; the diagonal mask overwrites them
      if (dead(n0, sb)) continue;
      const f16 *kr = k_sl(sc) + 32 * (NSUB * kh + sb) * D;
      floatx16 acc = mfma32(ld8<E>(kr + a_off[0]), qf[0], floatx16{});
#pragma unroll
      for (int cc = 1; cc < D / 16; ++cc) acc = mfma32(ld8<E>(kr + a_off[cc]), qf[cc], acc);
      s[sb] = acc;
    }
  };

  using C0 = std::integral_constant<int, 0>;
  using C1 = std::integral_constant<int, 1>;
  // ---- prologue: K(0), V(0) -> slot 0, K(1) -> K slot 1
  if (n_tiles > 0) {
    load_k(0, C0{});
    load_v(0, C0{});
  }
  if (n_tiles > 1) load_k(BN, C1{});
  {
    const int qr = min(qrow, nrows - 1);
    const f16 *qp = (SPLITKV ? a.q.head(b, hk * grp + qr % grp) + (int64_t)(qr / grp) * a.q.ss
                             : a.q.head(b, h) + (int64_t)qr * a.q.ss) + 8 * g;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) qf[c] = ld8<E>(qp + 16 * c);
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

  // Scores ping-pong between two register sets (no copy at the end of a
  // tile, which would wait for the next tile's S MFMAs right after issuing
  // them): tile t's scores live in s_a when t is even, s_b when odd.
  floatx16 s_a[NSUB], s_b[NSUB];
  if (n_tiles > 0) qk(C0{}, 0, s_a);
  // K slot 0 is refilled with K(2) at the start of the first iteration
  __syncthreads();

  floatx16 oacc[D / 32];
#pragma unroll
  for (int d = 0; d < D / 32; ++d) oacc[d] = floatx16{};
  float m_run = kNegInf;   // running max of c*s (log2 units), stale by <= log2 kFastSum
  float l_run = 0.0f;      // this lane's share of the running sum
  const float c = a.c;

  // One key tile; `pc` = t & 1 as a compile-time constant (the loop is
  // unrolled by two): S^T of tile t+1 reads K slot pc^1, P V reads V slot
  // pc, and the DMAs of K(t+2) / V(t+1) refill K slot pc / V slot pc^1,
  // whose last readers finished before the previous barrier.
  auto tile_step = [&](auto pcc, int t, floatx16 (&s_cur)[NSUB], floatx16 (&s_nxt)[NSUB]) {
    constexpr int pc = decltype(pcc)::value;
    using CP = std::integral_constant<int, pc>;
    using CQ = std::integral_constant<int, pc ^ 1>;
    const int n0 = t * BN;
    const bool more1 = t + 1 < n_tiles, more2 = t + 2 < n_tiles;
    if (more2) load_k_next(CP{});   // K(t + 2)
    if (more1) load_v_next(CQ{});   // V(t + 1)
    if (more1) qk(CQ{}, n0 + BN, s_nxt);

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

      // ---- P = exp2(c*s - m) rounded to E, against the running max m.
      // p >= 0, so the lane's sum of its rounded p bounds each of them: a
      // sum <= kFastSum proves every p inside E's range, and the tile needs
      // no row max.  Otherwise (the first tile with a visible key, or a
      // score grown past m by more than log2 kFastSum) the wave takes the
      // row max, rescales and recomputes.
      vec8<E> pf[NSUB][2];
      float l_tile = 0.0f;
      auto probs = [&](float neg_m) {
        l_tile = 0.0f;
#pragma unroll
        for (int sb = 0; sb < NSUB; ++sb) {
          if (dead(n0, sb)) continue;
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
              vec2<E> pr = __builtin_convertvector(
                  (floatx2){fast_exp2(__builtin_fmaf(s_cur[sb][8 * hh + j], c, neg_m)),
                            fast_exp2(__builtin_fmaf(s_cur[sb][8 * hh + j + 1], c, neg_m))},
                  vec2<E>);
              l_tile = dot2_acc(pr, l_tile);
              pf[sb][hh][j] = pr[0];
              pf[sb][hh][j + 1] = pr[1];
            }
          }
        }
      };
      probs(-m_run);
      const bool slow = m_run == kNegInf || !(l_tile <= kFastSum);
      if (__any(slow)) {
        float mx = s_cur[0][0];
#pragma unroll
        for (int sb = 0; sb < NSUB; ++sb)
#pragma unroll
          for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s_cur[sb][i]);
        mx = max_xor32(mx);
        const float m_new = fmaxf(m_run, mx * c);
        const bool grow = m_new > m_run;
        const float alpha = grow ? fast_exp2(m_run - m_new) : 1.0f;   // 0 from -inf
        m_run = grow ? m_new : m_run;
        l_run *= alpha;
#pragma unroll
        for (int d = 0; d < D / 32; ++d)
#pragma unroll
          for (int i = 0; i < 16; ++i) oacc[d][i] *= alpha;
        probs(m_run == kNegInf ? 0.0f : -m_run);
      }
      l_run += l_tile;

      // ---- O^T += V^T P^T
#pragma unroll
      for (int sb = 0; sb < NSUB; ++sb) {
        if (dead(n0, sb)) continue;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          // kperm rows 32 * (sub-block) + 16hh + 4g (+8): keys 16hh + 8g + 0..7
          const int rb = (32 * (NSUB * kh + sb) + 16 * hh) * D;
#pragma unroll
          for (int d = 0; d < D / 32; ++d)
            oacc[d] = mfma32(load_tr_pair<E>(v_sl(CP{}) + rb + t_off[d], 8 * D), pf[sb][hh],
                             oacc[d]);
        }
      }
    }

    if (more1) __builtin_amdgcn_s_waitcnt(0x0f70);   // this wave's DMAs into the next slots
    __syncthreads();
  };

  for (int t = 0; t < n_tiles; t += 2) {
    tile_step(C0{}, t, s_a, s_b);
    if (t + 1 < n_tiles) tile_step(C1{}, t + 1, s_b, s_a);
  }

  // ---- merge the two key halves of each query group (K slots reused; the
  // loop's last barrier ordered every read of them before these writes)
  if (KSPLIT == 2) {
    float *mbuf = reinterpret_cast<float *>(qg ? sk1 : sk0);
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
  if (SPLITKV) {
    // this split's normalised O and log2-domain LSE (-inf: no visible key)
    if (qrow < nrows) {
      const int hq = hk * grp + qrow % grp;
      const int64_t prow = (((int64_t)blockIdx.y * a.B + b) * a.H + hq) * Sq + qrow / grp;
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
struct CombineArgs {
  const float *part_o, *part_lse;   // as written by fa_fwd_kernel<..., SPLITKV>
  f16 *o;
  int64_t o_sb, o_ss, o_sh;
  float *lse;                       // (B, H, Sq) or nullptr
  int B, Sq, H, n_splits;
  int zgroups;                      // power of two, at most 256 / (D / 8)
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
  const int64_t rows = (int64_t)a.B * a.H * a.Sq;
  const int64_t row = (int64_t)blockIdx.x * rpb + rloc;
  const bool valid = row < rows;

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
  const int s = (int)(row % a.Sq);
  const int64_t bh = row / a.Sq;
  const int hh = (int)(bh % a.H), b = (int)(bh / a.H);
  vec8<E> out;
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = (E)(o8[i] * inv);
  *(vec8<E> *)(a.o + b * a.o_sb + s * a.o_ss + hh * a.o_sh + 8 * j) = out;
  if (a.lse != nullptr && j == 0) a.lse[row] = tot > 0.0f ? (mt + fast_log2(tot)) * kLn2 : kPosInf;
}

}  // namespace fa
