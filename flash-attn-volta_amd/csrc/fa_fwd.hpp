// fa_fwd.hpp -- forward FlashAttention kernel for gfx950.
//
// Computes, for one (query tile, batch*head), O = softmax(c * Q K^T) V with an
// online (streaming) softmax over key tiles, fp16 MFMA with fp32 accumulation,
// and the natural-log row LSE.  Behaviour follows the reference forward
// (flash_attn_volta/triton_fa.py:63-159): causal tiles above the diagonal are
// skipped (:110-117), masked scores are -inf (:123-126), O = acc / l
// (:146-150) and LSE = m + ln(l), +inf when a row saw no key (:152-159).
//
// MI355X layout of the work:
//   * workgroup = NW waves; each wave owns 32 consecutive queries, so a
//     workgroup covers BM = 32*NW queries of one (b, h);
//   * key/value tiles of BN = 64 rows stream through LDS, double-buffered:
//     K row-major [key][d] (A operand of S^T = K Q^T), V transposed [d][key]
//     (A operand of O^T = V^T P^T), each row padded by 8 halves;
//   * the wave's Q fragment stays in registers for the whole sweep;
//   * a lane owns one query row: the running max / sum and the O^T
//     accumulator column live in that lane, the only cross-lane step is one
//     exchange with lane ^ 32 per key tile for the row max;
//   * probabilities are rounded to fp16 once and the row sum accumulates
//     those rounded values (v_dot2_f32_f16), so numerator and denominator
//     see the same weights;
//   * the accumulator is rescaled only when a row max grows by more than
//     kRescaleLog2 (in log2 units): the stale max keeps p <= 2^kRescaleLog2,
//     well inside fp16, and the final O and LSE use the same max, so the
//     result is exact either way.
#pragma once

#include "fa_common.hpp"

namespace fa {

constexpr float kRescaleLog2 = 8.0f;

struct FwdArgs {
  TensorDesc q, k, v;
  f16 *o;
  int64_t o_sb, o_ss, o_sh;
  float *lse;          // (B, H, S) or nullptr
  int B, S, H;
  int n_qtiles;
  float c;             // |sm_scale| * log2(e), clamped away from 0
  int neg;             // 1 when sm_scale < 0: Q is negated on load
};

template <int D, int NW>
struct FwdTile {
  static constexpr int BM = 32 * NW;
  static constexpr int BN = 64;
  static constexpr int NT = 64 * NW;
  static constexpr int KS = D + 8;   // K tile row stride (halves)
  static constexpr int VS = BN + 8;  // V^T tile row stride (halves)
  static constexpr int K_CHUNKS = BN * D / 8;               // 16-byte chunks
  static constexpr int K_PER_T = (K_CHUNKS + NT - 1) / NT;
  static constexpr int V_UNITS = (BN / 8) * (D / 2);        // 8 keys x 2 d
  static constexpr int V_PER_T = (V_UNITS + NT - 1) / NT;
  static constexpr int LDS_K = BN * KS;
  static constexpr int LDS_V = D * VS;
};

template <int D, bool CAUSAL, int NW>
__global__ __launch_bounds__(64 * NW) void fa_fwd_kernel(FwdArgs a) {
  using T = FwdTile<D, NW>;
  constexpr int BM = T::BM, BN = T::BN, NT = T::NT, KS = T::KS, VS = T::VS;
  __shared__ __attribute__((aligned(16))) f16 sk[2][T::LDS_K];
  __shared__ __attribute__((aligned(16))) f16 sv[2][T::LDS_V];

  const int S = a.S;
  const int BH = a.B * a.H;
  const int bid = blockIdx.x;
  const int bh = bid % BH;
  // Heaviest causal tiles first; consecutive workgroups of one (b, h) are BH
  // apart, so with BH % 8 == 0 they land on one XCD and share its L2.
  const int qt = a.n_qtiles - 1 - bid / BH;
  const int b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int q0 = qt * BM;
  const int wq0 = q0 + 32 * w;   // first query of this wave
  const int qrow = wq0 + l32;    // query owned by this lane

  const f16 *qb = a.q.head(b, h);
  const f16 *kb = a.k.head(b, h);
  const f16 *vb = a.v.head(b, h);

  // ---- Q fragment (B operand of S^T = K Q^T): Q[qrow][16c + 8g .. +7]
  half8 qf[D / 16];
  if (qrow < S) {
    const f16 *qr = qb + (int64_t)qrow * a.q.ss + 8 * g;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) qf[c] = *(const half8 *)(qr + 16 * c);
    if (a.neg) {
#pragma unroll
      for (int c = 0; c < D / 16; ++c) qf[c] = neg8(qf[c]);
    }
  } else {
#pragma unroll
    for (int c = 0; c < D / 16; ++c) qf[c] = half8{};
  }

  int kv_end = S;
  if (CAUSAL) kv_end = min(S, q0 + BM);
  const int n_tiles = (kv_end + BN - 1) / BN;

  // ---- global -> register staging of one K/V tile
  u32x4 kreg[T::K_PER_T];
  uint32_t vreg[T::V_PER_T][8];

  auto load_tile = [&](int n0) {
#pragma unroll
    for (int i = 0; i < T::K_PER_T; ++i) {
      const int idx = tid + i * NT;
      if (idx < T::K_CHUNKS) {
        const int r = idx / (D / 8), c8 = idx % (D / 8);
        const int n = n0 + r;
        kreg[i] = (n < S) ? *(const u32x4 *)(kb + (int64_t)n * a.k.ss + 8 * c8)
                          : u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int i = 0; i < T::V_PER_T; ++i) {
      const int u = tid + i * NT;
      if (u < T::V_UNITS) {
        const int kg = u / (D / 2), dp = u % (D / 2);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int n = n0 + 8 * kg + j;
          vreg[i][j] = (n < S) ? *(const uint32_t *)(vb + (int64_t)n * a.v.ss + 2 * dp) : 0u;
        }
      }
    }
  };

  auto store_tile = [&](int st) {
#pragma unroll
    for (int i = 0; i < T::K_PER_T; ++i) {
      const int idx = tid + i * NT;
      if (idx < T::K_CHUNKS) {
        const int r = idx / (D / 8), c8 = idx % (D / 8);
        *(u32x4 *)(&sk[st][r * KS + 8 * c8]) = kreg[i];
      }
    }
#pragma unroll
    for (int i = 0; i < T::V_PER_T; ++i) {
      const int u = tid + i * NT;
      if (u < T::V_UNITS) {
        const int kg = u / (D / 2), dp = u % (D / 2);
        u32x4 lo, hi;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          lo[jj] = pack_lo(vreg[i][2 * jj], vreg[i][2 * jj + 1]);
          hi[jj] = pack_hi(vreg[i][2 * jj], vreg[i][2 * jj + 1]);
        }
        *(u32x4 *)(&sv[st][(2 * dp) * VS + 8 * kg]) = lo;
        *(u32x4 *)(&sv[st][(2 * dp + 1) * VS + 8 * kg]) = hi;
      }
    }
  };

  // ---- per-lane running state
  floatx16 oacc[D / 32];
#pragma unroll
  for (int d = 0; d < D / 32; ++d) oacc[d] = floatx16{};
  float m_run = kNegInf;   // running max of c*s (log2 units)
  float l_run = 0.0f;      // this lane's share of the running sum

  const int krow = kperm(l32);
  const float c = a.c;

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int st = t & 1;
    const int n0 = t * BN;
    if (t + 1 < n_tiles) load_tile(n0 + BN);

    // ---- S^T = K Q^T for the two 32-key sub-blocks
    floatx16 s[2];
    bool live[2];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int ns = n0 + 32 * sb;
      live[sb] = !CAUSAL || ns <= wq0 + 31;
      s[sb] = floatx16{};
      if (live[sb]) {
        const f16 *kr = &sk[st][(32 * sb + krow) * KS + 8 * g];
#pragma unroll
        for (int cc = 0; cc < D / 16; ++cc)
          s[sb] = mfma32(*(const half8 *)(kr + 16 * cc), qf[cc], s[sb]);
      }
    }

    // ---- masking (diagonal / ragged tiles only) and the tile row max
    float mx = kNegInf;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int ns = n0 + 32 * sb;
      if (!live[sb]) {
#pragma unroll
        for (int i = 0; i < 16; ++i) s[sb][i] = kNegInf;
        continue;
      }
      const bool need_mask = (CAUSAL && ns + 31 > wq0) || (ns + 31 >= S);
      if (need_mask) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = ns + slot_row(i, g);
          const bool vis = key < S && (!CAUSAL || key <= qrow);
          s[sb][i] = vis ? s[sb][i] : kNegInf;
        }
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[sb][i]);
    }
    mx = fmaxf(mx, xor32(mx));
    const float m_tile = mx * c;

    // ---- lazy rescale of the running state
    const float m_new = fmaxf(m_run, m_tile);
    const bool grow = m_new > m_run + kRescaleLog2;
    if (__any(grow)) {
      const float alpha = grow ? fast_exp2(m_run - m_new) : 1.0f;
      m_run = grow ? m_new : m_run;
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < D / 32; ++d)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[d][i] *= alpha;
    }
    const float neg_m = (m_run == kNegInf) ? 0.0f : -m_run;

    // ---- P = exp2(c*s - m), rounded to fp16; O^T += V^T P^T
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      if (!live[sb]) continue;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        half8 pf;
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          half2 pr = __builtin_convertvector(
              (floatx2){fast_exp2(__builtin_fmaf(s[sb][8 * hh + j], c, neg_m)),
                        fast_exp2(__builtin_fmaf(s[sb][8 * hh + j + 1], c, neg_m))},
              half2);
          l_run = dot2_acc(pr, l_run);
          pf[j] = pr[0];
          pf[j + 1] = pr[1];
        }
        const f16 *vr = &sv[st][l32 * VS + 32 * sb + 16 * hh + 8 * g];
#pragma unroll
        for (int d = 0; d < D / 32; ++d)
          oacc[d] = mfma32(*(const half8 *)(vr + 32 * d * VS), pf, oacc[d]);
      }
    }

    if (t + 1 < n_tiles) store_tile(st ^ 1);
    __syncthreads();
  }

  // ---- epilogue: O = acc / l, LSE = (m + log2 l) * ln2
  const float l_tot = l_run + xor32(l_run);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (qrow < S) {
    f16 *orow = a.o + b * a.o_sb + h * a.o_sh + (int64_t)qrow * a.o_ss;
#pragma unroll
    for (int d = 0; d < D / 32; ++d) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        half4 v4;
#pragma unroll
        for (int j = 0; j < 4; ++j) v4[j] = (f16)(oacc[d][4 * r + j] * inv);
        *(half4 *)(orow + 32 * d + c_row(4 * r, g)) = v4;
      }
    }
    if (a.lse != nullptr && g == 0) {
      const float lse = l_tot > 0.0f ? (m_run + fast_log2(l_tot)) * kLn2 : kPosInf;
      a.lse[(int64_t)bh * S + qrow] = lse;
    }
  }
}

}  // namespace fa
