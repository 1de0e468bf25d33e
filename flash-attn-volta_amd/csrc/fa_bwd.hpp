// fa_bwd.hpp -- backward FlashAttention kernels for gfx950.
//
// FlashAttention backward (Dao et al. 2022, Algorithm 4) as three launches,
// the same split as the reference (flash_attn_volta/triton_fa_bwd.py:636-700):
//   1. fa_bwd_preprocess_kernel : delta = rowsum(dO * O) in fp32
//                                 (reference: torch op at triton_fa_bwd.py:650)
//   2. fa_bwd_dkdv_kernel       : one workgroup per key block, sweeping query
//                                 tiles; dV = P^T dO, dK = scale * dS^T Q
//                                 (reference: _fa_bwd_dkdv_kernel_*, :319-580)
//   3. fa_bwd_dq_kernel         : one workgroup per query block, sweeping key
//                                 tiles; dQ = scale * dS K
//                                 (reference: _fa_bwd_dq_kernel_*, :73-307)
// with P = exp(scale * Q K^T - LSE) recomputed from the forward LSE and
// dS = P * (dO V^T - delta).  No atomics and no S x S buffer: every output
// element is written once by one lane, so results are bit-reproducible and a
// causal query row's dQ never reads a key block it cannot see.
//
// Fragment layouts follow fa_common.hpp.  The dK/dV kernel computes S = Q K^T
// with queries as the (permuted) A rows, so a lane owns one key and its
// P / dS values are directly the B operand of dV^T = dO^T P and
// dK^T = Q^T dS.  The dQ kernel computes S^T = K Q^T like the forward, so a
// lane owns one query and its dS^T values feed dQ^T = K^T dS^T.  The
// transposed tiles (Q^T, dO^T, K^T) are built in LDS from register
// transposes while staging.
#pragma once

#include "fa_common.hpp"

namespace fa {

struct BwdArgs {
  TensorDesc q, k, v, dout;
  const float *lse;     // (B, H, S) natural log
  const float *delta;   // (B, H, S)
  f16 *dq, *dk, *dv;
  int64_t dq_sb, dq_ss, dq_sh;
  int64_t dk_sb, dk_ss, dk_sh;
  int64_t dv_sb, dv_ss, dv_sh;
  int B, S, H;
  int n_blocks;         // query blocks (dQ) or key blocks (dK/dV)
  float c;              // |sm_scale| * log2(e), clamped away from 0
  float sm_scale;       // signed scale applied to dQ and dK
  int neg;              // 1 when sm_scale < 0 (K or Q negated in S recompute)
};

struct PreArgs {
  TensorDesc o, dout;
  float *delta;
  int B, S, H;
};

// ---------------------------------------------------------------------------
// delta[b,h,s] = sum_d O * dO.  Each group of D/8 lanes reduces one row from
// 16-byte loads; rows are enumerated in (b, h, s) order so delta writes are
// contiguous.
template <int D>
__global__ __launch_bounds__(256) void fa_bwd_preprocess_kernel(PreArgs a) {
  constexpr int LPR = D / 8;               // lanes per row
  constexpr int RPB = 256 / LPR;           // rows per block
  const int tid = threadIdx.x;
  const int64_t row = (int64_t)blockIdx.x * RPB + tid / LPR;
  const int part = tid % LPR;
  const int64_t total = (int64_t)a.B * a.H * a.S;
  float acc = 0.0f;
  if (row < total) {
    const int s = (int)(row % a.S);
    const int64_t bh = row / a.S;
    const int h = (int)(bh % a.H), b = (int)(bh / a.H);
    const half8 ov = *(const half8 *)(a.o.head(b, h) + (int64_t)s * a.o.ss + 8 * part);
    const half8 gv = *(const half8 *)(a.dout.head(b, h) + (int64_t)s * a.dout.ss + 8 * part);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc = __builtin_fmaf((float)ov[j], (float)gv[j], acc);
  }
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (row < total && part == 0) a.delta[row] = acc;
}

// ---------------------------------------------------------------------------
// Staging of a ROWS x D fp16 tile (rows r0 .. r0+ROWS-1 of one (b,h), rows
// >= S read as zero) into LDS, optionally both row-major [row][d] (stride
// RS halves) and transposed [d][row] (stride TS halves).  A unit is 8 rows x
// 2 columns: eight dword loads, then the row-major copy is eight dword
// stores and the transposed copy two 16-byte stores after a register
// transpose.
template <int ROWS, int D, int NT>
struct TileStager {
  static constexpr int UNITS = (ROWS / 8) * (D / 2);
  static constexpr int PER_T = (UNITS + NT - 1) / NT;
  uint32_t r[PER_T][8];

  __device__ __forceinline__ void load(const f16 *base, int64_t ss, int r0, int S, int tid) {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int u = tid + i * NT;
      if (u < UNITS) {
        const int rg = u / (D / 2), dp = u % (D / 2);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int n = r0 + 8 * rg + j;
          r[i][j] = (n < S) ? *(const uint32_t *)(base + (int64_t)n * ss + 2 * dp) : 0u;
        }
      }
    }
  }

  template <int RS, int TS>
  __device__ __forceinline__ void store(f16 *rowm, f16 *trans, int tid) const {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int u = tid + i * NT;
      if (u < UNITS) {
        const int rg = u / (D / 2), dp = u % (D / 2);
        if (rowm != nullptr) {
#pragma unroll
          for (int j = 0; j < 8; ++j)
            *(uint32_t *)(rowm + (8 * rg + j) * RS + 2 * dp) = r[i][j];
        }
        if (trans != nullptr) {
          u32x4 lo, hi;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            lo[jj] = pack_lo(r[i][2 * jj], r[i][2 * jj + 1]);
            hi[jj] = pack_hi(r[i][2 * jj], r[i][2 * jj + 1]);
          }
          *(u32x4 *)(trans + (2 * dp) * TS + 8 * rg) = lo;
          *(u32x4 *)(trans + (2 * dp + 1) * TS + 8 * rg) = hi;
        }
      }
    }
  }
};

// Row-major staging of a ROWS x D tile with 16-byte loads and stores.
template <int ROWS, int D, int NT>
struct RowStager {
  static constexpr int CHUNKS = ROWS * D / 8;
  static constexpr int PER_T = (CHUNKS + NT - 1) / NT;
  u32x4 r[PER_T];

  __device__ __forceinline__ void load(const f16 *base, int64_t ss, int r0, int S, int tid) {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int idx = tid + i * NT;
      if (idx < CHUNKS) {
        const int rr = idx / (D / 8), c8 = idx % (D / 8);
        const int n = r0 + rr;
        r[i] = (n < S) ? *(const u32x4 *)(base + (int64_t)n * ss + 8 * c8) : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }

  template <int RS>
  __device__ __forceinline__ void store(f16 *rowm, int tid) const {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int idx = tid + i * NT;
      if (idx < CHUNKS) {
        const int rr = idx / (D / 8), c8 = idx % (D / 8);
        *(u32x4 *)(rowm + rr * RS + 8 * c8) = r[i];
      }
    }
  }
};

// Store a D^T x 32 accumulator set (lane = row `row`, slots = columns) as
// fp16 row `row` of a (.., D) tensor, scaled by `mul`.
template <int D>
__device__ __forceinline__ void store_row_fp16(f16 *dst, const floatx16 (&acc)[D / 32], float mul, int g) {
#pragma unroll
  for (int d = 0; d < D / 32; ++d) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      half4 v4;
#pragma unroll
      for (int j = 0; j < 4; ++j) v4[j] = (f16)(acc[d][4 * r + j] * mul);
      *(half4 *)(dst + 32 * d + c_row(4 * r, g)) = v4;
    }
  }
}

// ---------------------------------------------------------------------------
// dK / dV: workgroup = NW waves, wave w owns keys k0 + 32w .. +31 (lane l32
// owns key k0 + 32w + l32).  Query tiles of BQ = 64 rows stream through LDS
// as Q, Q^T, dO, dO^T plus their LSE and delta.
template <int D, int NW>
struct DkdvTile {
  static constexpr int BK = 32 * NW;
  static constexpr int BQ = 64;
  static constexpr int NT = 64 * NW;
  static constexpr int RS = D + 8;
  static constexpr int TS = BQ + 8;
  static constexpr int LDS_ROW = BQ * RS;
  static constexpr int LDS_T = D * TS;
};

template <int D, bool CAUSAL, int NW>
__global__ __launch_bounds__(64 * NW) void fa_bwd_dkdv_kernel(BwdArgs a) {
  using T = DkdvTile<D, NW>;
  constexpr int BK = T::BK, BQ = T::BQ, NT = T::NT, RS = T::RS, TS = T::TS;
  __shared__ __attribute__((aligned(16))) f16 s_q[2][T::LDS_ROW];
  __shared__ __attribute__((aligned(16))) f16 s_qt[2][T::LDS_T];
  __shared__ __attribute__((aligned(16))) f16 s_do[2][T::LDS_ROW];
  __shared__ __attribute__((aligned(16))) f16 s_dot[2][T::LDS_T];
  __shared__ __attribute__((aligned(16))) float s_lse[2][BQ];
  __shared__ __attribute__((aligned(16))) float s_dl[2][BQ];

  const int S = a.S;
  const int BH = a.B * a.H;
  const int bid = blockIdx.x;
  const int bh = bid % BH;
  // Causal: low key blocks see the most queries, so run them first.
  const int kt = CAUSAL ? bid / BH : a.n_blocks - 1 - bid / BH;
  const int b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int k0 = kt * BK;
  const int wk0 = k0 + 32 * w;
  const int key = wk0 + l32;

  const f16 *qb = a.q.head(b, h);
  const f16 *kb = a.k.head(b, h);
  const f16 *vb = a.v.head(b, h);
  const f16 *gb = a.dout.head(b, h);
  const float *lse_b = a.lse + (int64_t)bh * S;
  const float *dl_b = a.delta + (int64_t)bh * S;

  // K^T and V^T fragments (B operands): K[key][16c + 8g .. +7]
  half8 kf[D / 16], vf[D / 16];
  if (key < S) {
    const f16 *kr = kb + (int64_t)key * a.k.ss + 8 * g;
    const f16 *vr = vb + (int64_t)key * a.v.ss + 8 * g;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      kf[c] = *(const half8 *)(kr + 16 * c);
      vf[c] = *(const half8 *)(vr + 16 * c);
    }
    if (a.neg) {
#pragma unroll
      for (int c = 0; c < D / 16; ++c) kf[c] = neg8(kf[c]);
    }
  } else {
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      kf[c] = half8{};
      vf[c] = half8{};
    }
  }

  floatx16 dk[D / 32], dv[D / 32];
#pragma unroll
  for (int d = 0; d < D / 32; ++d) {
    dk[d] = floatx16{};
    dv[d] = floatx16{};
  }

  const int m_begin = CAUSAL ? (k0 / BQ) * BQ : 0;
  const int n_tiles = (S > m_begin) ? (S - m_begin + BQ - 1) / BQ : 0;
  const int qperm = kperm(l32);
  const float c = a.c;

  TileStager<BQ, D, NT> stq, stg;
  float lse_r = 0.0f, dl_r = 0.0f;
  auto load_tile = [&](int m0) {
    stq.load(qb, a.q.ss, m0, S, tid);
    stg.load(gb, a.dout.ss, m0, S, tid);
    if (tid < BQ) {
      const int m = m0 + tid;
      // rows past S: +inf LSE makes P exactly 0 there
      lse_r = (m < S) ? lse_b[m] * kLog2e : kPosInf;
      dl_r = (m < S) ? dl_b[m] : 0.0f;
    }
  };
  auto store_tile = [&](int st) {
    stq.template store<RS, TS>(s_q[st], s_qt[st], tid);
    stg.template store<RS, TS>(s_do[st], s_dot[st], tid);
    if (tid < BQ) {
      s_lse[st][tid] = lse_r;
      s_dl[st][tid] = dl_r;
    }
  };

  if (n_tiles > 0) {
    load_tile(m_begin);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int st = t & 1;
    const int m0 = m_begin + t * BQ;
    if (t + 1 < n_tiles) load_tile(m0 + BQ);

#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      const int ms = m0 + 32 * qs;
      // whole sub-block above this wave's keys' diagonal: nothing visible
      if (CAUSAL && ms + 31 < wk0) continue;
      if (ms >= S) continue;

      floatx16 sacc = floatx16{}, dpacc = floatx16{};
      const f16 *qr = &s_q[st][(32 * qs + qperm) * RS + 8 * g];
      const f16 *gr = &s_do[st][(32 * qs + qperm) * RS + 8 * g];
#pragma unroll
      for (int cc = 0; cc < D / 16; ++cc) {
        sacc = mfma32(*(const half8 *)(qr + 16 * cc), kf[cc], sacc);
        dpacc = mfma32(*(const half8 *)(gr + 16 * cc), vf[cc], dpacc);
      }
      // slot i <-> query ms + slot_row(i, g); lane <-> key
      const bool need_mask = (CAUSAL && ms < wk0 + 31) || (ms + 31 >= S) || (wk0 + 31 >= S);
      half8 pf[2], dsf[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const floatx4 lse_lo = *(const floatx4 *)&s_lse[st][32 * qs + 16 * hh + 8 * g];
        const floatx4 lse_hi = *(const floatx4 *)&s_lse[st][32 * qs + 16 * hh + 8 * g + 4];
        const floatx4 dl_lo = *(const floatx4 *)&s_dl[st][32 * qs + 16 * hh + 8 * g];
        const floatx4 dl_hi = *(const floatx4 *)&s_dl[st][32 * qs + 16 * hh + 8 * g + 4];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int i = 8 * hh + j;
          const float l2 = j < 4 ? lse_lo[j] : lse_hi[j - 4];
          const float dl = j < 4 ? dl_lo[j] : dl_hi[j - 4];
          float p = fast_exp2(__builtin_fmaf(sacc[i], c, -l2));
          if (need_mask) {
            const int m = ms + slot_row(i, g);
            const bool vis = m < S && key < S && (!CAUSAL || key <= m);
            p = vis ? p : 0.0f;
          }
          const float ds = p * (dpacc[i] - dl);
          pf[hh][j] = (f16)p;
          dsf[hh][j] = (f16)ds;
        }
      }
      // dV^T += dO^T P ; dK^T += Q^T dS   (k = queries ms + 16hh + 8g ..)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const f16 *gt = &s_dot[st][l32 * TS + 32 * qs + 16 * hh + 8 * g];
        const f16 *qt = &s_qt[st][l32 * TS + 32 * qs + 16 * hh + 8 * g];
#pragma unroll
        for (int d = 0; d < D / 32; ++d) {
          dv[d] = mfma32(*(const half8 *)(gt + 32 * d * TS), pf[hh], dv[d]);
          dk[d] = mfma32(*(const half8 *)(qt + 32 * d * TS), dsf[hh], dk[d]);
        }
      }
    }

    if (t + 1 < n_tiles) store_tile(st ^ 1);
    __syncthreads();
  }

  if (key < S) {
    store_row_fp16<D>(a.dk + b * a.dk_sb + h * a.dk_sh + (int64_t)key * a.dk_ss, dk, a.sm_scale, g);
    store_row_fp16<D>(a.dv + b * a.dv_sb + h * a.dv_sh + (int64_t)key * a.dv_ss, dv, 1.0f, g);
  }
}

// ---------------------------------------------------------------------------
// dQ: workgroup = NW waves, wave w owns queries q0 + 32w .. +31 (lane l32
// owns one query).  Key tiles of BN = 64 rows stream through LDS as K, K^T
// and V.
template <int D, int NW>
struct DqTile {
  static constexpr int BM = 32 * NW;
  static constexpr int BN = 64;
  static constexpr int NT = 64 * NW;
  static constexpr int RS = D + 8;
  static constexpr int TS = BN + 8;
  static constexpr int LDS_ROW = BN * RS;
  static constexpr int LDS_T = D * TS;
};

template <int D, bool CAUSAL, int NW>
__global__ __launch_bounds__(64 * NW) void fa_bwd_dq_kernel(BwdArgs a) {
  using T = DqTile<D, NW>;
  constexpr int BM = T::BM, BN = T::BN, NT = T::NT, RS = T::RS, TS = T::TS;
  __shared__ __attribute__((aligned(16))) f16 s_k[2][T::LDS_ROW];
  __shared__ __attribute__((aligned(16))) f16 s_kt[2][T::LDS_T];
  __shared__ __attribute__((aligned(16))) f16 s_v[2][T::LDS_ROW];

  const int S = a.S;
  const int BH = a.B * a.H;
  const int bid = blockIdx.x;
  const int bh = bid % BH;
  const int qt = a.n_blocks - 1 - bid / BH;   // heaviest causal blocks first
  const int b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int q0 = qt * BM;
  const int wq0 = q0 + 32 * w;
  const int qrow = wq0 + l32;

  const f16 *qb = a.q.head(b, h);
  const f16 *kb = a.k.head(b, h);
  const f16 *vb = a.v.head(b, h);
  const f16 *gb = a.dout.head(b, h);

  half8 qf[D / 16], gf[D / 16];
  float l2 = kPosInf, dl = 0.0f;
  if (qrow < S) {
    const f16 *qr = qb + (int64_t)qrow * a.q.ss + 8 * g;
    const f16 *gr = gb + (int64_t)qrow * a.dout.ss + 8 * g;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      qf[c] = *(const half8 *)(qr + 16 * c);
      gf[c] = *(const half8 *)(gr + 16 * c);
    }
    if (a.neg) {
#pragma unroll
      for (int c = 0; c < D / 16; ++c) qf[c] = neg8(qf[c]);
    }
    l2 = a.lse[(int64_t)bh * S + qrow] * kLog2e;
    dl = a.delta[(int64_t)bh * S + qrow];
  } else {
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      qf[c] = half8{};
      gf[c] = half8{};
    }
  }

  floatx16 dq[D / 32];
#pragma unroll
  for (int d = 0; d < D / 32; ++d) dq[d] = floatx16{};

  int kv_end = S;
  if (CAUSAL) kv_end = min(S, q0 + BM);
  const int n_tiles = (kv_end + BN - 1) / BN;
  const int krow = kperm(l32);
  const float c = a.c;

  TileStager<BN, D, NT> stk;
  RowStager<BN, D, NT> stv;
  auto load_tile = [&](int n0) {
    stk.load(kb, a.k.ss, n0, S, tid);
    stv.load(vb, a.v.ss, n0, S, tid);
  };
  auto store_tile = [&](int st) {
    stk.template store<RS, TS>(s_k[st], s_kt[st], tid);
    stv.template store<RS>(s_v[st], tid);
  };

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int st = t & 1;
    const int n0 = t * BN;
    if (t + 1 < n_tiles) load_tile(n0 + BN);

#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int ns = n0 + 32 * sb;
      if (CAUSAL && ns > wq0 + 31) continue;
      if (ns >= S) continue;
      floatx16 sacc = floatx16{}, dpacc = floatx16{};
      const f16 *kr = &s_k[st][(32 * sb + krow) * RS + 8 * g];
      const f16 *vr = &s_v[st][(32 * sb + krow) * RS + 8 * g];
#pragma unroll
      for (int cc = 0; cc < D / 16; ++cc) {
        sacc = mfma32(*(const half8 *)(kr + 16 * cc), qf[cc], sacc);
        dpacc = mfma32(*(const half8 *)(vr + 16 * cc), gf[cc], dpacc);
      }
      const bool need_mask = (CAUSAL && ns + 31 > wq0) || (ns + 31 >= S);
      half8 dsf[2];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float p = fast_exp2(__builtin_fmaf(sacc[i], c, -l2));
        if (need_mask) {
          const int n = ns + slot_row(i, g);
          const bool vis = n < S && (!CAUSAL || n <= qrow);
          p = vis ? p : 0.0f;
        }
        dsf[i >> 3][i & 7] = (f16)(p * (dpacc[i] - dl));
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const f16 *ktr = &s_kt[st][l32 * TS + 32 * sb + 16 * hh + 8 * g];
#pragma unroll
        for (int d = 0; d < D / 32; ++d)
          dq[d] = mfma32(*(const half8 *)(ktr + 32 * d * TS), dsf[hh], dq[d]);
      }
    }

    if (t + 1 < n_tiles) store_tile(st ^ 1);
    __syncthreads();
  }

  if (qrow < S)
    store_row_fp16<D>(a.dq + b * a.dq_sb + h * a.dq_sh + (int64_t)qrow * a.dq_ss, dq, a.sm_scale, g);
}

}  // namespace fa
