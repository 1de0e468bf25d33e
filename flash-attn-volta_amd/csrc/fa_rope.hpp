// fa_rope.hpp -- fused QK-norm + rotary position embedding for q and k.
//
// The prologue of an attention layer in the Llama / Qwen2 / Qwen3 families
// (the reference routes them at flash_attn_volta/patch_hf.py:177, :291-303,
// :462, through transformers' Qwen3RMSNorm and apply_rotary_pos_emb):
//
//   n = x * rsqrt(mean_d(x^2) + eps)          (only when a norm weight w is given)
//   y = w * n                                 (else y = x)
//   out[d]       = y[d] cos[d]       - y[d + D/2] sin[d]          d < D/2
//   out[d + D/2] = y[d + D/2] cos[d + D/2] + y[d] sin[d + D/2]
//
// per row (b, s, head) of a (B, S, heads, D) tensor, with cos/sin given per
// (b, s) as (B or 1, S, D) tables.  Everything is computed in fp32 and
// rounded once at the store.
//
// Work mapping (HBM-bound elementwise work with a per-row reduction): a row
// is owned by D/16 adjacent lanes; lane j of a row holds the 16-byte chunks
// [8j, 8j+8) and [D/2 + 8j, D/2 + 8j + 8), i.e. the rotation pairs, so the
// rotation needs no lane exchange and the sum of squares needs log2(D/16)
// xor-shuffles.  Consecutive rows are consecutive heads of one position, so
// the lanes of a wave mostly read the same cos/sin chunks (one L2 line per
// chunk, broadcast by the address coalescer).  q and k are two halves of
// one launch (blockIdx.y).
//
// Backward, with g the gradient of `out`:
//   dy[d]       = g[d] cos[d]             + g[d + D/2] sin[d + D/2]
//   dy[d + D/2] = g[d + D/2] cos[d + D/2] - g[d] sin[d]
//   without a norm:  dx = dy
//   with a norm:     dn = w dy,  dx = r (dn - n mean_d(dn n)),  dw = sum over rows of dy n
// dw is reduced without atomics: each workgroup of the backward grid (a
// fixed, shape-determined count; grid-stride over rows) writes a partial
// (D) row, and fa_rope_dw_reduce_kernel sums the partials in a fixed order,
// so results are reproducible run to run.
#pragma once

#include "fa_common.hpp"

namespace fa {

struct RopeSide {
  const f16 *x;      // fwd: input (B, S, heads, D); bwd: the forward's input (norm only)
  const f16 *g;      // bwd: gradient of the forward's output
  f16 *y;            // fwd: output; bwd: gradient of x
  const f16 *w;      // RMSNorm weight (D), or nullptr
  float *partial;    // bwd with a norm: (gridDim.x, D) fp32 partial dw
  int64_t xb, xs, xh;   // strides of x (elements)
  int64_t gb, gs, gh;   // strides of g
  int64_t yb, ys, yh;   // strides of y
  int heads;
  int64_t rows;      // B * S * heads
};

struct RopeArgs {
  RopeSide side[2];  // q, k
  const f16 *cos;
  const f16 *sin;
  int64_t cb, cs;    // strides of cos / sin over (b, s); b may be 0 (shared table)
  int S;
  float eps;
};

constexpr int kRopeThreads = 256;
constexpr int kRopeUnroll = 1;   // rows per lane per pass (2 measured mixed: -9..+6 %)

template <typename E>
__device__ __forceinline__ void to_f32(u32x4 raw, float *f) {
  const vec8<E> v = __builtin_bit_cast(vec8<E>, raw);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = (float)v[i];
}

template <typename E>
__device__ __forceinline__ u32x4 from_f32(const float *f) {
  vec8<E> v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (E)f[i];
  return __builtin_bit_cast(u32x4, v);
}

__device__ __forceinline__ u32x4 ld16(const f16 *p) {
  return *reinterpret_cast<const u32x4 *>(p);
}

__device__ __forceinline__ void st16(f16 *p, u32x4 v) {
  *reinterpret_cast<u32x4 *>(p) = v;
}

// Sum over the LPR adjacent lanes that own one row.
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
#pragma unroll
  for (int m = 1; m < LPR; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Row index -> element offsets of that row (chunk 0) in a (B, S, heads, D)
// tensor with strides (sb, ss, sh), and of its cos/sin row.  Row indices
// are 32-bit (the launcher rejects more than 2^31 - 1 rows per side):
// 64-bit division by the runtime head count and length would cost several
// times the VALU work of the row itself.
struct RowPos {
  uint32_t b, s, h;
  __device__ __forceinline__ RowPos(uint32_t row, uint32_t heads, uint32_t S) {
    h = row % heads;
    const uint32_t bs = row / heads;
    s = bs % S;
    b = bs / S;
  }
  __device__ __forceinline__ int64_t off(int64_t sb, int64_t ss, int64_t sh) const {
    return (int64_t)b * sb + (int64_t)s * ss + (int64_t)h * sh;
  }
};

template <typename E, int D, bool NORM>
__device__ __forceinline__ void rope_fwd_side(const RopeArgs &a, const RopeSide &t) {
  constexpr int LPR = D / 16;                 // lanes per row
  constexpr int RPB = kRopeThreads / LPR;     // rows per workgroup per pass
  constexpr int U = kRopeUnroll;              // rows per lane per pass
  const int tid = threadIdx.x;
  const int j = tid % LPR;
  float wl[8], wh[8];
  if (NORM) {
    to_f32<E>(ld16(t.w + 8 * j), wl);
    to_f32<E>(ld16(t.w + D / 2 + 8 * j), wh);
  }
  for (int64_t row0 = (int64_t)blockIdx.x * RPB * U; row0 < t.rows;
       row0 += (int64_t)gridDim.x * RPB * U) {
    // all loads of the pass first (U rows per lane in flight), then the math
    u32x4 rx[U][2], rc[U][2], rs[U][2];
    int64_t yo[U];
    bool valid[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t row = row0 + u * RPB + tid / LPR;
      valid[u] = row < t.rows;                // uniform over the LPR lanes of a row
      const RowPos p(valid[u] ? (uint32_t)row : 0u, (uint32_t)t.heads, (uint32_t)a.S);
      const f16 *xp = t.x + p.off(t.xb, t.xs, t.xh) + 8 * j;
      const int64_t co = (int64_t)p.b * a.cb + (int64_t)p.s * a.cs + 8 * j;
      yo[u] = p.off(t.yb, t.ys, t.yh) + 8 * j;
      rx[u][0] = rx[u][1] = u32x4{0, 0, 0, 0};
      if (valid[u]) {
        rx[u][0] = ld16(xp);
        rx[u][1] = ld16(xp + D / 2);
      }
      rc[u][0] = ld16(a.cos + co);
      rc[u][1] = ld16(a.cos + co + D / 2);
      rs[u][0] = ld16(a.sin + co);
      rs[u][1] = ld16(a.sin + co + D / 2);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float xl[8], xh[8], cl[8], ch[8], sl[8], sh[8];
      to_f32<E>(rx[u][0], xl);
      to_f32<E>(rx[u][1], xh);
      to_f32<E>(rc[u][0], cl);
      to_f32<E>(rc[u][1], ch);
      to_f32<E>(rs[u][0], sl);
      to_f32<E>(rs[u][1], sh);
      if (NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += xl[i] * xl[i] + xh[i] * xh[i];
        ss = row_sum<LPR>(ss);
        const float r = rsqrtf(ss * (1.0f / D) + a.eps);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          xl[i] = xl[i] * r * wl[i];
          xh[i] = xh[i] * r * wh[i];
        }
      }
      float ol[8], oh[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        ol[i] = xl[i] * cl[i] - xh[i] * sl[i];
        oh[i] = xh[i] * ch[i] + xl[i] * sh[i];
      }
      if (valid[u]) {
        st16(t.y + yo[u], from_f32<E>(ol));
        st16(t.y + yo[u] + D / 2, from_f32<E>(oh));
      }
    }
  }
}

template <typename E, int D>
__global__ __launch_bounds__(kRopeThreads) void fa_rope_fwd_kernel(RopeArgs a) {
  const RopeSide &t = a.side[blockIdx.y];
  if (t.w != nullptr)
    rope_fwd_side<E, D, true>(a, t);
  else
    rope_fwd_side<E, D, false>(a, t);
}

template <typename E, int D, bool NORM>
__device__ __forceinline__ void rope_bwd_side(const RopeArgs &a, const RopeSide &t) {
  constexpr int LPR = D / 16;
  constexpr int RPB = kRopeThreads / LPR;
  const int tid = threadIdx.x;
  const int j = tid % LPR;
  float wl[8], wh[8], dwl[8], dwh[8];
  if (NORM) {
    to_f32<E>(ld16(t.w + 8 * j), wl);
    to_f32<E>(ld16(t.w + D / 2 + 8 * j), wh);
#pragma unroll
    for (int i = 0; i < 8; ++i) dwl[i] = dwh[i] = 0.0f;
  }
  for (int64_t row0 = (int64_t)blockIdx.x * RPB; row0 < t.rows; row0 += (int64_t)gridDim.x * RPB) {
    const int64_t row = row0 + tid / LPR;
    const bool valid = row < t.rows;
    const RowPos p(valid ? (uint32_t)row : 0u, (uint32_t)t.heads, (uint32_t)a.S);
    const f16 *gp = t.g + p.off(t.gb, t.gs, t.gh) + 8 * j;
    const int64_t co = (int64_t)p.b * a.cb + (int64_t)p.s * a.cs + 8 * j;
    u32x4 rgl = {0, 0, 0, 0}, rgh = {0, 0, 0, 0}, rxl = {0, 0, 0, 0}, rxh = {0, 0, 0, 0};
    if (valid) {
      rgl = ld16(gp);
      rgh = ld16(gp + D / 2);
      if (NORM) {
        const f16 *xp = t.x + p.off(t.xb, t.xs, t.xh) + 8 * j;
        rxl = ld16(xp);
        rxh = ld16(xp + D / 2);
      }
    }
    const u32x4 rcl = ld16(a.cos + co), rch = ld16(a.cos + co + D / 2);
    const u32x4 rsl = ld16(a.sin + co), rsh = ld16(a.sin + co + D / 2);
    float gl[8], gh[8], cl[8], ch[8], sl[8], sh[8], dl[8], dh[8];
    to_f32<E>(rgl, gl);
    to_f32<E>(rgh, gh);
    to_f32<E>(rcl, cl);
    to_f32<E>(rch, ch);
    to_f32<E>(rsl, sl);
    to_f32<E>(rsh, sh);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      dl[i] = gl[i] * cl[i] + gh[i] * sh[i];
      dh[i] = gh[i] * ch[i] - gl[i] * sl[i];
    }
    if (NORM) {
      float xl[8], xh[8];
      to_f32<E>(rxl, xl);
      to_f32<E>(rxh, xh);
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += xl[i] * xl[i] + xh[i] * xh[i];
      ss = row_sum<LPR>(ss);
      const float r = rsqrtf(ss * (1.0f / D) + a.eps);
      float dot = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        xl[i] *= r;   // n
        xh[i] *= r;
        dwl[i] += valid ? dl[i] * xl[i] : 0.0f;   // (a select: n may be NaN past the end)
        dwh[i] += valid ? dh[i] * xh[i] : 0.0f;
        dl[i] *= wl[i];   // dn
        dh[i] *= wh[i];
        dot += dl[i] * xl[i] + dh[i] * xh[i];
      }
      dot = row_sum<LPR>(dot) * (1.0f / D);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        dl[i] = r * (dl[i] - xl[i] * dot);
        dh[i] = r * (dh[i] - xh[i] * dot);
      }
    }
    if (valid) {
      f16 *yp = t.y + p.off(t.yb, t.ys, t.yh) + 8 * j;
      st16(yp, from_f32<E>(dl));
      st16(yp + D / 2, from_f32<E>(dh));
    }
  }
  if (NORM) {
    // Sum the lanes that hold the same chunk (same j) over the rows of the
    // wave, then the waves of the workgroup, into this workgroup's partial.
    __shared__ float s_dw[kRopeThreads / 64][D];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int m = LPR; m < 64; m <<= 1) {
        dwl[i] += __shfl_xor(dwl[i], m, 64);
        dwh[i] += __shfl_xor(dwh[i], m, 64);
      }
    }
    const int lane = tid % 64, w = tid / 64;
    if (lane < LPR) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        s_dw[w][8 * j + i] = dwl[i];
        s_dw[w][D / 2 + 8 * j + i] = dwh[i];
      }
    }
    __syncthreads();
    if (tid < D) {
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < kRopeThreads / 64; ++k) acc += s_dw[k][tid];
      t.partial[(int64_t)blockIdx.x * D + tid] = acc;
    }
  }
}

template <typename E, int D>
__global__ __launch_bounds__(kRopeThreads) void fa_rope_bwd_kernel(RopeArgs a) {
  const RopeSide &t = a.side[blockIdx.y];
  if (t.w != nullptr)
    rope_bwd_side<E, D, true>(a, t);
  else
    rope_bwd_side<E, D, false>(a, t);
}

// dw[side][d] = sum over nblk partials, in a fixed order.  Grid (D / 16, 2),
// 1024 threads: 16 columns x 64 interleaved partial subsets per workgroup,
// the subsets' loads unrolled so that many are in flight, then a tree over
// the 64 subsets in LDS.
constexpr int kRopeReduceThreads = 1024;

template <int D>
__global__ __launch_bounds__(kRopeReduceThreads) void fa_rope_dw_reduce_kernel(
    const float *partial_q, const float *partial_k, float *dw_q, float *dw_k, int nblk) {
  constexpr int SEGS = kRopeReduceThreads / 16;
  const float *part = blockIdx.y == 0 ? partial_q : partial_k;
  float *dw = blockIdx.y == 0 ? dw_q : dw_k;
  if (part == nullptr) return;
  __shared__ float s_acc[SEGS][17];
  const int c = threadIdx.x % 16, seg = threadIdx.x / 16;
  const int col = blockIdx.x * 16 + c;
  float acc = 0.0f;
#pragma unroll 8
  for (int blk = seg; blk < nblk; blk += SEGS) acc += part[(int64_t)blk * D + col];
  s_acc[seg][c] = acc;
  __syncthreads();
#pragma unroll
  for (int w = SEGS / 2; w >= 1; w >>= 1) {
    if (seg < w) s_acc[seg][c] += s_acc[seg + w][c];
    __syncthreads();
  }
  if (seg == 0) dw[col] = s_acc[0][c];
}

}  // namespace fa
