// fa_api.hip -- the extern "C" entry points declared in include/fa_mi355x.h.
//
// Each entry point validates its arguments on the host (before any HIP call,
// so the checks behave the same without a GPU), picks the kernel
// instantiation for (D, causal) and launches it asynchronously on the
// caller's stream.  Nothing here allocates device memory.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <atomic>
#include <type_traits>

#include "fa_mi355x.h"
#include "fa_bwd.hpp"
#include "fa_fwd.hpp"
#include "fa_rope.hpp"

namespace {

using fa::f16;

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Problem sizes: q, o, dout, dq are (B, Sq, H, D); k, v, dk, dv are
// (B, Sk, Hk, D); query head h uses key/value head h / (H / Hk).
struct Shape {
  int B, Sq, Sk, H, Hk, D;
  int dtype;   // FA_DTYPE_F16 or FA_DTYPE_BF16
};

int check_shape(const Shape &s) {
  if (s.dtype != FA_DTYPE_F16 && s.dtype != FA_DTYPE_BF16) return FA_ERR_DTYPE;
  if (s.B <= 0 || s.Sq <= 0 || s.Sk <= 0 || s.H <= 0 || s.Hk <= 0) return FA_ERR_SHAPE;
  if (s.H % s.Hk != 0) return FA_ERR_SHAPE;
  if (s.D != 32 && s.D != 64 && s.D != 128) return FA_ERR_HEAD_DIM;
  // Per-(b,h) row offsets use 32-bit query/key indices and the grid is 1-D.
  if (s.Sq > (1 << 30) || s.Sk > (1 << 30)) return FA_ERR_TOO_LARGE;
  const int64_t bh = (int64_t)s.B * s.H;
  if (bh > (int64_t)1 << 30) return FA_ERR_TOO_LARGE;
  if (bh * (int64_t)s.Sq > ((int64_t)1 << 40)) return FA_ERR_TOO_LARGE;
  return FA_OK;
}

// Rows of one head that the attention kernels stage per tile, at most (the
// dK/dV layouts' 128-key / 128-query tiles): inside a tile a lane addresses
// its row with a 32-bit buffer offset, row * seq_stride * 2 bytes
// (fa_common.hpp DmaStager), so (kMaxTileRows - 1) rows must span < 2^31.
constexpr int64_t kMaxTileRows = 128;

// True when the (b, s, h) rows of D elements never share an element: with
// the dimensions of size > 1 taken in increasing stride order, each stride
// is at least the extent of the rows nested inside it.  Every layout the
// wrappers produce (contiguous tensors, permuted and sliced views) passes;
// a written tensor that fails would have workgroups store the same bytes.
bool rows_disjoint(const int64_t *st, int B, int S, int H, int D) {
  int64_t stride[3] = {st[0], st[1], st[2]};
  int64_t size[3] = {B, S, H};
  for (int i = 1; i < 3; ++i)   // insertion sort of three dims by stride
    for (int j = i; j > 0 && stride[j] < stride[j - 1]; --j) {
      const int64_t ts = stride[j], tn = size[j];
      stride[j] = stride[j - 1];
      size[j] = size[j - 1];
      stride[j - 1] = ts;
      size[j - 1] = tn;
    }
  int64_t extent = D;
  for (int i = 0; i < 3; ++i) {
    if (size[i] == 1) continue;
    if (stride[i] < extent) return false;
    extent += stride[i] * (size[i] - 1);
  }
  return true;
}

// A (B, S, H, D) tensor with the given element strides.  `tile_rows` > 0
// bounds the sequence stride for kernels that address that many rows of a
// head with 32-bit offsets (0: every offset is 64-bit).  `output`: the
// tensor is written, so its rows must not overlap.
int check_tensor(const void *p, const int64_t *st, int B, int S, int H, int D, bool output,
                 int64_t tile_rows) {
  if (p == nullptr || st == nullptr) return FA_ERR_NULL_POINTER;
  if (!aligned16(p)) return FA_ERR_ALIGNMENT;
  if (st[3] != 1) return FA_ERR_STRIDE;
  for (int i = 0; i < 3; ++i) {
    if (st[i] < 0 || (st[i] & 7) != 0) return FA_ERR_STRIDE;
  }
  // Largest element offset must fit comfortably in int64.
  const double span = (double)(B - 1) * st[0] + (double)(S - 1) * st[1] +
                      (double)(H - 1) * st[2] + D;
  if (span > 4.0e18) return FA_ERR_TOO_LARGE;
  if (tile_rows > 0 && S > 1 && (tile_rows - 1) * st[1] * 2 + 2 * (int64_t)D > INT32_MAX)
    return FA_ERR_TOO_LARGE;
  if (output && !rows_disjoint(st, B, S, H, D)) return FA_ERR_STRIDE;
  return FA_OK;
}

int check_q_like(const void *p, const int64_t *st, const Shape &s, bool output = false) {
  return check_tensor(p, st, s.B, s.Sq, s.H, s.D, output, kMaxTileRows);
}

int check_kv_like(const void *p, const int64_t *st, const Shape &s, bool output = false) {
  return check_tensor(p, st, s.B, s.Sk, s.Hk, s.D, output, kMaxTileRows);
}

// Kernel view of a tensor with S rows per head; a single row's sequence
// stride is never used to address anything, so it is passed as 0 (a large
// one would otherwise wrap the 32-bit offsets of the rows a tile reads past
// the end).
fa::TensorDesc desc(const void *p, const int64_t *st, int S) {
  return fa::TensorDesc{static_cast<const f16 *>(p), st[0], S > 1 ? st[1] : 0, st[2]};
}

// Kernel-side score scale: |sm_scale| * log2(e), never exactly zero so that
// masked (-inf) scores stay -inf; a zero scale then gives scores of ~1e-30,
// whose exp2 is 1 to fp32 precision, i.e. uniform attention as intended.
float kernel_scale(float sm_scale) {
  float c = fabsf(sm_scale) * fa::kLog2e;
  return c < 1e-30f ? 1e-30f : c;
}

// fa::BwdArgs::lse_mul for kernel scale c: the dK/dV kernel's own
// definition of cr, in the same IEEE operations
float lse_seed_mul(float c, int dtype) {
  const float ck = dtype == FA_DTYPE_F16 ? fminf(c, 1.0f) : 1.0f;
  return -fa::kLog2e / (c / ck);
}

int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? FA_OK : FA_ERR_LAUNCH;
}

// Device of `stream`: kernels run on the device their stream belongs to,
// which need not be the host thread's current device.  The NULL stream (or
// a stream the runtime cannot place) means the current device.
int stream_device(hipStream_t stream) {
  int dev = -1;
  if (stream != nullptr) {
    if (hipStreamGetDevice(stream, &dev) == hipSuccess && dev >= 0) return dev;
    (void)hipGetLastError();   // not a launch error of the call
  }
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return -1;
  }
  return dev;
}

// The stream the current entry point launches on, per host thread: set by
// LaunchDevice at the top of each launching path (nested paths keep the
// outer one's), so the launch decisions below follow the stream's device
// without the stream passed through every helper.  The device is looked up
// on first use, after the arguments have been validated.
struct LaunchTarget {
  bool active = false;
  void *stream = nullptr;
  int dev = -2;   // -2: not looked up yet
};
thread_local LaunchTarget t_launch;

struct LaunchDevice {
  LaunchTarget saved;
  explicit LaunchDevice(void *stream) : saved(t_launch) {
    if (!t_launch.active || t_launch.stream != stream) t_launch = LaunchTarget{true, stream, -2};
  }
  ~LaunchDevice() { t_launch = saved; }
  LaunchDevice(const LaunchDevice &) = delete;
  LaunchDevice &operator=(const LaunchDevice &) = delete;
};

int launch_device() {
  if (t_launch.active) {
    if (t_launch.dev == -2) t_launch.dev = stream_device(static_cast<hipStream_t>(t_launch.stream));
    return t_launch.dev;
  }
  return stream_device(nullptr);
}

// Compute units of the launch device (cached per device; 256 on MI355X).
// The cache is atomic: entry points may be called from several host
// threads at once (they all store the same value).
int device_cus() {
  static std::atomic<int> cache[64];
  const int dev = launch_device();
  if (dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Split each tile's rows across two waves when the grid of 128-row
// workgroups would leave the GPU under-filled: fewer than one round of the
// resident workgroup slots (`per_cu` per CU), two rounds for causal, whose
// light blocks finish early and leave the heavy blocks' long sweeps as the
// critical path.  Used by the forward and both backward kernels (the split
// is over keys in the forward and dQ, over queries in dK/dV); `rows` is
// the length of the blocked dimension, `heads` the number of (b, head)
// pairs the grid covers.  per_cu = 2 for the kernels that run two
// workgroups per CU; 1 for D = 128 dK/dV, whose registers allow one
// (measured: unsplit is 11 % faster at (1,4096,8,128) non-causal and 4 %
// at (1,4096,16,128) causal, split stays 19 % faster at (1,4096,8,128)
// causal).
bool row_split(int rows, int64_t heads, bool causal, int per_cu = 2) {
  const int64_t wgs = (int64_t)((rows + 127) / 128) * heads;
  return wgs < (int64_t)(causal ? 2 : 1) * per_cu * device_cus();
}

// Workgroups of `Kernel` (launched with `threads` per workgroup) resident
// per CU, from the runtime's occupancy calculator; cached per kernel
// instantiation (the template argument is the kernel itself: kernels of
// one argument type share a function-pointer type) -- every device here is
// the same gfx950 part.  0 when the runtime cannot tell (not cached: a
// later call asks again).
template <auto Kernel>
int resident_per_cu(int threads) {
  static std::atomic<int> cache{0};
  int n = cache.load(std::memory_order_relaxed);
  if (n <= 0) {
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, Kernel, threads, 0) != hipSuccess) {
      // the failed query's error must not look like a launch error
      (void)hipGetLastError();
      return 0;
    }
    n = blocks > 0 ? blocks : 0;
    if (n > 0) cache.store(n, std::memory_order_relaxed);
  }
  return n;
}

// Causal block order of the forward and dQ kernels (zigzag flag): heaviest
// block first when the grid takes more than one round of resident
// workgroups, so that each slot freed takes the heaviest block left; zigzag
// heavy / light when the grid fits one round (then the order only decides
// which blocks share a CU, and mixing heavy with light evens the CUs'
// loads) or when a head has fewer than 16 blocks.  Measured against
// zigzag everywhere: several-round grids -4 to -12 % (forward) and -3.5 to
// -6 % (dQ); one-round grids +2 to +5 % with heaviest-first.
int zigzag_order(int64_t grid, int n_blocks, int per_cu) {
  if (per_cu <= 0 || n_blocks < 16) return 1;
  return grid <= (int64_t)per_cu * device_cus() ? 1 : 0;
}

// The forward kernel's pre-scaled mode (Q scaled by c in fp16, the score
// MFMAs seeded with -max): fp16 with c <= 1, where the scaled Q cannot
// overflow; bf16 and larger scales apply c in the softmax instead.
template <typename E>
bool fwd_prescaled(const fa::FwdArgs &a) {
  return std::is_same<E, fa::f16>::value && a.c <= 1.0f;
}

template <typename E, int D, bool CAUSAL, int KSPLIT, bool PRE, int NW = 4>
int launch_fwd_split(const fa::FwdArgs &args, hipStream_t stream) {
  using T = fa::FwdTile<D, KSPLIT, NW>;
  fa::FwdArgs a = args;
  a.n_qtiles = (a.Sq + T::BM - 1) / T::BM;
  const int64_t grid = (int64_t)a.n_qtiles * a.B * a.H;
  if (grid > 0x7fffffff) return FA_ERR_TOO_LARGE;
  constexpr auto kernel = fa::fa_fwd_kernel<E, D, CAUSAL, KSPLIT, false, PRE, false, NW>;
  a.zigzag = CAUSAL ? zigzag_order(grid, a.n_qtiles, resident_per_cu<kernel>(T::NT)) : 0;
  hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(T::NT), 0, stream, a);
  return launch_status();
}

template <typename E, int D, bool CAUSAL, int KSPLIT>
int launch_fwd_mode(const fa::FwdArgs &a, hipStream_t stream) {
  // Non-causal D = 64 grids of at least one 256-query tile per CU: eight
  // waves, 256 queries per workgroup sharing each K / V tile (half the
  // tile DMAs per query).
  if constexpr (D == 64 && !CAUSAL && KSPLIT == 1) {
    if ((int64_t)((a.Sq + 255) / 256) * a.B * a.H >= device_cus()) {
      if constexpr (std::is_same<E, fa::f16>::value) {
        if (fwd_prescaled<E>(a)) return launch_fwd_split<E, D, CAUSAL, 1, true, 8>(a, stream);
      }
      return launch_fwd_split<E, D, CAUSAL, 1, false, 8>(a, stream);
    }
  }
  // Non-causal D = 128 key-split grids of at least one 128-query tile per
  // CU: eight waves (four query groups x two key halves) sharing each K / V
  // tile.
  if constexpr (D == 128 && !CAUSAL && KSPLIT == 2) {
    if ((int64_t)((a.Sq + 127) / 128) * a.B * a.H >= device_cus()) {
      if constexpr (std::is_same<E, fa::f16>::value) {
        if (fwd_prescaled<E>(a)) return launch_fwd_split<E, D, CAUSAL, 2, true, 8>(a, stream);
      }
      return launch_fwd_split<E, D, CAUSAL, 2, false, 8>(a, stream);
    }
  }
  // (not the unsplit D = 128 layout: the -max seed's 16 registers would
  // push it past 256 VGPRs, measured +3-4 % on the grids that use it)
  if constexpr (std::is_same<E, fa::f16>::value && !(D == 128 && KSPLIT == 1)) {
    if (fwd_prescaled<E>(a)) return launch_fwd_split<E, D, CAUSAL, KSPLIT, true>(a, stream);
  }
  return launch_fwd_split<E, D, CAUSAL, KSPLIT, false>(a, stream);
}

template <typename E, int D, bool CAUSAL>
int launch_fwd(const fa::FwdArgs &a, hipStream_t stream) {
  // Non-causal grids of at most one 64-query workgroup per CU, where the
  // four-wave key-split layout would run one wave per SIMD: eight waves per
  // workgroup, each query group's keys in four parts of 128-key tiles --
  // twice the waves in flight on the same grid.
  if constexpr (!CAUSAL && D >= 64) {
    if ((int64_t)((a.Sq + 63) / 64) * a.B * a.H <= device_cus()) {
      if constexpr (std::is_same<E, fa::f16>::value) {
        if (fwd_prescaled<E>(a)) return launch_fwd_split<E, D, CAUSAL, 4, true, 8>(a, stream);
      }
      return launch_fwd_split<E, D, CAUSAL, 4, false, 8>(a, stream);
    }
  }
  return row_split(a.Sq, (int64_t)a.B * a.H, CAUSAL) ? launch_fwd_mode<E, D, CAUSAL, 2>(a, stream)
                                                     : launch_fwd_mode<E, D, CAUSAL, 1>(a, stream);
}

template <typename E, int D>
int launch_pre(const fa::PreArgs &a, hipStream_t stream) {
  constexpr int RPB = 128;   // two lanes per row, 128 rows of one (b, h) per workgroup
  const int64_t grid = (int64_t)a.B * a.H * ((a.S + RPB - 1) / RPB);
  if (grid > 0x7fffffff) return FA_ERR_TOO_LARGE;
  hipLaunchKernelGGL((fa::fa_bwd_preprocess_kernel<E, D>), dim3((unsigned)grid), dim3(256), 0,
                     stream, a);
  return launch_status();
}

template <typename E, int D, bool CAUSAL, int SPLIT>
int launch_dkdv_split(const fa::BwdArgs &args, hipStream_t stream) {
  using T = fa::DkdvTile<D, SPLIT>;
  fa::BwdArgs a = args;
  a.n_blocks = (a.Sk + T::BK - 1) / T::BK;
  // a split key block takes two workgroups
  const int64_t grid = ((int64_t)a.n_blocks + a.split_kt) * a.B * a.Hk;
  if (grid > 0x7fffffff) return FA_ERR_TOO_LARGE;
  constexpr auto kernel = fa::fa_bwd_dkdv_kernel<E, D, CAUSAL, SPLIT>;
  // Causal order (unsplit grids): heaviest first, except zigzag heavy /
  // light for long sweeps (>= 48 blocks per head) on grids of at most 1.5
  // rounds of resident workgroups.  Measured at three per CU (D = 64):
  // zigzag -3 % at (1,4096,16,64) (1.33 rounds), -1.4 % at (1,3072,16,64);
  // heaviest first -5 % at (1,2048,32,64) (32 blocks per head), -10 % at
  // (1,4096,32,64) (2.67 rounds), -17 % on the D = 128 grids.
  if (CAUSAL && a.split_kt == 0 && a.n_blocks >= 48) {
    const int per_cu = resident_per_cu<kernel>(T::NT);
    a.zigzag = per_cu > 0 && 2 * grid <= 3 * (int64_t)per_cu * device_cus() ? 1 : 0;
  } else {
    a.zigzag = 0;
  }
  hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(T::NT), 0, stream, a);
  return launch_status();
}

template <typename E, int D, bool CAUSAL, int SPLIT, bool PRE, int NW = 4>
int launch_dq_split(const fa::BwdArgs &args, hipStream_t stream) {
  using T = fa::DqTile<D, SPLIT, NW>;
  fa::BwdArgs a = args;
  a.n_blocks = (a.Sq + T::BM - 1) / T::BM;
  // a split query block takes two workgroups
  const int64_t grid = ((int64_t)a.n_blocks + a.dq_split) * a.B * a.H;
  if (grid > 0x7fffffff) return FA_ERR_TOO_LARGE;
  constexpr auto kernel = fa::fa_bwd_dq_kernel<E, D, CAUSAL, SPLIT, PRE, NW>;
  a.zigzag = CAUSAL ? zigzag_order(grid, a.n_blocks, resident_per_cu<kernel>(T::NT)) : 0;
  hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(T::NT), 0, stream, a);
  return launch_status();
}

template <typename E, int D, bool CAUSAL>
int launch_dkdv(const fa::BwdArgs &a, hipStream_t stream) {
  // the key-block split runs in the eight-wave D = 128 kernel and in the
  // D = 64 query-split kernel (dkdv_split_plan).  Causal D = 128 takes the
  // eight-wave layout on every grid: the layout of fa_bwd's fused launch,
  // so the separate launches give the same bits (the fused launch in this
  // layout ran the (1,2048,16,128) causal backward 19 % faster than the
  // dQ kernel and the four-wave query-split dK/dV kernel, one wave per
  // SIMD, that this grid used to take)
  if constexpr (D == 128 && CAUSAL) return launch_dkdv_split<E, D, CAUSAL, 1>(a, stream);
  if constexpr (D == 64 && CAUSAL) {
    if (a.split_kt > 0) return launch_dkdv_split<E, D, CAUSAL, 2>(a, stream);
  }
  return row_split(a.Sk, (int64_t)a.B * a.Hk, CAUSAL, D >= 128 ? 1 : 2)
             ? launch_dkdv_split<E, D, CAUSAL, 2>(a, stream)
             : launch_dkdv_split<E, D, CAUSAL, 1>(a, stream);
}

template <typename E, int D, bool CAUSAL>
int launch_dq(const fa::BwdArgs &a, hipStream_t stream) {
  const bool split = row_split(a.Sq, (int64_t)a.B * a.H, CAUSAL);
  // Non-causal grids of at least one eight-wave workgroup per CU: eight
  // waves sharing each K / V tile, as in the forward (D = 64: 256 queries,
  // no key split; D = 128 where the key split is chosen: 128 queries)
  if constexpr (!CAUSAL && D == 64) {
    if (!split && (int64_t)((a.Sq + 255) / 256) * a.B * a.H >= device_cus()) {
      if constexpr (std::is_same<E, fa::f16>::value) {
        if (a.c <= 1.0f) return launch_dq_split<E, D, CAUSAL, 1, true, 8>(a, stream);
      }
      return launch_dq_split<E, D, CAUSAL, 1, false, 8>(a, stream);
    }
  }
  if constexpr (!CAUSAL && D == 128) {
    if (split && (int64_t)((a.Sq + 127) / 128) * a.B * a.H >= device_cus()) {
      if constexpr (std::is_same<E, fa::f16>::value) {
        if (a.c <= 1.0f) return launch_dq_split<E, D, CAUSAL, 2, true, 8>(a, stream);
      }
      return launch_dq_split<E, D, CAUSAL, 2, false, 8>(a, stream);
    }
  }
  // the pre-scaled mode under the forward's condition (fp16, c <= 1), at
  // every D (at D = 128 its 16 seed registers fit beside two waves per SIMD
  // since the LDS offsets stopped taking a register per array and stage)
  if constexpr (std::is_same<E, fa::f16>::value) {
    if (a.c <= 1.0f)
      return split ? launch_dq_split<E, D, CAUSAL, 2, true>(a, stream)
                   : launch_dq_split<E, D, CAUSAL, 1, true>(a, stream);
  }
  return split ? launch_dq_split<E, D, CAUSAL, 2, false>(a, stream)
               : launch_dq_split<E, D, CAUSAL, 1, false>(a, stream);
}

// Fused causal backward (fa::fa_bwd_fused_kernel; bwd_fused decides): the pre-pass,
// which computes delta and zeroes the key-block split's counters, then
// one launch of every dK/dV block followed by every dQ block.
struct FusedBwd {
  fa::BwdArgs akv, aq;   // the dK/dV and dQ blocks' arguments
  fa::PreArgs pre;
  bool with_pre;         // launch the pre-pass first (false: delta is given)
  bool kv_split2;        // dK/dV layout: the query-split kernel (SPLIT = 2)
  bool q_split2;         // dQ layout: the key-split kernel (SPLIT = 2)
};

template <typename E, int D, bool CAUSAL, int KVS, int QS>
int launch_bwd_fused_as(FusedBwd f, hipStream_t stream) {
  using T = fa::DkdvTile<D, KVS>;
  using Q = fa::DqTile<D, QS, T::NW>;
  f.akv.n_blocks = (f.akv.Sk + T::BK - 1) / T::BK;
  f.aq.n_blocks = (f.aq.Sq + Q::BM - 1) / Q::BM;
  const int64_t n_kv = ((int64_t)f.akv.n_blocks + f.akv.split_kt) * f.akv.B * f.akv.Hk;
  const int64_t n_q = (int64_t)f.aq.n_blocks * f.aq.B * f.aq.H;
  if (n_kv + n_q > 0x7fffffff) return FA_ERR_TOO_LARGE;
  // heaviest blocks first in both parts: the last workgroups dispatched
  // are the lightest dQ blocks
  f.akv.zigzag = 0;
  f.aq.zigzag = 0;
  if (f.with_pre) {
    const int rc = launch_pre<E, D>(f.pre, stream);
    if (rc) return rc;
  }
  if constexpr (std::is_same<E, fa::f16>::value) {
    if (f.aq.c <= 1.0f) {
      hipLaunchKernelGGL((fa::fa_bwd_fused_kernel<E, D, CAUSAL, KVS, QS, true>),
                         dim3((unsigned)(n_kv + n_q)), dim3(T::NT), 0, stream, f.akv, f.aq, (int)n_kv);
      return launch_status();
    }
  }
  hipLaunchKernelGGL((fa::fa_bwd_fused_kernel<E, D, CAUSAL, KVS, QS, false>),
                     dim3((unsigned)(n_kv + n_q)), dim3(T::NT), 0, stream, f.akv, f.aq, (int)n_kv);
  return launch_status();
}

template <typename E, int D, bool CAUSAL>
int launch_bwd_fused(const FusedBwd &f, hipStream_t stream) {
  if constexpr (D <= 64 && CAUSAL) {
    if (f.kv_split2)
      return f.q_split2 ? launch_bwd_fused_as<E, D, CAUSAL, 2, 2>(f, stream)
                        : launch_bwd_fused_as<E, D, CAUSAL, 2, 1>(f, stream);
    return f.q_split2 ? launch_bwd_fused_as<E, D, CAUSAL, 1, 2>(f, stream)
                      : launch_bwd_fused_as<E, D, CAUSAL, 1, 1>(f, stream);
  } else if constexpr (D == 128 && CAUSAL) {
    // the eight-wave dK/dV layout beside eight-wave dQ blocks
    return f.q_split2 ? launch_bwd_fused_as<E, D, CAUSAL, 1, 2>(f, stream)
                      : launch_bwd_fused_as<E, D, CAUSAL, 1, 1>(f, stream);
  } else {
    (void)f;
    (void)stream;
    return FA_ERR_HEAD_DIM;   // run_bwd picks the fused path for causal grids only
  }
}

// (dtype, D, causal) -> one instantiation of launcher L<E, D, CAUSAL>.
#define FA_DISPATCH(L, s, causal, a, st)                                              \
  do {                                                                                \
    if ((s).dtype == FA_DTYPE_BF16) {                                                 \
      switch ((s).D) {                                                                \
        case 32: return causal ? L<fa::bf16, 32, true>(a, st) : L<fa::bf16, 32, false>(a, st);   \
        case 64: return causal ? L<fa::bf16, 64, true>(a, st) : L<fa::bf16, 64, false>(a, st);   \
        default: return causal ? L<fa::bf16, 128, true>(a, st) : L<fa::bf16, 128, false>(a, st); \
      }                                                                               \
    }                                                                                 \
    switch ((s).D) {                                                                  \
      case 32: return causal ? L<fa::f16, 32, true>(a, st) : L<fa::f16, 32, false>(a, st);       \
      case 64: return causal ? L<fa::f16, 64, true>(a, st) : L<fa::f16, 64, false>(a, st);       \
      default: return causal ? L<fa::f16, 128, true>(a, st) : L<fa::f16, 128, false>(a, st);     \
    }                                                                                 \
  } while (0)

// ---------------------------------------------------------------------------
// Split-KV forward (decode: a short query block against a long cache)

struct SplitPlan {
  int n_splits;   // 0: the split path does not apply
  int kv_split;   // keys per split, a multiple of the 64-key tile
};

// Split when one packed 64-row tile holds a key/value head's whole group of
// query rows (grp * Sq <= 64), the regular grid would leave the GPU
// under-filled, and there are enough keys: about 2 workgroups per CU, at
// least 128 keys per split (measured against 4 and 8 per CU and a 64- or
// 256-key minimum: equal or faster on every decode shape of bench.py).
SplitPlan splitkv_plan(const Shape &s) {
  const SplitPlan none{0, 0};
  const int64_t grp = s.H / s.Hk;
  if (grp * s.Sq > 64 || s.Sk < 256) return none;
  const int64_t cus = device_cus();
  const int64_t regular = (int64_t)((s.Sq + 63) / 64) * s.B * s.H;
  if (regular >= 2 * cus) return none;
  const int64_t heads = (int64_t)s.B * s.Hk;
  int64_t n = (2 * cus + heads - 1) / heads;
  const int64_t max_n = (s.Sk + 127) / 128;
  if (n > max_n) n = max_n;
  if (n < 2) return none;
  const int64_t kv = ((s.Sk + n - 1) / n + 63) / 64 * 64;
  n = (s.Sk + kv - 1) / kv;
  if (n < 2 || n > 65535) return none;
  return SplitPlan{(int)n, (int)kv};
}

// Workspace: part_o (n_splits, B, H, Sq, D) fp32, then part_lse (n_splits, B, H, Sq) fp32.
size_t splitkv_rows(const Shape &s, const SplitPlan &p) {
  return (size_t)p.n_splits * (size_t)s.B * (size_t)s.H * (size_t)s.Sq;
}

size_t splitkv_bytes(const Shape &s, const SplitPlan &p) {
  if (p.n_splits == 0) return 0;
  const size_t n = splitkv_rows(s, p) * (size_t)(s.D + 1) * sizeof(float);
  return (n + 255) & ~(size_t)255;
}

struct SplitLaunch {
  fa::FwdArgs f;
  fa::CombineArgs c;
  int n_splits;
};

template <typename E, int D, bool CAUSAL>
int launch_fwd_splitkv(const SplitLaunch &L, hipStream_t stream) {
  using T = fa::FwdTile<D, 2>;
  fa::FwdArgs a = L.f;
  a.n_qtiles = (a.grp * a.Sq + T::BM - 1) / T::BM;
  const int64_t gx = (int64_t)a.n_qtiles * a.B * (a.H / a.grp);
  if (gx > 0x7fffffff) return FA_ERR_TOO_LARGE;
  if constexpr (std::is_same<E, fa::f16>::value) {
    if (fwd_prescaled<E>(a))
      hipLaunchKernelGGL((fa::fa_fwd_kernel<E, D, CAUSAL, 2, true, true>),
                         dim3((unsigned)gx, L.n_splits), dim3(T::NT), 0, stream, a);
    else
      hipLaunchKernelGGL((fa::fa_fwd_kernel<E, D, CAUSAL, 2, true, false>),
                         dim3((unsigned)gx, L.n_splits), dim3(T::NT), 0, stream, a);
  } else {
    hipLaunchKernelGGL((fa::fa_fwd_kernel<E, D, CAUSAL, 2, true, false>),
                       dim3((unsigned)gx, L.n_splits), dim3(T::NT), 0, stream, a);
  }
  int rc = launch_status();
  if (rc) return rc;
  const int64_t rows = (int64_t)a.B * a.H * a.Sq;
  fa::CombineArgs c = L.c;
  constexpr int SLOTS = 256 / (D / 8);
  c.zgroups = 1;
  while (c.zgroups < SLOTS && c.zgroups < L.n_splits) c.zgroups *= 2;
  const int64_t rpb = SLOTS / c.zgroups;
  const int64_t gc = (rows + rpb - 1) / rpb;
  if (gc > 0x7fffffff) return FA_ERR_TOO_LARGE;
  hipLaunchKernelGGL((fa::fa_fwd_combine_kernel<E, D>), dim3((unsigned)gc), dim3(256), 0, stream,
                     c);
  return launch_status();
}

int check_fwd(const void *q, const void *k, const void *v, void *o, float *lse, const Shape &s,
              const int64_t *q_st, const int64_t *k_st, const int64_t *v_st, const int64_t *o_st,
              float sm_scale) {
  int rc = check_shape(s);
  if (rc) return rc;
  if ((rc = check_q_like(q, q_st, s))) return rc;
  if ((rc = check_kv_like(k, k_st, s))) return rc;
  if ((rc = check_kv_like(v, v_st, s))) return rc;
  if ((rc = check_q_like(o, o_st, s, true))) return rc;
  if (lse != nullptr && !aligned16(lse)) return FA_ERR_ALIGNMENT;
  if (!isfinite(sm_scale)) return FA_ERR_SCALE;
  return FA_OK;
}

fa::FwdArgs fwd_args(const void *q, const void *k, const void *v, void *o, float *lse,
                     const Shape &s, const int64_t *q_st, const int64_t *k_st,
                     const int64_t *v_st, const int64_t *o_st, float sm_scale) {
  fa::FwdArgs a{};
  a.q = desc(q, q_st, s.Sq);
  a.k = desc(k, k_st, s.Sk);
  a.v = desc(v, v_st, s.Sk);
  a.o = static_cast<f16 *>(o);
  a.o_sb = o_st[0];
  a.o_ss = o_st[1];
  a.o_sh = o_st[2];
  a.lse = lse;
  a.B = s.B;
  a.Sq = s.Sq;
  a.Sk = s.Sk;
  a.H = s.H;
  a.grp = s.H / s.Hk;
  a.off = s.Sk - s.Sq;
  a.c = kernel_scale(sm_scale);
  a.neg = sm_scale < 0.0f;
  return a;
}

int run_fwd(const void *q, const void *k, const void *v, void *o, float *lse, const Shape &s,
            const int64_t *q_st, const int64_t *k_st, const int64_t *v_st, const int64_t *o_st,
            float sm_scale, int causal, void *stream) {
  const LaunchDevice launch_dev(stream);
  int rc = check_fwd(q, k, v, o, lse, s, q_st, k_st, v_st, o_st, sm_scale);
  if (rc) return rc;
  const fa::FwdArgs a = fwd_args(q, k, v, o, lse, s, q_st, k_st, v_st, o_st, sm_scale);
  hipStream_t st = static_cast<hipStream_t>(stream);
  FA_DISPATCH(launch_fwd, s, causal, a, st);
}

int run_fwd_splitkv(const void *q, const void *k, const void *v, void *o, float *lse,
                    void *workspace, size_t workspace_bytes, const Shape &s, const int64_t *q_st,
                    const int64_t *k_st, const int64_t *v_st, const int64_t *o_st, float sm_scale,
                    int causal, void *stream) {
  const LaunchDevice launch_dev(stream);
  int rc = check_fwd(q, k, v, o, lse, s, q_st, k_st, v_st, o_st, sm_scale);
  if (rc) return rc;
  const SplitPlan plan = splitkv_plan(s);
  if (plan.n_splits == 0)
    return run_fwd(q, k, v, o, lse, s, q_st, k_st, v_st, o_st, sm_scale, causal, stream);
  if (workspace == nullptr || workspace_bytes < splitkv_bytes(s, plan)) return FA_ERR_WORKSPACE;
  if (!aligned16(workspace)) return FA_ERR_ALIGNMENT;
  SplitLaunch L{};
  L.f = fwd_args(q, k, v, o, lse, s, q_st, k_st, v_st, o_st, sm_scale);
  L.f.kv_split = plan.kv_split;
  L.f.part_o = static_cast<float *>(workspace);
  L.f.part_lse = L.f.part_o + splitkv_rows(s, plan) * (size_t)s.D;
  L.c.part_o = L.f.part_o;
  L.c.part_lse = L.f.part_lse;
  L.c.o = static_cast<f16 *>(o);
  L.c.o_sb = o_st[0];
  L.c.o_ss = o_st[1];
  L.c.o_sh = o_st[2];
  L.c.lse = lse;
  L.c.B = s.B;
  L.c.Sq = s.Sq;
  L.c.H = s.H;
  L.c.n_splits = plan.n_splits;
  L.n_splits = plan.n_splits;
  hipStream_t st = static_cast<hipStream_t>(stream);
  FA_DISPATCH(launch_fwd_splitkv, s, causal, L, st);
}

// ---------------------------------------------------------------------------
// Balanced causal forward (fa_fwd_bal_item in fa_fwd.hpp): causal tiles
// paired light with heavy, each pair cut in three work items dispatched
// largest first, the split heavy tiles' halves merged by
// fa_fwd_combine_kernel (pair mode).  For square causal grids (Sq == Sk)
// with at least kBalMinTiles 64-row tiles per head whose plain grid is at
// most half a workgroup per CU, one from 48 tiles per head, 1.75 from 64.  There the plain schedule ends on single
// workgroups sweeping every key tile alone (a lone workgroup's sweep runs
// at about 90 % of a CU's two-workgroup throughput, so splitting it is what
// shortens the kernel).  Measured on MI355X against the plain schedule
// (merge included): (1, 4096, 4, 128) -17 %, (1, 4096, 2, 128) -26 %,
// (1, 8192, 2, 128) -30 %, (1, 4096, 4, 64) -15 %, and at 1.25 - 1.5 tiles
// per CU (1, 4096, 5, 128) -16 %, (1, 4096, 6, 128) -11 %,
// (1, 4096, 6, 64) -11 %, (1, 8192, 3, 128) -19 %, at 1.75
// (1, 4096, 7, 64) -16 %, (1, 4096, 7, 128) -2.5 %; at 48 tiles per head
// (1, 3072, 2, 128) -21 %, (1, 3072, 4, 128) -13 %, (1, 3072, 4, 64) -8 %,
// but (1, 3072, 8, 64) (1.5 per CU) +4 %; at 32 tiles per head and half a
// tile per CU (1, 2048, 2, 128) -12 %, (1, 2048, 4, 128) -9 %,
// (2, 2048, 2, 128) -8 %, (1, 2048, 2, 64) -4 %; with fewer tiles per head
// or more workgroups per CU it loses (+3 to +50 %: every work item
// pays a workgroup's start-up of several microseconds, and the merge
// launch costs about 4 us): (1, 2048, 8, 128) +3 %, (1, 4096, 8, 128)
// +6 to +12 %, (1, 4096, 8, 64) +10 %, (4, 512, 4, 32) +50 %.

constexpr int kBalMinTiles = 32;

struct BalPlan {
  int nb;   // 64-row query tiles per (b, h); 0: the balanced schedule does not apply
};

BalPlan bal_plan(const Shape &s, int causal) {
  if (!causal || s.Sq != s.Sk) return BalPlan{0};
  if (!row_split(s.Sq, (int64_t)s.B * s.H, true)) return BalPlan{0};
  const int nb = (s.Sq + 63) / 64;
  const int64_t grid = (int64_t)nb * s.B * s.H;
  if (nb < kBalMinTiles) return BalPlan{0};
  const int64_t cus = device_cus();
  if (nb >= 64 ? 4 * grid > 7 * cus : nb >= 48 ? grid > cus : 2 * grid > cus) return BalPlan{0};
  return BalPlan{nb};
}

// Workspace: part_o (2, B, H, nb / 2, 64, D) fp32, then part_lse (2, B, H, nb / 2, 64) fp32.
size_t bal_rows(const Shape &s, const BalPlan &p) {
  return (size_t)s.B * (size_t)s.H * (size_t)(p.nb / 2) * 64;
}

size_t bal_bytes(const Shape &s, const BalPlan &p) {
  if (p.nb == 0) return 0;
  const size_t n = 2 * bal_rows(s, p) * (size_t)(s.D + 1) * sizeof(float);
  return (n + 255) & ~(size_t)255;
}

struct BalLaunch {
  fa::FwdArgs f;
  fa::CombineArgs c;
};

template <typename E, int D, bool PRE>
int launch_fwd_bal_mode(const BalLaunch &L, hipStream_t stream) {
  using T = fa::FwdTile<D, 2>;
  fa::FwdArgs a = L.f;
  a.n_qtiles = (a.Sq + T::BM - 1) / T::BM;
  a.zigzag = 0;
  const int64_t grid = (int64_t)fa::bal_items(a.n_qtiles) * a.B * a.H;
  if (grid > 0x7fffffff) return FA_ERR_TOO_LARGE;
  hipLaunchKernelGGL((fa::fa_fwd_kernel<E, D, true, 2, false, PRE, true>), dim3((unsigned)grid),
                     dim3(T::NT), 0, stream, a);
  int rc = launch_status();
  if (rc) return rc;
  fa::CombineArgs c = L.c;
  c.pair_bm = T::BM;
  c.nb = a.n_qtiles;
  c.bn = T::BN;
  c.Sk = a.Sk;
  c.off = a.off;
  c.n_splits = 2;
  c.zgroups = 1;
  constexpr int SLOTS = 256 / (D / 8);
  const int64_t rows = (int64_t)a.B * a.H * (a.n_qtiles / 2) * T::BM;
  const int64_t rpb = SLOTS / c.zgroups;
  const int64_t gc = (rows + rpb - 1) / rpb;
  if (gc > 0x7fffffff) return FA_ERR_TOO_LARGE;
  hipLaunchKernelGGL((fa::fa_fwd_combine_kernel<E, D>), dim3((unsigned)gc), dim3(256), 0, stream,
                     c);
  return launch_status();
}

template <typename E, int D, bool CAUSAL>
int launch_fwd_bal(const BalLaunch &L, hipStream_t stream) {
  if constexpr (!CAUSAL) {
    return FA_ERR_SHAPE;   // bal_plan applies to causal grids only
  } else {
    if constexpr (std::is_same<E, fa::f16>::value) {
      if (fwd_prescaled<E>(L.f)) return launch_fwd_bal_mode<E, D, true>(L, stream);
    }
    return launch_fwd_bal_mode<E, D, false>(L, stream);
  }
}

size_t fwd_ws_bytes(const Shape &s, int causal) {
  const SplitPlan kv = splitkv_plan(s);
  if (kv.n_splits) return splitkv_bytes(s, kv);
  return bal_bytes(s, bal_plan(s, causal));
}

int run_fwd_ws(const void *q, const void *k, const void *v, void *o, float *lse, void *workspace,
               size_t workspace_bytes, const Shape &s, const int64_t *q_st, const int64_t *k_st,
               const int64_t *v_st, const int64_t *o_st, float sm_scale, int causal,
               void *stream) {
  const LaunchDevice launch_dev(stream);
  int rc = check_fwd(q, k, v, o, lse, s, q_st, k_st, v_st, o_st, sm_scale);
  if (rc) return rc;
  // less than the schedule's workspace (none included): the plain forward
  const size_t need = fwd_ws_bytes(s, causal);
  if (need == 0 || workspace == nullptr || workspace_bytes < need)
    return run_fwd(q, k, v, o, lse, s, q_st, k_st, v_st, o_st, sm_scale, causal, stream);
  if (!aligned16(workspace)) return FA_ERR_ALIGNMENT;
  if (splitkv_plan(s).n_splits)
    return run_fwd_splitkv(q, k, v, o, lse, workspace, workspace_bytes, s, q_st, k_st, v_st, o_st,
                           sm_scale, causal, stream);
  const BalPlan plan = bal_plan(s, causal);
  if (plan.nb == 0)
    return run_fwd(q, k, v, o, lse, s, q_st, k_st, v_st, o_st, sm_scale, causal, stream);
  BalLaunch L{};
  L.f = fwd_args(q, k, v, o, lse, s, q_st, k_st, v_st, o_st, sm_scale);
  L.f.part_o = static_cast<float *>(workspace);
  L.f.part_lse = L.f.part_o + 2 * bal_rows(s, plan) * (size_t)s.D;
  L.c.part_o = L.f.part_o;
  L.c.part_lse = L.f.part_lse;
  L.c.o = static_cast<f16 *>(o);
  L.c.o_sb = o_st[0];
  L.c.o_ss = o_st[1];
  L.c.o_sh = o_st[2];
  L.c.lse = lse;
  L.c.B = s.B;
  L.c.Sq = s.Sq;
  L.c.H = s.H;
  hipStream_t st = static_cast<hipStream_t>(stream);
  FA_DISPATCH(launch_fwd_bal, s, causal, L, st);
}

// Backward workspace pieces: delta, then the row-group maxima.
size_t delta_bytes(int B, int Sq, int H) {
  const size_t n = (size_t)B * (size_t)H * (size_t)Sq * sizeof(float);
  return (n + 255) & ~(size_t)255;
}

// Row-group maxima (fa::BwdArgs::rmax): (B, H, ceil(Sq / 32), 2) fp32.
size_t rmax_bytes(int B, int Sq, int H) {
  const size_t n = (size_t)B * (size_t)H * (size_t)fa::row_groups(Sq) * 2 * sizeof(float);
  return (n + 255) & ~(size_t)255;
}

int run_pre(const void *o, const void *dout, float *delta, float *rmax, const Shape &s,
            const int64_t *o_st, const int64_t *do_st, void *stream) {
  const LaunchDevice launch_dev(stream);
  int rc = check_shape(s);
  if (rc) return rc;
  if ((rc = check_q_like(o, o_st, s))) return rc;
  if ((rc = check_q_like(dout, do_st, s))) return rc;
  if (delta == nullptr) return FA_ERR_NULL_POINTER;
  if (!aligned16(delta) || (rmax != nullptr && !aligned16(rmax))) return FA_ERR_ALIGNMENT;
  fa::PreArgs a{};
  a.o = desc(o, o_st, s.Sq);
  a.dout = desc(dout, do_st, s.Sq);
  a.delta = delta;
  a.rmax = rmax;
  a.B = s.B;
  a.S = s.Sq;
  a.H = s.H;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool bf = s.dtype == FA_DTYPE_BF16;
  switch (s.D) {
    case 32: return bf ? launch_pre<fa::bf16, 32>(a, st) : launch_pre<fa::f16, 32>(a, st);
    case 64: return bf ? launch_pre<fa::bf16, 64>(a, st) : launch_pre<fa::f16, 64>(a, st);
    default: return bf ? launch_pre<fa::bf16, 128>(a, st) : launch_pre<fa::f16, 128>(a, st);
  }
}

// Checks common to every backward step, then the kernel arguments; the
// output pointers that a step does not write stay NULL.
int bwd_common(const void *dout, const void *q, const void *k, const void *v, const float *lse,
               const float *delta, const Shape &s, const int64_t *do_st, const int64_t *q_st,
               const int64_t *k_st, const int64_t *v_st, float sm_scale, fa::BwdArgs *out) {
  int rc = check_shape(s);
  if (rc) return rc;
  if ((rc = check_q_like(dout, do_st, s))) return rc;
  if ((rc = check_q_like(q, q_st, s))) return rc;
  if ((rc = check_kv_like(k, k_st, s))) return rc;
  if ((rc = check_kv_like(v, v_st, s))) return rc;
  if (lse == nullptr || delta == nullptr) return FA_ERR_NULL_POINTER;
  if (!aligned16(lse) || !aligned16(delta)) return FA_ERR_ALIGNMENT;
  if (!isfinite(sm_scale)) return FA_ERR_SCALE;
  fa::BwdArgs a{};
  a.q = desc(q, q_st, s.Sq);
  a.k = desc(k, k_st, s.Sk);
  a.v = desc(v, v_st, s.Sk);
  a.dout = desc(dout, do_st, s.Sq);
  a.lse = lse;
  a.delta = delta;
  a.B = s.B;
  a.Sq = s.Sq;
  a.Sk = s.Sk;
  a.H = s.H;
  a.Hk = s.Hk;
  a.grp = s.H / s.Hk;
  a.off = s.Sk - s.Sq;
  a.c = kernel_scale(sm_scale);
  a.lse_mul = lse_seed_mul(a.c, s.dtype);
  a.sm_scale = sm_scale;
  a.neg = sm_scale < 0.0f;
  *out = a;
  return FA_OK;
}

// Causal key-block split of the dK/dV kernel (fa::BwdArgs::split_kt;
// the eight-wave D = 128 and the D = 64 query-split layouts).  When the
// grid of key blocks fits one round of resident workgroups, the causal
// sweep lengths set the time: block 0 sees every query tile, the last
// block one or two, and no other workgroup can take over.  The leading
// blocks with the longest sweeps are then swept by two workgroups each.
// Larger grids keep one workgroup per block: later rounds already fill in
// behind the long sweeps (heaviest blocks first).
struct DkdvSplit {
  int split_kt = 0;    // leading key blocks split, per (b, key/value head)
  int64_t slots = 0;   // split_kt * B * Hk
  int bk = 0, d = 0;   // the kernel's key block and head dimension
};

// Query tiles key block kt of a causal (B, Sq, Sk, H, Hk) problem sweeps
// with BK-key blocks and BQ-query tiles (the dK/dV kernel's m_begin / nt_h),
// counted over the H / Hk query heads of the group.
int64_t causal_tiles(const Shape &s, int64_t kt, int BK, int BQ) {
  const int64_t grp = s.H / s.Hk, off = (int64_t)s.Sk - s.Sq;
  const int64_t m_first = kt * BK - off > 0 ? kt * BK - off : 0;
  const int64_t m_begin = m_first / BQ * BQ;
  return s.Sq > m_begin ? (s.Sq - m_begin + BQ - 1) / BQ * grp : 0;
}

// Plan for one dK/dV layout T (BK keys per block, BQ-query tiles): split
// only grids that fit one round of resident workgroups (T::WAVES_PER_EU
// waves per SIMD, four SIMDs per CU) and whose block 0 sweeps at least 32
// tiles; then every leading block with more than `thr(t0)` tiles splits.
template <typename T, typename Thr>
DkdvSplit split_plan_for(const Shape &s, Thr thr_of) {
  DkdvSplit p;
  const int64_t bhk = (int64_t)s.B * s.Hk;
  const int64_t nb = (s.Sk + T::BK - 1) / T::BK;
  const int64_t per_cu = 4 * T::WAVES_PER_EU / T::NW;
  if (nb * bhk > per_cu * device_cus()) return p;
  const int64_t t0 = causal_tiles(s, 0, T::BK, T::BQ);
  if (t0 < 32) return p;
  const int64_t thr = thr_of(t0);
  int64_t kt = 0;
  while (kt < nb && causal_tiles(s, kt, T::BK, T::BQ) > thr) ++kt;
  p.split_kt = (int)kt;
  p.slots = kt * bhk;
  p.bk = T::BK;
  p.d = s.D;
  return p;
}

// Measured (fa_bwd time, same box): D = 128 (eight-wave kernel, one
// workgroup per CU) at (1,4096,8,128): thresholds of 1/2, 1/3, 1/4, 1/8 and
// 1/16 of block 0's tiles gave -7, -13, -14, -18 and -19 %; (1,1024,16,128)
// (16 tiles) lost ~1 % and stays unsplit.  D = 64 (query-split kernel,
// three per CU): 1/3 gave -18 % at (1,4096,8,64), -10 % at (1,2048,16,64),
// -34 % at (1,4096,16 heads / 4 kv heads,64); grids of more than one round
// lost 2-8 % ((1,4096,16,64), (1,2048,32,64)) and stay unsplit.
DkdvSplit dkdv_split_plan(const Shape &s, int causal) {
  if (!causal) return DkdvSplit{};
  if (s.D == 128) {
    // a full round whose block 0 sweeps under 64 tiles gains nothing since
    // the blocks go heaviest first ((1,2048,16,128): +3 %)
    using T = fa::DkdvTile<128, 1>;
    const int64_t blocks = (s.Sk + T::BK - 1) / T::BK * ((int64_t)s.B * s.Hk);
    if (causal_tiles(s, 0, T::BK, T::BQ) < 64 && 2 * blocks > device_cus()) return DkdvSplit{};
    return split_plan_for<T>(s, [](int64_t t0) { return t0 / 16 > 4 ? t0 / 16 : (int64_t)4; });
  }
  if (s.D == 64 && row_split(s.Sk, (int64_t)s.B * s.Hk, true, 2))
    return split_plan_for<fa::DkdvTile<64, 2>>(s, [](int64_t t0) { return t0 / 3; });
  return DkdvSplit{};
}

// Causal query-block split of the dQ kernel (fa::BwdArgs::dq_split): the
// mirror image of the key-block split, for dQ grids of at most half a
// round whose last query blocks sweep the most key tiles (measured with
// the dK/dV split: (1,4096,4,128) backward -20 % instead of -11 %,
// (1,2048,8,128) -11 % instead of -7 %).  The two halves' fp32 rows are
// added by the dK/dV kernel that follows (no counters: the dQ kernel runs
// first and nothing could zero them in time).
struct DqSplit {
  int split = 0;       // last query blocks split, per (b, h)
  int bm = 0;          // rows per block of the dQ layout in use
  int nblocks = 0;     // query blocks per (b, h)
  int64_t slots = 0;   // split * B * H
  int d = 0;
  int64_t sweep = 0;   // key tiles the last query block sweeps
};

DqSplit dq_split_plan(const Shape &s, int causal) {
  DqSplit p;
  if (!causal || (s.D != 64 && s.D != 128)) return p;
  const int64_t bh = (int64_t)s.B * s.H;
  const bool sp = row_split(s.Sq, bh, true);
  const int BM = s.D == 64 ? (sp ? fa::DqTile<64, 2>::BM : fa::DqTile<64, 1>::BM)
                           : (sp ? fa::DqTile<128, 2>::BM : fa::DqTile<128, 1>::BM);
  constexpr int BN = fa::DqTile<64, 1>::BN;
  // resident dQ workgroups per CU on gfx950 (VGPR-bound: 150-152 registers
  // at D = 64, 238-240 at D = 128)
  const int64_t per_cu = s.D == 64 ? 3 : 2;
  // at most half a round: on a full round the extra workgroups cost more
  // than the balance gains ((1,4096,8,128) +3.5 %, (1,2048,16,64) +6.5 %)
  const int64_t nq = (s.Sq + BM - 1) / BM;
  if (2 * nq * bh > per_cu * device_cus()) return p;
  const int64_t off = (int64_t)s.Sk - s.Sq;
  auto tiles = [&](int64_t qt) -> int64_t {
    int64_t end = (qt + 1) * BM + off;
    end = end < s.Sk ? end : s.Sk;
    return end > 0 ? (end + BN - 1) / BN : 0;
  };
  const int64_t tmax = tiles(nq - 1);
  if (tmax < 32) return p;
  const int64_t thr = tmax / 3;
  int64_t n = 0;
  while (n < nq && tiles(nq - 1 - n) > thr) ++n;
  p.split = (int)n;
  p.bm = BM;
  p.nblocks = (int)nq;
  p.slots = n * bh;
  p.d = s.D;
  p.sweep = tmax;
  return p;
}

// The fused backward launch (fa::fa_bwd_fused_kernel) runs the causal
// backwards without the dQ split (whose halves the dK/dV kernel adds after
// the dQ kernel), unsplit: every D = 32 / 64 one, and the D = 128 ones
// whose eight-wave dK/dV grid is at most four rounds.  `qplan` is the dQ
// split that will run (none without the workspace for it), so
// fa_bwd_blocks, which never splits, takes the path fa_bwd takes with the
// minimum workspace.  Measured (same-process A/B of the backward):
//   against the dQ kernel (delta folded in) then the dK/dV kernel, D = 128:
//   (1,2048,16,128) -18.6 %, (2,1100,32,128) -2.7 %, (1,4096,16,128)
//   -1.6 %, (2,4096,16,128) (four rounds) -1.0 %, (1,8192,16,128) -1.9 %;
//   on six rounds and more the separate pre-pass over O and dO costs more
//   than the fusion saves ((3,4096,16,128) +2.5 %, (6,1100,32,128)
//   +5.5 %, (4,4096,16,128) +2.0 %);
//   against the key-block split (inside the fused launch at D = 64, beside
//   it at D = 128) on grids of one round: (1,2048,16,64) -13.2 %,
//   (1,4096,8,64) -2.9 %, (1,4096,8,128) -9.9 %, (1,8192,4,128) -7.5 %,
//   (2,4096,4,128) -9.7 % -- the dQ blocks fill the slots the unequal
//   sweeps leave idle, as the split's second workgroups did, without its
//   partials.
bool bwd_fused(const Shape &s, int causal, const DqSplit &qplan) {
  if (!causal || qplan.split != 0) return false;
  if (s.D <= 64) return true;
  using T = fa::DkdvTile<128, 1>;
  const int64_t blocks = (s.Sk + T::BK - 1) / T::BK * ((int64_t)s.B * s.Hk);
  return blocks <= 4 * (int64_t)device_cus();
}

// Both backward splits for these sizes (what fa_bwd_gqa_workspace_bytes
// makes room for): the dQ split, and the key-block split beside it (the
// fused launch runs unsplit).  Where the fused launch can run instead, the
// dQ split runs only on sweeps of at least 64 key tiles (48 at D = 128);
// on shorter ones the fused launch is faster (same-process A/B of the
// backward, fused against the dQ split: (1,2048,8,64) -9.4 %,
// (2,2048,4,64) -9.0 %, (1,3072,8,64) -6.9 %, (1,2048,4,64) -4.6 %,
// (1,3072,4,64) -1.2 %, (1,2048,8,128) -5.4 %, (1,2048,4,128) -1.6 %,
// (2,2048,2,128) -1.5 %); from there on it is slower ((1,3072,4,128)
// +2.6 %, (1,3072,2,128) +7.7 %, (1,4096,4,64) +4.1 %, (1,4096,2,64)
// +6.9 %, (1,4096,4,128) +6.3 %, (1,8192,2,128) +14.9 %).
void bwd_plans(const Shape &s, int causal, DkdvSplit &plan, DqSplit &qplan) {
  qplan = dq_split_plan(s, causal);
  const int64_t min_sweep = s.D >= 128 ? 48 : 64;
  if (qplan.split != 0 && qplan.sweep < min_sweep && bwd_fused(s, causal, DqSplit{}))
    qplan = DqSplit{};
  plan = bwd_fused(s, causal, qplan) ? DkdvSplit{} : dkdv_split_plan(s, causal);
}

// two segments x BM rows x D fp32 per split query block
size_t dq_split_bytes(const DqSplit &p) {
  return p.split > 0 ? (size_t)p.slots * 2 * (size_t)p.bm * (size_t)p.d * sizeof(float) : 0;
}

size_t split_cnt_bytes(const DkdvSplit &p) {
  return ((size_t)p.slots * sizeof(unsigned) + 255) & ~(size_t)255;
}

// two segments x (dK, dV) x BK keys x D fp32 per split block
size_t split_part_bytes(const DkdvSplit &p) {
  return (size_t)p.slots * 2 * 2 * (size_t)p.bk * (size_t)p.d * sizeof(float);
}

size_t split_bytes(const DkdvSplit &p) {
  return p.split_kt > 0 ? split_cnt_bytes(p) + split_part_bytes(p) : 0;
}

// The dK/dV kernel's arguments (every check of run_dkdv).
int dkdv_args(const void *dout, const void *q, const void *k, const void *v, const float *lse,
              const float *delta, const float *rmax, void *dk, void *dv, const Shape &s,
              const int64_t *do_st, const int64_t *q_st, const int64_t *k_st,
              const int64_t *v_st, const int64_t *dk_st, const int64_t *dv_st, float sm_scale,
              int split_kt, unsigned *cnt, float *part, const DqSplit *dqs, float *dq_part,
              void *dq, const int64_t *dq_st, fa::BwdArgs *out) {
  fa::BwdArgs &a = *out;
  int rc = bwd_common(dout, q, k, v, lse, delta, s, do_st, q_st, k_st, v_st, sm_scale, &a);
  if (rc) return rc;
  if ((rc = check_kv_like(dk, dk_st, s, true))) return rc;
  if ((rc = check_kv_like(dv, dv_st, s, true))) return rc;
  if (rmax == nullptr) return FA_ERR_NULL_POINTER;
  if (!aligned16(rmax)) return FA_ERR_ALIGNMENT;
  a.rmax = rmax;
  a.split_kt = split_kt;
  a.cnt = cnt;
  a.part = part;
  if (dqs != nullptr && dqs->split > 0) {
    a.dq_split = dqs->split;
    a.dq_bm = dqs->bm;
    a.dq_nblocks = dqs->nblocks;
    a.dq_part = dq_part;
    a.dq = static_cast<f16 *>(dq);
    a.dq_sb = dq_st[0];
    a.dq_ss = dq_st[1];
    a.dq_sh = dq_st[2];
  }
  a.dk = static_cast<f16 *>(dk);
  a.dv = static_cast<f16 *>(dv);
  a.dk_sb = dk_st[0];
  a.dk_ss = dk_st[1];
  a.dk_sh = dk_st[2];
  a.dv_sb = dv_st[0];
  a.dv_ss = dv_st[1];
  a.dv_sh = dv_st[2];
  return FA_OK;
}

int run_dkdv(const void *dout, const void *q, const void *k, const void *v, const float *lse,
             const float *delta, const float *rmax, void *dk, void *dv, const Shape &s,
             const int64_t *do_st,
             const int64_t *q_st, const int64_t *k_st, const int64_t *v_st, const int64_t *dk_st,
             const int64_t *dv_st, float sm_scale, int causal, void *stream, int split_kt = 0,
             unsigned *cnt = nullptr, float *part = nullptr, const DqSplit *dqs = nullptr,
             float *dq_part = nullptr, void *dq = nullptr, const int64_t *dq_st = nullptr) {
  const LaunchDevice launch_dev(stream);
  fa::BwdArgs a;
  int rc = dkdv_args(dout, q, k, v, lse, delta, rmax, dk, dv, s, do_st, q_st, k_st, v_st, dk_st,
                     dv_st, sm_scale, split_kt, cnt, part, dqs, dq_part, dq, dq_st, &a);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  FA_DISPATCH(launch_dkdv, s, causal, a, st);
}

// The dQ kernel's arguments (every check of run_dq).
int dq_args(const void *dout, const void *q, const void *k, const void *v, const float *lse,
            const float *delta, void *dq, const Shape &s, const int64_t *do_st,
            const int64_t *q_st, const int64_t *k_st, const int64_t *v_st, const int64_t *dq_st,
            float sm_scale, const void *o, const int64_t *o_st, unsigned *cnt_zero,
            int n_cnt_zero, int dq_split, float *dq_part, float *rmax_out,
            fa::BwdArgs *out) {
  fa::BwdArgs &a = *out;
  int rc = bwd_common(dout, q, k, v, lse, delta, s, do_st, q_st, k_st, v_st, sm_scale, &a);
  if (rc) return rc;
  if ((rc = check_q_like(dq, dq_st, s, true))) return rc;
  if (o != nullptr) {
    // the full backward: delta and the row-group maxima computed here
    if ((rc = check_q_like(o, o_st, s))) return rc;
    a.o = desc(o, o_st, s.Sq);
    a.delta_out = const_cast<float *>(delta);
    a.rmax_out = rmax_out;
  }
  a.cnt_zero = cnt_zero;
  a.n_cnt_zero = n_cnt_zero;
  a.dq_split = dq_split;
  a.dq_part = dq_part;
  a.dq = static_cast<f16 *>(dq);
  a.dq_sb = dq_st[0];
  a.dq_ss = dq_st[1];
  a.dq_sh = dq_st[2];
  return FA_OK;
}

// dQ; with `o` given (the full backward), the kernel also computes delta
// from O and dO and writes it to `delta` instead of reading it.
int run_dq(const void *dout, const void *q, const void *k, const void *v, const float *lse,
           const float *delta, void *dq, const Shape &s, const int64_t *do_st, const int64_t *q_st,
           const int64_t *k_st, const int64_t *v_st, const int64_t *dq_st, float sm_scale,
           int causal, void *stream, const void *o = nullptr, const int64_t *o_st = nullptr,
           unsigned *cnt_zero = nullptr, int n_cnt_zero = 0, int dq_split = 0,
           float *dq_part = nullptr, float *rmax_out = nullptr) {
  const LaunchDevice launch_dev(stream);
  fa::BwdArgs a;
  int rc = dq_args(dout, q, k, v, lse, delta, dq, s, do_st, q_st, k_st, v_st, dq_st, sm_scale, o,
                   o_st, cnt_zero, n_cnt_zero, dq_split, dq_part, rmax_out, &a);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  FA_DISPATCH(launch_dq, s, causal, a, st);
}



// Every check of the full backward but the workspace's: a call that passes
// launches nothing invalid.
int check_bwd(const void *dout, const void *q, const void *k, const void *v, const void *o,
              const float *lse, void *dq, void *dk, void *dv, const Shape &s,
              const int64_t *do_st, const int64_t *q_st, const int64_t *k_st,
              const int64_t *v_st, const int64_t *o_st, const int64_t *dq_st,
              const int64_t *dk_st, const int64_t *dv_st, float sm_scale) {
  int rc = check_shape(s);
  if (rc) return rc;
  if ((rc = check_q_like(o, o_st, s))) return rc;
  if ((rc = check_q_like(dq, dq_st, s, true))) return rc;
  if ((rc = check_kv_like(dk, dk_st, s, true))) return rc;
  if ((rc = check_kv_like(dv, dv_st, s, true))) return rc;
  if ((rc = check_q_like(dout, do_st, s))) return rc;
  if ((rc = check_q_like(q, q_st, s))) return rc;
  if ((rc = check_kv_like(k, k_st, s))) return rc;
  if ((rc = check_kv_like(v, v_st, s))) return rc;
  if (lse == nullptr) return FA_ERR_NULL_POINTER;
  if (!aligned16(lse)) return FA_ERR_ALIGNMENT;
  if (!isfinite(sm_scale)) return FA_ERR_SCALE;
  return FA_OK;
}

int run_bwd(const void *dout, const void *q, const void *k, const void *v, const void *o,
            const float *lse, void *dq, void *dk, void *dv, void *workspace,
            size_t workspace_bytes, const Shape &s, const int64_t *do_st, const int64_t *q_st,
            const int64_t *k_st, const int64_t *v_st, const int64_t *o_st, const int64_t *dq_st,
            const int64_t *dk_st, const int64_t *dv_st, float sm_scale, int causal, void *stream) {
  const LaunchDevice launch_dev(stream);
  int rc = check_bwd(dout, q, k, v, o, lse, dq, dk, dv, s, do_st, q_st, k_st, v_st, o_st, dq_st,
                     dk_st, dv_st, sm_scale);
  if (rc) return rc;
  const size_t rbytes = rmax_bytes(s.B, s.Sq, s.H);
  if (workspace == nullptr || workspace_bytes < delta_bytes(s.B, s.Sq, s.H) + rbytes)
    return FA_ERR_WORKSPACE;
  if (!aligned16(workspace)) return FA_ERR_ALIGNMENT;
  float *delta = static_cast<float *>(workspace);
  // The key-block split runs when the workspace has room for it (see
  // fa_bwd_gqa_workspace_bytes): counters, then the fp32 partials.
  // Layout: delta, the row-group maxima, then the dK/dV split's counters
  // and partials, then the dQ split's partials -- both splits or neither,
  // by workspace size.  (`dbytes` below covers delta and the maxima.)
  DkdvSplit plan;
  DqSplit qplan;
  bwd_plans(s, causal, plan, qplan);
  float *rmax = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                          delta_bytes(s.B, s.Sq, s.H));
  const size_t dbytes = delta_bytes(s.B, s.Sq, s.H) + rbytes;
  if (workspace_bytes < dbytes + split_bytes(plan) + dq_split_bytes(qplan)) {
    plan = DkdvSplit{};
    qplan = DqSplit{};
  }
  char *ws = static_cast<char *>(workspace);
  unsigned *cnt = nullptr;
  float *part = nullptr;
  if (plan.split_kt > 0) {
    cnt = reinterpret_cast<unsigned *>(ws + dbytes);
    part = reinterpret_cast<float *>(ws + dbytes + split_cnt_bytes(plan));
  }
  float *dq_part =
      qplan.split > 0 ? reinterpret_cast<float *>(ws + dbytes + split_bytes(plan)) : nullptr;
  if (bwd_fused(s, causal, qplan)) {
    FusedBwd f{};
    if ((rc = dkdv_args(dout, q, k, v, lse, delta, rmax, dk, dv, s, do_st, q_st, k_st, v_st,
                        dk_st, dv_st, sm_scale, plan.split_kt, cnt, part, nullptr, nullptr,
                        nullptr, nullptr, &f.akv)))
      return rc;
    if ((rc = dq_args(dout, q, k, v, lse, delta, dq, s, do_st, q_st, k_st, v_st, dq_st, sm_scale,
                      nullptr, nullptr, nullptr, 0, 0, nullptr, nullptr, &f.aq)))
      return rc;
    f.pre.o = desc(o, o_st, s.Sq);
    f.pre.dout = desc(dout, do_st, s.Sq);
    f.pre.delta = delta;
    f.pre.rmax = rmax;
    f.pre.B = s.B;
    f.pre.S = s.Sq;
    f.pre.H = s.H;
    f.pre.cnt_zero = cnt;
    f.pre.n_cnt_zero = (int)plan.slots;
    f.with_pre = true;
    f.kv_split2 = plan.split_kt > 0 || row_split(s.Sk, (int64_t)s.B * s.Hk, true, 2);
    f.q_split2 = row_split(s.Sq, (int64_t)s.B * s.H, true);
    hipStream_t st = static_cast<hipStream_t>(stream);
    FA_DISPATCH(launch_bwd_fused, s, causal, f, st);
  }
  // dQ first: it computes delta and the row-group maxima (the pre-pass,
  // folded in) for the dK/dV kernel, which runs after it on the same
  // stream, zeroes the key-block split's counters and leaves its split
  // query blocks' halves for the dK/dV kernel to add.
  if ((rc = run_dq(dout, q, k, v, lse, delta, dq, s, do_st, q_st, k_st, v_st, dq_st, sm_scale,
                   causal, stream, o, o_st, cnt, (int)plan.slots, qplan.split, dq_part, rmax)))
    return rc;
  return run_dkdv(dout, q, k, v, lse, delta, rmax, dk, dv, s, do_st, q_st, k_st, v_st, dk_st,
                  dv_st, sm_scale, causal, stream, plan.split_kt, cnt, part, &qplan, dq_part, dq,
                  dq_st);
}

// Both gradient launches given delta (fa_bwd without its delta step):
// the fused launch where fa_bwd uses it (without a key-block split: there
// is no workspace), else the dQ kernel reading delta, then the dK/dV
// kernel.
int run_bwd_blocks(const void *dout, const void *q, const void *k, const void *v,
                   const float *lse, const float *delta, const float *rmax, void *dq, void *dk,
                   void *dv, const Shape &s, const int64_t *do_st, const int64_t *q_st,
                   const int64_t *k_st, const int64_t *v_st, const int64_t *dq_st,
                   const int64_t *dk_st, const int64_t *dv_st, float sm_scale, int causal,
                   void *stream) {
  const LaunchDevice launch_dev(stream);
  if (!bwd_fused(s, causal, DqSplit{})) {
    // every check before the first launch
    fa::BwdArgs chk;
    int rc = dkdv_args(dout, q, k, v, lse, delta, rmax, dk, dv, s, do_st, q_st, k_st, v_st,
                       dk_st, dv_st, sm_scale, 0, nullptr, nullptr, nullptr, nullptr, nullptr,
                       nullptr, &chk);
    if (rc) return rc;
    rc = run_dq(dout, q, k, v, lse, delta, dq, s, do_st, q_st, k_st, v_st, dq_st, sm_scale,
                causal, stream);
    if (rc) return rc;
    return run_dkdv(dout, q, k, v, lse, delta, rmax, dk, dv, s, do_st, q_st, k_st, v_st, dk_st,
                    dv_st, sm_scale, causal, stream);
  }
  FusedBwd f{};
  int rc = dkdv_args(dout, q, k, v, lse, delta, rmax, dk, dv, s, do_st, q_st, k_st, v_st, dk_st,
                     dv_st, sm_scale, 0, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                     &f.akv);
  if (rc) return rc;
  if ((rc = dq_args(dout, q, k, v, lse, delta, dq, s, do_st, q_st, k_st, v_st, dq_st, sm_scale,
                    nullptr, nullptr, nullptr, 0, 0, nullptr, nullptr, &f.aq)))
    return rc;
  f.with_pre = false;
  f.kv_split2 = row_split(s.Sk, (int64_t)s.B * s.Hk, true, 2);
  f.q_split2 = row_split(s.Sq, (int64_t)s.B * s.H, true);
  hipStream_t st = static_cast<hipStream_t>(stream);
  FA_DISPATCH(launch_bwd_fused, s, causal, f, st);
}

Shape square(int B, int S, int H, int D) { return Shape{B, S, S, H, H, D, FA_DTYPE_F16}; }

// ---------------------------------------------------------------------------
// QK-norm + rotary prologue

struct RopeShape {
  int B, S, H, Hk, D, dtype;
};

int check_rope_shape(const RopeShape &s) {
  if (s.dtype != FA_DTYPE_F16 && s.dtype != FA_DTYPE_BF16) return FA_ERR_DTYPE;
  if (s.B <= 0 || s.S <= 0 || s.H <= 0 || s.Hk <= 0) return FA_ERR_SHAPE;
  if (s.D != 16 && s.D != 32 && s.D != 64 && s.D != 128) return FA_ERR_HEAD_DIM;
  // Rows of the larger side, B * S * H, are indexed in 32 bits.
  if ((double)s.B * s.S * (s.H > s.Hk ? s.H : s.Hk) > 2147483647.0) return FA_ERR_TOO_LARGE;
  return FA_OK;
}

// Rows per 256-thread workgroup pass (a row takes D/16 lanes).
int64_t rope_rows_per_block(int D) { return fa::kRopeThreads / (D / 16); }

int64_t rope_rows(const RopeShape &s) {
  return (int64_t)s.B * s.S * (s.H > s.Hk ? s.H : s.Hk);
}

// Workgroups per side.  With a norm the backward writes one dw partial per
// workgroup, so its grid is capped (grid-stride beyond); everything else
// covers the rows in one pass.
constexpr int64_t kRopeNormBlocks = 1024;

int64_t rope_blocks(const RopeShape &s, bool capped) {
  const int64_t rpb = rope_rows_per_block(s.D);
  const int64_t need = (rope_rows(s) + rpb - 1) / rpb;
  // (a launch's x extent in work-items must stay below 2^32)
  const int64_t cap = capped ? kRopeNormBlocks : ((int64_t)1 << 22);
  return need < cap ? need : cap;
}

size_t rope_partial_bytes(const RopeShape &s) {
  return (size_t)rope_blocks(s, true) * (size_t)s.D * sizeof(float);
}

int check_rope_table(const void *cos, const void *sin, const int64_t *cs_st) {
  if (cos == nullptr || sin == nullptr || cs_st == nullptr) return FA_ERR_NULL_POINTER;
  if (!aligned16(cos) || !aligned16(sin)) return FA_ERR_ALIGNMENT;
  for (int i = 0; i < 2; ++i) {
    if (cs_st[i] < 0 || (cs_st[i] & 7) != 0) return FA_ERR_STRIDE;
  }
  return FA_OK;
}

int check_rope_eps(const void *wq, const void *wk, float eps) {
  if (wq != nullptr && !aligned16(wq)) return FA_ERR_ALIGNMENT;
  if (wk != nullptr && !aligned16(wk)) return FA_ERR_ALIGNMENT;
  if ((wq != nullptr || wk != nullptr) && !(isfinite(eps) && eps >= 0.0f)) return FA_ERR_EPS;
  return FA_OK;
}

void rope_strides(const int64_t *st, int64_t &b, int64_t &s, int64_t &h) {
  b = st[0];
  s = st[1];
  h = st[2];
}

template <typename E, int D>
int launch_rope_fwd(const fa::RopeArgs &a, int64_t blocks, hipStream_t st) {
  hipLaunchKernelGGL((fa::fa_rope_fwd_kernel<E, D>), dim3((unsigned)blocks, 2), dim3(fa::kRopeThreads),
                     0, st, a);
  return launch_status();
}

template <typename E, int D>
int launch_rope_bwd(const fa::RopeArgs &a, int64_t blocks, float *dwq, float *dwk,
                    hipStream_t st) {
  hipLaunchKernelGGL((fa::fa_rope_bwd_kernel<E, D>), dim3((unsigned)blocks, 2), dim3(fa::kRopeThreads),
                     0, st, a);
  int rc = launch_status();
  if (rc || (a.side[0].w == nullptr && a.side[1].w == nullptr)) return rc;
  hipLaunchKernelGGL(fa::fa_rope_dw_reduce_kernel<D>, dim3(D / 16, 2), dim3(fa::kRopeReduceThreads), 0, st,
                     a.side[0].partial, a.side[1].partial, dwq, dwk, (int)blocks);
  return launch_status();
}

// (dtype, D) -> one instantiation of launcher L<E, D>.
#define FA_ROPE_DISPATCH(L, s, ...)                                           \
  do {                                                                        \
    if ((s).dtype == FA_DTYPE_BF16) {                                         \
      switch ((s).D) {                                                        \
        case 16: return L<fa::bf16, 16>(__VA_ARGS__);                         \
        case 32: return L<fa::bf16, 32>(__VA_ARGS__);                         \
        case 64: return L<fa::bf16, 64>(__VA_ARGS__);                         \
        default: return L<fa::bf16, 128>(__VA_ARGS__);                        \
      }                                                                       \
    }                                                                         \
    switch ((s).D) {                                                          \
      case 16: return L<fa::f16, 16>(__VA_ARGS__);                            \
      case 32: return L<fa::f16, 32>(__VA_ARGS__);                            \
      case 64: return L<fa::f16, 64>(__VA_ARGS__);                            \
      default: return L<fa::f16, 128>(__VA_ARGS__);                           \
    }                                                                         \
  } while (0)

int run_rope_fwd(const void *q, const void *k, void *q_out, void *k_out, const void *cos,
                 const void *sin, const void *wq, const void *wk, float eps, const RopeShape &s,
                 const int64_t *q_st, const int64_t *k_st, const int64_t *qo_st,
                 const int64_t *ko_st, const int64_t *cs_st, void *stream) {
  const LaunchDevice launch_dev(stream);
  int rc = check_rope_shape(s);
  if (rc) return rc;
  if ((rc = check_tensor(q, q_st, s.B, s.S, s.H, s.D, false, 0))) return rc;
  if ((rc = check_tensor(k, k_st, s.B, s.S, s.Hk, s.D, false, 0))) return rc;
  if ((rc = check_tensor(q_out, qo_st, s.B, s.S, s.H, s.D, true, 0))) return rc;
  if ((rc = check_tensor(k_out, ko_st, s.B, s.S, s.Hk, s.D, true, 0))) return rc;
  if ((rc = check_rope_table(cos, sin, cs_st))) return rc;
  if ((rc = check_rope_eps(wq, wk, eps))) return rc;

  fa::RopeArgs a{};
  const void *x[2] = {q, k};
  void *y[2] = {q_out, k_out};
  const void *w[2] = {wq, wk};
  const int64_t *xs[2] = {q_st, k_st}, *ys[2] = {qo_st, ko_st};
  const int heads[2] = {s.H, s.Hk};
  for (int i = 0; i < 2; ++i) {
    fa::RopeSide &t = a.side[i];
    t.x = static_cast<const f16 *>(x[i]);
    t.y = static_cast<f16 *>(y[i]);
    t.w = static_cast<const f16 *>(w[i]);
    rope_strides(xs[i], t.xb, t.xs, t.xh);
    rope_strides(ys[i], t.yb, t.ys, t.yh);
    t.heads = heads[i];
    t.rows = (int64_t)s.B * s.S * heads[i];
  }
  a.cos = static_cast<const f16 *>(cos);
  a.sin = static_cast<const f16 *>(sin);
  a.cb = cs_st[0];
  a.cs = cs_st[1];
  a.S = s.S;
  a.eps = eps;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t blocks = rope_blocks(s, false);
  FA_ROPE_DISPATCH(launch_rope_fwd, s, a, blocks, st);
}

int run_rope_bwd(const void *dq_out, const void *dk_out, const void *q, const void *k,
                 const void *cos, const void *sin, const void *wq, const void *wk, float eps,
                 void *dq, void *dk, float *dwq, float *dwk, void *workspace,
                 size_t workspace_bytes, const RopeShape &s, const int64_t *dqo_st,
                 const int64_t *dko_st, const int64_t *q_st, const int64_t *k_st,
                 const int64_t *dq_st, const int64_t *dk_st, const int64_t *cs_st, void *stream) {
  const LaunchDevice launch_dev(stream);
  int rc = check_rope_shape(s);
  if (rc) return rc;
  if ((rc = check_tensor(dq_out, dqo_st, s.B, s.S, s.H, s.D, false, 0))) return rc;
  if ((rc = check_tensor(dk_out, dko_st, s.B, s.S, s.Hk, s.D, false, 0))) return rc;
  if ((rc = check_tensor(dq, dq_st, s.B, s.S, s.H, s.D, true, 0))) return rc;
  if ((rc = check_tensor(dk, dk_st, s.B, s.S, s.Hk, s.D, true, 0))) return rc;
  if ((rc = check_rope_table(cos, sin, cs_st))) return rc;
  if ((rc = check_rope_eps(wq, wk, eps))) return rc;
  const bool norm = wq != nullptr || wk != nullptr;
  // The forward's inputs and the dw outputs matter only for a normed side.
  if (wq != nullptr) {
    if ((rc = check_tensor(q, q_st, s.B, s.S, s.H, s.D, false, 0))) return rc;
    if (dwq == nullptr) return FA_ERR_NULL_POINTER;
    if (!aligned16(dwq)) return FA_ERR_ALIGNMENT;
  }
  if (wk != nullptr) {
    if ((rc = check_tensor(k, k_st, s.B, s.S, s.Hk, s.D, false, 0))) return rc;
    if (dwk == nullptr) return FA_ERR_NULL_POINTER;
    if (!aligned16(dwk)) return FA_ERR_ALIGNMENT;
  }
  if (norm) {
    if (workspace == nullptr || workspace_bytes < 2 * rope_partial_bytes(s)) return FA_ERR_WORKSPACE;
    if (!aligned16(workspace)) return FA_ERR_ALIGNMENT;
  }

  fa::RopeArgs a{};
  const void *x[2] = {q, k}, *g[2] = {dq_out, dk_out};
  void *y[2] = {dq, dk};
  const void *w[2] = {wq, wk};
  const int64_t *xs[2] = {q_st, k_st}, *gs[2] = {dqo_st, dko_st}, *ys[2] = {dq_st, dk_st};
  const int heads[2] = {s.H, s.Hk};
  for (int i = 0; i < 2; ++i) {
    fa::RopeSide &t = a.side[i];
    t.g = static_cast<const f16 *>(g[i]);
    t.y = static_cast<f16 *>(y[i]);
    t.w = static_cast<const f16 *>(w[i]);
    rope_strides(gs[i], t.gb, t.gs, t.gh);
    rope_strides(ys[i], t.yb, t.ys, t.yh);
    if (t.w != nullptr) {
      t.x = static_cast<const f16 *>(x[i]);
      rope_strides(xs[i], t.xb, t.xs, t.xh);
      t.partial = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                            (size_t)i * rope_partial_bytes(s));
    }
    t.heads = heads[i];
    t.rows = (int64_t)s.B * s.S * heads[i];
  }
  a.cos = static_cast<const f16 *>(cos);
  a.sin = static_cast<const f16 *>(sin);
  a.cb = cs_st[0];
  a.cs = cs_st[1];
  a.S = s.S;
  a.eps = eps;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t blocks = rope_blocks(s, norm);
  FA_ROPE_DISPATCH(launch_rope_bwd, s, a, blocks, dwq, dwk, st);
}

}  // namespace

// ---------------------------------------------------------------------------
// Allocation-free backward (fa_bwd_gqa_noalloc).  Its workspace -- delta,
// and the split schedule's counters and fp32 partials when they fit -- is
// this file-scope device array: each GPU the library runs on holds its own
// copy, FA_NOALLOC_SCRATCH_BYTES, until the process ends.  In host code the
// name is only a stand-in, never an address: the device copy's address is
// looked up once per device (with that device current) and that pointer is
// what the kernels get.  Nothing in the array needs clearing between calls:
// the dQ kernel writes delta and zeroes the split counters before the dK/dV
// kernel reads them, and every partial is written before it is read.
static __device__ __align__(256) unsigned char scratch[FA_NOALLOC_SCRATCH_BYTES];

namespace {

// Device address of `scratch` per device index (0: not looked up yet).  The
// lookup stores the same value from any thread, so the cache is race-free.
constexpr int kScratchDevices = 64;
std::atomic<uintptr_t> g_scratch_addr[kScratchDevices];

// The scratch array's address on the device of `stream` (stream_device):
// looked up with that device current, which is restored afterwards.
int scratch_for_stream(void *stream, void **out) {
  const int dev = stream_device(static_cast<hipStream_t>(stream));
  if (dev < 0) return FA_ERR_LAUNCH;
  const bool cached = dev < kScratchDevices;
  uintptr_t p = cached ? g_scratch_addr[dev].load(std::memory_order_relaxed) : 0;
  if (p == 0) {
    int cur = dev;
    if (hipGetDevice(&cur) != hipSuccess) cur = dev;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) {
      (void)hipGetLastError();
      return FA_ERR_LAUNCH;
    }
    void *addr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || addr == nullptr) {
      (void)hipGetLastError();   // not a launch error of the next call
      return FA_ERR_LAUNCH;
    }
    p = reinterpret_cast<uintptr_t>(addr);
    if (cached) g_scratch_addr[dev].store(p, std::memory_order_relaxed);
  }
  *out = reinterpret_cast<void *>(p);
  return FA_OK;
}

}  // namespace

extern "C" {

int fa_abi_version(void) { return FA_ABI_VERSION; }

const char *fa_strerror(int status) {
  switch (status) {
    case FA_OK: return "success";
    case FA_ERR_NULL_POINTER: return "a required pointer is NULL";
    case FA_ERR_HEAD_DIM: return "unsupported head_dim (supported: 32, 64, 128)";
    case FA_ERR_SHAPE:
      return "B, sequence lengths and head counts must be positive, and the query head "
             "count a multiple of the key/value head count";
    case FA_ERR_STRIDE:
      return "bad stride: the head_dim stride must be 1, the other strides non-negative "
             "multiples of 8 elements, and an output's rows must not overlap";
    case FA_ERR_ALIGNMENT: return "tensor data pointer is not 16-byte aligned";
    case FA_ERR_SCALE: return "sm_scale is not finite";
    case FA_ERR_WORKSPACE: return "workspace is NULL or smaller than fa_bwd_workspace_bytes()";
    case FA_ERR_TOO_LARGE:
      return "sizes or strides exceed the kernel's index or grid limits (a sequence stride "
             "must keep 127 rows under 2^31 bytes)";
    case FA_ERR_LAUNCH:
      return "the HIP runtime reported an error (a kernel launch, or the device address of "
             "the no-alloc scratch buffer)";
    case FA_ERR_SCRATCH:
      return "fa_bwd_gqa_noalloc: delta and the row-group maxima (fa_bwd_workspace_bytes) "
             "exceed the static scratch "
             "buffer (FA_NOALLOC_SCRATCH_BYTES)";
    case FA_ERR_DTYPE: return "unsupported dtype (supported: FA_DTYPE_F16, FA_DTYPE_BF16)";
    case FA_ERR_EPS: return "norm eps is negative or not finite";
    default: return "unknown status code";
  }
}

int fa_fwd(const void *q, const void *k, const void *v, void *o, float *lse,
           int B, int S, int H, int D,
           const int64_t q_strides[4], const int64_t k_strides[4],
           const int64_t v_strides[4], const int64_t o_strides[4],
           float sm_scale, int causal, void *stream) {
  return run_fwd(q, k, v, o, lse, square(B, S, H, D), q_strides, k_strides, v_strides, o_strides,
                 sm_scale, causal, stream);
}

int fa_fwd_gqa(const void *q, const void *k, const void *v, void *o, float *lse,
               int B, int Sq, int Sk, int H, int Hk, int D,
               const int64_t q_strides[4], const int64_t k_strides[4],
               const int64_t v_strides[4], const int64_t o_strides[4],
               float sm_scale, int causal, int dtype, void *stream) {
  return run_fwd(q, k, v, o, lse, Shape{B, Sq, Sk, H, Hk, D, dtype}, q_strides, k_strides, v_strides,
                 o_strides, sm_scale, causal, stream);
}

size_t fa_fwd_splitkv_workspace_bytes(int B, int Sq, int Sk, int H, int Hk, int D) {
  const Shape s{B, Sq, Sk, H, Hk, D, FA_DTYPE_F16};
  if (check_shape(s) != FA_OK) return 0;
  return splitkv_bytes(s, splitkv_plan(s));
}

int fa_fwd_splitkv(const void *q, const void *k, const void *v, void *o, float *lse,
                   void *workspace, size_t workspace_bytes,
                   int B, int Sq, int Sk, int H, int Hk, int D,
                   const int64_t q_strides[4], const int64_t k_strides[4],
                   const int64_t v_strides[4], const int64_t o_strides[4],
                   float sm_scale, int causal, int dtype, void *stream) {
  return run_fwd_splitkv(q, k, v, o, lse, workspace, workspace_bytes,
                         Shape{B, Sq, Sk, H, Hk, D, dtype}, q_strides, k_strides, v_strides,
                         o_strides, sm_scale, causal, stream);
}

size_t fa_fwd_workspace_bytes(int B, int Sq, int Sk, int H, int Hk, int D, int causal) {
  const Shape s{B, Sq, Sk, H, Hk, D, FA_DTYPE_F16};
  if (check_shape(s) != FA_OK) return 0;
  return fwd_ws_bytes(s, causal);
}

int fa_fwd_ws(const void *q, const void *k, const void *v, void *o, float *lse,
              void *workspace, size_t workspace_bytes,
              int B, int Sq, int Sk, int H, int Hk, int D,
              const int64_t q_strides[4], const int64_t k_strides[4],
              const int64_t v_strides[4], const int64_t o_strides[4],
              float sm_scale, int causal, int dtype, void *stream) {
  return run_fwd_ws(q, k, v, o, lse, workspace, workspace_bytes, Shape{B, Sq, Sk, H, Hk, D, dtype},
                    q_strides, k_strides, v_strides, o_strides, sm_scale, causal, stream);
}

int fa_bwd_preprocess(const void *o, const void *dout, float *delta, float *rowmax,
                      int B, int S, int H, int D,
                      const int64_t o_strides[4], const int64_t do_strides[4],
                      void *stream) {
  return run_pre(o, dout, delta, rowmax, square(B, S, H, D), o_strides, do_strides, stream);
}

size_t fa_bwd_workspace_bytes(int B, int S, int H, int D) {
  if (check_shape(square(B, S, H, D)) != FA_OK) return 0;
  return delta_bytes(B, S, H) + rmax_bytes(B, S, H);
}

size_t fa_bwd_rowmax_bytes(int B, int S, int H) {
  if (B <= 0 || S <= 0 || H <= 0) return 0;
  return rmax_bytes(B, S, H);
}

size_t fa_bwd_gqa_workspace_bytes(int B, int Sq, int Sk, int H, int Hk, int D, int causal) {
  const Shape s{B, Sq, Sk, H, Hk, D, FA_DTYPE_F16};
  if (check_shape(s) != FA_OK) return 0;
  DkdvSplit plan;
  DqSplit qplan;
  bwd_plans(s, causal, plan, qplan);
  return delta_bytes(B, Sq, H) + rmax_bytes(B, Sq, H) + split_bytes(plan) + dq_split_bytes(qplan);
}

int fa_bwd(const void *dout, const void *q, const void *k, const void *v,
           const void *o, const float *lse,
           void *dq, void *dk, void *dv,
           void *workspace, size_t workspace_bytes,
           int B, int S, int H, int D,
           const int64_t do_strides[4], const int64_t q_strides[4],
           const int64_t k_strides[4], const int64_t v_strides[4],
           const int64_t o_strides[4], const int64_t dq_strides[4],
           const int64_t dk_strides[4], const int64_t dv_strides[4],
           float sm_scale, int causal, void *stream) {
  return run_bwd(dout, q, k, v, o, lse, dq, dk, dv, workspace, workspace_bytes,
                 square(B, S, H, D), do_strides, q_strides, k_strides, v_strides, o_strides,
                 dq_strides, dk_strides, dv_strides, sm_scale, causal, stream);
}

int fa_bwd_gqa(const void *dout, const void *q, const void *k, const void *v,
               const void *o, const float *lse,
               void *dq, void *dk, void *dv,
               void *workspace, size_t workspace_bytes,
               int B, int Sq, int Sk, int H, int Hk, int D,
               const int64_t do_strides[4], const int64_t q_strides[4],
               const int64_t k_strides[4], const int64_t v_strides[4],
               const int64_t o_strides[4], const int64_t dq_strides[4],
               const int64_t dk_strides[4], const int64_t dv_strides[4],
               float sm_scale, int causal, int dtype, void *stream) {
  return run_bwd(dout, q, k, v, o, lse, dq, dk, dv, workspace, workspace_bytes,
                 Shape{B, Sq, Sk, H, Hk, D, dtype}, do_strides, q_strides, k_strides, v_strides,
                 o_strides, dq_strides, dk_strides, dv_strides, sm_scale, causal, stream);
}

int fa_bwd_gqa_noalloc(const void *dout, const void *q, const void *k, const void *v,
                       const void *o, const float *lse,
                       void *dq, void *dk, void *dv,
                       int B, int Sq, int Sk, int H, int Hk, int D,
                       const int64_t do_strides[4], const int64_t q_strides[4],
                       const int64_t k_strides[4], const int64_t v_strides[4],
                       const int64_t o_strides[4], const int64_t dq_strides[4],
                       const int64_t dk_strides[4], const int64_t dv_strides[4],
                       float sm_scale, int causal, int dtype, void *stream) {
  const Shape s{B, Sq, Sk, H, Hk, D, dtype};
  int rc = check_bwd(dout, q, k, v, o, lse, dq, dk, dv, s, do_strides, q_strides, k_strides,
                     v_strides, o_strides, dq_strides, dk_strides, dv_strides, sm_scale);
  if (rc) return rc;
  if (delta_bytes(B, Sq, H) + rmax_bytes(B, Sq, H) > (size_t)FA_NOALLOC_SCRATCH_BYTES)
    return FA_ERR_SCRATCH;
  void *ws = nullptr;
  if ((rc = scratch_for_stream(stream, &ws))) return rc;
  return run_bwd(dout, q, k, v, o, lse, dq, dk, dv, ws, FA_NOALLOC_SCRATCH_BYTES, s, do_strides,
                 q_strides, k_strides, v_strides, o_strides, dq_strides, dk_strides, dv_strides,
                 sm_scale, causal, stream);
}

int fa_bwd_dkdv(const void *dout, const void *q, const void *k, const void *v,
                const float *lse, const float *delta, const float *rowmax, void *dk, void *dv,
                int B, int S, int H, int D,
                const int64_t do_strides[4], const int64_t q_strides[4],
                const int64_t k_strides[4], const int64_t v_strides[4],
                const int64_t dk_strides[4], const int64_t dv_strides[4],
                float sm_scale, int causal, void *stream) {
  return run_dkdv(dout, q, k, v, lse, delta, rowmax, dk, dv, square(B, S, H, D), do_strides,
                  q_strides, k_strides, v_strides, dk_strides, dv_strides, sm_scale, causal,
                  stream);
}

int fa_bwd_dq(const void *dout, const void *q, const void *k, const void *v,
              const float *lse, const float *delta, void *dq,
              int B, int S, int H, int D,
              const int64_t do_strides[4], const int64_t q_strides[4],
              const int64_t k_strides[4], const int64_t v_strides[4],
              const int64_t dq_strides[4],
              float sm_scale, int causal, void *stream) {
  return run_dq(dout, q, k, v, lse, delta, dq, square(B, S, H, D), do_strides, q_strides,
                k_strides, v_strides, dq_strides, sm_scale, causal, stream);
}

int fa_bwd_blocks(const void *dout, const void *q, const void *k, const void *v,
                  const float *lse, const float *delta, const float *rowmax, void *dq, void *dk,
                  void *dv, int B, int S, int H, int D,
                  const int64_t do_strides[4], const int64_t q_strides[4],
                  const int64_t k_strides[4], const int64_t v_strides[4],
                  const int64_t dq_strides[4], const int64_t dk_strides[4],
                  const int64_t dv_strides[4],
                  float sm_scale, int causal, void *stream) {
  return run_bwd_blocks(dout, q, k, v, lse, delta, rowmax, dq, dk, dv, square(B, S, H, D),
                        do_strides, q_strides, k_strides, v_strides, dq_strides, dk_strides,
                        dv_strides, sm_scale, causal, stream);
}

size_t fa_rope_qk_workspace_bytes(int B, int S, int H, int Hk, int D) {
  const RopeShape s{B, S, H, Hk, D, FA_DTYPE_F16};
  if (check_rope_shape(s) != FA_OK) return 0;
  return 2 * rope_partial_bytes(s);
}

int fa_rope_qk_fwd(const void *q, const void *k, void *q_out, void *k_out,
                   const void *cos, const void *sin,
                   const void *q_norm_weight, const void *k_norm_weight, float eps,
                   int B, int S, int H, int Hk, int D,
                   const int64_t q_strides[4], const int64_t k_strides[4],
                   const int64_t q_out_strides[4], const int64_t k_out_strides[4],
                   const int64_t cs_strides[2], int dtype, void *stream) {
  return run_rope_fwd(q, k, q_out, k_out, cos, sin, q_norm_weight, k_norm_weight, eps,
                      RopeShape{B, S, H, Hk, D, dtype}, q_strides, k_strides, q_out_strides,
                      k_out_strides, cs_strides, stream);
}

int fa_rope_qk_bwd(const void *dq_out, const void *dk_out, const void *q, const void *k,
                   const void *cos, const void *sin,
                   const void *q_norm_weight, const void *k_norm_weight, float eps,
                   void *dq, void *dk, float *dq_norm_weight, float *dk_norm_weight,
                   void *workspace, size_t workspace_bytes,
                   int B, int S, int H, int Hk, int D,
                   const int64_t dq_out_strides[4], const int64_t dk_out_strides[4],
                   const int64_t q_strides[4], const int64_t k_strides[4],
                   const int64_t dq_strides[4], const int64_t dk_strides[4],
                   const int64_t cs_strides[2], int dtype, void *stream) {
  return run_rope_bwd(dq_out, dk_out, q, k, cos, sin, q_norm_weight, k_norm_weight, eps, dq, dk,
                      dq_norm_weight, dk_norm_weight, workspace, workspace_bytes,
                      RopeShape{B, S, H, Hk, D, dtype}, dq_out_strides, dk_out_strides, q_strides,
                      k_strides, dq_strides, dk_strides, cs_strides, stream);
}

}  // extern "C"
