// fa_common.hpp -- shared device helpers for the gfx950 FlashAttention kernels.
//
// Everything here is written for CDNA4 wave64 and the 32x32x16 16-bit MFMAs
// (v_mfma_f32_32x32x16_f16 / _bf16, 8 passes, 32768 FLOP per wave
// instruction).  Kernels are templated on the element type E (fp16 or
// bf16); pointers, LDS tiles and DMA staging carry raw 16-bit values typed
// `f16`, and only the fragments fed to the MFMAs and conversions are typed
// E.
//
// MFMA fragment conventions used by every kernel (lane = 0..63,
// l32 = lane % 32, g = lane / 32):
//   A operand  (32 x 16): lane holds A[row = l32][k = 8g .. 8g+7]
//   B operand  (16 x 32): lane holds B[k = 8g .. 8g+7][col = l32]
//   C/D result (32 x 32): lane holds C[row = 8*(i/4) + 4g + i%4][col = l32],
//                         i = 0..15
// The hardware's k order inside an operand is irrelevant as long as A and B
// agree, which they do because both are indexed by the same (lane, slot).
//
// The kernels compute transposed score tiles S^T = K Q^T, so a lane owns one
// query (the result column) and a per-lane subset of 16 keys (result rows).
// The A-operand rows of K are permuted with kperm() so that result slot i of
// lane group g is key 16*(i/8) + 8g + i%8: each 8-slot half of a lane's
// results is then 8 consecutive keys, exactly the k-slice the lane supplies
// when those probabilities are re-used as the B operand of the next MFMA.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace fa {

typedef _Float16 f16;
typedef __bf16 bf16;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
template <typename E> using vec8 = E __attribute__((ext_vector_type(8)));
template <typename E> using vec4 = E __attribute__((ext_vector_type(4)));
template <typename E> using vec2 = E __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();
constexpr float kPosInf = __builtin_inff();

__device__ __forceinline__ floatx16 mfma32(vec8<f16> a, vec8<f16> b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ floatx16 mfma32(vec8<bf16> a, vec8<bf16> b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Key (or query) index, inside a 32-block, of result slot i for lane group g.
__device__ __forceinline__ constexpr int slot_row(int i, int g) {
  return 16 * (i >> 3) + 8 * g + (i & 7);
}

// A-operand row permutation: the key that A-row r must hold so that the
// result row 8*(i/4) + 4g + i%4 (= r) carries key slot_row(i, g).
__device__ __forceinline__ int kperm(int r) {
  return 16 * (r >> 4) + 8 * ((r >> 2) & 1) + 4 * ((r >> 3) & 1) + (r & 3);
}

// Result-row index (inside a 32x32 C tile) of slot i for lane group g.
__device__ __forceinline__ constexpr int c_row(int i, int g) {
  return 8 * (i >> 2) + 4 * g + (i & 3);
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

__device__ __forceinline__ float fast_log2(float x) {
  return __builtin_amdgcn_logf(x);
}

// Value held by lane (lane ^ 32): the other half-wave owns the same query.
// v_permlane32_swap (below) leaves each lane {own, partner}; their bitwise
// xor with own is the partner, whichever order they come in (no LDS
// round trip).
__device__ __forceinline__ float xor32(float x) {
  const unsigned u = __float_as_uint(x);
  auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0] ^ r[1] ^ u);
}

// Value held by lane (lane ^ 1) (DPP quad_perm [1, 0, 3, 2]).
__device__ __forceinline__ float xor1(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
}

// max(x, value of lane ^ 32) without an LDS round trip.  v_permlane32_swap
// exchanges the upper half of its first operand with the lower half of its
// second; with both operands x, each lane ends up holding {own, partner} in
// some order.
__device__ __forceinline__ float max_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(x, fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])));
}

// Cross-lane maxima of non-negative floats, compared as unsigned bit
// patterns (they order non-negative floats as the floats do: one v_max_u32
// per step, no NaN canonicalisation), through DPP row operations instead
// of LDS-crossbar permutes.  One step: max with the lane DPP control CTRL
// names, in the rows of ROWS (other rows keep their value).
template <int CTRL, int ROWS>
__device__ __forceinline__ unsigned dpp_umax(unsigned m) {
  return max(m, (unsigned)__builtin_amdgcn_update_dpp((int)m, (int)m, CTRL, ROWS, 0xF, false));
}

// Maximum of x >= 0 over each 32-lane half of the wave, in the half's last
// lane (31, 63): within quads (lane ^ 1, lane ^ 2), 8-lane groups
// (row_half_mirror), 16-lane rows (row_mirror), then row 0's into row 1
// and row 2's into row 3 (row_bcast:15).
__device__ __forceinline__ unsigned max_halves_nonneg(float x) {
  unsigned m = __float_as_uint(x);
  m = dpp_umax<0xB1, 0xF>(m);    // quad_perm [1, 0, 3, 2]
  m = dpp_umax<0x4E, 0xF>(m);    // quad_perm [2, 3, 0, 1]
  m = dpp_umax<0x141, 0xF>(m);   // row_half_mirror
  m = dpp_umax<0x140, 0xF>(m);   // row_mirror
  return dpp_umax<0x142, 0xA>(m);   // row_bcast:15
}

// Maximum of x >= 0 over the wave, in lane 63 (row_bcast:31 brings lane
// 31's half maximum into rows 2 and 3).
__device__ __forceinline__ unsigned max_wave_nonneg(float x) {
  return dpp_umax<0x143, 0xC>(max_halves_nonneg(x));
}

// Sum of the two 16-bit values of `p` accumulated into fp32 `acc`
// (v_dot2_f32_f16 / v_dot2_f32_bf16 against (1, 1)).
__device__ __forceinline__ float dot2_acc(vec2<bf16> p, float acc) {
  const vec2<bf16> ones = {(bf16)1.0f, (bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(p, ones, acc, false);
}

__device__ __forceinline__ float dot2_acc(half2 p, float acc) {
  const half2 ones = {(f16)1.0f, (f16)1.0f};
  return __builtin_amdgcn_fdot2(p, ones, acc, false);
}

// Pack the low (or high) halves of two dwords into one dword.
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
  return (a & 0xffffu) | (b << 16);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
  return (a >> 16) | (b & 0xffff0000u);
}

// Flip the sign of 8 packed fp16 values (exact).
template <typename V>
__device__ __forceinline__ V neg8(V x) {
  u32x4 u = __builtin_bit_cast(u32x4, x);
  u ^= 0x80008000u;   // flip the sign bit of each 16-bit value (fp16 and bf16 alike)
  return __builtin_bit_cast(V, u);
}

// Buffer resource over rows [n0, S) of one (b, h) of a (B, S, H, D) tensor
// with row stride `ss` elements: raw (stride-0) buffer whose extent ends at
// the last element of row S-1, so a 16-byte load at byte offset
// r*ss*2 + 16*c (c < D/8) returns zeros for rows n0 + r >= S when ss >= D
// (and stays inside the tensor otherwise).  gfx9-family descriptor word 3.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const f16 *head, int64_t ss, int n0,
                                                            int S, int D) {
  // Scalar-only arithmetic (32-bit compares), so no VGPR temporaries: a
  // VALU 64-bit compare here would make the compiler wait for outstanding
  // tile loads that target the same registers.
  const f16 *base = head + (int64_t)n0 * ss;
  const int rows = S - n0;
  uint32_t ext = 0;
  if (rows > 0) {
    const uint64_t e = (uint64_t)(uint32_t)(rows - 1) * (uint64_t)(ss * 2) + (uint64_t)(2 * D);
    ext = (uint32_t)(e >> 32) != 0u ? 0xffffffffu : (uint32_t)e;
  }
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)ext, 0x00020000);
}

// rows_rsrc for a walk through a head in steps of a fixed number of rows:
// the base and the remaining byte count advance by a constant step, so each
// step costs a few scalar adds instead of rows_rsrc's 64-bit multiplies.
// rsrc() is the descriptor rows_rsrc(head, ss, r, S, D) gives at the
// cursor's row r (extent 0 once r >= S).
struct RowCursor {
  const char *base;   // row r of the head
  int64_t rem;        // bytes from row r to the end of row S-1
  int64_t step;       // bytes per step
  int left;           // rows S - r
  int rows_step;      // rows per step

  __device__ __forceinline__ void init(const f16 *head, int64_t ss, int r, int S, int D,
                                       int rows) {
    base = reinterpret_cast<const char *>(head + (int64_t)r * ss);
    rem = (int64_t)(S - 1 - r) * ss * 2 + 2 * D;
    step = (int64_t)rows * ss * 2;
    left = S - r;
    rows_step = rows;
  }
  __device__ __forceinline__ void advance() {
    base += step;
    rem -= step;
    left -= rows_step;
  }
  __device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc() const {
    uint32_t ext = 0;
    if (left > 0) ext = (rem >> 32) != 0 ? 0xffffffffu : (uint32_t)rem;
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)ext, 0x00020000);
  }
};

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

// LDS row holding in-tile row r when 32-row blocks are stored in kperm order
// (kperm swaps bits 2 and 3, so it is its own inverse).
__device__ __forceinline__ int kperm_row(int r) { return (r & ~31) + kperm(r & 31); }

// Causal work balance.  Workgroups are numbered bid = r * BH + bh; blocks
// with larger `heavy_rank` cost more (causal: more visible tiles).  Ranks are
// dealt heaviest-first for the first half of the grid and lightest-first for
// the second half, so the first-round and second-round workgroups that the
// dispatcher places on one CU (bid and bid + half * BH) carry complementary
// loads; with more workgroups than slots it degrades to longest-first.
// Returns the heavy rank (0 = heaviest) of rank r out of n.
__device__ __forceinline__ int zigzag_rank(int r, int n) {
  const int half = (n + 1) / 2;
  return r < half ? r : n - 1 - (r - half);
}

// f(integral_constant<int, 0>), ..., f(integral_constant<int, N - 1>): a loop
// whose index is a compile-time constant in the body (register arrays
// indexed by it stay in registers, and scheduling builtins take it).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F &f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Index of this thread's wave, as a wave-uniform (scalar) value.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// Per-lane LDS offsets inside a tile loop.  An LDS read's address is
// VGPR + 16-bit immediate, and the addresses of one lane's reads differ by
// compile-time constants (LDS array, stage, sub-block, 8-row step) once the
// lane's offset carries the wave-uniform part (its query or key group).  But
// LLVM hoists every (array + offset) sum out of the loop as a loop invariant,
// each into a VGPR of its own: one register per array, stage and chunk
// (measured: 34 address VGPRs in the D = 64 dK/dV loop, against 11 offsets).
// Passing the offsets through an empty asm at the top of every iteration
// makes those sums loop-variant, so each read takes the offset register plus
// an immediate.  No instruction is emitted.
// The offsets are kept in bytes (an element offset would need a shift per
// use) and ALIGN states what the reads may assume of them.
template <int ALIGN>
__device__ __forceinline__ void opaque(int &x) {
  asm volatile("" : "+v"(x));
  __builtin_assume((x & (ALIGN - 1)) == 0);
}

// ---------------------------------------------------------------------------
// Swizzled tiles staged straight from global memory into LDS.
//
// A tile is ROWS rows x D fp16, row stride 2*D bytes (unpadded except
// SW_PD's 16 bytes per KiB), with 32-row blocks in kperm row order.  Each row's 16-byte chunks are XOR-permuted:
// physical chunk = logical chunk ^ swz(row).  The LDS serves a wave's read
// in groups of lanes (gfx950: 64 banks of 4 bytes; 16 lanes of a 128-bit
// read, 32 lanes of a 64-bit transposed read per cycle), so a read is
// conflict-free when each group's bytes fall in distinct banks.  The two
// ways the kernels read tiles ask different things of the swizzle:
//   * A operands, ds_read_b128 of one logical chunk by lanes reading
//     consecutive rows (lane l32 reads row l32): any 16 consecutive rows
//     must land in 16 distinct 16-byte bank groups of a 256-byte window;
//   * transposed operands, ds_read_b64_tr_b16: an aligned group of 4 rows x
//     4 consecutive chunks {4q..4q+3} must cover 16 distinct groups of 256
//     bytes.
// Each map's output bits are parities of subsets of the row's low 4 bits,
// found by a search over all such maps (a map meeting only the 8-lane form
// of the first property measured 25-49 % bank-conflicted LDS cycles).
//   SW_A  (tiles read only as A operands): the first property.
//   SW_T  (tiles read only transposed): the second, with period 8 in the
//         row, so a transposed fragment's second read (8 rows further) is
//         the first's address plus an immediate.
//   SW_AT (tiles read both ways): both properties; period 16, so the second
//         transposed read takes its own offset (TrOffsets).
//   SW_P8 (tiles read both ways where the registers of those extra offsets
//         would cost occupancy): period 8, the 8-lane form of the first
//         property and the second at D <= 64.
//   SW_PD (tiles read both ways, D = 128): both properties with period 4
//         in the row, on a tile padded with 16 bytes after every KiB
//         (lds_row).  Rows 8 apart then share the chunk permutation (the
//         second transposed read is the first's address plus an immediate,
//         lds_row(8)) but sit 32 bytes apart in the bank window, which
//         gives 16 consecutive rows 16 distinct groups.  A tile costs 1/64
//         more LDS.  (The D = 64 analogue -- period 8, rows 8 apart 16 bytes
//         apart -- measured as many conflicts as SW_P8 on the query tiles
//         and more than SW_A on row-read tiles, so the model above is not
//         the whole story at D = 64; it is not used.)
enum { SW_A = 0, SW_T = 1, SW_AT = 2, SW_P8 = 3, SW_PD = 4 };
template <int D, int SW>
__device__ __forceinline__ constexpr int swz(int r) {
  static_assert(SW != SW_PD || D >= 128, "SW_PD is the D = 128 layout");
  if (SW == SW_A)
    return D >= 128 ? (r & 15)
         : D == 64  ? (((r >> 1) & 3) | (((r ^ (r >> 3)) & 1) << 2))
                    : (((r >> 2) & 1) | ((((r >> 1) ^ (r >> 3)) & 1) << 1));
  if (SW == SW_PD) return (r & 3) << 2;
  if (SW == SW_P8)
    return D >= 64 ? (((r & 3) << 1) | ((r >> 2) & 1)) : ((((r >> 1) & 1) << 1) | ((r >> 2) & 1));
  if (SW == SW_T)
    return D >= 128 ? ((r & 3) << 2)
         : D == 64  ? (((r & 3) << 1) | ((r >> 2) & 1))
                    : ((((r >> 1) & 1) << 1) | ((r >> 2) & 1));
  return D >= 128 ? ((r & 3) | (((r ^ (r >> 2)) & 3) << 2))
       : D == 64  ? (((r >> 1) & 1) | (((r ^ (r >> 2)) & 1) << 1) |
                     (((r ^ (r >> 1) ^ (r >> 3)) & 1) << 2))
                  : (((r >> 2) & 1) | ((((r >> 1) ^ (r >> 3)) & 1) << 1));
}

// Element offset of row r of a tile in LDS (rows of D fp16; an SW_PD tile
// has 8 elements of padding after every 512).  Linear in r over multiples
// of 4 rows at D = 128, so sub-block bases stay immediates.  lds_row(ROWS)
// is a tile's size.
template <int D, int SW>
__host__ __device__ __forceinline__ constexpr int lds_row(int r) {
  return SW == SW_PD ? r * D + 8 * ((r * D) >> 9) : r * D;
}

typedef __attribute__((address_space(3))) void lds_void;

// One buffer_load_dwordx4 ... lds: lane i's 16 bytes at byte offset `voff`
// of `rs` land at LDS byte (lds + 16 * i) (layout measured on gfx950); M0
// holds `lds`, which must be wave-uniform.  Tracked by vmcnt.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rs, const void *lds, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void *)lds, 16, voff, 0, 0, 0);
}

// Loads one ROWS-row tile (rows r0 .. r0+ROWS-1 of a (b, h) head, zeros
// past S) into a swizzled LDS slot: ROWS*D*2 bytes = ROWS*D/512 wave
// instructions of 1 KiB, ROWS*D/(512*NW) per wave of an NW-wave workgroup.
// No VGPRs hold tile data.
template <int D, int SW, int ROWS = 64, int NW = 4>
struct DmaStager {
  static constexpr int PER_WAVE = ROWS * D / (512 * NW);
  static_assert(PER_WAVE >= 1, "tile smaller than one DMA instruction per wave");
  int off[PER_WAVE];   // global byte offset of this lane's chunk, relative to row r0

  __device__ __forceinline__ void init(int w, int lane, int64_t ss) {
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int byte = (w * PER_WAVE + j) * 1024 + 16 * lane;
      const int p = byte / (2 * D), pc = (byte % (2 * D)) / 16;
      off[j] = kperm_row(p) * (int)ss * 2 + 16 * (pc ^ swz<D, SW>(p));
    }
  }
  __device__ __forceinline__ void load(f16 *slot, const f16 *head, int64_t ss, int r0, int S,
                                       int w) const {
    load(slot, rows_rsrc(head, ss, r0, S, D), w);
  }
  __device__ __forceinline__ void load(f16 *slot, __amdgpu_buffer_rsrc_t rs, int w) const {
    // one KiB per instruction, plus SW_PD's 16 bytes after each
    constexpr int kStride = lds_row<D, SW>(512 / D);
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) lds_dma16(rs, slot + (w * PER_WAVE + j) * kStride, off[j]);
  }
};

// A-operand (32 x 16) fragment of X^T from a row-major LDS tile X with two
// ds_read_b64_tr_b16 transpose loads, at `base + lo` and `base + hi`
// (elements).  Transpose-load lane layout (measured on gfx950): in each
// 16-lane group, source lane L addresses row L/4, columns 4*(L%4) .. +3 of a
// 4 x 16 block, and lane i receives column i of the four rows.  So with the
// lane's address of (row_lo + L/4, col0 + 16*((lane/16)%2) + 4*(L%4)) the
// lane receives X[row_lo + j][col0 + lane % 32] in slots j = 0..3, and from
// the same block 8 rows further the slots 4..7 (TrOffsets).  The transpose
// read moves 16-bit values without interpreting them, so one fp16-typed
// read serves both element types (the result is bit-cast).
template <typename E>
__device__ __forceinline__ vec8<E> load_tr_pair(const f16 *base, int lo, int hi) {
  typedef __fp16 h4 __attribute__((vector_size(8)));
  h4 a0 = __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) h4 *)(base + lo));
  h4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) h4 *)(base + hi));
  const u32x2 x = __builtin_bit_cast(u32x2, a0), y = __builtin_bit_cast(u32x2, a1);
  const u32x4 r = {x[0], x[1], y[0], y[1]};
  return __builtin_bit_cast(vec8<E>, r);
}

// load_tr_pair at byte offsets lo, hi from base.
template <typename E>
__device__ __forceinline__ vec8<E> load_tr_pair_b(const f16 *base, int lo, int hi) {
  typedef __fp16 h4 __attribute__((vector_size(8)));
  typedef __attribute__((address_space(3))) h4 lds_h4;
  const char *b = reinterpret_cast<const char *>(base);
  h4 a0 = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_h4 *)(b + lo));
  h4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_h4 *)(b + hi));
  const u32x2 x = __builtin_bit_cast(u32x2, a0), y = __builtin_bit_cast(u32x2, a1);
  const u32x4 r = {x[0], x[1], y[0], y[1]};
  return __builtin_bit_cast(vec8<E>, r);
}

// Per-lane element offsets of the transposed reads of a swizzled tile: for
// column block d (32 columns), rows 4g + (l16 >> 2) (`lo`) and 8 rows
// further (`hi`), column chunk 4d + 2((lane >> 4) & 1) + ((l16 >> 1) & 1),
// half 4 * (l16 & 1).  Row offsets that are multiples of 16 (sub-blocks of
// 32 rows, the 16-row halves; lds_row of them) keep the swizzle.  With
// SW_T, SW_P8 and SW_PD the swizzle repeats every 8 rows and hi(d) is
// lo(d) + lds_row(8), an immediate; with SW_AT the two reads take
// different chunk permutations and hi is a register.
template <int D, int SW>
struct TrOffsets {
  static constexpr bool SPLIT = SW == SW_A || SW == SW_AT;
  int lo_[D / 32];
  int hi_[SPLIT ? D / 32 : 1];
  __device__ __forceinline__ void init(int lane) {
    const int l16 = lane & 15, tr = 4 * (lane >> 5) + (l16 >> 2);
    const int half = 4 * (l16 & 1);
#pragma unroll
    for (int d = 0; d < D / 32; ++d) {
      const int c = 4 * d + 2 * ((lane >> 4) & 1) + ((l16 >> 1) & 1);
      lo_[d] = lds_row<D, SW>(tr) + ((c ^ swz<D, SW>(tr)) << 3) + half;
      if constexpr (SPLIT) hi_[d] = (tr + 8) * D + ((c ^ swz<D, SW>(tr + 8)) << 3) + half;
    }
  }
  __device__ __forceinline__ int lo(int d) const { return lo_[d]; }
  __device__ __forceinline__ int hi(int d) const {
    if constexpr (SPLIT) return hi_[d];
    else return lo_[d] + lds_row<D, SW>(8);
  }
};

// TrOffsets in bytes, hidden from loop-invariant code motion by hide() (see
// opaque()): for loops whose LDS arrays and stages are compile-time
// constants, so every transposed read is one register plus an immediate.
template <int D, int SW>
struct TrOffsetsB {
  static constexpr bool SPLIT = TrOffsets<D, SW>::SPLIT;
  int lo_[D / 32];
  int hi_[SPLIT ? D / 32 : 1];
  __device__ __forceinline__ void init(int lane, int base) {
    TrOffsets<D, SW> t;
    t.init(lane);
#pragma unroll
    for (int d = 0; d < D / 32; ++d) {
      lo_[d] = 2 * (t.lo(d) + base);
      if constexpr (SPLIT) hi_[d] = 2 * (t.hi(d) + base);
    }
  }
  __device__ __forceinline__ int lo(int d) const { return lo_[d]; }
  __device__ __forceinline__ int hi(int d) const {
    if constexpr (SPLIT) return hi_[d];
    else return lo_[d] + 2 * lds_row<D, SW>(8);
  }
  __device__ __forceinline__ void hide() {
#pragma unroll
    for (int d = 0; d < D / 32; ++d) {
      opaque<8>(lo_[d]);
      if constexpr (SPLIT) opaque<8>(hi_[d]);
    }
  }
};

// 8 consecutive 16-bit values at p (16-byte aligned), as an E vector.
template <typename E>
__device__ __forceinline__ vec8<E> ld8(const f16 *p) {
  return *reinterpret_cast<const vec8<E> *>(p);
}

// The same at a byte offset from p.
template <typename E>
__device__ __forceinline__ vec8<E> ld8_b(const f16 *p, int byte_off) {
  return *reinterpret_cast<const vec8<E> *>(reinterpret_cast<const char *>(p) + byte_off);
}

// Kernel arguments shared by the forward and backward launches. Strides are
// in elements of a (B, S, H, D) tensor whose D stride is 1.
struct TensorDesc {
  const f16 *ptr;
  int64_t sb, ss, sh;
  __device__ __forceinline__ const f16 *head(int b, int h) const {
    return ptr + b * sb + h * sh;
  }
};

}  // namespace fa
