// MFMA, fragment and LDS helpers for the ELSA HIP kernels (gfx950 / CDNA4 only).
//
// Every matrix product in this library is a 32x32 output tile on the wave64
// matrix cores:
//   fp16 : v_mfma_f32_32x32x16_f16   (A, B: 8 halves per lane, C/D: 16 floats)
//   bf16 : v_mfma_f32_32x32x16_bf16  (A, B: 8 bf16 per lane,  C/D: 16 floats)
//   fp32 : v_mfma_f32_32x32x2_f32    (A, B: 1 float per lane,  C/D: 16 floats)
//
// Operand layout (lane l, c = l % 32, g = l / 32, item t < KP):
//   A[i][k] : lane with c == i holds k = g*KP + t        (row of A per lane)
//   B[k][j] : lane with c == j holds k = g*KP + t        (column of B per lane)
//   D[i][j] : lane with c == j, register r holds row i = (r/4)*8 + 4*g + (r%4)
// Any assignment of k to (g, t) is valid as long as A and B use the same one;
// the kernels exploit that freedom (see key_of_reg). The layout is checked on
// the device by elsa_debug_mfma (tests/test_gpu_layout.py).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace elsa {

typedef _Float16 f16;
typedef __bf16 bf16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

template <typename T>
struct Mfma;

template <>
struct Mfma<f16> {
  static constexpr int KP = 8;
  typedef f16x8 frag;
  __device__ static inline f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<bf16> {
  static constexpr int KP = 8;
  typedef bf16x8 frag;
  __device__ static inline f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<float> {
  static constexpr int KP = 1;
  typedef float frag;
  __device__ static inline f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

// Row of the 32x32 D tile held by register r of a lane in lane-group g.
__device__ __host__ constexpr inline int drow(int r, int g) { return (r >> 2) * 8 + 4 * g + (r & 3); }

// Permutation of the 32 rows of an A operand: swapping bits 2 and 3 of the row
// position makes the D-layout register r of lane-group g correspond to key
// 16*(r/8) + 8*g + (r%8) (key_of_reg), so a lane's 8 consecutive registers are
// 8 consecutive keys and can feed the next MFMA's B operand directly.
__device__ __host__ constexpr inline int swap23(int i) {
  return (i & ~0xC) | ((i & 4) << 1) | ((i & 8) >> 1);
}
__device__ __host__ constexpr inline int key_of_reg(int r, int g) { return 16 * (r >> 3) + 8 * g + (r & 7); }

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Load KP elements (one MFMA operand fragment) from memory; `ok` false gives zeros.
template <typename T>
__device__ inline typename Mfma<T>::frag load_frag(const T* p, bool ok) {
  typedef typename Mfma<T>::frag F;
  if constexpr (Mfma<T>::KP == 1) {
    return ok ? *p : 0.0f;
  } else {
    F z = {};
    return ok ? *reinterpret_cast<const F*>(p) : z;
  }
}

// Build a B-operand fragment of type T from KP consecutive fp32 registers.
template <typename T, int R0>
__device__ inline typename Mfma<T>::frag pack_frag(const f32x16& v) {
  if constexpr (Mfma<T>::KP == 1) {
    return v[R0];
  } else {
    typename Mfma<T>::frag f;
#pragma unroll
    for (int t = 0; t < 8; ++t) f[t] = static_cast<T>(v[R0 + t]);
    return f;
  }
}

// Compile-time loop: f(std::integral_constant<int, I>) for I = B .. E-1.  Register
// staging arrays indexed through it see constant indices from the start, so they are
// split into VGPRs; indexed by a `#pragma unroll` loop variable they can instead be
// placed in LDS or scratch before the loop is unrolled.
template <int B, int E, typename Fn>
__device__ inline void static_for(Fn&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// 16-byte raw chunk used for global->LDS staging.  A vector type, not a struct: a
// struct copy is a memcpy, and a staging array of structs copied global -> array ->
// LDS by memcpy is not split into registers (it ends up in LDS or scratch).
typedef uint32_t Chunk16 __attribute__((ext_vector_type(4)));

// Raw buffer resource over [base, base + bytes): loads whose VGPR offset is >= bytes
// return zeros (callers keep the SGPR offset at 0 so that the whole offset is
// range-checked), which is the key-range masking the tile loaders need without compares.
// bytes must stay below 2^31 so that an offset pushed past it by kBufferOff never wraps.
constexpr uint32_t kBufferOff = 0x80000000u;
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
__device__ inline Chunk16 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(Chunk16, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
// 16 bytes per lane from a buffer straight into LDS (buffer_load_dwordx4 ... lds): lane i's bytes
// land at lds + 16 i (lds is wave-uniform: it goes to M0); offsets past the buffer range read zeros
__device__ inline void buffer_load16_lds(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

// acc + a + b with an fp32 accumulator (v_dot2_f32_f16 / v_dot2_f32_bf16 against (1, 1)).
__device__ inline float sum2(f16 a, f16 b, float acc) {
  const f16x2 v = {a, b}, one = {(f16)1.0f, (f16)1.0f};
  return __builtin_amdgcn_fdot2(v, one, acc, false);
}
__device__ inline float sum2(bf16 a, bf16 b, float acc) {
  const bf16x2 v = {a, b}, one = {(bf16)1.0f, (bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(v, one, acc, false);
}

// Unpadded LDS tiles of 64 two-byte elements per row (128 bytes) with the 16-byte chunk q of row r
// stored at chunk q ^ lds_swz(r), lds_swz(r) = 4 (m % 2) + m / 2 with m = (r / 2) % 8.  Both
// fragment reads of the kernels are then free of bank conflicts: the 16 lanes of a row-fragment
// read (one chunk of 16 rows) land on 16 distinct 4-bank groups, since the 8 rows of one parity
// take 8 distinct lds_swz values; the 32 lanes of a transposing read (rows r..r+3 for r a multiple
// of 4, 64 bytes each) land on disjoint groups, since rows r and r + 2 differ in bit 2 of lds_swz.
// No padded stride serves both: the row fragments need an odd multiple of 4 banks, the
// transposing reads 16 or 48.  lds_swz reads bits 1-3 of the row only, so offsets computed
// for one 16-row block hold in every other.
__device__ __host__ constexpr inline int lds_swz(int r) { return (((r >> 1) & 1) << 2) | ((r >> 2) & 3); }
__device__ __host__ constexpr inline int lds_swz_off(int r, int col) {
  return r * 64 + ((((col >> 3) ^ lds_swz(r)) << 3) | (col & 7));
}

// Transposing LDS read (ds_read_b64_tr_b16).  Within each 16-lane group, source
// lane s = 4t + a reads 4 16-bit elements at its own address; result lane
// i = 4a' + b' receives element b' of source lanes a' + 4t, t = 0..3.  Pointing
// source lane 4t + a at &M[k0 + t][d0 + 4a] of a row-major tile therefore gives
// lane i the column segment M[k0 .. k0+3][d0 + i].
__device__ inline i16x4 lds_read_tr16(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)p);
}

// Work-group coordinates in an XCD-aware order.  The dispatcher hands the work-groups
// of a launch (x fastest, then y, then z) to the 8 XCDs round-robin, and each XCD has
// its own L2.  Renumbering so that the work-groups running on one XCD cover one
// contiguous range of the logical grid (x fastest) keeps the K/V panel that neighbouring
// row blocks share in one L2, instead of fetching it into all eight.  The map is a
// bijection for any grid size.
struct WgCoord {
  int x, y, z;
};
__device__ inline int xcd_linear() {
  const int n = gridDim.x * gridDim.y * gridDim.z;
  const int lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const int per = n >> 3, rem = n & 7, xcd = lin & 7, slot = lin >> 3;
  return xcd * per + min(xcd, rem) + slot;
}
__device__ inline WgCoord xcd_order() {
  const int gx = gridDim.x, gy = gridDim.y, l = xcd_linear();
  return {l % gx, (l / gx) % gy, l / (gx * gy)};
}
// xcd_order for causal backward grids that fit the chip in one round of two work-groups per CU
// (more than 256, at most 512 work-groups of the 4-wave kernels), whose work-groups are numbered
// heaviest first within each head: the second half of each XCD's work-groups comes lightest
// first, so that the CU that takes the j-th work-group of the first half also takes the j-th
// lightest, and every CU gets about the same work.
__device__ inline WgCoord xcd_order_paired() {
  const int n = gridDim.x * gridDim.y * gridDim.z;
  const int lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const int per = n >> 3, rem = n & 7, xcd = lin & 7;
  int slot = lin >> 3;
  if (n > 256 && n <= 512 && rem == 0 && (per & 1) == 0 && slot >= per / 2) slot = per + per / 2 - 1 - slot;
  const int l = xcd * per + min(xcd, rem) + slot;
  const int gx = gridDim.x, gy = gridDim.y;
  return {l % gx, (l / gx) % gy, l / (gx * gy)};
}
// Non-causal Phase 1 (grid x = row block, y = head, z = K partition) with the panels (head,
// partition) dealt to the XCDs in turn, each panel whole: the dispatcher sends workgroup L to
// XCD L % 8, and the j-th workgroup of an XCD (j = L / 8) takes row block j % gx of panel
// L % 8 + 8 (j / gx), panel = head + gy * partition.  A short last partition then spreads its
// panels over all XCDs instead of leaving the last XCDs idle (B1 H8 N16K with 8190-key
// partitions: 96 workgroups of the full partitions on each of five XCDs against 64 on
// every XCD).  Panel counts that are not a multiple of 8 keep xcd_order.
__device__ inline WgCoord panel_order() {
  const int gx = gridDim.x, gy = gridDim.y, npan = gy * gridDim.z;
  if (npan & 7) return xcd_order();
  const int lin = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const int j = lin >> 3, pan = (lin & 7) + 8 * (j / gx);
  return {j % gx, pan % gy, pan / gy};
}
// Phase 1 order (grid x = row block, y = head, z = K partition).  Non-causal: panel_order
// (row blocks fastest, whole panels per XCD), so the workgroups resident on one XCD share one
// K/V partition panel in its L2: Phase 1 then fetches its algorithmic bytes (Q once per
// partition, K and V once; 101 MB at B1 H8 N16K d64 with 4 partitions), where a
// partition-fastest order fetched 244 MB in the same time.  Causal: the work of a row block
// grows with its index and vanishes for partitions past it; there the dispatcher's own
// round-robin over XCDs balances best, with the row blocks reversed so that the heaviest
// start first.
__device__ inline WgCoord phase1_order(bool causal) {
  if (causal) return {(int)gridDim.x - 1 - (int)blockIdx.x, (int)blockIdx.y, (int)blockIdx.z};
  return panel_order();
}

// Causal Phase 1 over the whole sequence (grid nrb row blocks x BH heads x P partitions, rpp =
// part_len / BM row blocks per partition): the dispatch order is longest first.  Row block r
// folds min(r - rpp*p, rpp - 1) + 1 key stages of partition p, none when r < rpp*p, and the
// same for every head, so the linear workgroup index L takes the head from L % BH (every XCD
// keeps the same heads when BH is a multiple of 8, and with them their K/V in its L2) and the
// (r, p) pair from L / BH in decreasing order of work: all pairs of the full level, then the
// diagonal levels from the longest down, then the empty pairs, which exit at once.  A greedy
// simulation of 512 resident workgroups at N = 16K, 4096-key partitions, 256-row blocks puts
// this order at 1.02 times the ideal makespan against 1.34 for phase1_order.
__device__ inline WgCoord causal_longest_first(int nrb, int BH, int P, int rpp) {
  const int L = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const int bh = L % BH;
  int j = L / BH;
  for (int p = 0; p < P; ++p) {  // rpp stages: r >= rpp*(p+1) - 1
    const int n = nrb - (rpp * p + rpp - 1);
    if (n <= 0) break;
    if (j < n) return {rpp * p + rpp - 1 + j, bh, p};
    j -= n;
  }
  for (int w = rpp - 2; w >= 0; --w) {  // w + 1 stages: r = rpp*p + w
    const int n = nrb > w ? min(P, (nrb - w + rpp - 1) / rpp) : 0;
    if (j < n) return {rpp * j + w, bh, j};
    j -= n;
  }
  for (int p = 1; p < P; ++p) {  // no keys: r < rpp*p
    const int n = min(nrb, rpp * p);
    if (j < n) return {j, bh, p};
    j -= n;
  }
  return {0, bh, 0};
}

// Combine the two 32-lane halves of a wave (lanes l and l ^ 32) with
// v_permlane32_swap: both results hold one value of each half.
__device__ inline float wave_max_pair(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float wave_sum_pair(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace elsa
