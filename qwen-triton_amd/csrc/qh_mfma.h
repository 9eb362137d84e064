// MFMA helpers shared by the GEMM and attention kernels (gfx950).
//
// v_mfma_f32_32x32x16_{bf16,f16} operand layout for lane l (0..63):
//   A (32 x 16): row l % 32, k = 8 * (l / 32) + e  (e = 0..7, one 16-byte register quad)
//   B (16 x 32): col l % 32, k = 8 * (l / 32) + e
//   C (32 x 32): col l % 32, row = 8 * g + 4 * (l / 32) + r for accumulator 4 * g + r
// The reduction over k is order-free, so A and B may use any common
// permutation of k; the attention kernels exploit this to feed a C-layout
// tile straight back in as the next product's B operand.
#pragma once

#include "qh_common.h"

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Mfma;
template <>
struct Mfma<bf16_t> {
  typedef bf16x8 v8;
  typedef bf16x4 v4;
  static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<f16_t> {
  typedef f16x8 v8;
  typedef f16x4 v4;
  static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// 16x16x32 products: lane l holds A row l%16 / B column l%16 with
// k = 8*(l/16)+e; C column l%16, rows 4*(l/16)+r.
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ f32x4 mma16(typename Mfma<T>::v8 a, typename Mfma<T>::v8 b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mma16<bf16_t>(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mma16<f16_t>(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int e = 0; e < 16; ++e) z[e] = 0.f;
  return z;
}

// Transpose an 8x8 block of 16-bit values: in[r] holds row r (8 values), out[c]
// receives column c.
__device__ __forceinline__ void transpose8x8(const uint4 (&in)[8], uint4 (&out)[8]) {
  const uint32_t* iw = reinterpret_cast<const uint32_t*>(in);
  uint32_t* ow = reinterpret_cast<uint32_t*>(out);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t a = iw[(2 * j) * 4 + (c >> 1)];
      const uint32_t b = iw[(2 * j + 1) * 4 + (c >> 1)];
      ow[c * 4 + j] = (c & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
    }
  }
}

// Workgroups are dealt round-robin to the 8 XCDs: renumber so each XCD walks a
// contiguous range of logical tiles (tile_order), then order tiles in groups of
// 8 M-tiles (tile_group_order, on a logical tile index) so concurrently running
// tiles share operand panels in the XCD's L2.
__device__ __forceinline__ void tile_group_order(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  constexpr int GROUP = 8;
  const int group_size = GROUP * tiles_n;
  const int g = pid / group_size;
  const int first_m = g * GROUP;
  const int gm = min(tiles_m - first_m, GROUP);
  const int in_group = pid - g * group_size;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}
__device__ __forceinline__ void tile_order(int tiles_m, int tiles_n, int& tm, int& tn) {
  int pid = blockIdx.x;
  const int nblk = gridDim.x;
  if ((nblk & 7) == 0) pid = (pid & 7) * (nblk >> 3) + (pid >> 3);
  tile_group_order(pid, tiles_m, tiles_n, tm, tn);
}
