// Shared device/host helpers for the gfx950 (MI355X) operator library.
//
// Everything here is written for CDNA4 only: 64-lane wavefronts, bf16 converts
// through the hardware v_cvt_pk_bf16_f32, 16-byte global accesses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <type_traits>

#include "qwen_hip.h"

typedef __bf16 bf16_t;
typedef _Float16 f16_t;

#define QH_WAVE 64

// ---------------------------------------------------------------------------
// Error reporting: every entry point returns 0 or a QH_E* code and records a
// thread-local message retrievable through qh_last_error().
// ---------------------------------------------------------------------------
namespace qh {

void set_error(const char* fmt, ...);

}  // namespace qh

#define QH_CHECK_ARG(cond, ...)                 \
  do {                                          \
    if (!(cond)) {                              \
      qh::set_error(__VA_ARGS__);               \
      return QH_E_ARG;                          \
    }                                           \
  } while (0)

#define QH_CHECK_LAUNCH(name)                                                  \
  do {                                                                         \
    hipError_t _e = hipGetLastError();                                         \
    if (_e != hipSuccess) {                                                    \
      qh::set_error("%s: launch failed: %s", name, hipGetErrorString(_e));     \
      return QH_E_HIP;                                                         \
    }                                                                          \
  } while (0)

#define QH_CHECK_HIP(expr, name)                                               \
  do {                                                                         \
    hipError_t _e = (expr);                                                    \
    if (_e != hipSuccess) {                                                    \
      qh::set_error("%s: %s", name, hipGetErrorString(_e));                    \
      return QH_E_HIP;                                                         \
    }                                                                          \
  } while (0)

// ---------------------------------------------------------------------------
// Kernel arguments read at the kernel's start. The compiler issues an argument's
// scalar load next to its first use, which may sit behind a branch or behind
// another argument's load (a product lookup, say): each such step is one more
// round trip before the first memory request, 0.5-0.7 us measured on a 5 us
// decode launch. sgpr_now(x) materialises x in scalar registers at that point;
// a run of them at a kernel's start has the loads issued together.
// ---------------------------------------------------------------------------
template <typename X>
__device__ __forceinline__ void sgpr_now(X& x) {
  asm volatile("" : "+s"(x));
}

// ---------------------------------------------------------------------------
// Scalar conversions
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float to_f32(T v) { return (float)v; }

template <typename T>
__device__ __forceinline__ T from_f32(float v) { return (T)v; }

// ---------------------------------------------------------------------------
// 16-byte vector of N elements of T (N * sizeof(T) == 16)
// ---------------------------------------------------------------------------
template <typename T>
struct Vec16 {
  static constexpr int N = 16 / sizeof(T);
  union {
    uint4 raw;
    T v[N];
  };
};

template <typename T>
__device__ __forceinline__ Vec16<T> ld16(const T* p) {
  Vec16<T> r;
  r.raw = *reinterpret_cast<const uint4*>(p);
  return r;
}

template <typename T>
__device__ __forceinline__ void st16(T* p, const Vec16<T>& v) {
  *reinterpret_cast<uint4*>(p) = v.raw;
}

// Non-temporal forms, for tensors streamed once that exceed the last-level
// cache (e.g. logits over a 151936-word vocabulary): they do not displace
// cached data.
typedef unsigned int qh_u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ Vec16<T> ld16_nt(const T* p) {
  const qh_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const qh_u32x4*>(p));
  Vec16<T> r;
  r.raw = make_uint4(v.x, v.y, v.z, v.w);
  return r;
}

template <typename T>
__device__ __forceinline__ void st16_nt(T* p, const Vec16<T>& v) {
  const qh_u32x4 w = {v.raw.x, v.raw.y, v.raw.z, v.raw.w};
  __builtin_nontemporal_store(w, reinterpret_cast<qh_u32x4*>(p));
}

// ---------------------------------------------------------------------------
// Wavefront reductions (64 lanes). `width` must be a power of two <= 64 and
// reduces within aligned groups of `width` lanes; every lane gets the result.
// ---------------------------------------------------------------------------
// DPP lane permutations (gfx9 encodings): quad_perm xor-1 / xor-2, and the
// half-row / row mirrors that pair lane i with 7-i / 15-i. Applied in sequence
// they all-reduce 16 lanes with plain VALU ops (no LDS crossbar traffic).
#define QH_DPP_XOR1 0xB1
#define QH_DPP_XOR2 0x4E
#define QH_DPP_HALF_MIRROR 0x141
#define QH_DPP_MIRROR 0x140

// Scalar access to a buffer whose dtype (QH_F32/F16/BF16) is only known at run time.
__device__ __forceinline__ float load_any(const void* p, int dtype, int64_t i) {
  if (dtype == QH_F32) return ((const float*)p)[i];
  if (dtype == QH_F16) return (float)((const f16_t*)p)[i];
  return (float)((const bf16_t*)p)[i];
}

// VN consecutive elements p[i .. i+VN) of a runtime-dtype buffer as fp32, with
// 16-byte loads when the buffer is 16-byte aligned (al16) and VN elements of the
// buffer's dtype span whole 16-byte words; i must be a multiple of VN.
template <int VN>
__device__ __forceinline__ void load_any_vec(const void* p, int dtype, int64_t i, bool al16, float (&out)[VN]) {
  if (al16 && dtype == QH_F32 && VN % 4 == 0) {
#pragma unroll
    for (int q = 0; q < VN; q += 4) {
      const float4 v = *reinterpret_cast<const float4*>((const float*)p + i + q);
      out[q] = v.x, out[q + 1] = v.y, out[q + 2] = v.z, out[q + 3] = v.w;
    }
  } else if (al16 && dtype == QH_BF16 && VN % 8 == 0) {
#pragma unroll
    for (int q = 0; q < VN; q += 8) {
      const Vec16<bf16_t> v = ld16((const bf16_t*)p + i + q);
#pragma unroll
      for (int j = 0; j < 8; ++j) out[q + j] = (float)v.v[j];
    }
  } else if (al16 && dtype == QH_F16 && VN % 8 == 0) {
#pragma unroll
    for (int q = 0; q < VN; q += 8) {
      const Vec16<f16_t> v = ld16((const f16_t*)p + i + q);
#pragma unroll
      for (int j = 0; j < 8; ++j) out[q + j] = (float)v.v[j];
    }
  } else {
#pragma unroll
    for (int j = 0; j < VN; ++j) out[j] = load_any(p, dtype, i + j);
  }
}

__device__ __forceinline__ void store_any(void* p, int dtype, int64_t i, float v) {
  if (dtype == QH_F32) ((float*)p)[i] = v;
  else if (dtype == QH_F16) ((f16_t*)p)[i] = (f16_t)v;
  else ((bf16_t*)p)[i] = (bf16_t)v;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

template <bool MAX>
__device__ __forceinline__ float red_op(float a, float b) {
  return MAX ? fmaxf(a, b) : a + b;
}

template <bool MAX>
__device__ __forceinline__ float group_reduce(float v, int width) {
  if (width >= 2) v = red_op<MAX>(v, dpp_f32<QH_DPP_XOR1>(v));
  if (width >= 4) v = red_op<MAX>(v, dpp_f32<QH_DPP_XOR2>(v));
  if (width >= 8) v = red_op<MAX>(v, dpp_f32<QH_DPP_HALF_MIRROR>(v));
  if (width >= 16) v = red_op<MAX>(v, dpp_f32<QH_DPP_MIRROR>(v));
  for (int o = 16; o < width; o <<= 1) v = red_op<MAX>(v, __shfl_xor(v, o, width));
  return v;
}

__device__ __forceinline__ float wave_sum(float v, int width = QH_WAVE) { return group_reduce<false>(v, width); }

__device__ __forceinline__ float wave_max(float v, int width = QH_WAVE) { return group_reduce<true>(v, width); }

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024). `red` must hold
// blockDim.x / 64 floats. The result is returned to every thread.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += red[i];  // fixed order: deterministic
  return t;
}

__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float t = -INFINITY;
  for (int i = 0; i < nw; ++i) t = fmaxf(t, red[i]);
  return t;
}

__device__ __forceinline__ float fast_exp(float x) { return __expf(x); }

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

static inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

static inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// QH_* dtype code of a storage type.
template <typename T>
constexpr int qh_dtype_of();
template <>
constexpr int qh_dtype_of<float>() { return QH_F32; }
template <>
constexpr int qh_dtype_of<f16_t>() { return QH_F16; }
template <>
constexpr int qh_dtype_of<bf16_t>() { return QH_BF16; }

// Dispatch a templated functor over the three storage dtypes.
#define QH_DISPATCH_DTYPE(dtype, T, name, ...)                         \
  switch (dtype) {                                                     \
    case QH_F32: { typedef float T; __VA_ARGS__; break; }              \
    case QH_F16: { typedef f16_t T; __VA_ARGS__; break; }              \
    case QH_BF16: { typedef bf16_t T; __VA_ARGS__; break; }            \
    default: qh::set_error("%s: unsupported dtype %d", name, (int)dtype); return QH_E_DTYPE; \
  }
