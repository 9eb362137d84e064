// Attention input preparation of one (token, head) row, shared by the fused
// prepare pass (qh_fused.hip) and the decode attention that prepares its own
// rows (qh_attention.hip), so both round exactly alike.
#pragma once
#include "qh_common.h"

// Per-lane parameters of a row: norm scale (w + wadd) and cos/sin of the lane's
// 8 columns (d0 .. d0 + 7; cos/sin only below rot, at (d mod half)).
struct RowParams {
  float w[8], c[8], s[8];
};

// Per-element loads (any alignment; wdtype fp32 or a 16-bit type).
template <typename C>
__device__ __forceinline__ RowParams load_row_params(const void* w, int wdtype, float wadd, int d0, bool act,
                                                     int half, int rot, const C* __restrict__ cs,
                                                     const C* __restrict__ sn, int64_t co_row) {
  RowParams rp;
#pragma unroll
  for (int e = 0; e < 8; ++e) rp.w[e] = act ? load_any(w, wdtype, d0 + e) + wadd : 0.f;
  if (d0 < rot) {
    const int64_t co = co_row + (d0 < half ? d0 : d0 - half);
#pragma unroll
    for (int e = 0; e < 8; ++e) rp.c[e] = to_f32(cs[co + e]), rp.s[e] = to_f32(sn[co + e]);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) rp.c[e] = 0.f, rp.s[e] = 0.f;
  }
  return rp;
}

// The same values from 16-byte words (w, cs and sn 16-byte aligned; C a 16-bit
// type; wdtype fp32 or C's dtype), in two steps: the raw 16-byte words, loaded with no
// branch (so that a caller can have them in flight together with its other
// loads before the first use: a branch ends the block the loads can be
// scheduled in), then their conversion. w1 is the second word of fp32 weights
// (bf16/f16 weights load the first word twice); lanes at or past rot load the
// row's first cos/sin word (in bounds) and get zeros.
struct RowRaw {
  uint4 w0, w1, c, s;
};

template <typename C>
__device__ __forceinline__ RowRaw load_row_raw(const void* w, int wdtype, int d0, bool act, int half, int rot,
                                               const C* __restrict__ cs, const C* __restrict__ sn, int64_t co_row) {
  static_assert(sizeof(C) == 2, "vector row parameters need a 16-bit cos/sin type");
  const bool f32 = wdtype == QH_F32;
  const char* wb = static_cast<const char*>(w) + (int64_t)(act ? d0 : 0) * (f32 ? 4 : 2);
  const int64_t co = co_row + (d0 < rot ? (d0 < half ? d0 : d0 - half) : 0);
  RowRaw r;
  r.w0 = *reinterpret_cast<const uint4*>(wb);
  r.w1 = *reinterpret_cast<const uint4*>(wb + (f32 ? 16 : 0));
  r.c = *reinterpret_cast<const uint4*>(cs + co);
  r.s = *reinterpret_cast<const uint4*>(sn + co);
  return r;
}

template <typename C>
__device__ __forceinline__ RowParams row_params_from(const RowRaw& r, int wdtype, float wadd, int d0, bool act,
                                                     int rot) {
  RowParams rp;
  if (wdtype == QH_F32) {
    const float f[8] = {__uint_as_float(r.w0.x), __uint_as_float(r.w0.y), __uint_as_float(r.w0.z),
                        __uint_as_float(r.w0.w), __uint_as_float(r.w1.x), __uint_as_float(r.w1.y),
                        __uint_as_float(r.w1.z), __uint_as_float(r.w1.w)};
#pragma unroll
    for (int e = 0; e < 8; ++e) rp.w[e] = act ? f[e] + wadd : 0.f;
  } else {
    Vec16<C> v;
    v.raw = r.w0;
#pragma unroll
    for (int e = 0; e < 8; ++e) rp.w[e] = act ? to_f32(v.v[e]) + wadd : 0.f;
  }
  Vec16<C> c, sv;
  c.raw = r.c;
  sv.raw = r.s;
  const bool in = d0 < rot;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    rp.c[e] = in ? to_f32(c.v[e]) : 0.f;
    rp.s[e] = in ? to_f32(sv.v[e]) : 0.f;
  }
  return rp;
}

// A row of D <= 128 elements on a 16-lane group, 8 per lane (lane g holds
// d0 = 8 g .. d0 + 7; act = d0 < D): RMSNorm over D (fp32 sums, the 16-lane
// DPP reduction of the norm kernel, rounded to T), then rotate-half RoPE of the
// first rot elements with the lane's cos/sin (rounded to T); the rest passes
// through. hl = half / 8 is the lane distance between the halves. All 16 lanes
// of the group must call it together.
template <typename T>
__device__ __forceinline__ Vec16<T> norm_rope_apply(const Vec16<T>& xv, bool act, const RowParams& rp, float eps,
                                                    int D, int d0, int hl, int half, int rot) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float f = to_f32(xv.v[e]);
    ss += f * f;
  }
  ss = wave_sum(ss, 16);
  const float inv = rsqrtf(ss / (float)D + eps);
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = act ? to_f32(from_f32<T>((to_f32(xv.v[e]) * inv) * rp.w[e])) : 0.f;
  float px[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) px[e] = __shfl_xor(y[e], hl, 16);
  Vec16<T> o;
  if (d0 < rot) {
    const bool lo = d0 < half;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float cc = rp.c[e], sv2 = rp.s[e];
      const float a = lo ? y[e] : px[e], bb = lo ? px[e] : y[e];
      o.v[e] = lo ? from_f32<T>(a * cc - bb * sv2) : from_f32<T>(bb * cc + a * sv2);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) o.v[e] = from_f32<T>(y[e]);
  }
  return o;
}

// load_row_params + norm_rope_apply.
template <typename T, typename C>
__device__ __forceinline__ Vec16<T> norm_rope_row(const Vec16<T>& xv, bool act, const void* w, int wdtype, float eps,
                                                  float wadd, int D, int d0, int hl, int half, int rot,
                                                  const C* __restrict__ cs, const C* __restrict__ sn,
                                                  int64_t co_row) {
  const RowParams rp = load_row_params<C>(w, wdtype, wadd, d0, act, half, rot, cs, sn, co_row);
  return norm_rope_apply<T>(xv, act, rp, eps, D, d0, hl, half, rot);
}
