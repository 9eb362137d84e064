// Bandwidth-bound operators: flat elementwise ops, residual add, RoPE, KV-cache
// write/append and embedding gather.
//
// Design (gfx950): every thread moves 16-byte vectors; grids are sized to a few
// waves per CU with grid-stride loops so a launch covers all 256 CUs without
// oversubscribing the dispatcher. fp32 math, one rounding on store.
#include "qh_common.h"

#include <algorithm>

namespace {

// ---------------------------------------------------------------------------
// Flat elementwise family
// ---------------------------------------------------------------------------
enum class EwOp { Add, SiluMul, SigmoidMul };

template <EwOp OP>
__device__ __forceinline__ float ew_apply(float a, float b) {
  if constexpr (OP == EwOp::Add) return a + b;
  if constexpr (OP == EwOp::SiluMul) return a * sigmoidf_(a) * b;  // silu(gate) * up
  return a * sigmoidf_(b);                                           // x * sigmoid(gate)
}

// Launches whose traffic reaches the last-level cache's size (256 MB) stream
// with non-temporal accesses (NT): caching them would only evict other data.
constexpr int64_t kStreamBytes = 256ll << 20;

template <bool NT, typename T>
__device__ __forceinline__ Vec16<T> ld16s(const T* p) {
  if constexpr (NT) return ld16_nt(p);
  else return ld16(p);
}
template <bool NT, typename T>
__device__ __forceinline__ void st16s(T* p, const Vec16<T>& v) {
  if constexpr (NT) st16_nt(p, v);
  else st16(p, v);
}

template <EwOp OP, typename T, bool NT>
__global__ __launch_bounds__(256) void ew_binary_vec(const T* __restrict__ a, const T* __restrict__ b,
                                                     T* __restrict__ o, int64_t nvec) {
  constexpr int VN = Vec16<T>::N;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nvec;
       i += (int64_t)gridDim.x * blockDim.x) {
    Vec16<T> va = ld16s<NT>(a + i * VN), vb = ld16s<NT>(b + i * VN), vo;
#pragma unroll
    for (int j = 0; j < VN; ++j) vo.v[j] = from_f32<T>(ew_apply<OP>(to_f32(va.v[j]), to_f32(vb.v[j])));
    st16s<NT>(o + i * VN, vo);
  }
}

template <EwOp OP, typename T>
__global__ __launch_bounds__(256) void ew_binary_scalar(const T* __restrict__ a, const T* __restrict__ b,
                                                        T* __restrict__ o, int64_t start, int64_t n) {
  for (int64_t i = start + blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    o[i] = from_f32<T>(ew_apply<OP>(to_f32(a[i]), to_f32(b[i])));
}

static int grid_for(int64_t work, int64_t per_block = 256) {
  int64_t g = ceil_div(work, per_block);
  if (g > 8192) g = 8192;
  if (g < 1) g = 1;
  return (int)g;
}

template <EwOp OP, typename T>
int launch_binary(const void* a, const void* b, void* o, int64_t n, hipStream_t st) {
  constexpr int VN = Vec16<T>::N;
  int64_t nvec = 0;
  if (aligned16(a) && aligned16(b) && aligned16(o)) nvec = n / VN;
  if (nvec > 0) {
    if (3 * nvec * 16 >= kStreamBytes)
      ew_binary_vec<OP, T, true><<<grid_for(nvec), 256, 0, st>>>((const T*)a, (const T*)b, (T*)o, nvec);
    else
      ew_binary_vec<OP, T, false><<<grid_for(nvec), 256, 0, st>>>((const T*)a, (const T*)b, (T*)o, nvec);
  }
  int64_t done = nvec * VN;
  if (done < n)
    ew_binary_scalar<OP, T><<<grid_for(n - done), 256, 0, st>>>((const T*)a, (const T*)b, (T*)o, done, n);
  return QH_OK;
}

// Backward of the two gated products: (ga, gb) from (a, b, g).
template <EwOp OP>
__device__ __forceinline__ void ew_grad(float a, float b, float g, float& ga, float& gb) {
  if constexpr (OP == EwOp::SiluMul) {  // a = gate, b = up
    float s = sigmoidf_(a);
    ga = g * b * s * (1.0f + a * (1.0f - s));
    gb = g * a * s;
  } else {  // a = x, b = gate
    float s = sigmoidf_(b);
    ga = g * s;
    gb = g * a * s * (1.0f - s);
  }
}

template <EwOp OP, typename T, bool NT>
__global__ __launch_bounds__(256) void ew_grad_vec(const T* __restrict__ a, const T* __restrict__ b,
                                                   const T* __restrict__ g, T* __restrict__ ga,
                                                   T* __restrict__ gb, int64_t nvec) {
  constexpr int VN = Vec16<T>::N;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nvec;
       i += (int64_t)gridDim.x * blockDim.x) {
    Vec16<T> va = ld16s<NT>(a + i * VN), vb = ld16s<NT>(b + i * VN), vg = ld16s<NT>(g + i * VN), oa, ob;
#pragma unroll
    for (int j = 0; j < VN; ++j) {
      float x, y;
      ew_grad<OP>(to_f32(va.v[j]), to_f32(vb.v[j]), to_f32(vg.v[j]), x, y);
      oa.v[j] = from_f32<T>(x);
      ob.v[j] = from_f32<T>(y);
    }
    st16s<NT>(ga + i * VN, oa);
    st16s<NT>(gb + i * VN, ob);
  }
}

template <EwOp OP, typename T>
__global__ __launch_bounds__(256) void ew_grad_scalar(const T* __restrict__ a, const T* __restrict__ b,
                                                      const T* __restrict__ g, T* __restrict__ ga,
                                                      T* __restrict__ gb, int64_t start, int64_t n) {
  for (int64_t i = start + blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    float x, y;
    ew_grad<OP>(to_f32(a[i]), to_f32(b[i]), to_f32(g[i]), x, y);
    ga[i] = from_f32<T>(x);
    gb[i] = from_f32<T>(y);
  }
}

template <EwOp OP, typename T>
int launch_grad(const void* a, const void* b, const void* g, void* ga, void* gb, int64_t n, hipStream_t st) {
  constexpr int VN = Vec16<T>::N;
  int64_t nvec = 0;
  if (aligned16(a) && aligned16(b) && aligned16(g) && aligned16(ga) && aligned16(gb)) nvec = n / VN;
  if (nvec > 0) {
    if (5 * nvec * 16 >= kStreamBytes)
      ew_grad_vec<OP, T, true><<<grid_for(nvec), 256, 0, st>>>((const T*)a, (const T*)b, (const T*)g, (T*)ga,
                                                               (T*)gb, nvec);
    else
      ew_grad_vec<OP, T, false><<<grid_for(nvec), 256, 0, st>>>((const T*)a, (const T*)b, (const T*)g, (T*)ga,
                                                                (T*)gb, nvec);
  }
  int64_t done = nvec * VN;
  if (done < n)
    ew_grad_scalar<OP, T><<<grid_for(n - done), 256, 0, st>>>((const T*)a, (const T*)b, (const T*)g,
                                                              (T*)ga, (T*)gb, done, n);
  return QH_OK;
}

// ---------------------------------------------------------------------------
// RoPE (rotate-half), strided input, contiguous output.
// Work item per row (b,h,s): half pairs + (D - rot) pass-through elements.
// ---------------------------------------------------------------------------
template <typename T, typename C>
__global__ __launch_bounds__(256) void rope_kernel(const T* __restrict__ x, int64_t sxb, int64_t sxh,
                                                   int64_t sxs, int64_t sxd, const C* __restrict__ cs,
                                                   const C* __restrict__ sn, int64_t scb, int64_t scs,
                                                   int64_t scd, int64_t cos_batch, T* __restrict__ out,
                                                   int64_t H, int64_t S, int64_t D, int64_t half,
                                                   int64_t rot, int64_t items, int64_t total, float sgn) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / items, w = i - row * items;
    const int64_t s = row % S;
    const int64_t bh = row / S;
    const int64_t h = bh % H, b = bh / H;
    const T* xr = x + b * sxb + h * sxh + s * sxs;
    T* orow = out + row * D;
    if (w < half) {
      const int64_t cb = (cos_batch == 1) ? 0 : b;
      const int64_t co = cb * scb + s * scs + w * scd;
      const float c = to_f32(cs[co]), sv = sgn * to_f32(sn[co]);
      const float x1 = to_f32(xr[w * sxd]), x2 = to_f32(xr[(w + half) * sxd]);
      orow[w] = from_f32<T>(x1 * c - x2 * sv);
      orow[w + half] = from_f32<T>(x2 * c + x1 * sv);
    } else {
      const int64_t d = rot + (w - half);
      orow[d] = xr[d * sxd];
    }
  }
}

// Vectorised RoPE for the common case: contiguous last dim, rot == D, half a
// multiple of the vector width. Each thread rotates VN pairs.
template <typename T, bool NT>
__global__ __launch_bounds__(256) void rope_vec_kernel(const T* __restrict__ x, int64_t sxb, int64_t sxh,
                                                       int64_t sxs, const T* __restrict__ cs,
                                                       const T* __restrict__ sn, int64_t scb, int64_t scs,
                                                       int64_t cos_batch, T* __restrict__ out, int64_t H,
                                                       int64_t S, int64_t D, int64_t half, int64_t total,
                                                       float sgn) {
  constexpr int VN = Vec16<T>::N;
  const int64_t vpr = half / VN;  // vectors per row (per half)
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / vpr, w = (i - row * vpr) * VN;
    const int64_t s = row % S;
    const int64_t bh = row / S;
    const int64_t h = bh % H, b = bh / H;
    const T* xr = x + b * sxb + h * sxh + s * sxs;
    const int64_t cb = (cos_batch == 1) ? 0 : b;
    const int64_t co = cb * scb + s * scs + w;
    Vec16<T> x1 = ld16s<NT>(xr + w), x2 = ld16s<NT>(xr + w + half), c = ld16(cs + co), sv = ld16(sn + co), o1, o2;
#pragma unroll
    for (int j = 0; j < VN; ++j) {
      const float a = to_f32(x1.v[j]), bb = to_f32(x2.v[j]), cc = to_f32(c.v[j]), ss = sgn * to_f32(sv.v[j]);
      o1.v[j] = from_f32<T>(a * cc - bb * ss);
      o2.v[j] = from_f32<T>(bb * cc + a * ss);
    }
    T* orow = out + row * D;
    st16s<NT>(orow + w, o1);
    st16s<NT>(orow + w + half, o2);
  }
}

// ---------------------------------------------------------------------------
// KV cache write-by-position and append.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void kv_write_vec(T* __restrict__ cache, int64_t scb, int64_t sch,
                                                    int64_t scs, const T* __restrict__ val, int64_t svb,
                                                    int64_t svh, int64_t svs, const int64_t* __restrict__ pos,
                                                    int64_t H, int64_t S, int64_t vpr, int64_t cap,
                                                    int64_t total) {
  constexpr int VN = Vec16<T>::N;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / vpr, d = (i - row * vpr) * VN;
    const int64_t s = row % S, bh = row / S;
    const int64_t h = bh % H, b = bh / H;
    // the value's address does not depend on its position: both loads are in flight at once
    const Vec16<T> v = ld16(val + b * svb + h * svh + s * svs + d);
    const int64_t p = pos[s];
    if (p < 0 || p >= cap) continue;
    st16(cache + b * scb + h * sch + p * scs + d, v);
  }
}

// The same write for planes of at least kKvPlaneMin 16-byte chunks per (sequence, head):
// blockIdx.y is the (b, h) pair, so the chunk index needs one 32-bit division (by the
// chunks per row), and each thread has kKvPlaneU value loads and their position loads in
// flight at once (chunks past the plane load its last chunk and store nothing).
constexpr int kKvPlaneU = 2, kKvPlaneMin = 1024;

template <typename T>
__global__ __launch_bounds__(256) void kv_write_plane(T* __restrict__ cache, int64_t scb, int64_t sch, int64_t scs,
                                                      const T* __restrict__ val, int64_t svb, int64_t svh,
                                                      int64_t svs, const int64_t* __restrict__ pos, int H, int S,
                                                      int vpr, int64_t cap) {
  constexpr int VN = Vec16<T>::N;
  const int b = (int)blockIdx.y / H, h = (int)blockIdx.y - b * H;
  T* cb = cache + b * scb + h * sch;
  const T* vb = val + b * svb + h * svh;
  const int plane = S * vpr;
  const int base = (int)blockIdx.x * (256 * kKvPlaneU) + (int)threadIdx.x;
  Vec16<T> t[kKvPlaneU];
  int64_t p[kKvPlaneU];
  int d[kKvPlaneU];
#pragma unroll
  for (int u = 0; u < kKvPlaneU; ++u) {
    const int i = min(base + u * 256, plane - 1);
    const int s = i / vpr;
    d[u] = (i - s * vpr) * VN;
    t[u] = ld16(vb + s * svs + d[u]);
    p[u] = pos[s];
  }
#pragma unroll
  for (int u = 0; u < kKvPlaneU; ++u)
    if (base + u * 256 < plane && p[u] >= 0 && p[u] < cap) st16(cb + p[u] * scs + d[u], t[u]);
}

template <typename T>
__global__ __launch_bounds__(256) void kv_write_scalar(T* __restrict__ cache, int64_t scb, int64_t sch,
                                                       int64_t scs, int64_t scd, const T* __restrict__ val,
                                                       int64_t svb, int64_t svh, int64_t svs, int64_t svd,
                                                       const int64_t* __restrict__ pos, int64_t H, int64_t S,
                                                       int64_t D, int64_t cap, int64_t total) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / D, d = i - row * D;
    const int64_t s = row % S, bh = row / S;
    const int64_t h = bh % H, b = bh / H;
    const int64_t p = pos[s];
    if (p < 0 || p >= cap) continue;
    cache[b * scb + h * sch + p * scs + d * scd] = val[b * svb + h * svh + s * svs + d * svd];
  }
}

template <typename T>
__global__ __launch_bounds__(256) void kv_append_kernel(const T* __restrict__ pre, const T* __restrict__ suf,
                                                        T* __restrict__ out, int64_t so, int64_t sn, int64_t D,
                                                        int64_t total) {
  const int64_t st = so + sn;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t d = i % D, r = i / D;
    const int64_t s = r % st, bh = r / st;
    out[i] = (s < so) ? pre[(bh * so + s) * D + d] : suf[(bh * sn + (s - so)) * D + d];
  }
}

template <typename T>
__global__ __launch_bounds__(256) void kv_append_vec(const T* __restrict__ pre, const T* __restrict__ suf,
                                                     T* __restrict__ out, int64_t so, int64_t sn, int64_t vpr,
                                                     int64_t total) {
  constexpr int VN = Vec16<T>::N;
  const int64_t st = so + sn, D = vpr * VN;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t d = (i % vpr) * VN, r = i / vpr;
    const int64_t s = r % st, bh = r / st;
    const T* src = (s < so) ? pre + (bh * so + s) * D + d : suf + (bh * sn + (s - so)) * D + d;
    st16(out + r * D + d, ld16(src));
  }
}

// ---------------------------------------------------------------------------
// Embedding gather: one 64-lane wave per token row.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void embedding_vec(const int64_t* __restrict__ ids, const T* __restrict__ w,
                                                     int64_t stride_w, T* __restrict__ out, int64_t n_tokens,
                                                     int64_t V, int64_t Hd) {
  constexpr int VN = Vec16<T>::N;
  const int64_t t = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (t >= n_tokens) return;
  const int64_t id = ids[t];
  const bool ok = id >= 0 && id < V;
  const T* src = w + (ok ? id : 0) * stride_w;
  T* dst = out + t * Hd;
  Vec16<T> z;
  z.raw = make_uint4(0, 0, 0, 0);
  for (int64_t c = lane * VN; c < Hd; c += 64 * VN) {
    if (ok) st16(dst + c, ld16(src + c));
    else st16(dst + c, z);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void embedding_scalar(const int64_t* __restrict__ ids, const T* __restrict__ w,
                                                        int64_t stride_w, T* __restrict__ out, int64_t n_tokens,
                                                        int64_t V, int64_t Hd) {
  const int64_t t = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (t >= n_tokens) return;
  const int64_t id = ids[t];
  const bool ok = id >= 0 && id < V;
  for (int64_t c = lane; c < Hd; c += 64) out[t * Hd + c] = ok ? w[id * stride_w + c] : from_f32<T>(0.f);
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
// dst = round(src * scale[0]) in T (fp32 src, scale read on the device).
template <typename T>
__global__ __launch_bounds__(256) void scale_cast_kernel(const float* __restrict__ src, T* __restrict__ dst,
                                                         int64_t n, const float* __restrict__ scale) {
  const float s = scale[0];
  const int64_t n4 = n / 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4; i += stride) {
    const float4 v = reinterpret_cast<const float4*>(src)[i];
    dst[4 * i] = from_f32<T>(v.x * s);
    dst[4 * i + 1] = from_f32<T>(v.y * s);
    dst[4 * i + 2] = from_f32<T>(v.z * s);
    dst[4 * i + 3] = from_f32<T>(v.w * s);
  }
  for (int64_t i = 4 * n4 + blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += stride)
    dst[i] = from_f32<T>(src[i] * s);
}

extern "C" int qh_scale_cast(const float* src, void* dst, int64_t n, const float* scale, int dtype, void* stream) {
  QH_CHECK_ARG(n >= 0 && src != nullptr && dst != nullptr && scale != nullptr, "qh_scale_cast: bad arguments");
  QH_CHECK_ARG(aligned16(src), "qh_scale_cast: src must be 16-byte aligned");
  if (n == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const int64_t grid = std::min<int64_t>(ceil_div(n / 4 + 1, 256), 4096);
  QH_DISPATCH_DTYPE(dtype, T, "qh_scale_cast",
                    scale_cast_kernel<T><<<(unsigned)grid, 256, 0, st>>>(src, (T*)dst, n, scale));
  QH_CHECK_LAUNCH("qh_scale_cast");
  return QH_OK;
}

extern "C" int qh_add(const void* x, const void* r, void* out, int64_t n, int dtype, void* stream) {
  QH_CHECK_ARG(n >= 0, "qh_add: negative n");
  if (n == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  QH_DISPATCH_DTYPE(dtype, T, "qh_add", launch_binary<EwOp::Add, T>(x, r, out, n, st));
  QH_CHECK_LAUNCH("qh_add");
  return QH_OK;
}

extern "C" int qh_silu_mul_fwd(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream) {
  QH_CHECK_ARG(n >= 0, "qh_silu_mul_fwd: negative n");
  if (n == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  QH_DISPATCH_DTYPE(dtype, T, "qh_silu_mul_fwd", launch_binary<EwOp::SiluMul, T>(gate, up, out, n, st));
  QH_CHECK_LAUNCH("qh_silu_mul_fwd");
  return QH_OK;
}

extern "C" int qh_silu_mul_bwd(const void* gate, const void* up, const void* gout, void* dgate, void* dup,
                               int64_t n, int dtype, void* stream) {
  QH_CHECK_ARG(n >= 0, "qh_silu_mul_bwd: negative n");
  if (n == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  QH_DISPATCH_DTYPE(dtype, T, "qh_silu_mul_bwd",
                    launch_grad<EwOp::SiluMul, T>(gate, up, gout, dgate, dup, n, st));
  QH_CHECK_LAUNCH("qh_silu_mul_bwd");
  return QH_OK;
}

extern "C" int qh_sigmoid_mul_fwd(const void* x, const void* gate, void* out, int64_t n, int dtype,
                                  void* stream) {
  QH_CHECK_ARG(n >= 0, "qh_sigmoid_mul_fwd: negative n");
  if (n == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  QH_DISPATCH_DTYPE(dtype, T, "qh_sigmoid_mul_fwd", launch_binary<EwOp::SigmoidMul, T>(x, gate, out, n, st));
  QH_CHECK_LAUNCH("qh_sigmoid_mul_fwd");
  return QH_OK;
}

extern "C" int qh_sigmoid_mul_bwd(const void* x, const void* gate, const void* gout, void* dx, void* dgate,
                                  int64_t n, int dtype, void* stream) {
  QH_CHECK_ARG(n >= 0, "qh_sigmoid_mul_bwd: negative n");
  if (n == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  QH_DISPATCH_DTYPE(dtype, T, "qh_sigmoid_mul_bwd",
                    launch_grad<EwOp::SigmoidMul, T>(x, gate, gout, dx, dgate, n, st));
  QH_CHECK_LAUNCH("qh_sigmoid_mul_bwd");
  return QH_OK;
}

template <typename T, typename C>
static int launch_rope(const void* x, int64_t sxb, int64_t sxh, int64_t sxs, int64_t sxd, const void* cs,
                       const void* sn, int64_t scb, int64_t scs, int64_t scd, int64_t cos_batch, void* out,
                       int64_t B, int64_t H, int64_t S, int64_t D, int64_t rot, float sgn, hipStream_t st) {
  const int64_t half = rot / 2;
  const int64_t rows = B * H * S;
  constexpr int VN = Vec16<T>::N;
  const bool vec = std::is_same<T, C>::value && rot == D && sxd == 1 && scd == 1 && half % VN == 0 &&
                   aligned16(x) && aligned16(cs) && aligned16(sn) && aligned16(out) && sxb % VN == 0 &&
                   sxh % VN == 0 && sxs % VN == 0 && scb % VN == 0 && scs % VN == 0;
  if (vec) {
    const int64_t total = rows * (half / VN);
    if (2 * rows * D * (int64_t)sizeof(T) >= kStreamBytes)
      rope_vec_kernel<T, true><<<grid_for(total), 256, 0, st>>>((const T*)x, sxb, sxh, sxs, (const T*)cs,
                                                                (const T*)sn, scb, scs, cos_batch, (T*)out, H, S, D,
                                                                half, total, sgn);
    else
      rope_vec_kernel<T, false><<<grid_for(total), 256, 0, st>>>((const T*)x, sxb, sxh, sxs, (const T*)cs,
                                                                 (const T*)sn, scb, scs, cos_batch, (T*)out, H, S, D,
                                                                 half, total, sgn);
  } else {
    const int64_t items = half + (D - rot);
    const int64_t total = rows * items;
    rope_kernel<T, C><<<grid_for(total), 256, 0, st>>>((const T*)x, sxb, sxh, sxs, sxd, (const C*)cs,
                                                       (const C*)sn, scb, scs, scd, cos_batch, (T*)out, H, S, D,
                                                       half, rot, items, total, sgn);
  }
  return QH_OK;
}

extern "C" int qh_rope(const void* x, int64_t sxb, int64_t sxh, int64_t sxs, int64_t sxd, const void* cos,
                       const void* sin, int64_t scb, int64_t scs, int64_t scd, int64_t cos_batch, void* out,
                       int64_t B, int64_t H, int64_t S, int64_t D, int64_t rot, int neg_sin, int dtype,
                       int cdtype, void* stream) {
  QH_CHECK_ARG(B >= 0 && H >= 0 && S >= 0 && D >= 0, "qh_rope: negative shape");
  QH_CHECK_ARG(rot >= 0 && rot <= D && rot % 2 == 0, "qh_rope: rotary dim %lld must be even and <= %lld",
               (long long)rot, (long long)D);
  QH_CHECK_ARG(cos_batch == 1 || cos_batch == B, "qh_rope: cos/sin batch %lld must be 1 or %lld",
               (long long)cos_batch, (long long)B);
  if (B * H * S * D == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const float sgn = neg_sin ? -1.0f : 1.0f;
#define QH_ROPE_C(T)                                                                                      \
  switch (cdtype) {                                                                                       \
    case QH_F32: launch_rope<T, float>(x, sxb, sxh, sxs, sxd, cos, sin, scb, scs, scd, cos_batch, out, B, H, S, D, rot, sgn, st); break; \
    case QH_F16: launch_rope<T, f16_t>(x, sxb, sxh, sxs, sxd, cos, sin, scb, scs, scd, cos_batch, out, B, H, S, D, rot, sgn, st); break; \
    case QH_BF16: launch_rope<T, bf16_t>(x, sxb, sxh, sxs, sxd, cos, sin, scb, scs, scd, cos_batch, out, B, H, S, D, rot, sgn, st); break; \
    default: qh::set_error("qh_rope: unsupported cos dtype %d", cdtype); return QH_E_DTYPE;                \
  }
  QH_DISPATCH_DTYPE(dtype, T, "qh_rope", QH_ROPE_C(T));
#undef QH_ROPE_C
  QH_CHECK_LAUNCH("qh_rope");
  return QH_OK;
}

extern "C" int qh_kv_write(void* cache, int64_t scb, int64_t sch, int64_t scs, int64_t scd, const void* values,
                           int64_t svb, int64_t svh, int64_t svs, int64_t svd, const int64_t* positions,
                           int64_t B, int64_t H, int64_t S, int64_t D, int64_t cap, int dtype, void* stream) {
  QH_CHECK_ARG(B >= 0 && H >= 0 && S >= 0 && D >= 0 && cap >= 0, "qh_kv_write: negative shape");
  if (B * H * S * D == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  QH_DISPATCH_DTYPE(dtype, T, "qh_kv_write", {
    constexpr int VN = Vec16<T>::N;
    const bool vec = scd == 1 && svd == 1 && D % VN == 0 && aligned16(cache) && aligned16(values) &&
                     scb % VN == 0 && sch % VN == 0 && scs % VN == 0 && svb % VN == 0 && svh % VN == 0 &&
                     svs % VN == 0;
    if (vec && S * (D / VN) >= kKvPlaneMin && S * (D / VN) < (1ll << 30) && B * H < 65536) {
      const int vpr = (int)(D / VN);
      const dim3 grid((unsigned)ceil_div(S * vpr, 256 * kKvPlaneU), (unsigned)(B * H));
      kv_write_plane<T><<<grid, 256, 0, st>>>((T*)cache, scb, sch, scs, (const T*)values, svb, svh, svs, positions,
                                              (int)H, (int)S, vpr, cap);
    } else if (vec) {
      const int64_t total = B * H * S * (D / VN);
      kv_write_vec<T><<<grid_for(total), 256, 0, st>>>((T*)cache, scb, sch, scs, (const T*)values, svb, svh, svs,
                                                       positions, H, S, D / VN, cap, total);
    } else {
      const int64_t total = B * H * S * D;
      kv_write_scalar<T><<<grid_for(total), 256, 0, st>>>((T*)cache, scb, sch, scs, scd, (const T*)values, svb,
                                                          svh, svs, svd, positions, H, S, D, cap, total);
    }
  });
  QH_CHECK_LAUNCH("qh_kv_write");
  return QH_OK;
}

extern "C" int qh_kv_append(const void* prefix, const void* suffix, void* out, int64_t B, int64_t H,
                            int64_t s_old, int64_t s_new, int64_t D, int dtype, void* stream) {
  QH_CHECK_ARG(B >= 0 && H >= 0 && s_old >= 0 && s_new >= 0 && D >= 0, "qh_kv_append: negative shape");
  const int64_t total = B * H * (s_old + s_new) * D;
  if (total == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  QH_DISPATCH_DTYPE(dtype, T, "qh_kv_append", {
    constexpr int VN = Vec16<T>::N;
    if (D % VN == 0 && aligned16(prefix) && aligned16(suffix) && aligned16(out)) {
      const int64_t tv = total / VN;
      kv_append_vec<T><<<grid_for(tv), 256, 0, st>>>((const T*)prefix, (const T*)suffix, (T*)out, s_old, s_new,
                                                     D / VN, tv);
    } else {
      kv_append_kernel<T><<<grid_for(total), 256, 0, st>>>((const T*)prefix, (const T*)suffix, (T*)out, s_old,
                                                           s_new, D, total);
    }
  });
  QH_CHECK_LAUNCH("qh_kv_append");
  return QH_OK;
}

extern "C" int qh_embedding_fwd(const int64_t* ids, const void* w, int64_t stride_w, void* out, int64_t n_tokens,
                                int64_t V, int64_t Hd, int dtype, void* stream) {
  QH_CHECK_ARG(n_tokens >= 0 && V >= 0 && Hd >= 0, "qh_embedding_fwd: negative shape");
  if (n_tokens == 0 || Hd == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const int grid = (int)ceil_div(n_tokens, 4);
  QH_DISPATCH_DTYPE(dtype, T, "qh_embedding_fwd", {
    constexpr int VN = Vec16<T>::N;
    if (Hd % VN == 0 && stride_w % VN == 0 && aligned16(w) && aligned16(out))
      embedding_vec<T><<<grid, 256, 0, st>>>(ids, (const T*)w, stride_w, (T*)out, n_tokens, V, Hd);
    else
      embedding_scalar<T><<<grid, 256, 0, st>>>(ids, (const T*)w, stride_w, (T*)out, n_tokens, V, Hd);
  });
  QH_CHECK_LAUNCH("qh_embedding_fwd");
  return QH_OK;
}
