// Deterministic scatter-add operators: embedding backward and index_add.
//
// Instead of float atomics (whose summation order depends on timing), the
// (row-index, source-position) pairs are sorted with a stable LSD radix sort
// (rocPRIM) and each destination row is produced by exactly one workgroup that
// sums its sources in source order in fp32 and rounds once.
#include <algorithm>
#include <cstring>
#include <rocprim/rocprim.hpp>

#include "qh_common.h"

namespace {

static int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

static size_t sort_temp_bytes(int64_t n) {
  size_t sz = 0;
  rocprim::radix_sort_pairs((void*)nullptr, sz, (const uint32_t*)nullptr, (uint32_t*)nullptr,
                            (const uint32_t*)nullptr, (uint32_t*)nullptr, (unsigned)n, 0, 32, (hipStream_t)0);
  return sz;
}

static int64_t scatter_ws_bytes(int64_t n) {
  if (n <= 0) return 0;
  return 4 * align256(n * 4) + align256((int64_t)sort_temp_bytes(n));
}

__global__ __launch_bounds__(256) void make_keys(const int64_t* __restrict__ idx, int64_t n, int64_t n_target,
                                                 uint32_t* __restrict__ keys, uint32_t* __restrict__ vals) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t v = idx[i];
    keys[i] = (v >= 0 && v < n_target) ? (uint32_t)v : (uint32_t)n_target;
    vals[i] = (uint32_t)i;
  }
}

// One workgroup per sorted position; only the first position of each key's
// run does work. ACC adds onto the existing destination row.
template <typename S, typename O, bool ACC>
__global__ __launch_bounds__(256) void segment_rows(const uint32_t* __restrict__ keys, const uint32_t* __restrict__ vals,
                                                    int64_t n, const S* __restrict__ src, int64_t stride_s,
                                                    O* __restrict__ dst, int64_t stride_d, int64_t D,
                                                    uint32_t n_target, int64_t skip_key) {
  const int64_t i = blockIdx.x;
  const uint32_t k = keys[i];
  if (k >= n_target) return;
  if (i > 0 && keys[i - 1] == k) return;
  if ((int64_t)k == skip_key) return;
  int64_t end = i + 1;
  while (end < n && keys[end] == k) ++end;
  O* drow = dst + (int64_t)k * stride_d;
  for (int64_t c = threadIdx.x; c < D; c += 256) {
    float acc = ACC ? to_f32(drow[c]) : 0.f;
    for (int64_t j = i; j < end; ++j) acc += to_f32(src[(int64_t)vals[j] * stride_s + c]);
    drow[c] = from_f32<O>(acc);
  }
}

// 8 consecutive elements of T as fp32 (16- or 32-byte aligned vector access).
template <typename T>
__device__ __forceinline__ void ld8f(const T* p, float (&o)[8]) {
  if constexpr (sizeof(T) == 4) {
    const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    o[0] = a.x, o[1] = a.y, o[2] = a.z, o[3] = a.w, o[4] = b.x, o[5] = b.y, o[6] = b.z, o[7] = b.w;
  } else {
    const Vec16<T> v = ld16(p);
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = to_f32(v.v[j]);
  }
}

template <typename T>
__device__ __forceinline__ void st8f(T* p, const float (&o)[8]) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(o[4], o[5], o[6], o[7]);
  } else {
    Vec16<T> v;
#pragma unroll
    for (int j = 0; j < 8; ++j) v.v[j] = from_f32<T>(o[j]);
    st16(p, v);
  }
}

// Sum of the source rows vals[s..e) (in that order, fp32, starting from
// `init`) for the 8-column chunk at element offset c.
template <typename S>
__device__ __forceinline__ void run_sum8(const uint32_t* __restrict__ vals, int64_t s, int64_t e,
                                         const S* __restrict__ src, int64_t stride_s, int64_t c, float (&acc)[8]) {
  for (int64_t j = s; j < e; ++j) {
    float t[8];
    ld8f(src + (int64_t)vals[j] * stride_s + c, t);
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] += t[q];
  }
}

// segment_rows with 8-column vector chunks: one wave per sorted position
// (D, both strides multiple of 8, 16-byte aligned rows). Same summation order.
template <typename S, typename O, bool ACC>
__global__ __launch_bounds__(64) void segment_rows_vec(const uint32_t* __restrict__ keys,
                                                       const uint32_t* __restrict__ vals, int64_t n,
                                                       const S* __restrict__ src, int64_t stride_s,
                                                       O* __restrict__ dst, int64_t stride_d, int64_t D,
                                                       uint32_t n_target, int64_t skip_key) {
  const int64_t i = blockIdx.x;
  const uint32_t k = keys[i];
  if (k >= n_target) return;
  if (i > 0 && keys[i - 1] == k) return;
  if ((int64_t)k == skip_key) return;
  int64_t end = i + 1;
  while (end < n && keys[end] == k) ++end;
  O* drow = dst + (int64_t)k * stride_d;
  for (int64_t c = threadIdx.x * 8; c < D; c += 64 * 8) {
    float acc[8];
    if (ACC) ld8f(drow + c, acc);
    else
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] = 0.f;
    run_sum8(vals, i, end, src, stride_s, c, acc);
    st8f(drow + c, acc);
  }
}

// Embedding weight gradient, every row written exactly once after the sort, by waves of two
// roles in one launch (no wave both loads gradient rows and streams stores: stores count in the
// same vmcnt as loads, so a load wait would also wait for the store stream).
// - Zero waves (the first zgrid workgroups): a wave owns rpw <= 128 consecutive rows, finds the
//   first sorted position with a key at or above its first row by a 64-way search (one load per
//   lane per step, about log64(n) steps), marks the rows some token hits (64 keys per load),
//   then writes zeros to the others (the padding row included).
// - Run waves (the rest, one per sorted position): the first position of each key's run sums
//   the run's gradient rows in position order (fp32, rounded once) into the row, except for the
//   padding row and ids outside [0, V).
constexpr int64_t kEmbRowsPerWave = 128;

template <typename S, typename O>
__global__ __launch_bounds__(256) void embedding_rows_roles(const uint32_t* __restrict__ keys,
                                                            const uint32_t* __restrict__ vals, int n,
                                                            const S* __restrict__ src, O* __restrict__ dst, int64_t V,
                                                            int64_t D, int64_t skip_key, int64_t rpw, int zgrid) {
  __shared__ uint32_t hitw[4][4];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if ((int)blockIdx.x >= zgrid) {  // run waves
    const int i = (blockIdx.x - zgrid) * 4 + wid;
    if (i >= n) return;
    const uint32_t k = keys[i];
    if ((int64_t)k >= V || (int64_t)k == skip_key || (i > 0 && keys[i - 1] == k)) return;
    int e = i + 1;
    while (e < n && keys[e] == k) ++e;
    O* drow = dst + (int64_t)k * D;
    for (int64_t c = lane * 8; c < D; c += 64 * 8) {
      float acc[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] = 0.f;
      run_sum8(vals, i, e, src, D, c, acc);
      st8f(drow + c, acc);
    }
    return;
  }
  const int64_t wave = (int64_t)blockIdx.x * 4 + wid;
  const int64_t a = wave * rpw, b = a + rpw < V ? a + rpw : V;
  if (lane < 4) hitw[wid][lane] = 0u;
  __syncthreads();  // every wave of a zero-role workgroup reaches both barriers (empty ranges too)
  // first position p in [0, n) with keys[p] >= a (n if none); wave-uniform throughout
  int lo = 0, len = a < b ? n : 0;
  while (len > 0) {
    const int step = (len + 63) / 64;
    const int idx = lo + lane * step;
    const bool less = idx < lo + len && (int64_t)keys[idx] < a;
    const int c = __popcll(__ballot(less));
    if (c == 0) break;
    const int nlo = lo + (c - 1) * step + 1;
    const int hi = lo + c * step < lo + len ? lo + c * step : lo + len;
    lo = nlo;
    len = hi - nlo;
  }
  // mark the hit rows of [a, b): 64 sorted keys per load
  for (int p = lo; a < b && p < n; p += 64) {
    const int64_t k = p + lane < n ? (int64_t)keys[p + lane] : V;
    if (k < b && k != skip_key) atomicOr(&hitw[wid][(k - a) >> 5], 1u << ((k - a) & 31));
    if (__any(k >= b)) break;  // keys are sorted: the range ends within these 64 keys
  }
  __syncthreads();
  float z[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) z[q] = 0.f;
  for (int64_t r = a; r < b; ++r) {
    if (hitw[wid][(r - a) >> 5] >> ((r - a) & 31) & 1) continue;
    O* drow = dst + r * D;
    for (int64_t c = lane * 8; c < D; c += 64 * 8) st8f(drow + c, z);
  }
}

template <bool ACC>
static int launch_segments(const uint32_t* keys, const uint32_t* vals, int64_t n, const void* src, int sdt,
                           int64_t stride_s, void* dst, int ddt, int64_t stride_d, int64_t D, uint32_t n_target,
                           int64_t skip_key, hipStream_t st) {
  const bool vec = D % 8 == 0 && stride_s % 8 == 0 && stride_d % 8 == 0 && aligned16(src) && aligned16(dst);
#define QH_SEG(S, O)                                                                                          \
  if (vec)                                                                                                    \
    segment_rows_vec<S, O, ACC><<<(unsigned)n, 64, 0, st>>>(keys, vals, n, (const S*)src, stride_s, (O*)dst, \
                                                            stride_d, D, n_target, skip_key);                 \
  else                                                                                                        \
    segment_rows<S, O, ACC><<<(unsigned)n, 256, 0, st>>>(keys, vals, n, (const S*)src, stride_s, (O*)dst,    \
                                                         stride_d, D, n_target, skip_key)
#define QH_SEG_O(S)                                        \
  switch (ddt) {                                           \
    case QH_F32: QH_SEG(S, float); break;                  \
    case QH_F16: QH_SEG(S, f16_t); break;                  \
    case QH_BF16: QH_SEG(S, bf16_t); break;                \
    default: qh::set_error("scatter: bad out dtype"); return QH_E_DTYPE; \
  }
  switch (sdt) {
    case QH_F32: QH_SEG_O(float); break;
    case QH_F16: QH_SEG_O(f16_t); break;
    case QH_BF16: QH_SEG_O(bf16_t); break;
    default: qh::set_error("scatter: bad src dtype"); return QH_E_DTYPE;
  }
#undef QH_SEG_O
#undef QH_SEG
  return QH_OK;
}

// Sort (idx -> key, position) pairs; returns pointers to the sorted arrays.
static int sort_indices(const int64_t* idx, int64_t n, int64_t n_target, void* ws, int64_t ws_bytes,
                        uint32_t** keys_sorted, uint32_t** vals_sorted, hipStream_t st, const char* name) {
  const int64_t need = scatter_ws_bytes(n);
  if (ws_bytes < need) {
    qh::set_error("%s: workspace %lld bytes < required %lld", name, (long long)ws_bytes, (long long)need);
    return QH_E_WORKSPACE;
  }
  char* base = (char*)ws;
  const int64_t a = align256(n * 4);
  uint32_t* k_in = (uint32_t*)(base);
  uint32_t* k_out = (uint32_t*)(base + a);
  uint32_t* v_in = (uint32_t*)(base + 2 * a);
  uint32_t* v_out = (uint32_t*)(base + 3 * a);
  void* temp = base + 4 * a;
  size_t temp_bytes = (size_t)(ws_bytes - 4 * a);
  int64_t g = ceil_div(n, 256);
  if (g > 4096) g = 4096;
  make_keys<<<(int)g, 256, 0, st>>>(idx, n, n_target, k_in, v_in);
  unsigned bits = 1;
  while (bits < 32 && (uint64_t(1) << bits) <= (uint64_t)n_target) ++bits;
  hipError_t e = rocprim::radix_sort_pairs(temp, temp_bytes, k_in, k_out, v_in, v_out, (unsigned)n, 0, bits, st);
  if (e != hipSuccess) {
    qh::set_error("%s: radix sort failed: %s", name, hipGetErrorString(e));
    return QH_E_HIP;
  }
  *keys_sorted = k_out;
  *vals_sorted = v_out;
  return QH_OK;
}

}  // namespace

// Sort space for the token ids (V is part of the signature; the rows need no table).
extern "C" int64_t qh_embedding_bwd_workspace(int64_t n_tokens, int64_t V) {
  if (n_tokens <= 0 || V <= 0) return 0;
  return scatter_ws_bytes(n_tokens);
}

extern "C" int64_t qh_index_add_workspace(int64_t n_src) { return scatter_ws_bytes(n_src); }

extern "C" int qh_embedding_bwd(const int64_t* ids, const void* gout, void* gw, void* ws, int64_t ws_bytes,
                                int64_t n_tokens, int64_t V, int64_t Hd, int64_t padding_idx, int gdtype, int wdtype,
                                void* stream) {
  QH_CHECK_ARG(n_tokens >= 0 && V >= 0 && Hd >= 0, "qh_embedding_bwd: negative shape");
  QH_CHECK_ARG(V < (1ll << 31) - 1 && n_tokens < (1ll << 31), "qh_embedding_bwd: sizes exceed 2^31");
  hipStream_t st = (hipStream_t)stream;
  const int wsz = wdtype == QH_F32 ? 4 : 2;
  if (n_tokens == 0 || Hd == 0 || V == 0) return qh_zero(gw, V * Hd * wsz, stream);
  const int64_t need = qh_embedding_bwd_workspace(n_tokens, V);
  if (ws_bytes < need) {
    qh::set_error("qh_embedding_bwd: workspace %lld bytes < required %lld", (long long)ws_bytes, (long long)need);
    return QH_E_WORKSPACE;
  }
  const int64_t sort_bytes = scatter_ws_bytes(n_tokens);
  const bool vec = Hd % 8 == 0 && aligned16(gout) && aligned16(gw);
  if (!vec) {
    uint32_t *keys = nullptr, *vals = nullptr;
    int rc = sort_indices(ids, n_tokens, V, ws, sort_bytes, &keys, &vals, st, "qh_embedding_bwd");
    if (rc) return rc;
    rc = qh_zero(gw, V * Hd * wsz, stream);
    if (rc) return rc;
    rc = launch_segments<false>(keys, vals, n_tokens, gout, gdtype, Hd, gw, wdtype, Hd, Hd, (uint32_t)V, padding_idx,
                                st);
    if (rc) return rc;
    QH_CHECK_LAUNCH("qh_embedding_bwd");
    return QH_OK;
  }
  uint32_t *keys = nullptr, *vals = nullptr;
  int rc = sort_indices(ids, n_tokens, V, ws, sort_bytes, &keys, &vals, st, "qh_embedding_bwd");
  if (rc) return rc;
  // zero waves: about 8 per CU (more for tables above 2048 x 128 rows), each over a contiguous
  // range of rows; then one run wave per sorted position
  const int64_t waves = std::max<int64_t>(std::min<int64_t>(ceil_div(V, 16), 2048), ceil_div(V, kEmbRowsPerWave));
  const int64_t rpw = ceil_div(V, waves);
  const int64_t zgrid = ceil_div(ceil_div(V, rpw), 4);
  const int64_t grid = zgrid + ceil_div(n_tokens, 4);
  QH_CHECK_ARG(grid < (1ll << 31), "qh_embedding_bwd: grid too large");
#define QH_EROWS(S, O)                                                                                   \
  embedding_rows_roles<S, O><<<(unsigned)grid, 256, 0, st>>>(keys, vals, (int)n_tokens, (const S*)gout, (O*)gw, V, \
                                                             Hd, padding_idx, rpw, (int)zgrid)
#define QH_EROWS_O(S)                                      \
  switch (wdtype) {                                        \
    case QH_F32: QH_EROWS(S, float); break;                \
    case QH_F16: QH_EROWS(S, f16_t); break;                \
    case QH_BF16: QH_EROWS(S, bf16_t); break;              \
    default: qh::set_error("qh_embedding_bwd: bad weight dtype"); return QH_E_DTYPE; \
  }
  switch (gdtype) {
    case QH_F32: QH_EROWS_O(float); break;
    case QH_F16: QH_EROWS_O(f16_t); break;
    case QH_BF16: QH_EROWS_O(bf16_t); break;
    default: qh::set_error("qh_embedding_bwd: bad grad dtype"); return QH_E_DTYPE;
  }
#undef QH_EROWS_O
#undef QH_EROWS
  QH_CHECK_LAUNCH("qh_embedding_bwd");
  return QH_OK;
}

extern "C" int qh_index_add(void* target, int64_t stride_t, const void* src, int64_t stride_s, const int64_t* index,
                            int64_t n_src, int64_t n_target, int64_t D, void* ws, int64_t ws_bytes, int dtype,
                            void* stream) {
  QH_CHECK_ARG(n_src >= 0 && n_target >= 0 && D >= 0, "qh_index_add: negative shape");
  QH_CHECK_ARG(n_target < (1ll << 31) - 1 && n_src < (1ll << 31), "qh_index_add: sizes exceed 2^31");
  if (n_src == 0 || D == 0 || n_target == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  uint32_t *keys = nullptr, *vals = nullptr;
  int rc = sort_indices(index, n_src, n_target, ws, ws_bytes, &keys, &vals, st, "qh_index_add");
  if (rc) return rc;
  rc = launch_segments<true>(keys, vals, n_src, src, dtype, stride_s, target, dtype, stride_t, D, (uint32_t)n_target,
                             -1, st);
  if (rc) return rc;
  QH_CHECK_LAUNCH("qh_index_add");
  return QH_OK;
}
