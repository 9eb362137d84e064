// Deterministic scatter-add operators: embedding backward and index_add.
//
// Instead of float atomics (whose summation order depends on timing), the
// (row-index, source-position) pairs are sorted with a stable LSD radix sort
// (rocPRIM) and each destination row is produced by exactly one workgroup that
// sums its sources in source order in fp32 and rounds once.
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

template <bool ACC>
static int launch_segments(const uint32_t* keys, const uint32_t* vals, int64_t n, const void* src, int sdt,
                           int64_t stride_s, void* dst, int ddt, int64_t stride_d, int64_t D, uint32_t n_target,
                           int64_t skip_key, hipStream_t st) {
#define QH_SEG(S, O)                                                                                        \
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

extern "C" int64_t qh_embedding_bwd_workspace(int64_t n_tokens) { return scatter_ws_bytes(n_tokens); }

extern "C" int64_t qh_index_add_workspace(int64_t n_src) { return scatter_ws_bytes(n_src); }

extern "C" int qh_embedding_bwd(const int64_t* ids, const void* gout, void* gw, void* ws, int64_t ws_bytes,
                                int64_t n_tokens, int64_t V, int64_t Hd, int64_t padding_idx, int gdtype, int wdtype,
                                void* stream) {
  QH_CHECK_ARG(n_tokens >= 0 && V >= 0 && Hd >= 0, "qh_embedding_bwd: negative shape");
  QH_CHECK_ARG(V < (1ll << 31) - 1 && n_tokens < (1ll << 31), "qh_embedding_bwd: sizes exceed 2^31");
  hipStream_t st = (hipStream_t)stream;
  const int wsz = wdtype == QH_F32 ? 4 : 2;
  int rc = qh_zero(gw, V * Hd * wsz, stream);
  if (rc) return rc;
  if (n_tokens == 0 || Hd == 0) return QH_OK;
  uint32_t *keys = nullptr, *vals = nullptr;
  rc = sort_indices(ids, n_tokens, V, ws, ws_bytes, &keys, &vals, st, "qh_embedding_bwd");
  if (rc) return rc;
  rc = launch_segments<false>(keys, vals, n_tokens, gout, gdtype, Hd, gw, wdtype, Hd, Hd, (uint32_t)V, padding_idx, st);
  if (rc) return rc;
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
