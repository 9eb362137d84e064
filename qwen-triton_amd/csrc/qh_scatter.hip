// Deterministic scatter-add operators: embedding backward and index_add.
//
// Instead of float atomics (whose summation order depends on timing), every
// destination row is produced by exactly one wave (or, for the slices of a hot
// embedding row, one wave per column slice) that sums its sources in source order
// in fp32 and rounds once. The embedding backward of up to 32768 tokens finds each
// workgroup's sources in LDS without a sort (embedding_bwd_interleaved); larger
// token counts and index_add sort the (row-index, source-position) pairs with a
// stable LSD radix sort (rocPRIM) first.
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

// U source rows from position j (all loads issued before the first add), added in order;
// 16-bit rows stay packed until their add, so a batch costs 4 registers per row.
template <int U, typename S>
__device__ __forceinline__ void run_batch8(const uint32_t* __restrict__ vals, int64_t j, const S* __restrict__ src,
                                           int64_t stride_s, int64_t c, float (&acc)[8]) {
  if constexpr (sizeof(S) == 4) {
    float t[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) ld8f(src + (int64_t)vals[j + u] * stride_s + c, t[u]);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] += t[u][q];
  } else {
    Vec16<S> t[U];
#pragma unroll
    for (int u = 0; u < U; ++u) t[u] = ld16(src + (int64_t)vals[j + u] * stride_s + c);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] += to_f32(t[u].v[q]);
  }
}

// Sum of the source rows vals[s..e) (in that order, fp32, onto acc) for the
// 8-column chunk at element offset c: batches of B rows of loads while B
// remain (at most 4 for fp32 rows), then single rows (a run of one row costs
// one load).
template <int BMAX = 8, typename S>
__device__ __forceinline__ void run_sum8(const uint32_t* __restrict__ vals, int64_t s, int64_t e,
                                         const S* __restrict__ src, int64_t stride_s, int64_t c, float (&acc)[8]) {
  constexpr int B = sizeof(S) == 4 && BMAX > 4 ? 4 : BMAX;
  int64_t j = s;
  for (; j + B <= e; j += B) run_batch8<B>(vals, j, src, stride_s, c, acc);
  for (; j < e; ++j) run_batch8<1>(vals, j, src, stride_s, c, acc);
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
      run_sum8<4>(vals, i, e, src, D, c, acc);
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

// Row pieces of VN elements for the single-launch embedding backward (16-byte aligned pieces of
// 8, naturally aligned pieces of 2).
template <typename T, int VN>
struct EmbPiece {
  static constexpr int B = VN * (int)sizeof(T);
  union {
    T v[VN];
    uint32_t w[B >= 4 ? B / 4 : 1];
  };
};

template <typename T, int VN>
__device__ __forceinline__ EmbPiece<T, VN> emb_load(const T* p) {
  EmbPiece<T, VN> r;
  constexpr int B = EmbPiece<T, VN>::B;
  if constexpr (B % 16 == 0) {
#pragma unroll
    for (int i = 0; i < B / 16; ++i) {
      const uint4 x = reinterpret_cast<const uint4*>(p)[i];
      r.w[4 * i] = x.x, r.w[4 * i + 1] = x.y, r.w[4 * i + 2] = x.z, r.w[4 * i + 3] = x.w;
    }
  } else if constexpr (B == 8) {
    const uint2 x = *reinterpret_cast<const uint2*>(p);
    r.w[0] = x.x, r.w[1] = x.y;
  } else if constexpr (B == 4) {
    r.w[0] = *reinterpret_cast<const uint32_t*>(p);
  } else {
    r.v[0] = *p;
  }
  return r;
}

typedef unsigned int qh_u32x2 __attribute__((ext_vector_type(2)));

template <typename T, int VN>
__device__ __forceinline__ void emb_store_nt(T* p, const float (&o)[VN]) {
  EmbPiece<T, VN> u;
#pragma unroll
  for (int k = 0; k < VN; ++k) u.v[k] = from_f32<T>(o[k]);
  constexpr int B = EmbPiece<T, VN>::B;
  if constexpr (B % 16 == 0) {
#pragma unroll
    for (int i = 0; i < B / 16; ++i) {
      const qh_u32x4 x = {u.w[4 * i], u.w[4 * i + 1], u.w[4 * i + 2], u.w[4 * i + 3]};
      __builtin_nontemporal_store(x, reinterpret_cast<qh_u32x4*>(p) + i);
    }
  } else if constexpr (B == 8) {
    const qh_u32x2 x = {u.w[0], u.w[1]};
    __builtin_nontemporal_store(x, reinterpret_cast<qh_u32x2*>(p));
  } else if constexpr (B == 4) {
    __builtin_nontemporal_store(u.w[0], reinterpret_cast<uint32_t*>(p));
  } else {
    uint16_t h;
    __builtin_memcpy(&h, &u.v[0], 2);
    __builtin_nontemporal_store(h, reinterpret_cast<uint16_t*>(p));
  }
}

// Embedding weight gradient in one launch, without a sort, for up to kEmbLdsTokens tokens.
// Workgroup g of G (a power of two) owns the rows v with v mod G = g, as local rows v / G. The
// interleave spreads the low ids, which BPE vocabularies give their most frequent tokens, over
// all workgroups.
// 1. Its threads read every token id once (coalesced) and stage, per position, an LDS entry
//    local_row << 16 | position for the tokens that hit its rows (none for ids outside [0, V)
//    and for the padding row), and count the hits per row.
// 2. A stable compaction turns the staged entries into the position-ordered list of hits: each
//    thread counts the hits of a contiguous block of positions, a block-wide exclusive scan
//    gives its offset. Wave 0 meanwhile lists the hit rows in two classes by hit count.
// 3. Every row of the workgroup is written once. The first kEmbZeroWaves waves write zeros to
//    the rows no token hits (16-byte non-temporal stores). The other waves take work items from
//    an LDS queue: first the kEmbHotCols-column slices of the rows with at least kEmbHot hits,
//    then the other hit rows whole. An item walks the list (64 entries per LDS read) and adds
//    the matching tokens' gradient rows in position order (fp32, rounded once), the loads of up
//    to U tokens in flight; a hot row's tokens so run as kEmbHotCols-column chains on several
//    waves at once. The zero waves join the queue when their rows are done.
// The sums and the rounding are those of the sorted form: the result is the same bit for bit.
constexpr int kEmbThreads = 1024, kEmbWaves = kEmbThreads / 64, kEmbZeroWaves = 12;
constexpr int kEmbIdsPerThread = 32;
constexpr int64_t kEmbLdsTokens = (int64_t)kEmbThreads * kEmbIdsPerThread;  // positions fit 16 bits
constexpr int kEmbMaxRows = 2048;  // local rows per workgroup
constexpr int kEmbHot = 32, kEmbHotVN = 2, kEmbHotU = 32;  // hot-row slices: 64 lanes x 2 columns
constexpr int kEmbHotCols = 64 * kEmbHotVN;

// acc[k][.] += the rows of the list's tokens on local row r, in list order, at the VN columns
// c + 64 VN k of this lane (columns at or past D are skipped); U tokens per batch of loads.
template <int VN, int NCH, int U, typename S>
__device__ __forceinline__ void emb_sum(const uint32_t* list, int L, uint32_t r, const S* __restrict__ src, int D,
                                        int c, float (&acc)[NCH][VN]) {
  const int lane = threadIdx.x & 63;
  for (int p = 0; p < L; p += 64) {
    const uint32_t e = p + lane < L ? list[p + lane] : 0xffffffffu;
    uint64_t mk = __ballot(e >> 16 == r);
    while (mk) {
      int pos[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        pos[u] = -1;
        if (mk) {
          const int j = __builtin_ctzll(mk);
          mk &= mk - 1;
          pos[u] = __builtin_amdgcn_readlane((int)e, j) & 0xffff;
        }
      }
      // Every load is issued, unconditionally, before the first add: an empty slot re-reads the
      // batch's first row and a column at or past D reads column 0 (neither is stored), and an
      // empty slot adds +0, which leaves an fp32 sum that starts at +0 unchanged bit for bit.
      EmbPiece<S, VN> t[U][NCH];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
          const int col = c + 64 * VN * k;
          t[u][k] = emb_load<S, VN>(src + (int64_t)(pos[u] >= 0 ? pos[u] : pos[0]) * D + (col < D ? col : 0));
        }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int k = 0; k < NCH; ++k)
#pragma unroll
          for (int q = 0; q < VN; ++q) acc[k][q] += pos[u] >= 0 ? to_f32(t[u][k].v[q]) : 0.f;
    }
  }
}

template <typename S, typename O>
__global__ __launch_bounds__(kEmbThreads) void embedding_bwd_interleaved(const int64_t* __restrict__ ids, int n,
                                                                         const S* __restrict__ src,
                                                                         O* __restrict__ dst, int64_t V, int D,
                                                                         int64_t pad, int shift, int R) {
  extern __shared__ uint32_t emb_sm[];
  uint32_t* list = emb_sm;  // n entries
  uint32_t* cnt = list + n;  // hits per local row
  uint32_t* hot = cnt + R;   // local rows with >= kEmbHot hits, ascending
  uint32_t* cold = hot + R;  // the other hit rows, ascending
  __shared__ int wsum[kEmbWaves];
  __shared__ int qnh, qnc, qhead;
  constexpr uint32_t kNone = 0xffffffffu;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t g = blockIdx.x, G = int64_t(1) << shift;
  const int rows = g < V ? (int)((V - 1 - g) >> shift) + 1 : 0;
  for (int i = tid; i < rows; i += kEmbThreads) cnt[i] = 0u;
  if (tid == 0) qhead = 0;
  __syncthreads();
  {
    int64_t v[kEmbIdsPerThread];
#pragma unroll
    for (int j = 0; j < kEmbIdsPerThread; ++j) {
      const int i = tid + j * kEmbThreads;
      v[j] = i < n ? ids[i] : -1;
    }
#pragma unroll
    for (int j = 0; j < kEmbIdsPerThread; ++j) {
      const int i = tid + j * kEmbThreads;
      if (i < n) {
        uint32_t e = kNone;
        if (v[j] >= 0 && v[j] < V && (v[j] & (G - 1)) == g && v[j] != pad) {
          const uint32_t r = (uint32_t)(v[j] >> shift);
          e = r << 16 | (uint32_t)i;
          atomicAdd(&cnt[r], 1u);
        }
        list[i] = e;
      }
    }
  }
  __syncthreads();
  // compaction: thread t takes positions [t J, t J + J)
  const int J = (n + kEmbThreads - 1) / kEmbThreads;
  uint32_t mine[kEmbIdsPerThread];
  int c = 0;
#pragma unroll
  for (int j = 0; j < kEmbIdsPerThread; ++j) {
    const int p = tid * J + j;
    mine[j] = j < J && p < n ? list[p] : kNone;
    c += mine[j] != kNone;
  }
  int incl = c;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(incl, o);
    if (lane >= o) incl += t;
  }
  if (lane == 63) wsum[wid] = incl;
  if (wid == 0) {  // hit rows by class, ascending
    int nh = 0, nc = 0;
    for (int r0 = 0; r0 < rows; r0 += 64) {
      const int r = r0 + lane;
      const uint32_t k = r < rows ? cnt[r] : 0u;
      const uint64_t hm = __ballot(k >= (uint32_t)kEmbHot), cm = __ballot(k > 0u && k < (uint32_t)kEmbHot);
      if (k >= (uint32_t)kEmbHot)
        hot[nh + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(hm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)hm, 0u))] = r;
      else if (k > 0u)
        cold[nc + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(cm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)cm, 0u))] = r;
      nh += __popcll(hm);
      nc += __popcll(cm);
    }
    if (lane == 0) qnh = nh, qnc = nc;
  }
  __syncthreads();  // every thread holds its entries; the wave totals and the row classes are in
  int off = incl - c, L = 0;
#pragma unroll
  for (int w = 0; w < kEmbWaves; ++w) {
    const int s = wsum[w];
    off += w < wid ? s : 0;
    L += s;
  }
#pragma unroll
  for (int j = 0; j < kEmbIdsPerThread; ++j)
    if (mine[j] != kNone) list[off++] = mine[j];
  __syncthreads();

  const int ns = (D + kEmbHotCols - 1) / kEmbHotCols;  // slices of a hot row
  const int nhi = qnh * ns, nitems = nhi + qnc;
  auto next = [&]() {
    int q = 0;
    if (lane == 0) q = atomicAdd(&qhead, 1);
    return __builtin_amdgcn_readfirstlane(q);
  };
  int q = next();
  for (; q < nhi; q = next()) {  // slices of the hot rows first: their chains are the longest
    const int h = q / ns, s = q - h * ns;
    const uint32_t r = hot[h];
    O* drow = dst + ((int64_t)r * G + g) * D;
    const int cc = s * kEmbHotCols + lane * kEmbHotVN;
    float acc[1][kEmbHotVN];
#pragma unroll
    for (int k = 0; k < kEmbHotVN; ++k) acc[0][k] = 0.f;
    emb_sum<kEmbHotVN, 1, kEmbHotU>(list, L, r, src, D, cc, acc);
    if (cc < D) emb_store_nt<O, kEmbHotVN>(drow + cc, acc[0]);
  }
  if (wid < kEmbZeroWaves) {  // local rows wid, wid + Z, wid + 2Z, ... that no token hits
    float z[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) z[k] = 0.f;
    for (int m0 = 0; wid + kEmbZeroWaves * m0 < rows; m0 += 64) {
      const int r = wid + kEmbZeroWaves * (m0 + lane);
      uint64_t mk = __ballot(r < rows && cnt[r] == 0u);
      while (mk) {
        const int j = __builtin_ctzll(mk);
        mk &= mk - 1;
        O* drow = dst + ((int64_t)(wid + kEmbZeroWaves * (m0 + j)) * G + g) * D;
        for (int cc = lane * 8; cc < D; cc += 64 * 8) emb_store_nt<O, 8>(drow + cc, z);
      }
    }
  }
  for (; q < nitems; q = next()) {  // the other hit rows whole, 1024 columns per pass
    const uint32_t r = cold[q - nhi];
    O* drow = dst + ((int64_t)r * G + g) * D;
    for (int c0 = 0; c0 < D; c0 += 2 * 64 * 8) {
      float acc[2][8];
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[0][k] = acc[1][k] = 0.f;
      const int cc = c0 + lane * 8;
      emb_sum<8, 2, 4>(list, L, r, src, D, cc, acc);
      if (cc < D) emb_store_nt<O, 8>(drow + cc, acc[0]);
      if (cc + 512 < D) emb_store_nt<O, 8>(drow + cc + 512, acc[1]);
    }
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

template <typename S, typename O>
static int launch_embedding_interleaved_t(const int64_t* ids, const void* gout, void* gw, int64_t n, int64_t V, int64_t D,
                                     int64_t pad, hipStream_t st) {
  // G = 256 workgroups (fewer for a smaller vocabulary, more when a workgroup would own more
  // than kEmbMaxRows rows), a power of two
  int shift = 0;
  while (shift < 8 && (int64_t(1) << shift) < V) ++shift;
  while (ceil_div(V, int64_t(1) << shift) > kEmbMaxRows) ++shift;
  const int64_t G = int64_t(1) << shift, R = ceil_div(V, G);
  QH_CHECK_ARG(G < (1ll << 31) && D < (1ll << 31), "qh_embedding_bwd: grid too large");
  const int lds = (int)(4 * (n + 3 * R));
  // the dynamic-LDS limit is raised once per instantiation and device
  static uint64_t attr_set = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    qh::set_error("qh_embedding_bwd: no current device");
    return QH_E_HIP;
  }
  if (!(attr_set >> dev & 1)) {
    const hipError_t e = hipFuncSetAttribute((const void*)embedding_bwd_interleaved<S, O>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             (int)(4 * (kEmbLdsTokens + 3 * kEmbMaxRows)));
    if (e != hipSuccess) {
      qh::set_error("qh_embedding_bwd: cannot raise the LDS limit: %s", hipGetErrorString(e));
      return QH_E_HIP;
    }
    attr_set |= 1ull << dev;
  }
  embedding_bwd_interleaved<S, O><<<(unsigned)G, kEmbThreads, lds, st>>>(ids, (int)n, (const S*)gout, (O*)gw, V,
                                                                          (int)D, pad, shift, (int)R);
  return QH_OK;
}

static int launch_embedding_interleaved(const int64_t* ids, const void* gout, void* gw, int64_t n, int64_t V, int64_t D,
                                   int64_t pad, int gdtype, int wdtype, hipStream_t st) {
  int rc = QH_OK;
#define QH_ER_O(S)                                                                                   \
  switch (wdtype) {                                                                                  \
    case QH_F32: rc = launch_embedding_interleaved_t<S, float>(ids, gout, gw, n, V, D, pad, st); break;   \
    case QH_F16: rc = launch_embedding_interleaved_t<S, f16_t>(ids, gout, gw, n, V, D, pad, st); break;   \
    case QH_BF16: rc = launch_embedding_interleaved_t<S, bf16_t>(ids, gout, gw, n, V, D, pad, st); break; \
    default: qh::set_error("qh_embedding_bwd: bad weight dtype"); return QH_E_DTYPE;                 \
  }
  switch (gdtype) {
    case QH_F32: QH_ER_O(float); break;
    case QH_F16: QH_ER_O(f16_t); break;
    case QH_BF16: QH_ER_O(bf16_t); break;
    default: qh::set_error("qh_embedding_bwd: bad grad dtype"); return QH_E_DTYPE;
  }
#undef QH_ER_O
  if (rc) return rc;
  QH_CHECK_LAUNCH("qh_embedding_bwd");
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
  if (n_tokens <= kEmbLdsTokens) return launch_embedding_interleaved(ids, gout, gw, n_tokens, V, Hd, padding_idx, gdtype,
                                                                wdtype, st);
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

// index_add of at most kIdxScanMax source rows in one launch, without the sort: wave i loads
// all n indices at once (one round trip) and exits unless position i is the first of its row;
// else it lists the row's positions in source order (a ballot per 64 positions) and adds those
// source rows onto the row in that order (fp32, rounded once): the sums of the sorted path.
// Any one wave scans n indices, so the launch reads n^2 indices from the L2 (32 MB at n = 2048).
constexpr int kIdxScanMax = 2048;

template <typename T>
__global__ __launch_bounds__(256) void index_add_scan(T* __restrict__ dst, int64_t stride_d, const T* __restrict__ src,
                                                      int64_t stride_s, const int64_t* __restrict__ idx, int n,
                                                      int64_t n_target, int64_t D) {
  constexpr int NB = kIdxScanMax / 64;
  __shared__ uint32_t runs[4][kIdxScanMax];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int i = (int)blockIdx.x * 4 + wid;
  if (i >= n) return;
  // every index load (clamped positions, unconditional) is issued before the first is used:
  // the empty asm keeps the compiler from sinking each into the block that tests it
  int64_t r = idx[i];
  int64_t v[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) v[b] = idx[min(b * 64 + lane, n - 1)];
  asm volatile("" : "+v"(r));
#pragma unroll
  for (int b = 0; b < NB; ++b) asm volatile("" : "+v"(v[b]));
  if (r < 0 || r >= n_target) return;
  uint32_t* run = runs[wid];
  int cnt = 0;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (b * 64 >= n) break;
    const uint64_t m = __ballot(b * 64 + lane < n && v[b] == r);
    const int p0 = b * 64;
    // positions p0 + bit below i that hold the row: i is not its first position
    const int below = i - p0;  // bits [0, below) lie before i
    const uint64_t before = below <= 0 ? 0ull : (below >= 64 ? ~0ull : ((1ull << below) - 1));
    if (m & before) return;
    const uint64_t after = m & ~before;
    if ((after >> lane) & 1ull) run[cnt + __popcll(after & ((1ull << lane) - 1))] = (uint32_t)(p0 + lane);
    cnt += __popcll(after);
  }
  __builtin_amdgcn_wave_barrier();  // (LDS runs in order within the wave: the list is written before it is read)
  // four 8-column chunks per lane at a time (clamped to the row, so every load is issued; only
  // the stores are guarded): the row's chunks and each source row's chunks load together
  constexpr int CW = 4;
  T* drow = dst + r * stride_d;
  for (int64_t c0 = lane * 8; c0 < D; c0 += 64 * 8 * CW) {
    int64_t cw[CW];
#pragma unroll
    for (int w = 0; w < CW; ++w) cw[w] = min(c0 + (int64_t)w * 512, D - 8);
    float acc[CW][8];
#pragma unroll
    for (int w = 0; w < CW; ++w) ld8f(drow + cw[w], acc[w]);
    for (int j = 0; j < cnt; ++j) {
      const T* srow = src + (int64_t)run[j] * stride_s;
      float t[CW][8];
#pragma unroll
      for (int w = 0; w < CW; ++w) ld8f(srow + cw[w], t[w]);
#pragma unroll
      for (int w = 0; w < CW; ++w)
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[w][q] += t[w][q];
    }
#pragma unroll
    for (int w = 0; w < CW; ++w)
      if (c0 + w * 512 < D) st8f(drow + c0 + w * 512, acc[w]);
  }
}

extern "C" int qh_index_add(void* target, int64_t stride_t, const void* src, int64_t stride_s, const int64_t* index,
                            int64_t n_src, int64_t n_target, int64_t D, void* ws, int64_t ws_bytes, int dtype,
                            void* stream) {
  QH_CHECK_ARG(n_src >= 0 && n_target >= 0 && D >= 0, "qh_index_add: negative shape");
  QH_CHECK_ARG(n_target < (1ll << 31) - 1 && n_src < (1ll << 31), "qh_index_add: sizes exceed 2^31");
  if (n_src == 0 || D == 0 || n_target == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const bool vec = D % 8 == 0 && stride_s % 8 == 0 && stride_t % 8 == 0 && aligned16(src) && aligned16(target);
  if (vec && n_src <= kIdxScanMax) {
    const unsigned grid = (unsigned)((n_src + 3) / 4);
    switch (dtype) {
      case QH_F32:
        index_add_scan<float><<<grid, 256, 0, st>>>((float*)target, stride_t, (const float*)src, stride_s, index,
                                                    (int)n_src, n_target, D);
        break;
      case QH_F16:
        index_add_scan<f16_t><<<grid, 256, 0, st>>>((f16_t*)target, stride_t, (const f16_t*)src, stride_s, index,
                                                    (int)n_src, n_target, D);
        break;
      case QH_BF16:
        index_add_scan<bf16_t><<<grid, 256, 0, st>>>((bf16_t*)target, stride_t, (const bf16_t*)src, stride_s,
                                                     index, (int)n_src, n_target, D);
        break;
      default: qh::set_error("qh_index_add: bad dtype"); return QH_E_DTYPE;
    }
    QH_CHECK_LAUNCH("qh_index_add");
    return QH_OK;
  }
  uint32_t *keys = nullptr, *vals = nullptr;
  int rc = sort_indices(index, n_src, n_target, ws, ws_bytes, &keys, &vals, st, "qh_index_add");
  if (rc) return rc;
  rc = launch_segments<true>(keys, vals, n_src, src, dtype, stride_s, target, dtype, stride_t, D, (uint32_t)n_target,
                             -1, st);
  if (rc) return rc;
  QH_CHECK_LAUNCH("qh_index_add");
  return QH_OK;
}
