// MoE token dispatch and combine (the data movement around the grouped expert
// GEMM, qh_moe_gemm).
//
// Dispatch: the T*k (token, slot) assignments are sorted by expert with a
// stable radix sort (rocPRIM), so expert e's rows form one contiguous segment
// in (token, slot) order. From the sorted keys: segment offsets (binary
// search, no atomics), the first 128-row M-tile of each expert, and per
// sorted row its token, its routing weight and (inverse map) its position.
//
// Combine: out[t] = sum over t's k expert rows in ascending expert order, with
// a rounding to the dtype after every add — the order and rounding of the
// reference's per-expert index_add into a zero tensor.
#include <cstring>
#include <rocprim/rocprim.hpp>

#include "qh_common.h"

namespace {

static int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

static size_t sort_temp_bytes(int64_t n, int bits) {
  size_t sz = 0;
  rocprim::radix_sort_pairs((void*)nullptr, sz, (const uint32_t*)nullptr, (uint32_t*)nullptr,
                            (const uint32_t*)nullptr, (uint32_t*)nullptr, (unsigned)n, 0, bits, (hipStream_t)0);
  return sz;
}

static int key_bits(int64_t E) {
  int b = 1;
  while ((1ll << b) <= E) ++b;  // keys 0..E (E marks an out-of-range expert id)
  return b;
}

__global__ __launch_bounds__(256) void moe_keys(const int64_t* __restrict__ sel, int64_t n, int64_t E,
                                                uint32_t* __restrict__ keys, uint32_t* __restrict__ vals) {
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t e = sel[i];
    keys[i] = (e >= 0 && e < E) ? (uint32_t)e : (uint32_t)E;
    vals[i] = (uint32_t)i;
  }
}

// seg[e] = first sorted position with key >= e, e = 0..E (lower bound).
__global__ __launch_bounds__(256) void moe_segments(const uint32_t* __restrict__ keys, int64_t n, int E,
                                                    int32_t* __restrict__ seg) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e > E) return;
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (keys[mid] < (uint32_t)e) lo = mid + 1;
    else hi = mid;
  }
  seg[e] = (int32_t)lo;
}

// toff[e] = sum over e' < e of ceil(n_e' / tile_m) (one workgroup, E <= 65536).
__global__ __launch_bounds__(1024) void moe_tile_offsets(const int32_t* __restrict__ seg, int E, int tile_m,
                                                         int32_t* __restrict__ toff) {
  __shared__ int32_t part[1024];
  const int per = (E + 1023) / 1024;
  const int b0 = threadIdx.x * per;
  int32_t s = 0;
  for (int e = b0; e < b0 + per && e < E; ++e) s += (seg[e + 1] - seg[e] + tile_m - 1) / tile_m;
  part[threadIdx.x] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t run = 0;
    for (int i = 0; i < 1024; ++i) {
      const int32_t v = part[i];
      part[i] = run;
      run += v;
    }
  }
  __syncthreads();
  int32_t run = part[threadIdx.x];
  for (int e = b0; e < b0 + per && e < E; ++e) {
    toff[e] = run;
    run += (seg[e + 1] - seg[e] + tile_m - 1) / tile_m;
  }
  if (threadIdx.x == 1023) toff[E] = run;  // blocks past E add nothing: this is the total
}

template <typename T>
__global__ __launch_bounds__(256) void moe_rows(const uint32_t* __restrict__ vals, int64_t n, int k,
                                                const T* __restrict__ w, int32_t* __restrict__ rows,
                                                T* __restrict__ wsorted, int32_t* __restrict__ inv) {
  for (int64_t r = blockIdx.x * 256ll + threadIdx.x; r < n; r += (int64_t)gridDim.x * 256) {
    const uint32_t a = vals[r];
    rows[r] = (int32_t)(a / (uint32_t)k);
    wsorted[r] = w[a];
    inv[a] = (int32_t)r;
  }
}

// One workgroup per token; each thread owns 8 consecutive columns. With
// weights, row j contributes round(Y[p] * w[t, j]) (the routing-weight scaling
// of the expert output), else Y[p] itself.
template <typename T, int KMAX>
__global__ __launch_bounds__(256) void moe_combine_kernel(const T* __restrict__ Y, int64_t ldy,
                                                          const int32_t* __restrict__ inv,
                                                          const int64_t* __restrict__ sel,
                                                          const T* __restrict__ w, int k, int64_t E,
                                                          T* __restrict__ out, int64_t H) {
  const int64_t t = blockIdx.x;
  // The token's k slots are loaded together (slots past k repeat slot 0 and are dropped), then
  // ordered by expert id in registers (ids of one token are distinct; out-of-range ids sort last
  // and are dropped). The empty asm statements keep every load of a group issued before the
  // first use: the compiler otherwise sinks each guarded load into the block that tests it and
  // waits for it there, one round trip per slot.
  int64_t ek[KMAX];
  int32_t pk[KMAX];
  float wk[KMAX];
  uint32_t wr[KMAX];  // the weights' 16-bit patterns
  const uint16_t* wb = reinterpret_cast<const uint16_t*>(w);
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    const int64_t jj = t * k + (j < k ? j : 0);
    ek[j] = sel[jj];
    pk[j] = inv[jj];
  }
  if (w) {
#pragma unroll
    for (int j = 0; j < KMAX; ++j) wr[j] = wb[t * k + (j < k ? j : 0)];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) asm volatile("" : "+v"(wr[j]));
  }
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    asm volatile("" : "+v"(ek[j]), "+v"(pk[j]));
    wk[j] = w ? to_f32(__builtin_bit_cast(T, (uint16_t)wr[j])) : 1.f;
    ek[j] = (j >= k || ek[j] < 0 || ek[j] >= E) ? E : ek[j];
  }
  int nk = 0;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) nk += ek[j] < E ? 1 : 0;
#pragma unroll
  for (int j = 1; j < KMAX; ++j)
#pragma unroll
    for (int q = j; q > 0; --q) {
      const bool sw = ek[q - 1] > ek[q];
      const int64_t e0 = ek[q - 1], e1 = ek[q];
      const int32_t p0 = pk[q - 1], p1 = pk[q];
      const float w0 = wk[q - 1], w1 = wk[q];
      ek[q - 1] = sw ? e1 : e0;
      ek[q] = sw ? e0 : e1;
      pk[q - 1] = sw ? p1 : p0;
      pk[q] = sw ? p0 : p1;
      wk[q - 1] = sw ? w1 : w0;
      wk[q] = sw ? w0 : w1;
    }
  for (int64_t c = threadIdx.x * 8; c < H; c += 256 * 8) {
    Vec16<T> acc;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc.v[e] = (T)0.f;
    if (nk > 0) {
      // every row is requested before the ordered sum consumes them (rows past nk repeat the first);
      // non-temporal: the expert rows are read once and exceed the last-level cache
      Vec16<T> y[KMAX];
#pragma unroll
      for (int j = 0; j < KMAX; ++j) y[j] = ld16_nt(Y + (int64_t)pk[j < nk ? j : 0] * ldy + c);
#pragma unroll
      for (int j = 0; j < KMAX; ++j) {
        qh_u32x4 r = __builtin_bit_cast(qh_u32x4, y[j].raw);
        asm volatile("" : "+v"(r));
        y[j].raw = __builtin_bit_cast(uint4, r);
      }
#pragma unroll
      for (int j = 0; j < KMAX; ++j) {
        if (j >= nk) break;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float yv = w ? to_f32(from_f32<T>(to_f32(y[j].v[e]) * wk[j])) : to_f32(y[j].v[e]);
          acc.v[e] = from_f32<T>(to_f32(acc.v[e]) + yv);
        }
      }
    }
    st16(out + t * H + c, acc);
  }
}

// Xs[r] = X[rows[r]] (one workgroup per 8 rows, two rows per wave, 16-byte vectors): both row
// indices load together, then up to eight 16-byte loads are in flight before their stores.
template <typename T>
__global__ __launch_bounds__(256) void moe_gather_kernel(const T* __restrict__ X, int64_t ldx,
                                                         const int32_t* __restrict__ rows, int64_t R, int64_t H,
                                                         T* __restrict__ Xs, int64_t lds) {
  const int64_t r0 = (blockIdx.x * 4ll + (threadIdx.x >> 6)) * 2;
  if (r0 >= R) return;
  const bool two = r0 + 1 < R;
  const T* src0 = X + (int64_t)rows[r0] * ldx;
  const T* src1 = X + (int64_t)rows[two ? r0 + 1 : r0] * ldx;
  T* dst0 = Xs + r0 * lds;
  T* dst1 = dst0 + lds;
  for (int64_t c0 = (threadIdx.x & 63) * 8; c0 < H; c0 += 4 * 64 * 8) {
    // clamped columns: every load is issued, only the stores are guarded
    int64_t cc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) cc[u] = min(c0 + (int64_t)u * 512, H - 8);
    Vec16<T> v0[4], v1[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      v0[u] = ld16(src0 + cc[u]);
      v1[u] = ld16(src1 + cc[u]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (c0 + u * 512 < H) {
        st16(dst0 + c0 + u * 512, v0[u]);
        if (two) st16(dst1 + c0 + u * 512, v1[u]);
      }
  }
}

// Backward of the routing-weight scaling, one workgroup per token t: for each
// of its expert rows p (slot j), dD[p] = round(dout[t] * w[t, j]) and
// dw[t, j] = round(sum_c dout[t, c] * D[p, c]) (fp32, fixed-order block sum).
// Slots with an out-of-range expert id get dw = 0.
template <typename T>
__global__ __launch_bounds__(256) void moe_scale_bwd_kernel(const T* __restrict__ dout, int64_t ldo,
                                                            const T* __restrict__ D, int64_t ldd,
                                                            const T* __restrict__ w, const int32_t* __restrict__ inv,
                                                            const int64_t* __restrict__ sel, int k, int64_t E,
                                                            int64_t H, T* __restrict__ dD, int64_t ldg,
                                                            T* __restrict__ dw) {
  __shared__ float red[4];
  const int64_t t = blockIdx.x;
  const T* go = dout + t * ldo;
  for (int j = 0; j < k; ++j) {
    const int64_t e = sel[t * k + j];
    if (e < 0 || e >= E) {
      if (threadIdx.x == 0) dw[t * k + j] = (T)0.f;
      continue;
    }
    const int64_t p = inv[t * k + j];
    const float wj = to_f32(w[t * k + j]);
    const T* drow = D + p * ldd;
    T* grow = dD + p * ldg;
    float s = 0.f;
    for (int64_t c = threadIdx.x * 8; c < H; c += 256 * 8) {
      const Vec16<T> g = ld16(go + c), d = ld16(drow + c);
      Vec16<T> o;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const float gf = to_f32(g.v[q]);
        o.v[q] = from_f32<T>(gf * wj);
        s += gf * to_f32(d.v[q]);
      }
      st16(grow + c, o);
    }
    s = block_sum(s, red);
    if (threadIdx.x == 0) dw[t * k + j] = from_f32<T>(s);
  }
}

// The same for top_k <= 8, with every load of a token in flight at once: its slots (expert, row,
// weight), then its gradient row with every slot's D row, and the k dot products reduced
// together (one barrier). Per-slot sums and their order are those of moe_scale_bwd_kernel, so
// the results are equal bit for bit.
template <typename T>
__global__ __launch_bounds__(256) void moe_scale_bwd8_kernel(const T* __restrict__ dout, int64_t ldo,
                                                             const T* __restrict__ D, int64_t ldd,
                                                             const T* __restrict__ w,
                                                             const int32_t* __restrict__ inv,
                                                             const int64_t* __restrict__ sel, int k, int64_t E,
                                                             int64_t H, T* __restrict__ dD, int64_t ldg,
                                                             T* __restrict__ dw) {
  constexpr int KM = 8;
  __shared__ float red[KM][4];
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const uint16_t* wb = reinterpret_cast<const uint16_t*>(w);
  int64_t ek[KM];
  int32_t pk[KM];
  uint32_t wr[KM];
#pragma unroll
  for (int j = 0; j < KM; ++j) {
    const int64_t jj = t * k + (j < k ? j : 0);
    ek[j] = sel[jj];
    pk[j] = inv[jj];
    wr[j] = wb[jj];
  }
  // (empty asm: every slot load is issued before the first is used)
#pragma unroll
  for (int j = 0; j < KM; ++j) asm volatile("" : "+v"(ek[j]), "+v"(pk[j]), "+v"(wr[j]));
  bool ok[KM];
  int pfirst = -1;
#pragma unroll
  for (int j = KM - 1; j >= 0; --j) {
    ok[j] = j < k && ek[j] >= 0 && ek[j] < E;
    if (ok[j]) pfirst = pk[j];
  }
  float s[KM];
#pragma unroll
  for (int j = 0; j < KM; ++j) s[j] = 0.f;
  if (pfirst >= 0) {  // (token-uniform) some slot has a row; the others read that row and drop it
    const T* go = dout + t * ldo;
    for (int64_t c = threadIdx.x * 8; c < H; c += 256 * 8) {
      const Vec16<T> g = ld16(go + c);
      Vec16<T> d[KM];
#pragma unroll
      for (int j = 0; j < KM; ++j)  // (non-temporal: D is read once and exceeds the last-level cache)
        d[j] = ld16_nt(D + (int64_t)(ok[j] ? pk[j] : pfirst) * ldd + c);
#pragma unroll
      for (int j = 0; j < KM; ++j) {
        qh_u32x4 r = __builtin_bit_cast(qh_u32x4, d[j].raw);
        asm volatile("" : "+v"(r));
        d[j].raw = __builtin_bit_cast(uint4, r);
      }
#pragma unroll
      for (int j = 0; j < KM; ++j) {
        if (!ok[j]) continue;
        const float wj = to_f32(__builtin_bit_cast(T, (uint16_t)wr[j]));
        Vec16<T> o;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const float gf = to_f32(g.v[q]);
          o.v[q] = from_f32<T>(gf * wj);
          s[j] += gf * to_f32(d[j].v[q]);
        }
        st16(dD + (int64_t)pk[j] * ldg + c, o);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < KM; ++j) s[j] = wave_sum(s[j]);
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < KM; ++j) red[j][wid] = s[j];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int j = 0; j < KM; ++j) {
      if (j >= k) break;
      float tsum = 0.f;
      for (int i = 0; i < 4; ++i) tsum += red[j][i];  // the wave order of block_sum
      dw[t * k + j] = ok[j] ? from_f32<T>(tsum) : (T)0.f;
    }
  }
}

}  // namespace

extern "C" int64_t qh_moe_dispatch_workspace(int64_t n_tokens, int64_t top_k, int64_t n_experts) {
  const int64_t n = n_tokens * top_k;
  if (n <= 0 || n_experts <= 0) return 0;
  return 4 * align256(n * 4) + align256((int64_t)sort_temp_bytes(n, key_bits(n_experts)));
}

extern "C" int qh_moe_dispatch(const int64_t* selected, const void* weights, int64_t n_tokens, int64_t top_k,
                               int64_t n_experts, int64_t tile_m, void* ws, int64_t ws_bytes, int32_t* rows,
                               void* wsorted, int32_t* inv, int32_t* seg_off, int32_t* tile_off, int dtype,
                               void* stream) {
  QH_CHECK_ARG(n_tokens >= 0 && top_k > 0 && n_experts > 0 && n_experts <= 65536 && tile_m > 0,
               "qh_moe_dispatch: bad shape");
  const int64_t n = n_tokens * top_k;
  QH_CHECK_ARG(n < (1ll << 31), "qh_moe_dispatch: too many assignments");
  QH_CHECK_ARG(dtype >= QH_F32 && dtype <= QH_BF16, "qh_moe_dispatch: bad dtype");
  const int64_t need = qh_moe_dispatch_workspace(n_tokens, top_k, n_experts);
  if (ws_bytes < need) {
    qh::set_error("qh_moe_dispatch: workspace %lld < %lld", (long long)ws_bytes, (long long)need);
    return QH_E_WORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  const int E = (int)n_experts;
  if (n == 0) {
    int rc = qh_zero(seg_off, (E + 1) * 4, stream);
    return rc ? rc : qh_zero(tile_off, (E + 1) * 4, stream);
  }
  char* p = (char*)ws;
  uint32_t* keys_in = (uint32_t*)p; p += align256(n * 4);
  uint32_t* keys_out = (uint32_t*)p; p += align256(n * 4);
  uint32_t* vals_in = (uint32_t*)p; p += align256(n * 4);
  uint32_t* vals_out = (uint32_t*)p; p += align256(n * 4);
  const int bits = key_bits(n_experts);
  size_t temp = sort_temp_bytes(n, bits);
  const unsigned g = (unsigned)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
  moe_keys<<<g, 256, 0, st>>>(selected, n, n_experts, keys_in, vals_in);
  if (rocprim::radix_sort_pairs((void*)p, temp, keys_in, keys_out, vals_in, vals_out, (unsigned)n, 0, bits, st) !=
      hipSuccess) {
    qh::set_error("qh_moe_dispatch: radix sort failed");
    return QH_E_HIP;
  }
  moe_segments<<<(E + 1 + 255) / 256, 256, 0, st>>>(keys_out, n, E, seg_off);
  moe_tile_offsets<<<1, 1024, 0, st>>>(seg_off, E, (int)tile_m, tile_off);
#define QH_ROWS(T) moe_rows<T><<<g, 256, 0, st>>>(vals_out, n, (int)top_k, (const T*)weights, rows, (T*)wsorted, inv)
  if (dtype == QH_BF16) QH_ROWS(bf16_t); else if (dtype == QH_F16) QH_ROWS(f16_t); else QH_ROWS(float);
#undef QH_ROWS
  QH_CHECK_LAUNCH("qh_moe_dispatch");
  return QH_OK;
}

extern "C" int qh_moe_combine(const void* Y, int64_t ldy, const int32_t* inv, const int64_t* selected,
                              const void* weights, int64_t n_tokens, int64_t top_k, int64_t n_experts, void* out,
                              int64_t H, int dtype, void* stream) {
  QH_CHECK_ARG(n_tokens >= 0 && top_k > 0 && top_k <= 32 && H > 0 && n_experts > 0, "qh_moe_combine: bad shape");
  QH_CHECK_ARG(H % 8 == 0 && ldy % 8 == 0 && aligned16(Y) && aligned16(out),
               "qh_moe_combine: rows must be 16-byte aligned with H, ldy multiples of 8");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_moe_combine: bf16/f16 only");
  QH_CHECK_ARG(n_tokens < (1ll << 31), "qh_moe_combine: too many tokens");
  if (n_tokens == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
#define QH_COMB(T, KM) \
  moe_combine_kernel<T, KM><<<(unsigned)n_tokens, 256, 0, st>>>((const T*)Y, ldy, inv, selected, (const T*)weights, \
                                                                 (int)top_k, n_experts, (T*)out, H)
  if (dtype == QH_BF16) {
    if (top_k <= 8) QH_COMB(bf16_t, 8); else QH_COMB(bf16_t, 32);
  } else {
    if (top_k <= 8) QH_COMB(f16_t, 8); else QH_COMB(f16_t, 32);
  }
#undef QH_COMB
  QH_CHECK_LAUNCH("qh_moe_combine");
  return QH_OK;
}

extern "C" int qh_moe_gather(const void* X, int64_t ldx, const int32_t* rows, int64_t R, int64_t H, void* Xs,
                             int64_t lds, int dtype, void* stream) {
  QH_CHECK_ARG(R >= 0 && H > 0 && R < (1ll << 33), "qh_moe_gather: bad shape");
  QH_CHECK_ARG(H % 8 == 0 && ldx % 8 == 0 && lds % 8 == 0 && lds >= H && aligned16(X) && aligned16(Xs),
               "qh_moe_gather: rows must be 16-byte aligned with H and strides multiples of 8");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_moe_gather: bf16/f16 only");
  if (R == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const unsigned g = (unsigned)((R + 7) / 8);
  if (dtype == QH_BF16)
    moe_gather_kernel<bf16_t><<<g, 256, 0, st>>>((const bf16_t*)X, ldx, rows, R, H, (bf16_t*)Xs, lds);
  else
    moe_gather_kernel<f16_t><<<g, 256, 0, st>>>((const f16_t*)X, ldx, rows, R, H, (f16_t*)Xs, lds);
  QH_CHECK_LAUNCH("qh_moe_gather");
  return QH_OK;
}

extern "C" int qh_moe_scale_bwd(const void* dout, int64_t ldo, const void* D, int64_t ldd, const void* weights,
                                const int32_t* inv, const int64_t* selected, int64_t n_tokens, int64_t top_k,
                                int64_t n_experts, int64_t H, void* dD, int64_t ldg, void* dw, int dtype,
                                void* stream) {
  QH_CHECK_ARG(n_tokens >= 0 && top_k > 0 && H > 0 && n_experts > 0 && n_tokens < (1ll << 31),
               "qh_moe_scale_bwd: bad shape");
  QH_CHECK_ARG(H % 8 == 0 && ldo % 8 == 0 && ldd % 8 == 0 && ldg % 8 == 0 && aligned16(dout) && aligned16(D) &&
                   aligned16(dD),
               "qh_moe_scale_bwd: rows must be 16-byte aligned with H and strides multiples of 8");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_moe_scale_bwd: bf16/f16 only");
  if (n_tokens == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
#define QH_SB(T)                                                                                              \
  if (top_k <= 8)                                                                                             \
    moe_scale_bwd8_kernel<T><<<(unsigned)n_tokens, 256, 0, st>>>((const T*)dout, ldo, (const T*)D, ldd,       \
                                                                 (const T*)weights, inv, selected, (int)top_k, \
                                                                 n_experts, H, (T*)dD, ldg, (T*)dw);          \
  else                                                                                                        \
    moe_scale_bwd_kernel<T><<<(unsigned)n_tokens, 256, 0, st>>>((const T*)dout, ldo, (const T*)D, ldd,        \
                                                                (const T*)weights, inv, selected, (int)top_k, \
                                                                n_experts, H, (T*)dD, ldg, (T*)dw)
  if (dtype == QH_BF16) QH_SB(bf16_t); else QH_SB(f16_t);
#undef QH_SB
  QH_CHECK_LAUNCH("qh_moe_scale_bwd");
  return QH_OK;
}
