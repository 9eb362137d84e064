// Flash attention with fp32 inputs and outputs (forward and backward) on the
// fp32 matrix cores (v_mfma_f32_16x16x4_f32), for the fp32 q/k/v calls that the
// reference also runs through its kernel (qwen_triton/kernels/flash_attention.py:
// 280-314 forward, 317-367 backward). The bf16/fp16 kernels of qh_attention.hip
// carry the configurations' workloads; these keep fp32 calls on the GPU path with
// fp32 accuracy (every product and sum in fp32), at the fp32 MFMA rate.
//
// MFMA 16x16x4 f32: lane l supplies A[m = l % 16][k = l / 16] and B[k = l / 16]
// [n = l % 16] (one value each) and holds D[4 (l / 16) + r][l % 16], r = 0..3.
// The k index of a product is a label: each kernel maps lane group g = l / 16 of
// step j to whichever key or head-dim index it needs, the same way for A and B.
// Two mappings are used:
//   * head-dim steps: group g, step j <-> d = g DP/4 + j, so a lane's operand
//     row is DP/4 contiguous values (16-byte LDS reads);
//   * key (or query) steps over a 16-row C tile: group g, step (t, r) <->
//     row 16 t + 4 g + r, exactly the rows that lane holds in the C layout, so
//     a product's output is the next product's B operand without moving data.
// Scores are computed transposed where that mapping needs it (S^T = K Q^T in the
// forward and dQ passes, S = Q K^T in the dK/dV pass), as in the bf16 kernels.
// Deterministic: fixed loop orders, no atomics. LDS tiles are [64][DP + 4]
// floats; the 4-float pad makes the 16-row fragment reads conflict-free.
#include "qh_common.h"

namespace {

typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2eF = 1.4426950408889634f;
constexpr float kLn2F = 0.6931471805599453f;
constexpr int kT = 64;  // rows per tile (queries or keys) and per workgroup

__device__ __forceinline__ f4_t mma4(float a, float b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// Stage rows [r0, r0 + 64) of a [rows, D] operand (row stride ld, unit d stride)
// into an LDS tile [64][DP + 4]; rows past `rows` and columns past D read as zero.
template <int DP>
__device__ __forceinline__ void stage_tile(float* __restrict__ dst, const float* __restrict__ src, int64_t ld, int r0,
                                           int rows, int D) {
  constexpr int LD = DP + 4, C4 = DP / 4;
  for (int i = threadIdx.x; i < kT * C4; i += 256) {
    const int r = i / C4, c = (i - r * C4) * 4;
    f4_t v = {0.f, 0.f, 0.f, 0.f};
    if (r0 + r < rows && c < D) v = *reinterpret_cast<const f4_t*>(src + (int64_t)(r0 + r) * ld + c);
    *reinterpret_cast<f4_t*>(dst + r * LD + c) = v;
  }
}

// A lane's operand row for head-dim steps: DP/4 values from d = g DP/4 (zero past D).
template <int DP>
__device__ __forceinline__ void load_row(float (&x)[DP / 4], const float* __restrict__ row, bool ok, int g, int D) {
#pragma unroll
  for (int j = 0; j < DP / 4; j += 4) {
    const int d = g * (DP / 4) + j;
    f4_t v = {0.f, 0.f, 0.f, 0.f};
    if (ok && d < D) v = *reinterpret_cast<const f4_t*>(row + d);
#pragma unroll
    for (int e = 0; e < 4; ++e) x[j + e] = v[e];
  }
}

// out[t] (C layout, 16 rows x 16 columns) = tile rows 16 t + (l % 16) as A (from LDS) times
// the lane's row x as B, over head-dim steps.
template <int DP>
__device__ __forceinline__ void tile_rows_times(f4_t (&out)[4], const float* __restrict__ tile,
                                                const float (&x)[DP / 4], int lane) {
  constexpr int LD = DP + 4;
  const int li = lane & 15, g = lane >> 4;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    f4_t acc = {0.f, 0.f, 0.f, 0.f};
    const float* row = tile + (16 * t + li) * LD + g * (DP / 4);
#pragma unroll
    for (int j = 0; j < DP / 4; j += 4) {
      const f4_t a = *reinterpret_cast<const f4_t*>(row + j);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = mma4(a[e], x[j + e], acc);
    }
    out[t] = acc;
  }
}

// acc[dt] (C layout: rows d = 16 dt + 4 g + r, column = the lane's n) += sum over the 64 tile
// rows k of tile[k][d] * p[k][n], where p is held in the C layout of four 16-row tiles.
template <int DP>
__device__ __forceinline__ void tileT_times(f4_t (&acc)[DP / 16], const float* __restrict__ tile, const f4_t (&p)[4],
                                            int lane) {
  constexpr int LD = DP + 4;
  const int li = lane & 15, g = lane >> 4;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float* row = tile + (16 * t + 4 * g + r) * LD + li;
#pragma unroll
      for (int dt = 0; dt < DP / 16; ++dt) acc[dt] = mma4(row[16 * dt], p[t][r], acc[dt]);
    }
}

// ---------------------------------------------------------------------------
// Forward: one workgroup per 64 queries of one (b, q-head); wave w owns queries
// 16 w .. 16 w + 15 (lane: query l % 16). Per 64-key tile: S^T = K Q^T, online
// softmax per query (the 64 keys of a query are spread over its 4 lane groups),
// O^T += V^T P^T.
template <int DP>
__global__ __launch_bounds__(256) void fa32_fwd_kernel(const float* __restrict__ Q, int64_t sqb, int64_t sqh,
                                                       int64_t sqs, const float* __restrict__ K, int64_t skb,
                                                       int64_t skh, int64_t sks, const float* __restrict__ V,
                                                       int64_t svb, int64_t svh, int64_t svs, float* __restrict__ O,
                                                       int64_t sob, int64_t soh, int64_t sos, float* __restrict__ LSE,
                                                       int Hq, int groups, int Sq, int Sk, int D, float scale_log2,
                                                       int causal, int coff) {
  constexpr int LD = DP + 4;
  __shared__ __attribute__((aligned(16))) float Ks[kT * LD];
  __shared__ __attribute__((aligned(16))) float Vs[kT * LD];
  const int bh = blockIdx.y, b = bh / Hq, hq = bh % Hq, hk = hq / groups;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
  const int q0 = blockIdx.x * kT, qi = q0 + 16 * w + li;
  const float* Kb = K + b * skb + hk * skh;
  const float* Vb = V + b * svb + hk * svh;
  float qr[DP / 4];
  load_row<DP>(qr, Q + b * sqb + hq * sqh + (int64_t)qi * sqs, qi < Sq, g, D);
  f4_t oacc[DP / 16];
#pragma unroll
  for (int dt = 0; dt < DP / 16; ++dt) oacc[dt] = f4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  int kend = Sk;
  if (causal) kend = min(Sk, max(0, q0 + kT - 1 + coff + 1));
  for (int kv0 = 0; kv0 < kend; kv0 += kT) {
    stage_tile<DP>(Ks, Kb, sks, kv0, Sk, D);
    stage_tile<DP>(Vs, Vb, svs, kv0, Sk, D);
    __syncthreads();
    f4_t s[4];
    tile_rows_times<DP>(s, Ks, qr, lane);  // s[t][r] = S^T[key 16 t + 4 g + r][query li]
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kv0 + 16 * t + 4 * g + r;
        const bool ok = key < Sk && (!causal || key <= qi + coff);
        s[t][r] = ok ? s[t][r] * scale_log2 : -INFINITY;
        mx = fmaxf(mx, s[t][r]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    if (mx > m) {
      const float a = m == -INFINITY ? 0.f : ex2(m - mx);
      l *= a;
#pragma unroll
      for (int dt = 0; dt < DP / 16; ++dt) oacc[dt] *= a;
      m = mx;
    }
    const float mr = m == -INFINITY ? 0.f : m;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s[t][r] = ex2(s[t][r] - mr);
        l += s[t][r];
      }
    tileT_times<DP>(oacc, Vs, s, lane);  // O^T[d][query] += V^T P^T
    __syncthreads();
  }
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (qi < Sq) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    float* Ob = O + b * sob + hq * soh + (int64_t)qi * sos;
#pragma unroll
    for (int dt = 0; dt < DP / 16; ++dt) {
      const int d = 16 * dt + 4 * g;
      if (d < D) *reinterpret_cast<f4_t*>(Ob + d) = oacc[dt] * inv;
    }
    if (g == 0 && LSE) LSE[(int64_t)bh * Sq + qi] = l > 0.f ? (m + __log2f(l)) * kLn2F : -INFINITY;
  }
}

// ---------------------------------------------------------------------------
// Backward. Per query row: Delta = rowsum(O dO) and the LSE in log2 units, in
// rows of sqp floats per (b, q-head) (the layout of the bf16 backward's workspace).
__global__ __launch_bounds__(256) void fa32_bwd_prep_kernel(const float* __restrict__ O, const float* __restrict__ dO,
                                                            const float* __restrict__ LSE, float* __restrict__ delta,
                                                            float* __restrict__ lse2, int64_t rows, int Sq,
                                                            int64_t sqp, int D) {
  const int64_t prow = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int li = threadIdx.x & 15;
  const int64_t bh = prow / sqp;
  const int q = (int)(prow - bh * sqp);
  const bool real = prow < rows && q < Sq;
  const int64_t row = bh * Sq + q;
  float s = 0.f;
  if (real)
    for (int d = li * 4; d < D; d += 64) {
      const f4_t a = *reinterpret_cast<const f4_t*>(O + row * D + d);
      const f4_t c = *reinterpret_cast<const f4_t*>(dO + row * D + d);
      s += a[0] * c[0] + a[1] * c[1] + a[2] * c[2] + a[3] * c[3];
    }
  s = wave_sum(s, 16);
  if (prow < rows && li == 0) {
    delta[prow] = s;
    lse2[prow] = real ? LSE[row] * kLog2eF : 0.f;
  }
}

// dK, dV for 64 keys of one (b, kv-head); wave w owns keys 16 w .. 16 w + 15 (lane: key
// l % 16), its K and V rows in registers. Over every q-head of the group and every visible
// 64-query tile: S = Q K^T and dP = dO V^T (C layout: rows = queries, column = key),
// P = exp2(S scale_log2 - lse2), dS = P (dP - Delta), dV^T += dO^T P, dK^T += Q^T dS.
template <int DP>
__global__ __launch_bounds__(256) void fa32_bwd_dkdv_kernel(
    const float* __restrict__ Q, int64_t sqb, int64_t sqh, int64_t sqs, const float* __restrict__ K, int64_t skb,
    int64_t skh, int64_t sks, const float* __restrict__ V, int64_t svb, int64_t svh, int64_t svs,
    const float* __restrict__ dO, const float* __restrict__ lse2, const float* __restrict__ delta, int64_t sqp,
    float* __restrict__ dK, float* __restrict__ dV, int Hq, int Hkv, int groups, int Sq, int Sk, int D,
    float scale_log2, float scale, int causal, int coff) {
  constexpr int LD = DP + 4;
  __shared__ __attribute__((aligned(16))) float Qs[kT * LD];
  __shared__ __attribute__((aligned(16))) float dOs[kT * LD];
  __shared__ float ls[kT], dl[kT];
  const int bk = blockIdx.y, b = bk / Hkv, hk = bk % Hkv;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
  const int k0 = blockIdx.x * kT, key = k0 + 16 * w + li;
  float kr[DP / 4], vr[DP / 4];
  load_row<DP>(kr, K + b * skb + hk * skh + (int64_t)key * sks, key < Sk, g, D);
  load_row<DP>(vr, V + b * svb + hk * svh + (int64_t)key * svs, key < Sk, g, D);
  f4_t dkT[DP / 16], dvT[DP / 16];
#pragma unroll
  for (int dt = 0; dt < DP / 16; ++dt) dkT[dt] = dvT[dt] = f4_t{0.f, 0.f, 0.f, 0.f};
  // first query that sees key k0 under the causal mask: q + coff >= k0
  const int qstart = causal ? max(0, (k0 - coff) / kT * kT) : 0;
  for (int gi = 0; gi < groups; ++gi) {
    const int hq = hk * groups + gi;
    const float* Qb = Q + b * sqb + hq * sqh;
    const float* dOb = dO + ((int64_t)b * Hq + hq) * Sq * D;
    const float* lrow = lse2 + ((int64_t)b * Hq + hq) * sqp;
    const float* drow = delta + ((int64_t)b * Hq + hq) * sqp;
    for (int q0 = qstart; q0 < Sq; q0 += kT) {
      stage_tile<DP>(Qs, Qb, sqs, q0, Sq, D);
      stage_tile<DP>(dOs, dOb, D, q0, Sq, D);
      if (threadIdx.x < kT) {
        ls[threadIdx.x] = lrow[q0 + threadIdx.x];  // rows past Sq read the zero tail
        dl[threadIdx.x] = drow[q0 + threadIdx.x];
      }
      __syncthreads();
      f4_t p[4], dp[4];
      tile_rows_times<DP>(p, Qs, kr, lane);   // S[query 16 t + 4 g + r][key li]
      tile_rows_times<DP>(dp, dOs, vr, lane);  // dP, same layout
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int qr = 16 * t + 4 * g + r, q = q0 + qr;
          const bool ok = q < Sq && key < Sk && (!causal || key <= q + coff);
          const float pv = ok ? ex2(p[t][r] * scale_log2 - ls[qr]) : 0.f;
          p[t][r] = pv;
          dp[t][r] = pv * (dp[t][r] - dl[qr]);
        }
      tileT_times<DP>(dvT, dOs, p, lane);   // dV^T[d][key] += dO^T P
      tileT_times<DP>(dkT, Qs, dp, lane);   // dK^T[d][key] += Q^T dS
      __syncthreads();
    }
  }
  if (key < Sk) {
    float* dkr = dK + (((int64_t)b * Hkv + hk) * Sk + key) * D;
    float* dvr = dV + (((int64_t)b * Hkv + hk) * Sk + key) * D;
#pragma unroll
    for (int dt = 0; dt < DP / 16; ++dt) {
      const int d = 16 * dt + 4 * g;
      if (d < D) {
        *reinterpret_cast<f4_t*>(dkr + d) = dkT[dt] * scale;
        *reinterpret_cast<f4_t*>(dvr + d) = dvT[dt];
      }
    }
  }
}

// dQ for 64 queries of one (b, q-head); wave w owns queries 16 w .. 16 w + 15 (lane: query
// l % 16), its Q and dO rows in registers. Per visible 64-key tile: S^T = K Q^T and
// dP^T = V dO^T, P^T = exp2(S^T scale_log2 - lse2), dS^T = P^T (dP^T - Delta),
// dQ^T += K^T dS^T.
template <int DP>
__global__ __launch_bounds__(256) void fa32_bwd_dq_kernel(
    const float* __restrict__ Q, int64_t sqb, int64_t sqh, int64_t sqs, const float* __restrict__ K, int64_t skb,
    int64_t skh, int64_t sks, const float* __restrict__ V, int64_t svb, int64_t svh, int64_t svs,
    const float* __restrict__ dO, const float* __restrict__ lse2, const float* __restrict__ delta, int64_t sqp,
    float* __restrict__ dQ, int Hq, int groups, int Sq, int Sk, int D, float scale_log2, float scale, int causal,
    int coff) {
  constexpr int LD = DP + 4;
  __shared__ __attribute__((aligned(16))) float Ks[kT * LD];
  __shared__ __attribute__((aligned(16))) float Vs[kT * LD];
  const int bh = blockIdx.y, b = bh / Hq, hq = bh % Hq, hk = hq / groups;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
  const int q0 = blockIdx.x * kT, qi = q0 + 16 * w + li;
  float qr[DP / 4], dor[DP / 4];
  load_row<DP>(qr, Q + b * sqb + hq * sqh + (int64_t)qi * sqs, qi < Sq, g, D);
  load_row<DP>(dor, dO + (((int64_t)b * Hq + hq) * Sq + qi) * D, qi < Sq, g, D);
  const int64_t prow = ((int64_t)b * Hq + hq) * sqp + qi;  // padded rows: qi < sqp always
  const float lq = lse2[prow], dq_delta = delta[prow];
  const float* Kb = K + b * skb + hk * skh;
  const float* Vb = V + b * svb + hk * svh;
  f4_t dqT[DP / 16];
#pragma unroll
  for (int dt = 0; dt < DP / 16; ++dt) dqT[dt] = f4_t{0.f, 0.f, 0.f, 0.f};
  int kend = Sk;
  if (causal) kend = min(Sk, max(0, q0 + kT - 1 + coff + 1));
  for (int kv0 = 0; kv0 < kend; kv0 += kT) {
    stage_tile<DP>(Ks, Kb, sks, kv0, Sk, D);
    stage_tile<DP>(Vs, Vb, svs, kv0, Sk, D);
    __syncthreads();
    f4_t s[4], dp[4];
    tile_rows_times<DP>(s, Ks, qr, lane);    // S^T[key 16 t + 4 g + r][query li]
    tile_rows_times<DP>(dp, Vs, dor, lane);  // dP^T, same layout
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kv0 + 16 * t + 4 * g + r;
        const bool ok = qi < Sq && key < Sk && (!causal || key <= qi + coff);
        const float pv = ok ? ex2(s[t][r] * scale_log2 - lq) : 0.f;
        s[t][r] = pv * (dp[t][r] - dq_delta);
      }
    tileT_times<DP>(dqT, Ks, s, lane);  // dQ^T[d][query] += K^T dS^T
    __syncthreads();
  }
  if (qi < Sq) {
    float* dqr = dQ + (((int64_t)b * Hq + hq) * Sq + qi) * D;
#pragma unroll
    for (int dt = 0; dt < DP / 16; ++dt) {
      const int d = 16 * dt + 4 * g;
      if (d < D) *reinterpret_cast<f4_t*>(dqr + d) = dqT[dt] * scale;
    }
  }
}

int pick_dp32(int64_t D) { return D <= 32 ? 32 : (D <= 64 ? 64 : (D <= 128 ? 128 : 0)); }

}  // namespace

// Called by qh_flash_fwd / qh_flash_bwd (qh_attention.hip) for dtype QH_F32, after
// their shape checks; same arguments.
int qh_flash_fwd_f32(const float* q, int64_t sqb, int64_t sqh, int64_t sqs, const float* k, int64_t skb, int64_t skh,
                     int64_t sks, const float* v, int64_t svb, int64_t svh, int64_t svs, float* o, int64_t sob,
                     int64_t soh, int64_t sos, float* lse, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk,
                     int64_t D, float scale, int causal, int64_t coff, hipStream_t st) {
  const int dp = pick_dp32(D);
  dim3 grid((unsigned)ceil_div(Sq, kT), (unsigned)(B * Hq));
  const float sl2 = scale * kLog2eF;
  const int groups = (int)(Hq / Hkv);
#define QH_F32F(DPV)                                                                                              \
  fa32_fwd_kernel<DPV><<<grid, 256, 0, st>>>(q, sqb, sqh, sqs, k, skb, skh, sks, v, svb, svh, svs, o, sob, soh, sos, \
                                             lse, (int)Hq, groups, (int)Sq, (int)Sk, (int)D, sl2, causal, (int)coff)
  if (dp == 32) QH_F32F(32); else if (dp == 64) QH_F32F(64); else QH_F32F(128);
#undef QH_F32F
  return QH_OK;
}

int qh_flash_bwd_f32(const float* q, int64_t sqb, int64_t sqh, int64_t sqs, const float* k, int64_t skb, int64_t skh,
                     int64_t sks, const float* v, int64_t svb, int64_t svh, int64_t svs, const float* o,
                     const float* dout, const float* lse, float* dq, float* dk, float* dv, float* delta, float* lse2,
                     int64_t sqp, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D, float scale,
                     int causal, int64_t coff, hipStream_t st) {
  const int dp = pick_dp32(D);
  const int64_t rows = B * Hq * sqp;
  const float sl2 = scale * kLog2eF;
  const int groups = (int)(Hq / Hkv);
  fa32_bwd_prep_kernel<<<(unsigned)ceil_div(rows, 16), 256, 0, st>>>(o, dout, lse, delta, lse2, rows, (int)Sq, sqp,
                                                                     (int)D);
  dim3 gkv((unsigned)ceil_div(Sk, kT), (unsigned)(B * Hkv));
  dim3 gq((unsigned)ceil_div(Sq, kT), (unsigned)(B * Hq));
#define QH_F32B(DPV)                                                                                               \
  do {                                                                                                             \
    if (Sk > 0)                                                                                                    \
      fa32_bwd_dkdv_kernel<DPV><<<gkv, 256, 0, st>>>(q, sqb, sqh, sqs, k, skb, skh, sks, v, svb, svh, svs, dout,    \
                                                     lse2, delta, sqp, dk, dv, (int)Hq, (int)Hkv, groups, (int)Sq, \
                                                     (int)Sk, (int)D, sl2, scale, causal, (int)coff);              \
    fa32_bwd_dq_kernel<DPV><<<gq, 256, 0, st>>>(q, sqb, sqh, sqs, k, skb, skh, sks, v, svb, svh, svs, dout, lse2,   \
                                                delta, sqp, dq, (int)Hq, groups, (int)Sq, (int)Sk, (int)D, sl2,     \
                                                scale, causal, (int)coff);                                         \
  } while (0)
  if (dp == 32) QH_F32B(32); else if (dp == 64) QH_F32B(64); else QH_F32B(128);
#undef QH_F32B
  return QH_OK;
}
