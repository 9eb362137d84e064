// Gated delta rule (Qwen3-Next / Qwen3.5 linear attention) over whole sequences, one launch.
//
// Per (sequence b, head h) the fp32 state S [K, Vd] evolves token by token:
//   S   = S * exp(g_t)
//   kv  = S^T k_t                 (the state's prediction of v_t)
//   d   = (v_t - kv) * beta_t
//   S   = S + k_t d^T
//   o_t = S^T (q_t * scale)        (q_t * scale rounded to the input dtype, as the reference does)
// The reference launches one kernel per token (qwen_triton/kernels/linear_attention.py:54-101,
// driven by the Python loop of :130-189), reloading and storing the state each time. Here a
// workgroup owns one (b, h, 64-column value block) for the whole sequence and keeps its slice of
// S in registers: wave w takes value columns 16 w .. 16 w + 15, and lane (kg, vi) = (lane / 16,
// lane % 16) holds rows kg * KPL .. kg * KPL + KPL - 1 of column vi, so the two K reductions of a
// token are in-lane sums plus an xor tree over the four row groups. The inputs of kGdrChunk
// tokens at a time (q, k, this block's v columns, g, beta) are loaded by the whole workgroup with
// coalesced loads into registers while the previous chunk's tokens are processed, then written
// (q and k widened to fp32) to the other half of a double-buffered LDS stage (one barrier per chunk): a token's loads are
// requested a chunk ahead rather than one token ahead, so their latency (far longer than a
// token's arithmetic) is not waited for per token, and each lane reads its rows from LDS as
// broadcasts. The state is read and written once per launch.
#include "qh_common.h"

namespace {

constexpr int kGdrCols = 64;   // value columns per workgroup
constexpr int kGdrChunk = 32;  // tokens per LDS stage
constexpr int kGdrKMax = 128;  // key head dim the stage rows hold

// x[l] + x[l ^ 16] and x[l] + x[l ^ 32] in registers (v_permlane16/32_swap with x in both operands
// hand each lane the pair in a fixed order; the sum is the same on both lanes of a pair), instead of
// LDS permutes, whose latency sits on every token's dependent chain.
__device__ __forceinline__ float pair16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <typename T, int KPL>
__global__ __launch_bounds__(256) void gdr_kernel(const T* __restrict__ Q, const T* __restrict__ Kt,
                                                  const T* __restrict__ Vt, int64_t sqb, int64_t sqs, int64_t sqh,
                                                  int64_t svb, int64_t svs, int64_t svh, const float* __restrict__ G,
                                                  const float* __restrict__ Beta, int64_t sgb, int64_t sgs,
                                                  int64_t sgh, const float* __restrict__ state_in,
                                                  float* __restrict__ state_out, T* __restrict__ O, int64_t sob,
                                                  int64_t sos, int64_t soh, int S, int H, int K, int Vd,
                                                  float scale) {
  const int vblocks = (Vd + kGdrCols - 1) / kGdrCols;
  const int bh = blockIdx.x / vblocks, vb = blockIdx.x % vblocks;
  const int b = bh / H, h = bh % H;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int kg = lane >> 4, vi = lane & 15;
  const int col = vb * kGdrCols + w * 16 + vi;
  const bool cok = col < Vd;
  const int k0 = kg * KPL;

  float st[KPL];
  const float* sin_ = state_in ? state_in + ((int64_t)bh * K) * Vd : nullptr;
#pragma unroll
  for (int i = 0; i < KPL; ++i) st[i] = (sin_ && cok && k0 + i < K) ? sin_[(int64_t)(k0 + i) * Vd + col] : 0.f;

  const T* qb = Q + (int64_t)b * sqb + (int64_t)h * sqh;
  const T* kb = Kt + (int64_t)b * sqb + (int64_t)h * sqh;
  const T* vbp = Vt + (int64_t)b * svb + (int64_t)h * svh;
  const float* gb = G + (int64_t)b * sgb + (int64_t)h * sgh;
  const float* bb = Beta + (int64_t)b * sgb + (int64_t)h * sgh;
  T* ob = O + (int64_t)b * sob + (int64_t)h * soh;

  // Chunk staging: thread tid loads q/k elements tid + 256 j of the chunk's [C, K] rows, v
  // elements tid + 256 j of its [C, 64] block, and (tid < C) g / (64 <= tid < 64 + C) beta.
  constexpr int C = kGdrChunk, NQK = C * kGdrKMax / 256, NV = C * kGdrCols / 256;
  // q and k staged as fp32 (q already scaled and rounded to T), so a token's rows need no conversion
  __shared__ float qs[2][C][kGdrKMax], ks[2][C][kGdrKMax];
  __shared__ T vs[2][C][kGdrCols];
  __shared__ float gs[2][C], bs[2][C];
  const int tid = threadIdx.x;
  T rq[NQK], rk[NQK], rv[NV];
  float rg = 0.f;
  auto stage_load = [&](int t0) {
#pragma unroll
    for (int j = 0; j < NQK; ++j) {
      const int e = tid + 256 * j, tt = e / K, d = e - tt * K;
      const bool ok = tt < C && t0 + tt < S;
      rq[j] = ok ? qb[(int64_t)(t0 + tt) * sqs + d] : (T)0.f;
      rk[j] = ok ? kb[(int64_t)(t0 + tt) * sqs + d] : (T)0.f;
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int e = tid + 256 * j, tt = e / kGdrCols, c = e - tt * kGdrCols, gc = vb * kGdrCols + c;
      rv[j] = (t0 + tt < S && gc < Vd) ? vbp[(int64_t)(t0 + tt) * svs + gc] : (T)0.f;
    }
    if (tid < C) rg = t0 + tid < S ? gb[(int64_t)(t0 + tid) * sgs] : 0.f;
    else if (tid >= 64 && tid < 64 + C) rg = t0 + tid - 64 < S ? bb[(int64_t)(t0 + tid - 64) * sgs] : 0.f;
  };
  auto stage_store = [&](int buf) {
#pragma unroll
    for (int j = 0; j < NQK; ++j) {
      const int e = tid + 256 * j, tt = e / K, d = e - tt * K;
      if (tt < C) {
        // q * scale rounded to T, as the reference scales the query tensor before the recurrence
        qs[buf][tt][d] = to_f32(from_f32<T>(to_f32(rq[j]) * scale));
        ks[buf][tt][d] = to_f32(rk[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int e = tid + 256 * j, tt = e / kGdrCols, c = e - tt * kGdrCols;
      vs[buf][tt][c] = rv[j];
    }
    if (tid < C) gs[buf][tid] = rg;
    else if (tid >= 64 && tid < 64 + C) bs[buf][tid - 64] = rg;
  };
  // Stage rows hold kGdrKMax entries; those at or past K are never staged: zero them once, so the
  // token loop reads every row entry a lane owns (k0 + i < 4 KPL <= kGdrKMax) without a guard (a
  // zero q/k entry meets a zero state row, as a masked one would).
  for (int e = tid; e < 2 * C * (kGdrKMax - K); e += 256) {
    const int bufz = e / (C * (kGdrKMax - K)), r = e % (C * (kGdrKMax - K));
    const int tt = r / (kGdrKMax - K), d = K + r % (kGdrKMax - K);
    qs[bufz][tt][d] = 0.f;
    ks[bufz][tt][d] = 0.f;
  }
  if (S > 0) {
    stage_load(0);
    stage_store(0);
  }
  __syncthreads();
  for (int t0 = 0; t0 < S; t0 += C) {
    const int buf = (t0 / C) & 1;
    const bool more = t0 + C < S;
    if (more) stage_load(t0 + C);  // in flight while this chunk's tokens run
    const int nt = S - t0 < C ? S - t0 : C;
    for (int tt = 0; tt < nt; ++tt) {
      float q[KPL], k[KPL];
#pragma unroll
      for (int i = 0; i < KPL; ++i) {  // unguarded: every entry is staged or zero
        q[i] = qs[buf][tt][k0 + i];
        k[i] = ks[buf][tt][k0 + i];
      }
      const float v = to_f32(vs[buf][tt][w * 16 + vi]);  // columns past Vd are staged as zero
      const float decay = __expf(gs[buf][tt]), beta = bs[buf][tt];
      float kv = 0.f;
#pragma unroll
      for (int i = 0; i < KPL; ++i) {
        st[i] *= decay;
        kv += st[i] * k[i];
      }
      kv = pair32_sum(pair16_sum(kv));
      const float d = (v - kv) * beta;
      float o = 0.f;
#pragma unroll
      for (int i = 0; i < KPL; ++i) {
        st[i] += k[i] * d;
        o += st[i] * q[i];
      }
      o = pair32_sum(pair16_sum(o));
      if (kg == 0 && cok) ob[(int64_t)(t0 + tt) * sos + col] = from_f32<T>(o);
    }
    if (more) stage_store(buf ^ 1);  // the other stage held the previous chunk, read by all before the last barrier
    __syncthreads();
  }
  if (state_out && cok) {
    float* so = state_out + ((int64_t)bh * K) * Vd;
#pragma unroll
    for (int i = 0; i < KPL; ++i)
      if (k0 + i < K) so[(int64_t)(k0 + i) * Vd + col] = st[i];
  }
}

}  // namespace

extern "C" int qh_gated_delta_rule(const void* q, const void* k, int64_t sqb, int64_t sqs, int64_t sqh, const void* v,
                                   int64_t svb, int64_t svs, int64_t svh, const float* g, const float* beta,
                                   int64_t sgb, int64_t sgs, int64_t sgh, const float* state_in, float* state_out,
                                   void* out, int64_t sob, int64_t sos, int64_t soh, int64_t B, int64_t S, int64_t H,
                                   int64_t K, int64_t Vd, float scale, int dtype, void* stream) {
  QH_CHECK_ARG(B >= 0 && S >= 0 && H > 0 && K > 0 && Vd > 0, "qh_gated_delta_rule: bad shape");
  QH_CHECK_ARG(K <= 128, "qh_gated_delta_rule: key head dim %lld > 128", (long long)K);
  QH_CHECK_ARG(B * H * ((Vd + kGdrCols - 1) / kGdrCols) < (1ll << 31) && S < (1ll << 31),
               "qh_gated_delta_rule: too large");
  if (B == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const unsigned grid = (unsigned)(B * H * ((Vd + kGdrCols - 1) / kGdrCols));
  const int kpl = (int)((K + 3) / 4);
#define QH_GDR(TT, KP)                                                                                           \
  gdr_kernel<TT, KP><<<grid, 256, 0, st>>>((const TT*)q, (const TT*)k, (const TT*)v, sqb, sqs, sqh, svb, svs, svh, \
                                           g, beta, sgb, sgs, sgh, state_in, state_out, (TT*)out, sob, sos, soh,  \
                                           (int)S, (int)H, (int)K, (int)Vd, scale)
#define QH_GDR_K(TT) \
  if (kpl <= 4) QH_GDR(TT, 4); else if (kpl <= 8) QH_GDR(TT, 8); else if (kpl <= 16) QH_GDR(TT, 16); \
  else QH_GDR(TT, 32);
  switch (dtype) {
    case QH_BF16: QH_GDR_K(bf16_t) break;
    case QH_F16: QH_GDR_K(f16_t) break;
    case QH_F32: QH_GDR_K(float) break;
    default: qh::set_error("qh_gated_delta_rule: unsupported dtype %d", dtype); return QH_E_DTYPE;
  }
#undef QH_GDR_K
#undef QH_GDR
  QH_CHECK_LAUNCH("qh_gated_delta_rule");
  return QH_OK;
}
