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
// token are in-lane sums plus an xor tree over the four row groups. The next token's q, k, v, g
// and beta are loaded while the current token updates the state. The state is read and written
// once per launch.
#include "qh_common.h"

namespace {

constexpr int kGdrCols = 64;  // value columns per workgroup

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

  float qn[KPL], kn[KPL], vn = 0.f, gn = 0.f, betan = 0.f;
  auto load = [&](int t) {
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const bool ok = k0 + i < K;
      // q * scale rounded to T, as the reference scales the query tensor before the recurrence
      qn[i] = ok ? to_f32(from_f32<T>(to_f32(qb[(int64_t)t * sqs + k0 + i]) * scale)) : 0.f;
      kn[i] = ok ? to_f32(kb[(int64_t)t * sqs + k0 + i]) : 0.f;
    }
    vn = cok ? to_f32(vbp[(int64_t)t * svs + col]) : 0.f;
    gn = gb[(int64_t)t * sgs];
    betan = bb[(int64_t)t * sgs];
  };
  if (S > 0) load(0);
  for (int t = 0; t < S; ++t) {
    float q[KPL], k[KPL];
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      q[i] = qn[i];
      k[i] = kn[i];
    }
    const float v = vn, decay = __expf(gn), beta = betan;
    if (t + 1 < S) load(t + 1);
    float kv = 0.f;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      st[i] *= decay;
      kv += st[i] * k[i];
    }
    kv += __shfl_xor(kv, 16);
    kv += __shfl_xor(kv, 32);
    const float d = (v - kv) * beta;
    float o = 0.f;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      st[i] += k[i] * d;
      o += st[i] * q[i];
    }
    o += __shfl_xor(o, 16);
    o += __shfl_xor(o, 32);
    if (kg == 0 && cok) ob[(int64_t)t * sos + col] = from_f32<T>(o);
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
