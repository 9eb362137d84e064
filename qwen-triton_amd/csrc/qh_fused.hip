// Fused passes for the inference path of the attention block and the decoder
// layer. Each replaces a chain of the single-op kernels with one launch and
// one pass over the data, with the same per-element arithmetic and rounding
// points as that chain (so results match it exactly).
#include "qh_prep.h"

namespace {

// Attention input preparation, one 16-lane group per (token, head) row of D
// (<= 128) elements, 8 per lane:
//   q, k rows: RMSNorm over D (rounded to T, as the norm kernel), then
//              rotate-half RoPE with cos/sin[.., :rot/2] (rounded to T);
//              q goes to q_out [B, Hq, S, D], k into its cache at pos[s];
//   v rows:    copied into the value cache at pos[s].
// The lane layout and the DPP reduction are those of the 16-lane RMSNorm
// kernel and the RoPE expressions are those of the RoPE kernel.
// VEC (16-bit cos/sin, 16-byte aligned norm weights and cos/sin rows): every
// load of a row (the row, its norm weights, cos/sin, the position) is issued
// before the first use, with no branch in between (load_row_raw), and the row
// type decides only afterwards what is computed and stored. Same values.
template <typename T, typename C, bool VEC = false>
__global__ __launch_bounds__(256) void attn_prepare_kernel(
    const T* __restrict__ q, int64_t sq, const T* __restrict__ k, int64_t sk, const T* __restrict__ v, int64_t sv,
    const void* __restrict__ qw, const void* __restrict__ kw, int wdtype, float eps, float wadd,
    const C* __restrict__ cs, const C* __restrict__ sn, int64_t scb, int64_t scs, int64_t cos_batch, int half,
    int rot, T* __restrict__ q_out, T* __restrict__ kc, int64_t kcb, int64_t kch, int64_t kcs, T* __restrict__ vc,
    int64_t vcb, int64_t vch, int64_t vcs, const int64_t* __restrict__ pos, int S, int Hq, int Hkv, int D,
    int64_t cap, int64_t rows) {
  const int grp = threadIdx.x >> 4, g = threadIdx.x & 15;
  const int HT = Hq + 2 * Hkv;
  const int d0 = g * 8;
  const bool act = d0 < D;
  const int hl = half / 8;  // lane distance between the two rotated halves
  for (int64_t row = blockIdx.x * 16ll + grp; row < rows; row += (int64_t)gridDim.x * 16) {
    const int64_t t = row / HT;
    const int j = (int)(row - t * HT);
    const int64_t b = t / S;
    const int s = (int)(t - b * S);
    if constexpr (VEC) {
      const bool isq = j < Hq, isv = j >= Hq + Hkv;
      const int h = isq ? j : (isv ? j - Hq - Hkv : j - Hq);
      const T* src = isq ? q + t * sq : (isv ? v + t * sv : k + t * sk);
      Vec16<T> xv = ld16(src + h * D + (act ? d0 : 0));
      const RowRaw rr = load_row_raw<C>(isq ? qw : kw, wdtype, d0, act, half, rot, cs, sn,
                                        (cos_batch == 1 ? 0 : b) * scb + s * scs);
      const int64_t p = pos[s];
      if (!act) xv.raw = make_uint4(0, 0, 0, 0);
      if (isv) {
        if (act && p >= 0 && p < cap) st16(vc + b * vcb + h * vch + p * vcs + d0, xv);
        continue;
      }
      const RowParams rp = row_params_from<C>(rr, wdtype, wadd, d0, act, rot);
      const Vec16<T> o = norm_rope_apply<T>(xv, act, rp, eps, D, d0, hl, half, rot);
      if (!act) continue;
      if (isq) st16(q_out + ((b * Hq + h) * (int64_t)S + s) * D + d0, o);
      else if (p >= 0 && p < cap) st16(kc + b * kcb + h * kch + p * kcs + d0, o);
      continue;
    }
    const int64_t p = pos[s];
    Vec16<T> xv;
    xv.raw = make_uint4(0, 0, 0, 0);
    if (j >= Hq + Hkv) {  // value row: copy into the cache
      const int h = j - Hq - Hkv;
      if (act) xv = ld16(v + t * sv + h * D + d0);
      if (act && p >= 0 && p < cap) st16(vc + b * vcb + h * vch + p * vcs + d0, xv);
      continue;
    }
    const bool isq = j < Hq;
    const int h = isq ? j : j - Hq;
    if (act) xv = ld16(isq ? q + t * sq + h * D + d0 : k + t * sk + h * D + d0);
    const Vec16<T> o = norm_rope_row<T, C>(xv, act, isq ? qw : kw, wdtype, eps, wadd, D, d0, hl, half, rot, cs, sn,
                                           (cos_batch == 1 ? 0 : b) * scb + s * scs);
    if (!act) continue;
    if (isq) st16(q_out + ((b * Hq + h) * (int64_t)S + s) * D + d0, o);
    else if (p >= 0 && p < cap) st16(kc + b * kcb + h * kch + p * kcs + d0, o);
  }
}

// Launch of attn_prepare_kernel, the vector form where it applies (16-bit cos/sin).
template <typename T, typename C>
void launch_attn_prepare(bool vec, unsigned grid, hipStream_t st, const T* q, int64_t sq, const T* k, int64_t sk,
                         const T* v, int64_t sv, const void* qw, const void* kw, int wdtype, float eps, float wadd,
                         const C* cs, const C* sn, int64_t scb, int64_t scs, int64_t cos_batch, int half, int rot,
                         T* q_out, T* kc, int64_t kcb, int64_t kch, int64_t kcs, T* vc, int64_t vcb, int64_t vch,
                         int64_t vcs, const int64_t* pos, int S, int Hq, int Hkv, int D, int64_t cap, int64_t rows) {
  if constexpr (sizeof(C) == 2) {
    if (vec) {
      attn_prepare_kernel<T, C, true><<<grid, 256, 0, st>>>(q, sq, k, sk, v, sv, qw, kw, wdtype, eps, wadd, cs, sn, scb,
                                                           scs, cos_batch, half, rot, q_out, kc, kcb, kch, kcs, vc,
                                                           vcb, vch, vcs, pos, S, Hq, Hkv, D, cap, rows);
      return;
    }
  }
  attn_prepare_kernel<T, C, false><<<grid, 256, 0, st>>>(q, sq, k, sk, v, sv, qw, kw, wdtype, eps, wadd, cs, sn, scb, scs,
                                                        cos_batch, half, rot, q_out, kc, kcb, kch, kcs, vc, vcb, vch,
                                                        vcs, pos, S, Hq, Hkv, D, cap, rows);
}

}  // namespace

extern "C" int qh_attn_prepare(const void* q, int64_t sq, const void* k, int64_t sk, const void* v, int64_t sv,
                               const void* qw, const void* kw, float eps, int one_plus, const void* cos,
                               const void* sin, int64_t scb, int64_t scs, int64_t cos_batch, int64_t rot,
                               void* q_out, void* k_cache, int64_t kcb, int64_t kch, int64_t kcs, void* v_cache,
                               int64_t vcb, int64_t vch, int64_t vcs, const int64_t* positions, int64_t B,
                               int64_t S, int64_t Hq, int64_t Hkv, int64_t D, int64_t cap, int dtype, int wdtype,
                               int cdtype, void* stream) {
  QH_CHECK_ARG(B >= 0 && S >= 0 && Hq > 0 && Hkv > 0 && cap >= 0, "qh_attn_prepare: bad shape");
  QH_CHECK_ARG(D > 0 && D <= 128 && D % 8 == 0, "qh_attn_prepare: head dim %lld must be a multiple of 8 and <= 128",
               (long long)D);
  const int64_t half = rot / 2;
  QH_CHECK_ARG(rot >= 16 && rot <= D && rot % 16 == 0 && ((half / 8) & (half / 8 - 1)) == 0,
               "qh_attn_prepare: rotary dim %lld must be 16 * 2^k <= D", (long long)rot);
  QH_CHECK_ARG(cos_batch == 1 || cos_batch == B, "qh_attn_prepare: cos/sin batch must be 1 or B");
  QH_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(q_out) && aligned16(k_cache) &&
                   aligned16(v_cache),
               "qh_attn_prepare: pointers must be 16-byte aligned");
  QH_CHECK_ARG(sq % 8 == 0 && sk % 8 == 0 && sv % 8 == 0 && kcb % 8 == 0 && kch % 8 == 0 && kcs % 8 == 0 &&
                   vcb % 8 == 0 && vch % 8 == 0 && vcs % 8 == 0,
               "qh_attn_prepare: strides must be multiples of 8 elements");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_attn_prepare: bf16/f16 only");
  QH_CHECK_ARG(wdtype == QH_F32 || wdtype == dtype, "qh_attn_prepare: norm weights must be fp32 or the input dtype");
  QH_CHECK_ARG(cdtype == QH_F32 || cdtype == dtype, "qh_attn_prepare: cos/sin must be fp32 or the input dtype");
  const int64_t rows = B * S * (Hq + 2 * Hkv);
  if (rows == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const float wadd = one_plus ? 1.f : 0.f;
  const int64_t nblk = (rows + 15) / 16;
  const unsigned grid = (unsigned)(nblk < 65536 ? nblk : 65536);
  const bool vec = cdtype != QH_F32 && aligned16(qw) && aligned16(kw) && aligned16(cos) && aligned16(sin) &&
                   scb % 8 == 0 && scs % 8 == 0;
#define QH_PREP(T, C)                                                                                            \
  launch_attn_prepare<T, C>(vec, grid, st, (const T*)q, sq, (const T*)k, sk, (const T*)v, sv, qw, kw, wdtype, eps, \
                            wadd, (const C*)cos, (const C*)sin, scb, scs, cos_batch, (int)half, (int)rot, (T*)q_out, \
                            (T*)k_cache, kcb, kch, kcs, (T*)v_cache, vcb, vch, vcs, positions, (int)S, (int)Hq,    \
                            (int)Hkv, (int)D, cap, rows)
  if (dtype == QH_BF16) {
    if (cdtype == QH_F32) {
      QH_PREP(bf16_t, float);
    } else {
      QH_PREP(bf16_t, bf16_t);
    }
  } else {
    if (cdtype == QH_F32) {
      QH_PREP(f16_t, float);
    } else {
      QH_PREP(f16_t, f16_t);
    }
  }
#undef QH_PREP
  QH_CHECK_LAUNCH("qh_attn_prepare");
  return QH_OK;
}
