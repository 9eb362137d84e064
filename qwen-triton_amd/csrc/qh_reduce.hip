// Row-reduction operators: RMSNorm (fwd/bwd), softmax (fwd/bwd), cross-entropy
// (fwd/bwd), top-k and one-hot.
//
// Row kernels map a row onto a group of G lanes (G in {8,16,32,64}) that each
// keep NV 16-byte vectors of the row in registers, so a row is read from HBM
// exactly once and reductions are register + DPP shuffles only. Rows that do
// not fit that shape take a one-block-per-row path. Every reduction uses a fixed
// order, so results are bitwise reproducible run to run (no float atomics).
#include "qh_common.h"

namespace {

static int grid_cap(int64_t work, int64_t cap = 8192) {
  if (work < 1) return 1;
  return (int)(work < cap ? work : cap);
}

// Pick a (lanes-per-row G, vectors-per-lane NV) shape for a row of `cols`
// elements of a type with VN elements per 16 bytes. 0 = no fast path.
static int pick_row_shape(int64_t cols, int VN, int& G, int& NV) {
  if (cols <= 0 || cols % VN) return 0;
  const int64_t nv = cols / VN;
  if (nv <= 8) { G = 8; NV = 1; }
  else if (nv <= 16) { G = 16; NV = 1; }
  else if (nv <= 32) { G = 32; NV = 1; }
  else if (nv <= 64) { G = 64; NV = 1; }
  else if (nv <= 128) { G = 64; NV = 2; }
  else if (nv <= 256) { G = 64; NV = 4; }
  else if (nv <= 512) { G = 64; NV = 8; }
  else return 0;
  return 1;
}



// ===========================================================================
// RMSNorm
// ===========================================================================
// Per-lane scale (w + wadd) of the columns a lane owns in the (G, NV) row
// shape, loaded once per workgroup; columns past the row end get 0.
template <int VN, int NV, int G>
__device__ __forceinline__ void load_row_scale(const void* w, int wdtype, int cols, int g, float wadd,
                                               float (&sw)[NV][VN]) {
  const bool al16 = (reinterpret_cast<uintptr_t>(w) & 15) == 0;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * G + g) * VN;
    if (c < cols) {
      load_any_vec<VN>(w, wdtype, c, al16, sw[i]);
#pragma unroll
      for (int j = 0; j < VN; ++j) sw[i][j] += wadd;
    } else {
#pragma unroll
      for (int j = 0; j < VN; ++j) sw[i][j] = 0.f;
    }
  }
}

template <typename T, int G, int NV>
__global__ __launch_bounds__(256) void rmsnorm_fwd_fast(const T* __restrict__ x, const void* __restrict__ w,
                                                        int wdtype, T* __restrict__ y, int64_t rows, int cols,
                                                        float eps, float wadd) {
  constexpr int VN = Vec16<T>::N;
  constexpr int RPB = 256 / G;
  const int grp = threadIdx.x / G, g = threadIdx.x % G;
  float sw[NV][VN];
  load_row_scale<VN, NV, G>(w, wdtype, cols, g, wadd, sw);
  for (int64_t row = blockIdx.x * (int64_t)RPB + grp; row < rows; row += (int64_t)gridDim.x * RPB) {
    const T* xr = x + row * cols;
    Vec16<T> xv[NV];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * G + g) * VN;
      if (c < cols) {
        xv[i] = ld16(xr + c);
#pragma unroll
        for (int j = 0; j < VN; ++j) {
          const float f = to_f32(xv[i].v[j]);
          ss += f * f;
        }
      }
    }
    ss = wave_sum(ss, G);
    const float inv = rsqrtf(ss / (float)cols + eps);
    T* yr = y + row * cols;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * G + g) * VN;
      if (c < cols) {
        Vec16<T> o;
#pragma unroll
        for (int j = 0; j < VN; ++j) o.v[j] = from_f32<T>((to_f32(xv[i].v[j]) * inv) * sw[i][j]);
        st16(yr + c, o);
      }
    }
  }
}

// Residual add fused with RMSNorm: sum = x + r (rounded to T, as the add
// kernel), y = RMSNorm(sum) with the row shape and summation order of
// rmsnorm_fwd_fast, so both outputs equal the two separate kernels'.
template <typename T, int G, int NV>
__global__ __launch_bounds__(256) void add_rmsnorm_fast(const T* __restrict__ x, const T* __restrict__ r,
                                                        const void* __restrict__ w, int wdtype, T* __restrict__ sum,
                                                        T* __restrict__ y, int64_t rows, int cols, float eps,
                                                        float wadd) {
  constexpr int VN = Vec16<T>::N;
  constexpr int RPB = 256 / G;
  const int grp = threadIdx.x / G, g = threadIdx.x % G;
  float sw[NV][VN];
  load_row_scale<VN, NV, G>(w, wdtype, cols, g, wadd, sw);
  for (int64_t row = blockIdx.x * (int64_t)RPB + grp; row < rows; row += (int64_t)gridDim.x * RPB) {
    Vec16<T> xv[NV];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * G + g) * VN;
      if (c < cols) {
        const Vec16<T> a = ld16(x + row * cols + c), b = ld16(r + row * cols + c);
#pragma unroll
        for (int j = 0; j < VN; ++j) xv[i].v[j] = from_f32<T>(to_f32(a.v[j]) + to_f32(b.v[j]));
        st16(sum + row * cols + c, xv[i]);
#pragma unroll
        for (int j = 0; j < VN; ++j) {
          const float f = to_f32(xv[i].v[j]);
          ss += f * f;
        }
      }
    }
    ss = wave_sum(ss, G);
    const float inv = rsqrtf(ss / (float)cols + eps);
    T* yr = y + row * cols;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * G + g) * VN;
      if (c < cols) {
        Vec16<T> o;
#pragma unroll
        for (int j = 0; j < VN; ++j) o.v[j] = from_f32<T>((to_f32(xv[i].v[j]) * inv) * sw[i][j]);
        st16(yr + c, o);
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_fwd_generic(const T* __restrict__ x, const void* __restrict__ w,
                                                           int wdtype, T* __restrict__ y, int64_t rows,
                                                           int64_t cols, float eps, float wadd) {
  __shared__ float red[4];
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const T* xr = x + row * cols;
    float ss = 0.f;
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
      const float f = to_f32(xr[c]);
      ss += f * f;
    }
    ss = block_sum(ss, red);
    const float inv = rsqrtf(ss / (float)cols + eps);
    for (int64_t c = threadIdx.x; c < cols; c += 256)
      y[row * cols + c] = from_f32<T>((to_f32(xr[c]) * inv) * (load_any(w, wdtype, c) + wadd));
  }
}

// Backward, fast path. BT threads per workgroup, RPB = BT / G row groups. Each
// row group accumulates its dW partial in registers over the rows it visits;
// at the end the groups' partials are summed in LDS in group order and the
// workgroup writes one partial row ws[blockIdx.x, :].
template <typename T, int G, int NV, int BT>
__global__ __launch_bounds__(BT) void rmsnorm_bwd_fast(const T* __restrict__ x, const void* __restrict__ w,
                                                       int wdtype, const T* __restrict__ gy, T* __restrict__ gx,
                                                       float* __restrict__ ws, int64_t rows, int cols, float eps,
                                                       float wadd) {
  constexpr int VN = Vec16<T>::N;
  constexpr int RPB = BT / G;
  const int grp = threadIdx.x / G, g = threadIdx.x % G;
  float pw[NV][VN];
  float sw[NV][VN];
  load_row_scale<VN, NV, G>(w, wdtype, cols, g, wadd, sw);
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int j = 0; j < VN; ++j) pw[i][j] = 0.f;
  const float inv_cols = 1.0f / (float)cols;
  const int64_t step = (int64_t)gridDim.x * RPB;
  // With at most two vectors per lane the next row's x and dy are loaded before this row's sums
  // (clamped to the last row: every load stays in bounds, a group's surplus last loads go unused),
  // so a group waits for memory once rather than once per row. With more, the extra registers
  // cost more than the overlap gains.
  constexpr bool kAhead = NV <= 2;
  Vec16<T> xn[NV], gn[NV];
  if constexpr (kAhead) {
    const int64_t r0 = min((int64_t)blockIdx.x * RPB + grp, rows - 1);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = min((i * G + g) * VN, cols - VN);
      xn[i] = ld16(x + r0 * cols + c);
      gn[i] = ld16(gy + r0 * cols + c);
    }
  }
  for (int64_t row = blockIdx.x * (int64_t)RPB + grp; row < rows; row += step) {
    const T* xr = x + row * cols;
    const T* gr = gy + row * cols;
    Vec16<T> xv[NV], gv[NV];
    if constexpr (kAhead) {
      const int64_t rn = min(row + step, rows - 1);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        xv[i] = xn[i];
        gv[i] = gn[i];
        const int c = min((i * G + g) * VN, cols - VN);
        xn[i] = ld16(x + rn * cols + c);
        gn[i] = ld16(gy + rn * cols + c);
      }
    }
    float ss = 0.f, dot = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * G + g) * VN;
      if (c < cols) {
        if constexpr (!kAhead) {
          xv[i] = ld16(xr + c);
          gv[i] = ld16(gr + c);
        }
#pragma unroll
        for (int j = 0; j < VN; ++j) {
          const float xf = to_f32(xv[i].v[j]), gf = to_f32(gv[i].v[j]);
          ss += xf * xf;
          dot += gf * sw[i][j] * xf;
        }
      }
    }
    ss = wave_sum(ss, G);
    dot = wave_sum(dot, G);
    const float inv = rsqrtf(ss * inv_cols + eps);
    const float k3 = inv * inv * inv * inv_cols * dot;
    T* gxr = gx + row * cols;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * G + g) * VN;
      if (c < cols) {
        Vec16<T> o;
#pragma unroll
        for (int j = 0; j < VN; ++j) {
          const float xf = to_f32(xv[i].v[j]), gf = to_f32(gv[i].v[j]);
          o.v[j] = from_f32<T>(gf * sw[i][j] * inv - xf * k3);
          pw[i][j] += gf * (xf * inv);
        }
        st16(gxr + c, o);
      }
    }
  }
  // The RPB groups' partials side by side in LDS (acc[grp][cols]), then each
  // column summed over the groups in group order: the workgroup's partial row.
  extern __shared__ float acc[];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = (i * G + g) * VN;
    if (c < cols) {
#pragma unroll
      for (int j = 0; j < VN; ++j) acc[grp * cols + c + j] = pw[i][j];
    }
  }
  __syncthreads();
  float* wr = ws + (int64_t)blockIdx.x * cols;
  for (int c = threadIdx.x; c < cols; c += BT) {
    float t = acc[c];
    for (int s2 = 1; s2 < RPB; ++s2) t += acc[s2 * cols + c];
    wr[c] = t;
  }
}

// Backward, generic path: block owns ws row blockIdx.x; thread t owns columns
// t, t+256, ... of that row, so the partial needs no atomics.
template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_bwd_generic(const T* __restrict__ x, const void* __restrict__ w,
                                                           int wdtype, const T* __restrict__ gy,
                                                           T* __restrict__ gx, float* __restrict__ ws,
                                                           int64_t rows, int64_t cols, float eps, float wadd) {
  __shared__ float red[4];
  float* wr = ws + (int64_t)blockIdx.x * cols;
  for (int64_t c = threadIdx.x; c < cols; c += 256) wr[c] = 0.f;
  const float inv_cols = 1.0f / (float)cols;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const T* xr = x + row * cols;
    const T* gr = gy + row * cols;
    float ss = 0.f, dot = 0.f;
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
      const float xf = to_f32(xr[c]), gf = to_f32(gr[c]);
      ss += xf * xf;
      dot += gf * (load_any(w, wdtype, c) + wadd) * xf;
    }
    ss = block_sum(ss, red);
    dot = block_sum(dot, red);
    const float inv = rsqrtf(ss * inv_cols + eps);
    const float k3 = inv * inv * inv * inv_cols * dot;
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
      const float xf = to_f32(xr[c]), gf = to_f32(gr[c]);
      gx[row * cols + c] = from_f32<T>(gf * (load_any(w, wdtype, c) + wadd) * inv - xf * k3);
      wr[c] += gf * (xf * inv);
    }
  }
}

// Stage 2: gw[c] = sum_r ws[r, c]. A block owns 64 columns; each of its 16
// waves sums every 16th partial row with four interleaved accumulators (rows
// w, w+16, w+32, w+48 of each 64-row step), and the 16 wave sums are added in
// wave order. The order is fixed by the code, so results are deterministic.
__global__ __launch_bounds__(1024) void colsum_partials(const float* __restrict__ ws, int64_t nrows, int64_t cols,
                                                        void* __restrict__ out, int odtype) {
  __shared__ float part[16][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t c = blockIdx.x * 64 + lane;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  if (c < cols) {
    int64_t r = wv;
    // four 64-row steps' loads issued together (same order of additions as the loop below)
    for (; r + 48 + 192 < nrows; r += 256) {
      float v[4][4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int q = 0; q < 4; ++q) v[u][q] = ws[(r + 64 * u + 16 * q) * cols + c];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        a0 += v[u][0];
        a1 += v[u][1];
        a2 += v[u][2];
        a3 += v[u][3];
      }
    }
    for (; r + 48 < nrows; r += 64) {
      a0 += ws[r * cols + c];
      a1 += ws[(r + 16) * cols + c];
      a2 += ws[(r + 32) * cols + c];
      a3 += ws[(r + 48) * cols + c];
    }
    for (; r < nrows; r += 16) a0 += ws[r * cols + c];
  }
  part[wv][lane] = (a0 + a1) + (a2 + a3);
  __syncthreads();
  if (wv == 0 && c < cols) {
    float t = 0.f;
    for (int i = 0; i < 16; ++i) t += part[i][lane];
    store_any(out, odtype, c, t);
  }
}

// Workgroups of the backward row kernels (one fp32 partial row each): 1024 of
// 256 threads for the generic kernel; the fast kernel keeps the same 4096 waves
// in larger workgroups where its registers allow (fewer partial rows to sum).
static const int kRmsBwdBlocks = 1024;

// Threads per workgroup of rmsnorm_bwd_fast for NV vectors per lane: 1024 (four
// waves per SIMD, 128 registers) while the row's values fit, then 512, 256.
static int rms_bwd_threads(int NV) { return NV <= 2 ? 1024 : NV == 4 ? 512 : 256; }

// ===========================================================================
// Softmax
// ===========================================================================
template <typename T, int G, int NV>
__global__ __launch_bounds__(256) void softmax_fwd_fast(const T* __restrict__ x, T* __restrict__ y, int64_t rows,
                                                        int cols) {
  constexpr int VN = Vec16<T>::N;
  constexpr int RPB = 256 / G;
  const int grp = threadIdx.x / G, g = threadIdx.x % G;
  for (int64_t row = blockIdx.x * (int64_t)RPB + grp; row < rows; row += (int64_t)gridDim.x * RPB) {
    const T* xr = x + row * cols;
    float v[NV][VN];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * G + g) * VN;
      if (c < cols) {
        Vec16<T> t = ld16(xr + c);
#pragma unroll
        for (int j = 0; j < VN; ++j) {
          v[i][j] = to_f32(t.v[j]);
          m = fmaxf(m, v[i][j]);
        }
      }
    }
    m = wave_max(m, G);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * G + g) * VN;
      if (c < cols) {
#pragma unroll
        for (int j = 0; j < VN; ++j) {
          v[i][j] = fast_exp(v[i][j] - m);
          s += v[i][j];
        }
      }
    }
    s = wave_sum(s, G);
    const float rs = 1.0f / s;
    T* yr = y + row * cols;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * G + g) * VN;
      if (c < cols) {
        Vec16<T> o;
#pragma unroll
        for (int j = 0; j < VN; ++j) o.v[j] = from_f32<T>(v[i][j] * rs);
        st16(yr + c, o);
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_fwd_generic(const T* __restrict__ x, T* __restrict__ y,
                                                           int64_t rows, int64_t cols) {
  __shared__ float red[4];
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const T* xr = x + row * cols;
    float m = -INFINITY;
    for (int64_t c = threadIdx.x; c < cols; c += 256) m = fmaxf(m, to_f32(xr[c]));
    m = block_max(m, red);
    float s = 0.f;
    for (int64_t c = threadIdx.x; c < cols; c += 256) s += fast_exp(to_f32(xr[c]) - m);
    s = block_sum(s, red);
    const float rs = 1.0f / s;
    for (int64_t c = threadIdx.x; c < cols; c += 256) y[row * cols + c] = from_f32<T>(fast_exp(to_f32(xr[c]) - m) * rs);
  }
}

template <typename T, int G, int NV>
__global__ __launch_bounds__(256) void softmax_bwd_fast(const T* __restrict__ y, const T* __restrict__ gy,
                                                        T* __restrict__ gx, int64_t rows, int cols) {
  constexpr int VN = Vec16<T>::N;
  constexpr int RPB = 256 / G;
  const int grp = threadIdx.x / G, g = threadIdx.x % G;
  for (int64_t row = blockIdx.x * (int64_t)RPB + grp; row < rows; row += (int64_t)gridDim.x * RPB) {
    Vec16<T> yv[NV], gv[NV];
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * G + g) * VN;
      if (c < cols) {
        yv[i] = ld16(y + row * cols + c);
        gv[i] = ld16(gy + row * cols + c);
#pragma unroll
        for (int j = 0; j < VN; ++j) dot += to_f32(yv[i].v[j]) * to_f32(gv[i].v[j]);
      }
    }
    dot = wave_sum(dot, G);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = (i * G + g) * VN;
      if (c < cols) {
        Vec16<T> o;
#pragma unroll
        for (int j = 0; j < VN; ++j) o.v[j] = from_f32<T>(to_f32(yv[i].v[j]) * (to_f32(gv[i].v[j]) - dot));
        st16(gx + row * cols + c, o);
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_bwd_generic(const T* __restrict__ y, const T* __restrict__ gy,
                                                           T* __restrict__ gx, int64_t rows, int64_t cols) {
  __shared__ float red[4];
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    float dot = 0.f;
    for (int64_t c = threadIdx.x; c < cols; c += 256) dot += to_f32(y[row * cols + c]) * to_f32(gy[row * cols + c]);
    dot = block_sum(dot, red);
    for (int64_t c = threadIdx.x; c < cols; c += 256)
      gx[row * cols + c] = from_f32<T>(to_f32(y[row * cols + c]) * (to_f32(gy[row * cols + c]) - dot));
  }
}

// ===========================================================================
// Cross-entropy: one 256-thread block per row, single pass online logsumexp.
// ===========================================================================
__device__ __forceinline__ void lse_merge(float& m, float& s, float m2, float s2) {
  const float M = fmaxf(m, m2);
  if (M == -INFINITY) return;
  const float a = (m == -INFINITY) ? 0.f : s * fast_exp(m - M);
  const float b = (m2 == -INFINITY) ? 0.f : s2 * fast_exp(m2 - M);
  m = M;
  s = a + b;
}

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void ce_fwd_kernel(const T* __restrict__ logits, int64_t stride,
                                                     const int64_t* __restrict__ tgt, float* __restrict__ lse,
                                                     float* __restrict__ loss, int64_t V, int64_t ignore) {
  __shared__ float sm[4], ssum[4];
  const int64_t row = blockIdx.x;
  const int64_t t = tgt[row];
  if (t == ignore) {
    if (threadIdx.x == 0) {
      loss[row] = 0.f;
      lse[row] = 0.f;
    }
    return;
  }
  const T* xr = logits + row * stride;
  float m = -INFINITY, s = 0.f;
  if constexpr (VEC) {
    constexpr int VN = Vec16<T>::N;
    for (int64_t c = threadIdx.x * VN; c < V; c += 256 * VN) {
      Vec16<T> v = ld16_nt(xr + c);
      float lm = -INFINITY;
#pragma unroll
      for (int j = 0; j < VN; ++j) lm = fmaxf(lm, to_f32(v.v[j]));
      if (lm > m) {
        s = (m == -INFINITY) ? 0.f : s * fast_exp(m - lm);
        m = lm;
      }
      if (m != -INFINITY) {
#pragma unroll
        for (int j = 0; j < VN; ++j) s += fast_exp(to_f32(v.v[j]) - m);
      }
    }
  } else {
    for (int64_t c = threadIdx.x; c < V; c += 256) {
      const float f = to_f32(xr[c]);
      if (f > m) {
        s = (m == -INFINITY) ? 0.f : s * fast_exp(m - f);
        m = f;
      }
      if (m != -INFINITY) s += fast_exp(f - m);
    }
  }
  // wave merge (fixed xor tree), then block merge in wave order
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(s, o);
    lse_merge(m, s, m2, s2);
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) {
    sm[wid] = m;
    ssum[wid] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = sm[0], S = ssum[0];
    for (int i = 1; i < 4; ++i) lse_merge(M, S, sm[i], ssum[i]);
    const float l = M + __logf(S);
    const float xt = (t >= 0 && t < V) ? to_f32(xr[t]) : __int_as_float(0x7fc00000);
    lse[row] = l;
    loss[row] = l - xt;
  }
}

// loss_out = sum(loss) / max(1, n_valid); nvalid_out = n_valid.
__global__ __launch_bounds__(1024) void ce_finalize(const float* __restrict__ loss, const int64_t* __restrict__ tgt,
                                                    int64_t N, int64_t ignore, float* __restrict__ loss_out,
                                                    float* __restrict__ nvalid_out) {
  __shared__ float red[16];
  float s = 0.f, n = 0.f;
  for (int64_t i = threadIdx.x; i < N; i += 1024) {
    s += loss[i];
    n += (tgt[i] != ignore) ? 1.f : 0.f;
  }
  s = block_sum(s, red);
  n = block_sum(n, red);
  if (threadIdx.x == 0) {
    loss_out[0] = s / fmaxf(n, 1.f);
    nvalid_out[0] = n;
  }
}

// g may be logits itself (same stride): each element is read and then written by one thread.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void ce_bwd_kernel(const T* logits, int64_t stride,
                                                     const int64_t* __restrict__ tgt, const float* __restrict__ lse,
                                                     const float* __restrict__ gloss, const float* __restrict__ nvalid,
                                                     T* g, int64_t gstride, int64_t V, int64_t ignore) {
  const int64_t row = blockIdx.x;
  const int64_t t = tgt[row];
  T* gr = g + row * gstride;
  const T* xr = logits + row * stride;
  const bool ign = (t == ignore);
  const float scale = gloss[0] / fmaxf(nvalid[0], 1.f);
  const float l = lse[row];
  if constexpr (VEC) {
    constexpr int VN = Vec16<T>::N;
    for (int64_t c = threadIdx.x * VN; c < V; c += 256 * VN) {
      Vec16<T> o;
      if (ign) {
        o.raw = make_uint4(0, 0, 0, 0);
      } else {
        Vec16<T> v = ld16_nt(xr + c);
#pragma unroll
        for (int j = 0; j < VN; ++j) {
          const float p = fast_exp(to_f32(v.v[j]) - l);
          o.v[j] = from_f32<T>((p - ((c + j) == t ? 1.f : 0.f)) * scale);
        }
      }
      st16_nt(gr + c, o);
    }
  } else {
    for (int64_t c = threadIdx.x; c < V; c += 256) {
      float r = 0.f;
      if (!ign) r = (fast_exp(to_f32(xr[c]) - l) - (c == t ? 1.f : 0.f)) * scale;
      gr[c] = from_f32<T>(r);
    }
  }
}

// ===========================================================================
// Top-k: one wave per row. Selection order: larger value first, equal values
// by lower index. Round r picks the best element strictly after the (r-1)-th
// pick in that order, so the input is never modified.
// ===========================================================================
__device__ __forceinline__ bool topk_better(float v, int i, float bv, int bi) {
  return bi < 0 || v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ bool topk_after(float v, int i, float lv, int li) {
  return v < lv || (v == lv && i > li);
}

template <typename T, int CPL>
__global__ __launch_bounds__(256) void topk_kernel(const T* __restrict__ x, T* __restrict__ vals,
                                                   int64_t* __restrict__ idx, int64_t N, int C, int k) {
  const int64_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= N) return;
  const T* xr = x + row * C;
  float cv[CPL > 0 ? CPL : 1];
  if constexpr (CPL > 0) {
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = i * 64 + lane;
      cv[i] = (c < C) ? to_f32(xr[c]) : -INFINITY;
    }
  }
  float lv = INFINITY;
  int li = -1;
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY;
    int bi = -1;
    if constexpr (CPL > 0) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = i * 64 + lane;
        if (c < C && topk_after(cv[i], c, lv, li) && topk_better(cv[i], c, bv, bi)) {
          bv = cv[i];
          bi = c;
        }
      }
    } else {
      for (int c = lane; c < C; c += 64) {
        const float v = to_f32(xr[c]);
        if (topk_after(v, c, lv, li) && topk_better(v, c, bv, bi)) {
          bv = v;
          bi = c;
        }
      }
    }
    for (int o = 32; o > 0; o >>= 1) {
      const float v2 = __shfl_xor(bv, o);
      const int i2 = __shfl_xor(bi, o);
      if (i2 >= 0 && topk_better(v2, i2, bv, bi)) {
        bv = v2;
        bi = i2;
      }
    }
    if (lane == 0) {
      vals[row * k + r] = from_f32<T>(bi >= 0 ? bv : __int_as_float(0x7fc00000));
      idx[row * k + r] = bi;
    }
    lv = bv;
    li = bi;
    if (bi < 0) lv = -INFINITY, li = 0x7fffffff;
  }
}

// Rows wider than 1024 columns (e.g. an argmax over a vocabulary): one
// 1024-thread workgroup per row. Each round scans the row with 16-byte loads
// (four in flight per thread), keeps the best element strictly after the
// previous pick in (value desc, column asc) order, and reduces the 16
// wavefronts' candidates through LDS. Same selection rule as topk_kernel.
template <typename T, bool VEC>
__global__ __launch_bounds__(1024) void topk_wide_kernel(const T* __restrict__ x, T* __restrict__ vals,
                                                         int64_t* __restrict__ idx, int64_t N, int C, int k) {
  constexpr int VN = Vec16<T>::N;
  __shared__ float sv[16];
  __shared__ int si[16];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * (int64_t)C;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  float lv = INFINITY;
  int li = -1;
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY;
    int bi = -1;
    if (VEC && k == 1) {
      // Top-1: each thread visits its columns in increasing order, so a strict > keeps the
      // lowest index of equal maxima; NaN is never taken (topk_after is false for it) and the
      // first non-NaN value is taken whatever it is (bi < 0 in topk_better).
      const int nv = C / VN;
      for (int v0 = tid; v0 < nv; v0 += 8 * 1024) {
        Vec16<T> buf[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (v0 + u * 1024 < nv) buf[u] = ld16(xr + (int64_t)(v0 + u * 1024) * VN);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (v0 + u * 1024 < nv) {
#pragma unroll
            for (int e = 0; e < VN; ++e) {
              const float v = to_f32(buf[u].v[e]);
              if (v > bv || (bi < 0 && v == v)) {
                bv = v;
                bi = (v0 + u * 1024) * VN + e;
              }
            }
          }
        }
      }
    } else if constexpr (VEC) {
      const int nv = C / VN;  // C is a multiple of VN
      for (int v0 = tid; v0 < nv; v0 += 4 * 1024) {
        Vec16<T> buf[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (v0 + u * 1024 < nv) buf[u] = ld16(xr + (int64_t)(v0 + u * 1024) * VN);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (v0 + u * 1024 < nv) {
#pragma unroll
            for (int e = 0; e < VN; ++e) {
              const int c = (v0 + u * 1024) * VN + e;
              const float v = to_f32(buf[u].v[e]);
              if (topk_after(v, c, lv, li) && topk_better(v, c, bv, bi)) {
                bv = v;
                bi = c;
              }
            }
          }
        }
      }
    } else {
      for (int c = tid; c < C; c += 1024) {
        const float v = to_f32(xr[c]);
        if (topk_after(v, c, lv, li) && topk_better(v, c, bv, bi)) {
          bv = v;
          bi = c;
        }
      }
    }
    for (int o = 32; o > 0; o >>= 1) {
      const float v2 = __shfl_xor(bv, o);
      const int i2 = __shfl_xor(bi, o);
      if (i2 >= 0 && topk_better(v2, i2, bv, bi)) {
        bv = v2;
        bi = i2;
      }
    }
    if (lane == 0) {
      sv[wid] = bv;
      si[wid] = bi;
    }
    __syncthreads();
    bv = -INFINITY;
    bi = -1;
    for (int w = 0; w < 16; ++w)
      if (si[w] >= 0 && topk_better(sv[w], si[w], bv, bi)) {
        bv = sv[w];
        bi = si[w];
      }
    __syncthreads();  // sv / si are rewritten next round
    if (tid == 0) {
      vals[row * k + r] = from_f32<T>(bi >= 0 ? bv : __int_as_float(0x7fc00000));
      idx[row * k + r] = bi;
    }
    lv = bv;
    li = bi;
    if (bi < 0) lv = -INFINITY, li = 0x7fffffff;
  }
}

// Top-k for rows of C <= 128 and k <= 16: 16 lanes per row, each holding 8
// values as 64-bit keys (order-preserving value bits << 32 | ~column), so one
// unsigned max gives "largest value, then lowest column" -- the order of
// topk_better/topk_after. NaN gets key 0 and is never selected, as there. Each
// lane sorts its 8 keys (Batcher's 19-comparator network); each of the k rounds
// takes the 16-lane max of the list heads with DPP and the winning lane pops
// its head. Values are re-read from the row so they keep their exact bits.
__device__ __forceinline__ uint64_t topk_key(float v, int c) {
  if (v != v) return 0;
  if (v == 0.f) v = 0.f;
  const uint32_t u = __float_as_uint(v);
  const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)o << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)c);
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xF, 0xF, true);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, true);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ void cas_desc(uint64_t& a, uint64_t& b) {
  const uint64_t hi = max_u64(a, b), lo = a > b ? b : a;
  a = hi;
  b = lo;
}

template <typename T>
__global__ __launch_bounds__(256) void topk16_kernel(const T* __restrict__ x, T* __restrict__ vals,
                                                     int64_t* __restrict__ idx, int64_t N, int C, int k) {
  constexpr int VN = Vec16<T>::N;
  constexpr int NL = 8 / VN;
  const int64_t row = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int g = threadIdx.x & 15;
  if (row >= N) return;  // whole 16-lane groups leave together
  const T* xr = x + row * C;
  uint64_t key[8];
#pragma unroll
  for (int l = 0; l < NL; ++l) {
    const int c0 = (l * 16 + g) * VN;
    if (c0 < C) {
      const Vec16<T> v = ld16(xr + c0);
#pragma unroll
      for (int j = 0; j < VN; ++j) key[l * VN + j] = topk_key(to_f32(v.v[j]), c0 + j);
    } else {
#pragma unroll
      for (int j = 0; j < VN; ++j) key[l * VN + j] = 0;
    }
  }
  cas_desc(key[0], key[1]); cas_desc(key[2], key[3]); cas_desc(key[4], key[5]); cas_desc(key[6], key[7]);
  cas_desc(key[0], key[2]); cas_desc(key[1], key[3]); cas_desc(key[4], key[6]); cas_desc(key[5], key[7]);
  cas_desc(key[1], key[2]); cas_desc(key[5], key[6]);
  cas_desc(key[0], key[4]); cas_desc(key[1], key[5]); cas_desc(key[2], key[6]); cas_desc(key[3], key[7]);
  cas_desc(key[2], key[4]); cas_desc(key[3], key[5]);
  cas_desc(key[1], key[2]); cas_desc(key[3], key[4]); cas_desc(key[5], key[6]);
  int my_col = -1;
  for (int r = 0; r < k; ++r) {
    uint64_t m = key[0];
    m = max_u64(m, dpp_u64<QH_DPP_XOR1>(m));
    m = max_u64(m, dpp_u64<QH_DPP_XOR2>(m));
    m = max_u64(m, dpp_u64<QH_DPP_HALF_MIRROR>(m));
    m = max_u64(m, dpp_u64<QH_DPP_MIRROR>(m));
    if (g == r) my_col = m ? (int)(0xFFFFFFFFu - (uint32_t)m) : -1;
    if (m != 0 && key[0] == m) {
#pragma unroll
      for (int j = 0; j < 7; ++j) key[j] = key[j + 1];
      key[7] = 0;
    }
  }
  if (g < k) {
    vals[row * k + g] = my_col >= 0 ? xr[my_col] : from_f32<T>(__int_as_float(0x7fc00000));
    idx[row * k + g] = my_col;
  }
}

__global__ __launch_bounds__(256) void one_hot_kernel(const int64_t* __restrict__ idx, int64_t* __restrict__ out,
                                                      int64_t N, int64_t C, int64_t total) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i / C, c = i - n * C;
    out[i] = (idx[n] == c) ? 1 : 0;
  }
}


// ---------------------------------------------------------------------------
// Host launchers (shape selection happens here, outside the dtype dispatch)
// ---------------------------------------------------------------------------
#define QH_SHAPE_SWITCH(KERNEL, ...)                                             \
  if (G == 8 && NV == 1) KERNEL<T, 8, 1><<<grid, 256, 0, st>>>(__VA_ARGS__);     \
  else if (G == 16 && NV == 1) KERNEL<T, 16, 1><<<grid, 256, 0, st>>>(__VA_ARGS__); \
  else if (G == 32 && NV == 1) KERNEL<T, 32, 1><<<grid, 256, 0, st>>>(__VA_ARGS__); \
  else if (G == 64 && NV == 1) KERNEL<T, 64, 1><<<grid, 256, 0, st>>>(__VA_ARGS__); \
  else if (G == 64 && NV == 2) KERNEL<T, 64, 2><<<grid, 256, 0, st>>>(__VA_ARGS__); \
  else if (G == 64 && NV == 4) KERNEL<T, 64, 4><<<grid, 256, 0, st>>>(__VA_ARGS__); \
  else if (G == 64 && NV == 8) KERNEL<T, 64, 8><<<grid, 256, 0, st>>>(__VA_ARGS__);

template <typename T>
static void launch_rms_fwd(const void* x, const void* w, int wdtype, void* y, int64_t rows, int64_t cols, float eps,
                           float wadd, hipStream_t st) {
  int G = 0, NV = 0;
  if (pick_row_shape(cols, Vec16<T>::N, G, NV) && aligned16(x) && aligned16(y)) {
    const int grid = grid_cap(ceil_div(rows, 256 / G));
    QH_SHAPE_SWITCH(rmsnorm_fwd_fast, (const T*)x, w, wdtype, (T*)y, rows, (int)cols, eps, wadd)
  } else {
    rmsnorm_fwd_generic<T><<<grid_cap(rows), 256, 0, st>>>((const T*)x, w, wdtype, (T*)y, rows, cols, eps, wadd);
  }
}

template <typename T>
static void launch_softmax_fwd(const void* x, void* y, int64_t rows, int64_t cols, hipStream_t st) {
  int G = 0, NV = 0;
  if (pick_row_shape(cols, Vec16<T>::N, G, NV) && aligned16(x) && aligned16(y)) {
    const int grid = grid_cap(ceil_div(rows, 256 / G));
    QH_SHAPE_SWITCH(softmax_fwd_fast, (const T*)x, (T*)y, rows, (int)cols)
  } else {
    softmax_fwd_generic<T><<<grid_cap(rows), 256, 0, st>>>((const T*)x, (T*)y, rows, cols);
  }
}

template <typename T>
static void launch_softmax_bwd(const void* y, const void* gy, void* gx, int64_t rows, int64_t cols, hipStream_t st) {
  int G = 0, NV = 0;
  if (pick_row_shape(cols, Vec16<T>::N, G, NV) && aligned16(y) && aligned16(gy) && aligned16(gx)) {
    const int grid = grid_cap(ceil_div(rows, 256 / G));
    QH_SHAPE_SWITCH(softmax_bwd_fast, (const T*)y, (const T*)gy, (T*)gx, rows, (int)cols)
  } else {
    softmax_bwd_generic<T><<<grid_cap(rows), 256, 0, st>>>((const T*)y, (const T*)gy, (T*)gx, rows, cols);
  }
}

template <typename T>
static void launch_topk(const void* x, void* vals, int64_t* idx, int64_t N, int64_t C, int64_t k, hipStream_t st) {
  if (C <= 128 && k <= 16 && (C * (int64_t)sizeof(T)) % 16 == 0 && aligned16(x)) {
    topk16_kernel<T><<<(int)ceil_div(N, 16), 256, 0, st>>>((const T*)x, (T*)vals, idx, N, (int)C, (int)k);
    return;
  }
  const int grid = (int)ceil_div(N, 4);
  const int cpl = (int)ceil_div(C, 64);
  if (cpl <= 1) topk_kernel<T, 1><<<grid, 256, 0, st>>>((const T*)x, (T*)vals, idx, N, (int)C, (int)k);
  else if (cpl <= 2) topk_kernel<T, 2><<<grid, 256, 0, st>>>((const T*)x, (T*)vals, idx, N, (int)C, (int)k);
  else if (cpl <= 4) topk_kernel<T, 4><<<grid, 256, 0, st>>>((const T*)x, (T*)vals, idx, N, (int)C, (int)k);
  else if (cpl <= 8) topk_kernel<T, 8><<<grid, 256, 0, st>>>((const T*)x, (T*)vals, idx, N, (int)C, (int)k);
  else if (cpl <= 16) topk_kernel<T, 16><<<grid, 256, 0, st>>>((const T*)x, (T*)vals, idx, N, (int)C, (int)k);
  else if (aligned16(x) && (C * (int64_t)sizeof(T)) % 16 == 0)
    topk_wide_kernel<T, true><<<(unsigned)N, 1024, 0, st>>>((const T*)x, (T*)vals, idx, N, (int)C, (int)k);
  else
    topk_wide_kernel<T, false><<<(unsigned)N, 1024, 0, st>>>((const T*)x, (T*)vals, idx, N, (int)C, (int)k);
}


// ---------------------------------------------------------------------------
// Greedy decode step: the argmax of each row of the last logits (torch.argmax
// semantics: NaN counts as the largest value, ties go to the lowest column)
// and the step's bookkeeping in device memory. An element's key is
// (order-preserving value bits, NaN above +inf) << 32 | ~column, so the
// largest key is the answer whatever the reduction order; -0.0 keys as +0.0
// (the two compare equal, so the lower column wins between them).
constexpr int kGreedyMaxRows = 64;  // rows one launch serves

__device__ __forceinline__ uint64_t greedy_key(float v, int c) {
  uint32_t b = v == 0.f ? 0u : __float_as_uint(v);
  b = (v != v) ? 0xFFFFFFFFu : (b ^ ((b >> 31) ? 0xFFFFFFFFu : 0x80000000u));
  return ((uint64_t)b << 32) | (uint32_t)~(uint32_t)c;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t k2 = ((uint64_t)(uint32_t)__shfl_xor((int)(k >> 32), o) << 32) |
                        (uint32_t)__shfl_xor((int)(uint32_t)k, o);
    k = k2 > k ? k2 : k;
  }
  return k;
}

// Columns one first-stage workgroup keys: one 16-byte load per thread.
template <typename T>
__host__ __device__ constexpr int greedy_cols() { return 256 * (16 / (int)sizeof(T)); }

// Stage 1: workgroup (p, row) reduces its greedy_cols<T>() columns to one key.
template <typename T>
__global__ __launch_bounds__(256) void greedy_partial_kernel(const T* __restrict__ x, int64_t ld, int V,
                                                             uint64_t* __restrict__ part, int P) {
  constexpr int VN = Vec16<T>::N;
  __shared__ uint64_t sk[4];
  const int row = blockIdx.y, p = blockIdx.x;
  const T* xr = x + (int64_t)row * ld;
  const int c0 = p * greedy_cols<T>() + threadIdx.x * VN;
  uint64_t best = 0;  // below every element's key
  if (c0 + VN <= V) {
    const Vec16<T> v = ld16(xr + c0);
#pragma unroll
    for (int e = 0; e < VN; ++e) {
      const uint64_t k = greedy_key(to_f32(v.v[e]), c0 + e);
      best = k > best ? k : best;
    }
  } else {
    for (int c = c0; c < V && c < c0 + VN; ++c) {
      const uint64_t k = greedy_key(to_f32(xr[c]), c);
      best = k > best ? k : best;
    }
  }
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) sk[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = sk[0];
    for (int w = 1; w < 4; ++w) b = sk[w] > b ? sk[w] : b;
    part[(int64_t)row * P + p] = b;
  }
}

// Stage 2 (one workgroup, a 16-lane group per row): each row's answer from its P partial
// keys, then the step's bookkeeping: ids[b] = tokens[b, col] = answer, seqlens[b] += 1 (the
// row's group), col += 1, positions += 1 (thread 0, after every group has read col). Each
// pointer is optional.
__global__ __launch_bounds__(kGreedyMaxRows * 16) void greedy_finish_kernel(
    const uint64_t* __restrict__ part, int P, int B, int64_t* __restrict__ ids, int64_t* __restrict__ tokens,
    int64_t ldt, int64_t ncols, int64_t* __restrict__ col, int64_t* __restrict__ positions,
    int32_t* __restrict__ seqlens) {
  const int b = threadIdx.x >> 4, l = threadIdx.x & 15;
  const int64_t c = col ? col[0] : -1;
  if (b < B) {
    uint64_t best = 0;
    for (int p = l; p < P; p += 16) {
      const uint64_t k = part[(int64_t)b * P + p];
      best = k > best ? k : best;
    }
    for (int o = 8; o > 0; o >>= 1) {  // within the 16-lane group
      const uint64_t k2 = ((uint64_t)(uint32_t)__shfl_xor((int)(best >> 32), o) << 32) |
                          (uint32_t)__shfl_xor((int)(uint32_t)best, o);
      best = k2 > best ? k2 : best;
    }
    if (l == 0) {
      const int64_t ans = (int64_t)(uint32_t)~(uint32_t)best;
      if (ids) ids[b] = ans;
      if (tokens && c >= 0 && c < ncols) tokens[(int64_t)b * ldt + c] = ans;
      if (seqlens) seqlens[b] += 1;
    }
  }
  __syncthreads();  // every read of col has completed
  if (threadIdx.x == 0) {
    if (col) col[0] = c + 1;
    if (positions) positions[0] += 1;
  }
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" int qh_rmsnorm_fwd(const void* x, const void* w, void* y, int64_t rows, int64_t cols, float eps,
                              int one_plus, int dtype, int wdtype, void* stream) {
  QH_CHECK_ARG(rows >= 0 && cols >= 0, "qh_rmsnorm_fwd: negative shape");
  QH_CHECK_ARG(wdtype >= QH_F32 && wdtype <= QH_BF16, "qh_rmsnorm_fwd: bad weight dtype");
  if (rows == 0 || cols == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const float wadd = one_plus ? 1.f : 0.f;
  QH_DISPATCH_DTYPE(dtype, T, "qh_rmsnorm_fwd", launch_rms_fwd<T>(x, w, wdtype, y, rows, cols, eps, wadd, st));
  QH_CHECK_LAUNCH("qh_rmsnorm_fwd");
  return QH_OK;
}

extern "C" int qh_add_rmsnorm(const void* x, const void* r, const void* w, void* sum, void* y, int64_t rows,
                              int64_t cols, float eps, int one_plus, int dtype, int wdtype, void* stream) {
  QH_CHECK_ARG(rows >= 0 && cols >= 0, "qh_add_rmsnorm: negative shape");
  QH_CHECK_ARG(wdtype >= QH_F32 && wdtype <= QH_BF16, "qh_add_rmsnorm: bad weight dtype");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_add_rmsnorm: bf16/f16 only");
  if (rows == 0 || cols == 0) return QH_OK;
  int G = 0, NV = 0;
  const bool fast = pick_row_shape(cols, 8, G, NV) && aligned16(x) && aligned16(r) && aligned16(sum) && aligned16(y);
  if (!fast) {  // the two kernels in sequence
    int rc = qh_add(x, r, sum, rows * cols, dtype, stream);
    return rc ? rc : qh_rmsnorm_fwd(sum, w, y, rows, cols, eps, one_plus, dtype, wdtype, stream);
  }
  hipStream_t st = (hipStream_t)stream;
  const float wadd = one_plus ? 1.f : 0.f;
  const int grid = grid_cap(ceil_div(rows, 256 / G));
#define QH_ADDRMS(T) \
  QH_SHAPE_SWITCH(add_rmsnorm_fast, (const T*)x, (const T*)r, w, wdtype, (T*)sum, (T*)y, rows, (int)cols, eps, wadd)
  if (dtype == QH_BF16) {
    typedef bf16_t T;
    QH_ADDRMS(T)
  } else {
    typedef f16_t T;
    QH_ADDRMS(T)
  }
#undef QH_ADDRMS
  QH_CHECK_LAUNCH("qh_add_rmsnorm");
  return QH_OK;
}

static int64_t rms_bwd_partial_rows(int64_t rows, int64_t cols, int dtype, int* fast_grid, int* G_out, int* NV_out) {
  const int VN = dtype == QH_F32 ? 4 : 8;
  int G = 0, NV = 0;
  if (pick_row_shape(cols, VN, G, NV)) {
    const int bt = rms_bwd_threads(NV);
    const int rpb = bt / G;
    int64_t grid = ceil_div(rows, rpb);
    const int64_t cap = (int64_t)kRmsBwdBlocks * 256 / bt;
    if (grid > cap) grid = cap;
    if (grid < 1) grid = 1;
    if (fast_grid) *fast_grid = (int)grid;
    if (G_out) *G_out = G;
    if (NV_out) *NV_out = NV;
    return grid;
  }
  if (fast_grid) *fast_grid = 0;
  return 0;
}

template <typename T>
static int64_t launch_rms_bwd(const void* x, const void* w, int wdtype, const void* gy, void* gx, void* ws,
                              int64_t rows, int64_t cols, float eps, float wadd, int dtype, hipStream_t st) {
  int grid = 0, G = 0, NV = 0;
  const int64_t fr = rms_bwd_partial_rows(rows, cols, dtype, &grid, &G, &NV);
  if (fr > 0 && aligned16(x) && aligned16(gy) && aligned16(gx)) {
    const int bt = rms_bwd_threads(NV);
    const size_t lds = (size_t)(bt / G) * cols * sizeof(float);  // at most 64 KB for the shapes served
#define QH_RBW(GG, NN, BB)                                                                                        \
  rmsnorm_bwd_fast<T, GG, NN, BB><<<grid, BB, lds, st>>>((const T*)x, w, wdtype, (const T*)gy, (T*)gx, (float*)ws, \
                                                        rows, (int)cols, eps, wadd)
    if (G == 8) QH_RBW(8, 1, 1024);
    else if (G == 16) QH_RBW(16, 1, 1024);
    else if (G == 32) QH_RBW(32, 1, 1024);
    else if (NV == 1) QH_RBW(64, 1, 1024);
    else if (NV == 2) QH_RBW(64, 2, 1024);
    else if (NV == 4) QH_RBW(64, 4, 512);
    else QH_RBW(64, 8, 256);
#undef QH_RBW
    return fr;
  }
  const int g = (int)(rows < kRmsBwdBlocks ? rows : kRmsBwdBlocks);
  rmsnorm_bwd_generic<T><<<g, 256, 0, st>>>((const T*)x, w, wdtype, (const T*)gy, (T*)gx, (float*)ws, rows, cols,
                                            eps, wadd);
  return g;
}

extern "C" int64_t qh_rmsnorm_bwd_workspace(int64_t rows, int64_t cols, int dtype) {
  if (rows <= 0 || cols <= 0) return 0;
  const int64_t fast_rows = rms_bwd_partial_rows(rows, cols, dtype, nullptr, nullptr, nullptr);
  const int64_t gen_rows = rows < kRmsBwdBlocks ? rows : kRmsBwdBlocks;
  const int64_t r = fast_rows > gen_rows ? fast_rows : gen_rows;
  return r * cols * (int64_t)sizeof(float);
}

extern "C" int qh_rmsnorm_bwd(const void* x, const void* w, const void* gy, void* gx, void* gw, void* ws,
                              int64_t ws_bytes, int64_t rows, int64_t cols, float eps, int one_plus, int dtype,
                              int wdtype, void* stream) {
  QH_CHECK_ARG(rows >= 0 && cols >= 0, "qh_rmsnorm_bwd: negative shape");
  QH_CHECK_ARG(wdtype >= QH_F32 && wdtype <= QH_BF16, "qh_rmsnorm_bwd: bad weight dtype");
  if (cols == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  if (rows == 0) return qh_zero(gw, cols * (wdtype == QH_F32 ? 4 : 2), stream);
  const int64_t need = qh_rmsnorm_bwd_workspace(rows, cols, dtype);
  if (ws_bytes < need) {
    qh::set_error("qh_rmsnorm_bwd: workspace %lld bytes < required %lld", (long long)ws_bytes, (long long)need);
    return QH_E_WORKSPACE;
  }
  const float wadd = one_plus ? 1.f : 0.f;
  int64_t prow = 0;
  QH_DISPATCH_DTYPE(dtype, T, "qh_rmsnorm_bwd",
                    prow = launch_rms_bwd<T>(x, w, wdtype, gy, gx, ws, rows, cols, eps, wadd, dtype, st));
  colsum_partials<<<(int)ceil_div(cols, 64), 1024, 0, st>>>((const float*)ws, prow, cols, gw, wdtype);
  QH_CHECK_LAUNCH("qh_rmsnorm_bwd");
  return QH_OK;
}

extern "C" int qh_softmax_fwd(const void* x, void* y, int64_t rows, int64_t cols, int dtype, void* stream) {
  QH_CHECK_ARG(rows >= 0 && cols >= 0, "qh_softmax_fwd: negative shape");
  if (rows == 0 || cols == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  QH_DISPATCH_DTYPE(dtype, T, "qh_softmax_fwd", launch_softmax_fwd<T>(x, y, rows, cols, st));
  QH_CHECK_LAUNCH("qh_softmax_fwd");
  return QH_OK;
}

extern "C" int qh_softmax_bwd(const void* y, const void* gy, void* gx, int64_t rows, int64_t cols, int dtype,
                              void* stream) {
  QH_CHECK_ARG(rows >= 0 && cols >= 0, "qh_softmax_bwd: negative shape");
  if (rows == 0 || cols == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  QH_DISPATCH_DTYPE(dtype, T, "qh_softmax_bwd", launch_softmax_bwd<T>(y, gy, gx, rows, cols, st));
  QH_CHECK_LAUNCH("qh_softmax_bwd");
  return QH_OK;
}

extern "C" int qh_ce_fwd(const void* logits, int64_t stride, const int64_t* targets, float* lse, float* loss_rows,
                         float* loss_out, float* nvalid_out, int64_t N, int64_t V, int64_t ignore_index, int dtype, void* stream) {
  QH_CHECK_ARG(N >= 0 && V > 0 && stride >= V, "qh_ce_fwd: bad shape N=%lld V=%lld stride=%lld", (long long)N,
               (long long)V, (long long)stride);
  QH_CHECK_ARG(N < (1ll << 31), "qh_ce_fwd: too many rows");
  hipStream_t st = (hipStream_t)stream;
  if (N > 0) {
    QH_DISPATCH_DTYPE(dtype, T, "qh_ce_fwd", {
      constexpr int VN = Vec16<T>::N;
      if (aligned16(logits) && V % VN == 0 && stride % VN == 0)
        ce_fwd_kernel<T, true><<<(int)N, 256, 0, st>>>((const T*)logits, stride, targets, lse, loss_rows, V,
                                                       ignore_index);
      else
        ce_fwd_kernel<T, false><<<(int)N, 256, 0, st>>>((const T*)logits, stride, targets, lse, loss_rows, V,
                                                        ignore_index);
    });
  }
  ce_finalize<<<1, 1024, 0, st>>>(loss_rows, targets, N, ignore_index, loss_out, nvalid_out);
  QH_CHECK_LAUNCH("qh_ce_fwd");
  return QH_OK;
}

extern "C" int qh_ce_bwd(const void* logits, int64_t stride, const int64_t* targets, const float* lse,
                         const float* grad_loss, const float* nvalid, void* glogits, int64_t gstride, int64_t N,
                         int64_t V, int64_t ignore_index, int dtype, void* stream) {
  QH_CHECK_ARG(N >= 0 && V > 0 && stride >= V && gstride >= V, "qh_ce_bwd: bad shape");
  QH_CHECK_ARG(N < (1ll << 31), "qh_ce_bwd: too many rows");
  if (N == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  QH_DISPATCH_DTYPE(dtype, T, "qh_ce_bwd", {
    constexpr int VN = Vec16<T>::N;
    if (aligned16(logits) && aligned16(glogits) && V % VN == 0 && stride % VN == 0 && gstride % VN == 0)
      ce_bwd_kernel<T, true><<<(int)N, 256, 0, st>>>((const T*)logits, stride, targets, lse, grad_loss, nvalid,
                                                     (T*)glogits, gstride, V, ignore_index);
    else
      ce_bwd_kernel<T, false><<<(int)N, 256, 0, st>>>((const T*)logits, stride, targets, lse, grad_loss, nvalid,
                                                      (T*)glogits, gstride, V, ignore_index);
  });
  QH_CHECK_LAUNCH("qh_ce_bwd");
  return QH_OK;
}

extern "C" int qh_topk(const void* x, void* vals, int64_t* idx, int64_t N, int64_t C, int64_t k, int dtype,
                       void* stream) {
  QH_CHECK_ARG(N >= 0 && C >= 0 && k >= 0, "qh_topk: negative shape");
  QH_CHECK_ARG(k <= C, "qh_topk: k=%lld > C=%lld", (long long)k, (long long)C);
  QH_CHECK_ARG(C < (1ll << 30) && N < (1ll << 31), "qh_topk: too large");
  if (N == 0 || k == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  QH_DISPATCH_DTYPE(dtype, T, "qh_topk", launch_topk<T>(x, vals, idx, N, C, k, st));
  QH_CHECK_LAUNCH("qh_topk");
  return QH_OK;
}

extern "C" int64_t qh_greedy_step_workspace(int64_t B, int64_t V) {
  return B * ((V + greedy_cols<float>() - 1) / greedy_cols<float>()) * (int64_t)sizeof(uint64_t);
}

extern "C" int qh_greedy_step(const void* logits, int64_t ld, int64_t B, int64_t V, int64_t* ids, int64_t* tokens,
                              int64_t ldt, int64_t ncols, int64_t* col, int64_t* positions, int32_t* seqlens,
                              void* ws, int64_t ws_bytes, int dtype, void* stream) {
  QH_CHECK_ARG(B >= 1 && B <= kGreedyMaxRows && V >= 1 && V < (1ll << 31) && ld >= V,
               "qh_greedy_step: bad shape B=%lld V=%lld ld=%lld", (long long)B, (long long)V, (long long)ld);
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16 || dtype == QH_F32, "qh_greedy_step: bf16/f16/f32 logits");
  QH_CHECK_ARG(aligned16(logits) && (ld * (dtype == QH_F32 ? 4 : 2)) % 16 == 0,
               "qh_greedy_step: logits rows must be 16-byte aligned");
  QH_CHECK_ARG(ws != nullptr && ws_bytes >= qh_greedy_step_workspace(B, V), "qh_greedy_step: workspace too small");
  hipStream_t st = (hipStream_t)stream;
  uint64_t* part = (uint64_t*)ws;
  int P = 0;
#define QH_GREEDY(TT)                                                                                \
  P = (int)((V + greedy_cols<TT>() - 1) / greedy_cols<TT>());                                         \
  greedy_partial_kernel<TT><<<dim3((unsigned)P, (unsigned)B), 256, 0, st>>>((const TT*)logits, ld, (int)V, part, P)
  if (dtype == QH_BF16) { QH_GREEDY(bf16_t); } else if (dtype == QH_F16) { QH_GREEDY(f16_t); } else { QH_GREEDY(float); }
#undef QH_GREEDY
  greedy_finish_kernel<<<1, kGreedyMaxRows * 16, 0, st>>>(part, P, (int)B, ids, tokens, ldt, ncols, col, positions,
                                                         seqlens);
  QH_CHECK_LAUNCH("qh_greedy_step");
  return QH_OK;
}

extern "C" int qh_one_hot(const int64_t* idx, int64_t* out, int64_t N, int64_t C, void* stream) {
  QH_CHECK_ARG(N >= 0 && C >= 0, "qh_one_hot: negative shape");
  const int64_t total = N * C;
  if (total == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  one_hot_kernel<<<grid_cap(ceil_div(total, 256)), 256, 0, st>>>(idx, out, N, C, total);
  QH_CHECK_LAUNCH("qh_one_hot");
  return QH_OK;
}
