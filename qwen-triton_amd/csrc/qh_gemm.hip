// GEMM for the Linear layers: C[M,N] = A(M,K) * B(N,K)^T (+ bias[N]).
//
// Operand views (element (i, k) of each logical operand):
//   A(m,k) = A[m*lda + k]  (row-major, "N")   or  A[k*lda + m]  ("T")
//   B(n,k) = B[n*ldb + k]  (row-major, "N")   or  B[k*ldb + n]  ("T")
// which covers the three Linear products without copying any operand:
//   forward  y  = x  W^T : A = x  [M,K] N, B = W  [N,K] N
//   grad in  dx = dy W   : A = dy [M,N] N, B = W  [N,K] T
//   grad wt  dW = dy^T x : A = dy [T,N] T, B = x  [T,K] T
//
// gfx950 design:
//  * bf16/fp16 operands on v_mfma_f32_32x32x16_{bf16,f16}; fp32 accumulation.
//  * 256-thread workgroups (4 wavefronts, 2x2), BK = 64, double-buffered LDS
//    tiles stored k-contiguous with 16-byte row padding (conflict-free
//    ds_read_b128 fragment loads); the next k-tile is fetched into registers
//    while the current one feeds the matrix cores.
//  * "T" operands are transposed while staging: each thread loads an 8x8 block
//    with eight 16-byte loads and re-packs it with byte permutes, so every
//    operand lands in LDS in the same k-contiguous layout.
//  * Tile order is XCD-aware: the 8 XCDs each take a contiguous run of tiles
//    (grouped 8 M-tiles at a time) so operand panels are reused out of the
//    XCD's own L2.
//  * 4 < M <= 128 (batched decode, short prefill) uses 1024-thread workgroups
//    of MFMA 16x16x32 over R x 32 or R x 16 tiles whose operands stream
//    through a ring of LDS stages, 16 wavefronts splitting K into 4 or 16
//    slices (by K alone) summed through LDS in a fixed order; M <= 4 one
//    wavefront per output column.
#include "qh_mfma.h"
#include "qh_lds.h"

// Large-tile and split-K paths (qh_gemm_tile.hip).
int qh_gemm_tile_dispatch(int ta, int tb, int M, int N, int K, const void* A, int64_t lda, const void* B,
                          int64_t ldb, void* C, int64_t ldc, const void* bias, int dtype, int out_dtype,
                          hipStream_t st);
int qh_gemm_splitk_count(int64_t M, int64_t N, int64_t K);
int qh_gemm_splitk_dispatch(int ta, int tb, int M, int N, int K, const void* A, int64_t lda, const void* B,
                            int64_t ldb, void* C, int64_t ldc, const void* bias, int dtype, int out_dtype, int S,
                            void* ws, hipStream_t st);

namespace {

constexpr int BK = 64;
constexpr int LDS_LD = BK + 8;  // padded row length (elements) of an LDS tile

// Stage one operand tile (ROWS x BK) for k-tile starting at k0 into registers.
// Non-transposed: 16-byte chunk c -> row c/8, k-chunk c%8.
// Transposed:     8x8 sub-block sb -> row-block sb % (ROWS/8), k-block sb / (ROWS/8).
// NT: non-temporal loads (operands read exactly once, e.g. the weights of a
// product with a single row of output tiles).
template <typename T, int ROWS, bool TR, bool NT = false>
struct TileLoader {
  static constexpr int SUBS = (ROWS + 255) / 256;          // 8x8 sub-blocks per thread (transposed)
  static constexpr int NREG = TR ? 8 * SUBS : ROWS / 32;   // uint4 staging registers per thread
  uint4 r[NREG];

  __device__ __forceinline__ void load(const T* __restrict__ P, int64_t ld, int row0, int rows, int k0, int K) {
    const int tid = threadIdx.x;
    const uint4 z = make_uint4(0, 0, 0, 0);
    if constexpr (!TR) {
#pragma unroll
      for (int i = 0; i < NREG; ++i) {
        const int c = tid + i * 256;
        const int row = c >> 3, kc = c & 7;
        const int gr = row0 + row, gk = k0 + kc * 8;
        if (gr < rows && gk < K) {
          const T* src = P + (int64_t)gr * ld + gk;
          if constexpr (NT) {
            typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
            const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
            r[i] = make_uint4(v.x, v.y, v.z, v.w);
          } else {
            r[i] = *reinterpret_cast<const uint4*>(src);
          }
        } else {
          r[i] = z;
        }
      }
    } else {
#pragma unroll
      for (int s = 0; s < SUBS; ++s) {
        const int sb = tid + s * 256;
        if (sb < ROWS) {
          const int rb = sb % (ROWS / 8), kb = sb / (ROWS / 8);
          const int gr = row0 + rb * 8;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int gk = k0 + kb * 8 + j;
            if (gr < rows && gk < K) r[s * 8 + j] = *reinterpret_cast<const uint4*>(P + (int64_t)gk * ld + gr);
            else r[s * 8 + j] = z;
          }
        }
      }
    }
  }

  __device__ __forceinline__ void store(T* __restrict__ S) const {
    const int tid = threadIdx.x;
    if constexpr (!TR) {
#pragma unroll
      for (int i = 0; i < NREG; ++i) {
        const int c = tid + i * 256;
        const int row = c >> 3, kc = c & 7;
        *reinterpret_cast<uint4*>(S + row * LDS_LD + kc * 8) = r[i];
      }
    } else {
#pragma unroll
      for (int s = 0; s < SUBS; ++s) {
        const int sb = tid + s * 256;
        if (sb < ROWS) {
          const int rb = sb % (ROWS / 8), kb = sb / (ROWS / 8);
          uint4 in[8], out[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) in[j] = r[s * 8 + j];
          transpose8x8(in, out);
#pragma unroll
          for (int c = 0; c < 8; ++c) *reinterpret_cast<uint4*>(S + (rb * 8 + c) * LDS_LD + kb * 8) = out[c];
        }
      }
    }
  }
};


template <typename T, typename OT, int BM, int BN, int WM, int WN, bool AT, bool BT, bool BNT = false>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(const T* __restrict__ A, int64_t lda, const T* __restrict__ B,
                                                        int64_t ldb, OT* __restrict__ C, int64_t ldc,
                                                        const T* __restrict__ bias, int M, int N, int K,
                                                        int tiles_m, int tiles_n) {
  static_assert(WM * WN == 4, "4 wavefronts per workgroup");
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(TM >= 1 && TN >= 1, "wave tile must cover whole 32x32 MFMA tiles");
  typedef typename Mfma<T>::v8 v8;

  __shared__ __attribute__((aligned(16))) T smem[2][(BM + BN) * LDS_LD];

  int tm_, tn_;
  tile_order(tiles_m, tiles_n, tm_, tn_);
  const int m0 = tm_ * BM, n0 = tn_ * BN;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid / WN, wn = wid % WN;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  TileLoader<T, BM, AT> la;
  TileLoader<T, BN, BT, BNT> lb;
  const int nk = (K + BK - 1) / BK;

  la.load(A, lda, m0, M, 0, K);
  lb.load(B, ldb, n0, N, 0, K);
  la.store(smem[0]);
  lb.store(smem[0] + BM * LDS_LD);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      la.load(A, lda, m0, M, (kt + 1) * BK, K);
      lb.load(B, ldb, n0, N, (kt + 1) * BK, K);
    }
    const T* As = smem[buf];
    const T* Bs = smem[buf] + BM * LDS_LD;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      v8 af[TM], bf[TN];
      const int koff = kk * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const v8*>(As + (wm * WTM + i * 32 + (lane & 31)) * LDS_LD + koff);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bf[j] = *reinterpret_cast<const v8*>(Bs + (wn * WTN + j * 32 + (lane & 31)) * LDS_LD + koff);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = Mfma<T>::mma(af[i], bf[j], acc[i][j]);
    }
    if (more) {
      la.store(smem[buf ^ 1]);
      lb.store(smem[buf ^ 1] + BM * LDS_LD);
    }
    __syncthreads();
  }

  // Epilogue. MFMA 32x32 output layout: lane holds column (lane % 32) and rows
  // 8g + 4*(lane / 32) + r for register 4g + r.
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int col = n0 + wn * WTN + j * 32 + (lane & 31);
    if (col >= N) continue;
    const float bv = bias ? to_f32(bias[col]) : 0.f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int rbase = m0 + wm * WTM + i * 32 + (lane >> 5) * 4;
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = rbase + g * 8 + r;
          if (row < M) C[(int64_t)row * ldc + col] = from_f32<OT>(acc[i][j][g * 4 + r] + bv);
        }
    }
  }
}

// ---------------------------------------------------------------------------
// Decode products (M <= 128): the operand set of one launch, the norm fusion
// parameters, and helpers shared by the batch-1 and the chunked kernels.
// ---------------------------------------------------------------------------
constexpr int kMaxProducts = 4;
template <typename T, typename OT>
struct DecodeProducts {
  const T* B[kMaxProducts];
  OT* C[kMaxProducts];
  const T* bias[kMaxProducts];
  const T* res[kMaxProducts];
  int64_t ldb[kMaxProducts], ldc[kMaxProducts], ldr[kMaxProducts];
  int N[kMaxProducts];
  int tile0[kMaxProducts + 1];  // first workgroup of each product
  int count;
};

struct DecodeNorm {
  const void* w;  // RMSNorm weight [K] in the activation dtype, nullptr = no norm (unless folded)
  float eps, wadd;
  int folded;  // 1: the weight is folded into B (row factor only)
};

// One product's fields as a kernel uses them. Product 0's are read with constant offsets, so
// the kernel's argument loads are issued together at its start; only a launch of several
// products looks its product up (a chain of dependent argument loads measured 0.5-0.7 us of a
// 5-6 us launch). The model's decode launches all have one product (q/k/v concatenated, gate
// and up as one gated pair).
template <typename T, typename OT>
struct ProductView {
  const T* B;
  int64_t ldb;
  int N, first;
  OT* C;
  int64_t ldc;
  const T* bias;
  const T* res;
  int64_t ldr;
};
template <typename T, typename OT>
__device__ __forceinline__ ProductView<T, OT> product_view(const DecodeProducts<T, OT>& P, int i) {
  return ProductView<T, OT>{P.B[i], P.ldb[i], P.N[i], P.tile0[i], P.C[i], P.ldc[i], P.bias[i], P.res[i], P.ldr[i]};
}
template <typename T, typename OT>
__device__ __forceinline__ void view_now(ProductView<T, OT>& v) {
  sgpr_now(v.B);
  sgpr_now(v.ldb);
  sgpr_now(v.N);
  sgpr_now(v.first);
  sgpr_now(v.C);
  sgpr_now(v.ldc);
  sgpr_now(v.bias);
  sgpr_now(v.res);
  sgpr_now(v.ldr);
}
// The product of column tile (or column) t: the last i < count with first[i] <= t.
template <typename T, typename OT>
__device__ __forceinline__ int product_of(const DecodeProducts<T, OT>& P, int t) {
  int pi = 0;
  while (pi + 1 < P.count && t >= P.tile0[pi + 1]) ++pi;
  return pi;
}

// NORM template mode: 0 none, 1 weight applied in the kernel, 2 folded into B
// (3: folded, K slices in several chunks; chosen at launch).
__host__ __device__ constexpr int decode_norm_mode(const DecodeNorm* n) {
  return n == nullptr ? 0 : (n->folded ? 2 : (n->w != nullptr ? 1 : 0));
}

// acc + sum of the squares of 8 packed 16-bit values, two per v_dot2 (fp32 sums).
template <typename T>
__device__ __forceinline__ float sumsq8(const typename Mfma<T>::v8& v, float acc) {
  if constexpr (std::is_same<T, bf16_t>::value) {
    typedef __bf16 p2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const p2 x = {v[e], v[e + 1]};
      acc = __builtin_amdgcn_fdot2_f32_bf16(x, x, acc, false);
    }
  } else {
    typedef _Float16 p2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const p2 x = {(_Float16)v[e], (_Float16)v[e + 1]};
      acc = __builtin_amdgcn_fdot2(x, x, acc, false);
    }
  }
  return acc;
}


// Decode products of at most kGemvMaxRows activation rows (batch-1 and small-
// batch decode): one wavefront per output column of every product, each wave
// streaming its weight row over the whole K range with all of a chunk's
// 16-byte loads in flight (non-temporal: the weights are read once per step),
// fp32 sums per lane, then a fixed-order xor-tree sum across the wave. The
// MFMA decode kernel would use 1..4 of its 16 MFMA rows here, and gives each
// workgroup 16 columns, so o_proj/down (1024 columns) ran on 64 workgroups;
// this kernel gives every 4 columns a workgroup (256+ for 1024 columns) and
// measured 2.9-4.1 us for the 4-12 MB config-0 products against 4.8-7.3 us.
// Same fusions as gemm_decode_kernel: NORM (row factor rsqrt(mean(h^2) + eps)
// after the sum; here the activation operand round(h * (w + wadd)) is the one
// rounded, 8 MR values per lane and step, where the MFMA kernel rounds the
// weight operand), bias, residual round(round(product) + R), GATED
// silu(round(g)) * round(u).
constexpr int kGemvMaxRows = 4;

// 16-byte loads per lane and operand row in one chunk (512 K values each).
__host__ __device__ constexpr int gemv_chunk(int mr, bool gated, int rc) {
  return rc > 1 ? 2 : (mr == 1 ? (gated ? 4 : 8) : (mr == 2 ? 4 : 2));
}
// Columns a wave takes in a single wide product (the LM head): a wave of one
// column there lives for one memory round trip, and the 152K waves of a
// vocabulary-wide output then queue for wave slots.
constexpr int kGemvWideCols = 4;
constexpr int kGemvWideMin = 32768;
constexpr int kGemvTwoColMin = 4096;

// NB weight rows per column (2: gate and up); RC columns per wave (non-gated
// products whose widths are multiples of RC; the wave's NB = RC rows are
// consecutive columns of one product).
template <typename T, typename OT, int MR, bool GATED, int NORM, int RC = 1>
__global__ __launch_bounds__(256) void gemv_decode_kernel(const T* __restrict__ A, int64_t lda,
                                                          const DecodeProducts<T, OT> P, const DecodeNorm nrm, int M,
                                                          int K, int ncols, int count) {
  static_assert(RC == 1 || !GATED, "a wave takes several columns of non-gated products only");
  constexpr bool SCALE = NORM == 1, ROWS = NORM != 0;  // activation scaled here; row factor applied
  constexpr int NB = GATED ? 2 : RC;
  constexpr int CH = gemv_chunk(MR, GATED, RC);
  typedef typename Mfma<T>::v8 v8;
  const int lane = threadIdx.x & 63;
  // P.tile0 holds the first column of each product here; a gated launch has one product
  ProductView<T, OT> pv = product_view(P, 0);
  view_now(pv);
  const T* Bup = P.B[1];  // GATED: the up projection
  int64_t ldbup = P.ldb[1];
  const T* biasup = P.bias[1];
  if constexpr (GATED) {
    sgpr_now(Bup);
    sgpr_now(ldbup);
    sgpr_now(biasup);
  }
  // count (= P.count) is a direct argument: the trailing ints then fill the 16-byte argument
  // load they share, so no other argument is loaded into its padding register (after a wait)
  sgpr_now(count);
  sgpr_now(A);
  sgpr_now(lda);
  const int col = ((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6)) * RC;
  if (col >= ncols) return;
  if (count > 1) pv = product_view(P, product_of(P, col));
  const int n = col - pv.first;
  const int Np = pv.N;
  const T* brow[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int nj = RC > 1 ? min(n + j, Np - 1) : n;  // columns past N re-read the last row
    const T* bj = GATED && j == 1 ? Bup : pv.B;
    const int64_t lj = GATED && j == 1 ? ldbup : pv.ldb;
    brow[j] = bj + (int64_t)nj * lj;
  }
  // Bias and residual of the row this lane writes (lane i writes row i), loaded before the
  // weight stream so their latency is not added after the reduction. C may be the residual
  // itself: each element is read and then written by this lane only.
  float pb[NB], pr[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) pb[j] = 0.f, pr[j] = 0.f;
  if (lane < MR && lane < M) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const T* bias = GATED && j == 1 ? biasup : pv.bias;
      if (bias != nullptr) pb[j] = to_f32(bias[RC > 1 ? min(n + j, Np - 1) : n]);
      if constexpr (!GATED) {
        if (pv.res != nullptr && (RC == 1 || n + j < Np))
          pr[j] = to_f32(pv.res[(int64_t)lane * pv.ldr + n + (RC > 1 ? j : 0)]);
      }
    }
  }
  float acc[NB][MR], ss[MR];
#pragma unroll
  for (int i = 0; i < MR; ++i) {
    ss[i] = 0.f;
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[j][i] = 0.f;
  }
  v8 zero;
#pragma unroll
  for (int e = 0; e < 8; ++e) zero[e] = (T)0.f;
  for (int k0 = 0; k0 < K; k0 += 512 * CH) {
    v8 b[CH][NB], a[CH][MR];
    v8 wr[SCALE ? CH : 1];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int k = k0 + u * 512 + lane * 8;
      const bool kok = k < K;
#pragma unroll
      for (int j = 0; j < NB; ++j)
        b[u][j] = kok ? __builtin_nontemporal_load(reinterpret_cast<const v8*>(brow[j] + k)) : zero;
#pragma unroll
      for (int i = 0; i < MR; ++i)
        a[u][i] = (kok && i < M) ? *reinterpret_cast<const v8*>(A + (int64_t)i * lda + k) : zero;
      if constexpr (SCALE) wr[u] = kok ? *reinterpret_cast<const v8*>((const T*)nrm.w + k) : zero;
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) {
#pragma unroll
      for (int i = 0; i < MR; ++i) {
        if constexpr (ROWS) ss[i] = sumsq8<T>(a[u][i], ss[i]);
        if constexpr (SCALE) {
#pragma unroll
          for (int e = 0; e < 8; ++e) a[u][i][e] = from_f32<T>(to_f32(a[u][i][e]) * (to_f32(wr[u][e]) + nrm.wadd));
        }
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[j][i] += to_f32(b[u][j][e]) * to_f32(a[u][i][e]);
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
#pragma unroll
    for (int i = 0; i < MR; ++i) {
      if constexpr (ROWS) ss[i] += __shfl_xor(ss[i], o);
#pragma unroll
      for (int j = 0; j < NB; ++j) acc[j][i] += __shfl_xor(acc[j][i], o);
    }
  }
  // lane i writes row i
#pragma unroll
  for (int i = 0; i < MR; ++i) {
    if (lane != i || i >= M) continue;
    float v[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      v[j] = acc[j][i];
      if constexpr (ROWS) v[j] *= rsqrtf(ss[i] / (float)K + nrm.eps);
      v[j] += pb[j];
    }
    OT* const Cp = pv.C;
    const int64_t ldc = pv.ldc;
    if constexpr (RC > 1) {
      const bool res = pv.res != nullptr;
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        if (n + j >= Np) continue;
        OT o = from_f32<OT>(v[j]);
        if (res) o = from_f32<OT>(to_f32(o) + pr[j]);
        Cp[(int64_t)i * ldc + n + j] = o;
      }
    } else if constexpr (GATED) {
      const float gt = to_f32(from_f32<OT>(v[0])), up = to_f32(from_f32<OT>(v[1]));
      Cp[(int64_t)i * ldc + n] = from_f32<OT>(gt * sigmoidf_(gt) * up);
    } else {
      OT o = from_f32<OT>(v[0]);
      if (pv.res != nullptr) o = from_f32<OT>(to_f32(o) + pr[0]);
      Cp[(int64_t)i * ldc + n] = o;
    }
  }
}

template <typename T, typename OT>
void launch_gemv_products(const T* a, int64_t lda, DecodeProducts<T, OT>& P, int M, int K, bool gated,
                          const DecodeNorm& nz, hipStream_t st) {
  const int nprod = gated ? 1 : P.count;  // the gated pair shares its columns
  P.tile0[0] = 0;
  for (int i = 0; i < nprod; ++i) P.tile0[i + 1] = P.tile0[i] + P.N[i];
  if (gated) P.count = 1;
  const int ncols = P.tile0[nprod];
  const int nmode = decode_norm_mode(&nz);
  // Columns per wave: 4 for a vocabulary-wide product; 2 when that still gives 2048+ waves and
  // no wave straddles two products (each wave re-reads the activation row and the norm weights,
  // so fewer waves read less: the config-0 q/k/v launch, 4096 columns, 4.7 us against 7.5 us at
  // one column); else 1 (o_proj/down, 1024 columns, are fastest at 1).
  int rc = 1;
  if (!gated && nprod == 1 && ncols >= kGemvWideMin) {
    rc = kGemvWideCols;
  } else if (!gated && ncols >= kGemvTwoColMin) {
    rc = 2;
    for (int i = 0; i < nprod; ++i) rc = P.N[i] % 2 ? 1 : rc;
  }
  if (rc > 1) {
    const unsigned grid = (unsigned)((ncols + 4 * rc - 1) / (4 * rc));
#define QH_GR(MRV, NV, RCV) gemv_decode_kernel<T, OT, MRV, false, NV, RCV><<<grid, 256, 0, st>>>(a, lda, P, nz, M, K, ncols, P.count)
#define QH_GW(MRV, NV) \
  if (rc == 2) QH_GR(MRV, NV, 2); else QH_GR(MRV, NV, kGemvWideCols);
    if constexpr (std::is_same<T, OT>::value) {
      if (nmode == 1) {
        if (M == 1) { QH_GW(1, 1) } else if (M == 2) { QH_GW(2, 1) } else { QH_GW(4, 1) }
        return;
      }
      if (nmode == 2) {
        if (M == 1) { QH_GW(1, 2) } else if (M == 2) { QH_GW(2, 2) } else { QH_GW(4, 2) }
        return;
      }
    }
    if (M == 1) { QH_GW(1, 0) } else if (M == 2) { QH_GW(2, 0) } else { QH_GW(4, 0) }
#undef QH_GW
#undef QH_GR
    return;
  }
  const unsigned grid = (unsigned)((ncols + 3) / 4);
#define QH_GV(MRV, GV, NV) gemv_decode_kernel<T, OT, MRV, GV, NV><<<grid, 256, 0, st>>>(a, lda, P, nz, M, K, ncols, P.count)
#define QH_GV_M(MRV)                                                      \
  if constexpr (std::is_same<T, OT>::value) {                             \
    if (nmode == 1) {                                                     \
      if (gated) QH_GV(MRV, true, 1); else QH_GV(MRV, false, 1);          \
      return;                                                             \
    }                                                                     \
    if (nmode == 2) {                                                     \
      if (gated) QH_GV(MRV, true, 2); else QH_GV(MRV, false, 2);          \
      return;                                                             \
    }                                                                     \
  }                                                                       \
  if (gated) QH_GV(MRV, true, 0); else QH_GV(MRV, false, 0);
  if (M == 1) { QH_GV_M(1) } else if (M == 2) { QH_GV_M(2) } else { QH_GV_M(4) }
#undef QH_GV_M
#undef QH_GV
}

// ---------------------------------------------------------------------------
// Decode products for 4 < M <= 128 rows (batched decode, short prefill), both
// operands k-contiguous: one 1024-thread workgroup (16 wavefronts) per tile of
// R activation rows by C = 32 or 16 weight rows (output columns), all K:
//  * the tile's operands stream through a ring of NST LDS stages, chunk by
//    chunk of K: direct-to-LDS loads by the whole workgroup (1 KB per wave and
//    instruction, whole 128-byte lines), 16-byte slots XOR-swizzled per row so
//    the fragment reads are conflict-free; NST - 1 chunks are in flight while
//    one is multiplied, and a chunk's stage is refilled right after the
//    barrier that follows its last reader;
//  * per CU this moves R x K activation and C x K weight bytes, with R and C
//    chosen so that about one workgroup runs per CU (a 64-row q/k/v product:
//    32 x 32 tiles, 128 KB per CU, where a copy of all 64 rows per 16 weight
//    columns moved 160 KB);
//  * the 16 waves are KS K slices x 16 / KS (row group, column block) pairs;
//    slice s takes the 32-wide MFMA k-steps t = s (mod KS) in increasing order,
//    then the slices are summed in order through LDS. KS = 4 for K <= 1536,
//    else 16, so the summation order of every output depends on K alone: the
//    grouped, gated and single products of one K give equal bits, whatever the
//    tile shape or the number of columns.
// Several products sharing A (q/k/v, gate/up) are served by one launch: tiles
// are dealt to the products' columns in order. GATED (two products of equal N):
// a tile holds gate and up columns side by side (two column blocks, KS = 4, or
// the halves of one block, KS = 16) and the epilogue writes silu(gate) * up,
// each rounded to OT first, as separate products and the SiLU-mul kernel would.
// NORM: the rows of A are RMSNorm inputs h; the products use the weight
// operand round((w + wadd) * B) (formed here from the LDS fragments with
// scale_b, else folded into B beforehand: equal bits) and each output row is
// scaled by rsqrt(mean_k(h^2) + eps) after the sum over K (the row sums of
// squares: this lane's pairs by v_dot2, the four lane groups of a row, then
// the slices in order), then bias. Residual (per product, optional):
// C = round(round(product) + R), the residual-add kernel's rounding.
// ---------------------------------------------------------------------------
template <int N>
__device__ __forceinline__ void wait_vm_upto(int n) {
  // wait until at most n vector memory instructions of this wave are in flight (n <= N)
  if constexpr (N > 0) {
    if (n >= N) {
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(N));
      return;
    }
    wait_vm_upto<N - 1>(n);
  } else {
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  }
}

template <typename T, typename OT, int WR, int KS, int U, int NST, bool GATED, bool NORM>
__global__ __launch_bounds__(1024) void gemm_decode_kernel(const T* __restrict__ A, int64_t lda,
                                                           const DecodeProducts<T, OT> P, const DecodeNorm nrm, int M,
                                                           int K, int ms, int tiles, int scale_b) {
  constexpr int NWC = KS == 4 ? 2 : 1;           // 16-column blocks per tile
  constexpr int NWR = KS == 4 ? 2 : 1;           // row groups of waves
  constexpr int R = 16 * NWR * WR, C = 16 * NWC;  // tile rows and weight rows
  constexpr int OC = GATED ? C / 2 : C;           // output columns per tile
  constexpr int KC = 32 * KS * U;                 // K per chunk
  constexpr int S16 = KC / 8;                     // 16-byte slots per staged row
  constexpr int STAGE = (R + C) * KC * 2;
  constexpr int SLOTS = (R + C) * S16;            // slots per stage
  constexpr int D = (SLOTS + 1023) / 1024;        // loads per thread and chunk
  static_assert(S16 >= 16 && SLOTS % 64 == 0, "row swizzle and per-wave loads");
  static_assert(NST * STAGE <= 144 * 1024, "LDS stages");
  static_assert(16 * WR * 64 * 16 <= NST * STAGE, "K-slice partials reuse the stages");
  static_assert(D * (NST - 1) <= 63, "vmcnt");
  typedef typename Mfma<T>::v8 v8;
  __shared__ __align__(16) unsigned char smem[NST * STAGE];
  __shared__ float nss[NORM ? KS : 1][R];  // row sums of squares per K slice
  // workgroup -> (column tile, row group): the ms row groups of a tile get ids equal mod 8,
  // so they run on one XCD and read the tile's weights through the same L2
  ProductView<T, OT> pv = product_view(P, 0);  // a gated launch has one product
  view_now(pv);
  const T* Bup = P.B[1];  // GATED: the up projection
  int64_t ldbup = P.ldb[1];
  const T* biasup = P.bias[1];
  int count = P.count;
  if constexpr (GATED) {
    sgpr_now(Bup);
    sgpr_now(ldbup);
    sgpr_now(biasup);
  }
  sgpr_now(count);
  sgpr_now(A);
  sgpr_now(lda);
  const int bid = (int)blockIdx.x;
  const int rest = bid >> 3;
  const int mg = rest % ms;
  const int gtile = (rest / ms) * 8 + (bid & 7);
  if (gtile >= tiles) return;
  if (count > 1) pv = product_view(P, product_of(P, gtile));
  const int tile = gtile - pv.first;
  const int N = pv.N;
  const int m0 = mg * R;
  const int tid = (int)threadIdx.x, lane = tid & 63, wid = tid >> 6;
  // Non-gated epilogue: element e of the tile is output (grow, gn); thread tid writes the
  // elements tid, tid + 1024, ... Their residual is loaded here, before the weight stream,
  // so that its latency is not added after the reduction (C may be the residual: each
  // element is read and then written by the same thread).
  constexpr int EN = NWR * NWC * WR * 256;
  constexpr int EPT = GATED ? 1 : (EN + 1023) / 1024;
  auto epi_index = [&](int e, int& grow, int& gn) {
    const int g = e / (NWC * WR * 256), c = (e / (WR * 256)) % NWC, i = (e >> 8) % WR;
    const int r = (e >> 6) & 3, l = e & 63;
    grow = m0 + (g * WR + i) * 16 + (l >> 4) * 4 + r;
    gn = tile * OC + c * 16 + (l & 15);
  };
  float rpre[EPT];
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    rpre[k] = 0.f;
    if constexpr (!GATED) {
      const int e = tid + k * 1024;
      int grow, gn;
      epi_index(e, grow, gn);
      if (pv.res != nullptr && e < EN && grow < M && gn < N) rpre[k] = to_f32(pv.res[(int64_t)grow * pv.ldr + gn]);
    }
  }
  const int ks = wid % KS, st = wid / KS, rb = st / NWC, cb = st % NWC;
  const int li = lane & 15, q = lane >> 4;
  // source row of each of this thread's stage slots (fixed over the chunks): staged rows
  // 0..R-1 are activation rows (rows past M repeat row M - 1; their outputs are not
  // stored), R..R+C-1 weight rows (past N: row N - 1)
  const T* src[D];
  int soff[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int p = min(d * 1024 + tid, SLOTS - 1);
    const int r = p / S16;
    soff[d] = ((p % S16) ^ (r & 15)) * 8;
    if (r < R) {
      src[d] = A + (int64_t)min(m0 + r, M - 1) * lda;
    } else {
      const int j = r - R;
      int sel = 0, col;
      if constexpr (GATED) {
        sel = j / OC;  // gate rows, then up rows
        col = tile * OC + j % OC;
      } else {
        col = tile * C + j;
      }
      const T* bp = GATED && sel ? Bup : pv.B;
      const int64_t ldbp = GATED && sel ? ldbup : pv.ldb;
      src[d] = bp + (int64_t)min(col, N - 1) * ldbp;
    }
  }
  const uint32_t sbase = lds_addr(smem);
  int dw = 0;  // loads this wave issues per chunk (SLOTS is a multiple of 64)
#pragma unroll
  for (int d = 0; d < D; ++d) dw += d * 1024 + wid * 64 < SLOTS ? 1 : 0;
  auto issue = [&](int c) {
    const int k0 = c * KC;
    const uint32_t lb = sbase + (uint32_t)((c % NST) * STAGE);
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (d * 1024 + wid * 64 < SLOTS) {  // wave-uniform
        const int k = k0 + soff[d];
        lds_dma16(src[d] + (k < K ? k : 0), lb + (uint32_t)((d * 1024 + wid * 64) * 16));
      }
    }
  };
  const int nch = (K + KC - 1) / KC;
  for (int c = 0; c < min(nch, NST - 1); ++c) issue(c);
  v8 zero;
#pragma unroll
  for (int e = 0; e < 8; ++e) zero[e] = (T)0.f;
  f32x4 acc[WR];
  float sq[WR];
#pragma unroll
  for (int i = 0; i < WR; ++i) {
    acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    sq[i] = 0.f;
  }
  // NORM with scale_b: the weight row's norm-weight factor per lane (gate and up share it)
  for (int c = 0; c < nch; ++c) {
    wait_vm_upto<D * (NST - 2)>(dw * (min(nch, c + NST - 1) - 1 - c));  // chunk c has landed
    __syncthreads();  // ... for every wave, and chunk c - 1's stage is free
    if (c + NST - 1 < nch) issue(c + NST - 1);
    const unsigned char* sp = smem + (c % NST) * STAGE;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int sl = (u * KS + ks) * 4 + q;  // logical slot: k = c KC + 8 sl .. + 7
      const int k = c * KC + sl * 8;
      const bool kok = k < K;
      const int rB = R + cb * 16 + li;
      v8 b = kok ? *reinterpret_cast<const v8*>(sp + rB * (KC * 2) + ((sl ^ (rB & 15)) << 4)) : zero;
      if constexpr (NORM) {
        if (scale_b && kok) {  // round((w + wadd) * B), as the folded weights hold it
          const v8 w = *reinterpret_cast<const v8*>((const T*)nrm.w + k);
#pragma unroll
          for (int e = 0; e < 8; ++e) b[e] = from_f32<T>(to_f32(b[e]) * (to_f32(w[e]) + nrm.wadd));
        }
      }
#pragma unroll
      for (int i = 0; i < WR; ++i) {
        const int r = (rb * WR + i) * 16 + li;
        const v8 a = kok ? *reinterpret_cast<const v8*>(sp + r * (KC * 2) + ((sl ^ (r & 15)) << 4)) : zero;
        if constexpr (NORM) {
          if (cb == 0) sq[i] = sumsq8<T>(a, sq[i]);
        }
        acc[i] = mma16<T>(a, b, acc[i]);
      }
    }
  }
  if constexpr (NORM) {
#pragma unroll
    for (int i = 0; i < WR; ++i) {
      float v = sq[i];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      if (cb == 0 && q == 0) nss[ks][(rb * WR + i) * 16 + li] = v;
    }
  }
  __syncthreads();  // every wave's fragment reads are done: the partials reuse the stages
  f32x4* red = reinterpret_cast<f32x4*>(smem);
#pragma unroll
  for (int i = 0; i < WR; ++i) red[(wid * WR + i) * 64 + lane] = acc[i];
  __syncthreads();
  // element (row group g, column block c, row block i, lane l, row r of the lane's four):
  // the K slices summed in order
  auto slice_sum = [&](int g, int c, int i, int l, int r) {
    float v = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < KS; ++s2) v += red[(((g * NWC + c) * KS + s2) * WR + i) * 64 + l][r];
    return v;
  };
  auto row_factor = [&](int row) {
    float ss = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < KS; ++s2) ss += nss[s2][row];
    return rsqrtf(ss / (float)K + nrm.eps);
  };
  if constexpr (GATED) {
    constexpr int E = NWR * WR * (KS == 4 ? 256 : 128);
    for (int e = tid; e < E; e += 1024) {
      int g, i, l, lu, cu, oc, r;
      if constexpr (KS == 4) {  // column block 0 gate, 1 up
        g = e / (WR * 256);
        i = (e >> 8) % WR;
        r = (e >> 6) & 3;
        l = e & 63;
        lu = l;
        cu = 1;
        oc = l & 15;
      } else {  // lanes 0-7 of a block gate, 8-15 up
        g = 0;
        i = e >> 7;
        r = (e >> 5) & 3;
        const int lq = (e >> 3) & 3, lc = e & 7;
        l = lq * 16 + lc;
        lu = l + 8;
        cu = 0;
        oc = lc;
      }
      const int row = (g * WR + i) * 16 + (l >> 4) * 4 + r;
      const int grow = m0 + row, gn = tile * OC + oc;
      if (grow >= M || gn >= N) continue;
      float vg = slice_sum(g, 0, i, l, r), vu = slice_sum(g, cu, i, lu, r);
      if constexpr (NORM) {
        const float f = row_factor(row);
        vg *= f;
        vu *= f;
      }
      const T* bg = pv.bias;
      const T* bu = biasup;
      const float gt = to_f32(from_f32<OT>(vg + (bg ? to_f32(bg[gn]) : 0.f)));
      const float up = to_f32(from_f32<OT>(vu + (bu ? to_f32(bu[gn]) : 0.f)));
      pv.C[(int64_t)grow * pv.ldc + gn] = from_f32<OT>(gt * sigmoidf_(gt) * up);
    }
  } else {
    const T* bias = pv.bias;
    const bool has_res = pv.res != nullptr;
    OT* const Cp = pv.C;
    const int64_t ldc = pv.ldc;
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int e = tid + k * 1024;
      if (e >= EN) break;
      const int g = e / (NWC * WR * 256), c = (e / (WR * 256)) % NWC, i = (e >> 8) % WR;
      const int r = (e >> 6) & 3, l = e & 63;
      const int row = (g * WR + i) * 16 + (l >> 4) * 4 + r;
      int grow, gn;
      epi_index(e, grow, gn);
      if (grow >= M || gn >= N) continue;
      float v = slice_sum(g, c, i, l, r);
      if constexpr (NORM) v *= row_factor(row);
      v += bias ? to_f32(bias[gn]) : 0.f;
      OT o = from_f32<OT>(v);
      if (has_res) o = from_f32<OT>(to_f32(o) + rpre[k]);
      Cp[(int64_t)grow * ldc + gn] = o;
    }
  }
}

// Launch shape: K slices (4 or 16, by K alone), rows per tile (R = 16 x NWR x WR), row groups
// per column tile (ms, until about one workgroup per CU), and the chunk ring (U k-steps per
// slice and chunk, NST stages of at most 48 KB).
struct DecodePlan {
  int ks, wr, ms, oc, tiles;
};

static DecodePlan decode_plan(int M, int K, bool gated, int count, const int* N) {
  DecodePlan p{};
  p.ks = K <= 1536 ? 4 : 16;
  const int nwr = p.ks == 4 ? 2 : 1, c = p.ks == 4 ? 32 : 16;
  const int wrmax = p.ks == 4 ? 4 : 2;
  p.oc = gated ? c / 2 : c;
  p.tiles = 0;
  for (int i = 0; i < (gated ? 1 : count); ++i) p.tiles += (N[i] + p.oc - 1) / p.oc;
  const int mtu = (M + 16 * nwr - 1) / (16 * nwr);
  int ms = 1;
  while ((mtu + ms - 1) / ms > wrmax) ms *= 2;
  while (ms < mtu && p.tiles * ms * 2 <= 256) ms *= 2;
  const int wr = (mtu + ms - 1) / ms;
  p.wr = wr <= 1 ? 1 : (wr <= 2 ? 2 : 4);
  p.ms = ms;
  return p;
}

template <typename T, typename OT>
int launch_decode_products(const T* a, int64_t lda, DecodeProducts<T, OT>& P, int M, int K, bool gated,
                           hipStream_t st, const DecodeNorm* nrm = nullptr) {
  const int nmode = decode_norm_mode(nrm);
  const bool norm = nmode != 0;
  if (norm && !std::is_same<T, OT>::value) return QH_E_ARG;
  const DecodeNorm nz = norm ? *nrm : DecodeNorm{nullptr, 0.f, 0.f, 0};
  if (M <= kGemvMaxRows) {
    launch_gemv_products<T, OT>(a, lda, P, M, K, gated, nz, st);
    return QH_OK;
  }
  const DecodePlan d = decode_plan(M, K, gated, P.count, P.N);
  const int nprod = gated ? 1 : P.count;
  P.tile0[0] = 0;
  for (int i = 0; i < nprod; ++i) P.tile0[i + 1] = P.tile0[i] + (P.N[i] + d.oc - 1) / d.oc;
  if (gated) P.count = 1;
  const int grid = (d.tiles + 7) / 8 * 8 * d.ms;
  const int scale_b = nmode == 1 ? 1 : 0;
  // (WR, KS, U, NST): stages of 32 x 32 + 32 rows x 256 k (32 KB), 64 + 32 x 256 (48 KB),
  // 128 + 32 x 128 (40 KB), 16 + 16 x 512 (32 KB), 32 + 16 x 512 (48 KB)
#define QH_DK(WRV, KSV, UV, NSTV, GV, NV)                                                     \
  gemm_decode_kernel<T, OT, WRV, KSV, UV, NSTV, GV, NV><<<grid, 1024, 0, st>>>(a, lda, P, nz, M, K, d.ms, \
                                                                               d.tiles, scale_b)
#define QH_DK_S(GV, NV)                                               \
  if (d.ks == 4) {                                                    \
    if (d.wr == 1) QH_DK(1, 4, 2, 4, GV, NV);                         \
    else if (d.wr == 2) QH_DK(2, 4, 2, 3, GV, NV);                    \
    else QH_DK(4, 4, 1, 3, GV, NV);                                   \
  } else {                                                            \
    if (d.wr == 1) QH_DK(1, 16, 1, 4, GV, NV);                        \
    else QH_DK(2, 16, 1, 3, GV, NV);                                  \
  }
  if constexpr (std::is_same<T, OT>::value) {
    if (gated) {
      if (norm) { QH_DK_S(true, true) } else { QH_DK_S(true, false) }
      return QH_OK;
    }
    if (norm) {
      QH_DK_S(false, true)
      return QH_OK;
    }
  }
  QH_DK_S(false, false)
#undef QH_DK_S
#undef QH_DK
  return QH_OK;
}

// A norm-prologue launch fits every shape qh_gemm_multi takes (M <= 128): the batch-1 kernel
// and the chunked kernel both sum the squares over any K.
static bool decode_norm_fits(int M, int K, bool gated, int count, const int64_t* N) {
  (void)M;
  (void)K;
  (void)gated;
  (void)count;
  (void)N;
  return true;
}

template <typename T, typename OT>
void launch_decode_gemm(const T* a, int64_t lda, const T* b, int64_t ldb, OT* c, int64_t ldc, const T* bi, int M,
                        int N, int K, hipStream_t st) {
  DecodeProducts<T, OT> P = {};
  P.B[0] = b;
  P.C[0] = c;
  P.bias[0] = bi;
  P.ldb[0] = ldb;
  P.ldc[0] = ldc;
  P.N[0] = N;
  P.count = 1;
  launch_decode_products<T, OT>(a, lda, P, M, K, false, st);
}

// ---------------------------------------------------------------------------
// Grouped GEMM over expert segments (MoE). The rows of the left operand are
// grouped by expert: segment e is rows [seg[e], seg[e+1]) and multiplies
// expert e's weight matrix, found through a device table of pointers (the
// experts' parameters stay separate tensors). M-tiles never straddle a
// segment: toff[e] is the first M-tile of expert e (prefix sum of
// ceil(n_e / 128)) and the grid's x extent is an upper bound (extra
// workgroups exit). Modes:
//   MOE_GATED:  A rows gathered from X through rows[] (token of each routed
//               row); the 128 B-tile rows are 32-row blocks of gate and up
//               weights in turn, so a wave's two 32-column MFMA tiles hold
//               the same columns of gate and up and the epilogue writes
//               silu(gate) * up (each rounded to T first, as the expert MLP's
//               two GEMMs and SiLU-mul kernel would);
//   MOE_SCALED: A rows contiguous; the epilogue writes round(acc) * w[row]
//               rounded, the routing-weight scaling of the expert output.
// ---------------------------------------------------------------------------
enum { MOE_GATED = 0, MOE_SCALED = 1 };

// Rows of a ROWS x BK tile read through one row pointer per staging register
// (nullptr = zero row); k-contiguous LDS layout as TileLoader<.., false>.
template <typename T, int ROWS>
struct RowTileLoader {
  static constexpr int NREG = ROWS / 32;
  uint4 r[NREG];
  const T* rowp[NREG];
  __device__ __forceinline__ void load(int k0, int K) {
    const int tid = threadIdx.x;
    const uint4 z = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < NREG; ++i) {
      const int gk = k0 + ((tid + i * 256) & 7) * 8;
      if (rowp[i] != nullptr && gk < K) r[i] = *reinterpret_cast<const uint4*>(rowp[i] + gk);
      else r[i] = z;
    }
  }
  __device__ __forceinline__ void store(T* __restrict__ S) const {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < NREG; ++i) {
      const int c = tid + i * 256;
      *reinterpret_cast<uint4*>(S + (c >> 3) * LDS_LD + (c & 7) * 8) = r[i];
    }
  }
  // tile row of staging register i
  static __device__ __forceinline__ int row_of(int i) { return (threadIdx.x + i * 256) >> 3; }
};

template <typename T, int MODE>
__global__ __launch_bounds__(256) void moe_gemm_kernel(const T* __restrict__ A, int64_t lda,
                                                       const int* __restrict__ rows, const T* const* __restrict__ Bt,
                                                       int64_t ldb, T* __restrict__ C, int64_t ldc,
                                                       const T* __restrict__ wrow, const int* __restrict__ seg,
                                                       const int* __restrict__ toff, int E, int N, int K) {
  constexpr int BM = 128, BN = 128, WM = 2, WN = 2;
  constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
  typedef typename Mfma<T>::v8 v8;
  __shared__ __attribute__((aligned(16))) T smem[2][(BM + BN) * LDS_LD];

  const int tm = blockIdx.x;
  if (tm >= toff[E]) return;
  int lo = 0, hi = E;  // largest e with toff[e] <= tm
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (toff[mid] <= tm) lo = mid;
    else hi = mid;
  }
  const int e = lo;
  const int r0 = seg[e] + (tm - toff[e]) * BM, r1 = seg[e + 1];
  // MOE_GATED covers 64 output columns (gate and up), MOE_SCALED 128.
  const int n0 = blockIdx.y * (MODE == MOE_GATED ? 64 : 128);

  RowTileLoader<T, BM> la;
  RowTileLoader<T, BN> lb;
#pragma unroll
  for (int i = 0; i < RowTileLoader<T, BM>::NREG; ++i) {
    const int r = r0 + RowTileLoader<T, BM>::row_of(i);
    const int src = MODE == MOE_GATED ? (r < r1 ? rows[r] : -1) : (r < r1 ? r : -1);
    la.rowp[i] = src >= 0 ? A + (int64_t)src * lda : nullptr;
  }
#pragma unroll
  for (int i = 0; i < RowTileLoader<T, BN>::NREG; ++i) {
    const int tr = RowTileLoader<T, BN>::row_of(i);
    const T* W;
    int col;
    if (MODE == MOE_GATED) {
      const int blk = tr >> 5;
      W = Bt[2 * e + (blk & 1)];
      col = n0 + (blk >> 1) * 32 + (tr & 31);
    } else {
      W = Bt[e];
      col = n0 + tr;
    }
    lb.rowp[i] = col < N ? W + (int64_t)col * ldb : nullptr;
  }

  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid / WN, wn = wid % WN;
  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = zero16();

  const int nk = (K + BK - 1) / BK;
  la.load(0, K);
  lb.load(0, K);
  la.store(smem[0]);
  lb.store(smem[0] + BM * LDS_LD);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      la.load((kt + 1) * BK, K);
      lb.load((kt + 1) * BK, K);
    }
    const T* As = smem[buf];
    const T* Bs = smem[buf] + BM * LDS_LD;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      v8 af[TM], bf[TN];
      const int koff = kk * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const v8*>(As + (wm * WTM + i * 32 + (lane & 31)) * LDS_LD + koff);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bf[j] = *reinterpret_cast<const v8*>(Bs + (wn * WTN + j * 32 + (lane & 31)) * LDS_LD + koff);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = Mfma<T>::mma(af[i], bf[j], acc[i][j]);
    }
    if (more) {
      la.store(smem[buf ^ 1]);
      lb.store(smem[buf ^ 1] + BM * LDS_LD);
    }
    __syncthreads();
  }

  // C layout of a 32x32 tile: column lane % 32, rows 8 g + 4 (lane / 32) + r.
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int rbase = r0 + wm * WTM + i * 32 + (lane >> 5) * 4;
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = rbase + g * 8 + r;
        if (row >= r1) continue;
        if constexpr (MODE == MOE_GATED) {
          const int col = n0 + wn * 32 + (lane & 31);
          if (col < N) {
            const float gt = to_f32((T)acc[i][0][g * 4 + r]), up = to_f32((T)acc[i][1][g * 4 + r]);
            C[(int64_t)row * ldc + col] = from_f32<T>(gt * sigmoidf_(gt) * up);
          }
        } else {
          const float w = to_f32(wrow[row]);
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * WTN + j * 32 + (lane & 31);
            if (col < N) C[(int64_t)row * ldc + col] = from_f32<T>(to_f32((T)acc[i][j][g * 4 + r]) * w);
          }
        }
      }
  }
}

// ---------------------------------------------------------------------------
// Generic VALU GEMM (fp32 and shapes the MFMA path does not take). 64x64 tile,
// 256 threads each owning a 4x4 block, fp32 accumulation.
// ---------------------------------------------------------------------------
template <typename T, typename OT, bool AT, bool BT>
__global__ __launch_bounds__(256) void gemm_generic_kernel(const T* __restrict__ A, int64_t lda,
                                                           const T* __restrict__ B, int64_t ldb, OT* __restrict__ C,
                                                           int64_t ldc, const T* __restrict__ bias, int M, int N,
                                                           int K) {
  __shared__ float As[16][64 + 1];
  __shared__ float Bs[16][64 + 1];
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int e = threadIdx.x; e < 16 * 64; e += 256) {
      const int kk = e / 64, ii = e % 64;
      const int gk = k0 + kk;
      const int gm = m0 + ii, gn = n0 + ii;
      float a = 0.f, b = 0.f;
      if (gk < K && gm < M) a = to_f32(AT ? A[(int64_t)gk * lda + gm] : A[(int64_t)gm * lda + gk]);
      if (gk < K && gn < N) b = to_f32(BT ? B[(int64_t)gk * ldb + gn] : B[(int64_t)gn * ldb + gk]);
      As[kk][ii] = a;
      Bs[kk][ii] = b;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * b[j];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = m0 + ty * 4 + i;
    if (row >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = n0 + tx * 4 + j;
      if (col < N) C[(int64_t)row * ldc + col] = from_f32<OT>(acc[i][j] + (bias ? to_f32(bias[col]) : 0.f));
    }
  }
}

template <typename T, typename OT, int BM, int BN, int WM, int WN, bool AT, bool BT>
void launch_mfma(const T* A, int64_t lda, const T* B, int64_t ldb, OT* C, int64_t ldc, const T* bias, int M, int N,
                 int K, hipStream_t st) {
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  if (tm == 1 && !BT)  // one row of tiles: every weight element is read once (the batched LM head)
    gemm_mfma_kernel<T, OT, BM, BN, WM, WN, AT, BT, true><<<tn, 256, 0, st>>>(A, lda, B, ldb, C, ldc, bias, M, N, K,
                                                                              tm, tn);
  else
    gemm_mfma_kernel<T, OT, BM, BN, WM, WN, AT, BT><<<tm * tn, 256, 0, st>>>(A, lda, B, ldb, C, ldc, bias, M, N, K,
                                                                             tm, tn);
}

template <typename T, typename OT, bool AT, bool BT>
void launch_mfma_pick(const T* A, int64_t lda, const T* B, int64_t ldb, OT* C, int64_t ldc, const T* bias, int M,
                      int N, int K, hipStream_t st) {
  if (M > 64)
    launch_mfma<T, OT, 128, 128, 2, 2, AT, BT>(A, lda, B, ldb, C, ldc, bias, M, N, K, st);
  else
    launch_mfma<T, OT, 64, 128, 1, 4, AT, BT>(A, lda, B, ldb, C, ldc, bias, M, N, K, st);
}

template <typename T, typename OT>
int gemm_typed(int ta, int tb, int M, int N, int K, const void* A, int64_t lda, const void* B, int64_t ldb, void* C,
               int64_t ldc, const void* bias, void* ws, int64_t ws_bytes, hipStream_t st) {
  const T* a = (const T*)A;
  const T* b = (const T*)B;
  OT* c = (OT*)C;
  const T* bi = (const T*)bias;
  constexpr bool is_mfma_type = !std::is_same<T, float>::value;
  if constexpr (is_mfma_type) {
    // Decode path for small M (up to 128 rows: decode batches and short
    // prefills), both operands k-contiguous; wide outputs with M > 16 (the
    // batched LM head) stream better through the tiled kernel.
    if (M <= 128 && !(M > 16 && N > 8192) && !ta && !tb && K % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 &&
        aligned16(A) && aligned16(B)) {
      launch_decode_gemm<T, OT>(a, lda, b, ldb, c, ldc, bi, M, N, K, st);
      return QH_OK;
    }
    // MFMA path: 16-byte aligned operand rows along their contiguous dimension.
    const bool a_ok = aligned16(A) && lda % 8 == 0 && (ta ? M % 8 == 0 : K % 8 == 0);
    const bool b_ok = aligned16(B) && ldb % 8 == 0 && (tb ? N % 8 == 0 : K % 8 == 0);
    if (a_ok && b_ok) {
      // Few output tiles and long K: split K when the caller gave a workspace.
      const int splits = qh_gemm_splitk_count(M, N, K);
      if (splits > 1 && ws != nullptr && ws_bytes >= (int64_t)splits * M * N * 4)
        return qh_gemm_splitk_dispatch(ta, tb, M, N, K, A, lda, B, ldb, C, ldc, bias, qh_dtype_of<T>(),
                                       qh_dtype_of<OT>(), splits, ws, st);
      // Large outputs: the 256x256 direct-to-LDS tile kernel.
      const int64_t big_tiles = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
      if (M >= 256 && N >= 256 && big_tiles >= 128)
        return qh_gemm_tile_dispatch(ta, tb, M, N, K, A, lda, B, ldb, C, ldc, bias, qh_dtype_of<T>(),
                                     qh_dtype_of<OT>(), st);
      if (!ta && !tb) launch_mfma_pick<T, OT, false, false>(a, lda, b, ldb, c, ldc, bi, M, N, K, st);
      else if (!ta && tb) launch_mfma_pick<T, OT, false, true>(a, lda, b, ldb, c, ldc, bi, M, N, K, st);
      else if (ta && tb) launch_mfma_pick<T, OT, true, true>(a, lda, b, ldb, c, ldc, bi, M, N, K, st);
      else launch_mfma_pick<T, OT, true, false>(a, lda, b, ldb, c, ldc, bi, M, N, K, st);
      return QH_OK;
    }
  }
  dim3 grid((N + 63) / 64, (M + 63) / 64);
  if (!ta && !tb) gemm_generic_kernel<T, OT, false, false><<<grid, 256, 0, st>>>(a, lda, b, ldb, c, ldc, bi, M, N, K);
  else if (!ta && tb) gemm_generic_kernel<T, OT, false, true><<<grid, 256, 0, st>>>(a, lda, b, ldb, c, ldc, bi, M, N, K);
  else if (ta && tb) gemm_generic_kernel<T, OT, true, true><<<grid, 256, 0, st>>>(a, lda, b, ldb, c, ldc, bi, M, N, K);
  else gemm_generic_kernel<T, OT, true, false><<<grid, 256, 0, st>>>(a, lda, b, ldb, c, ldc, bi, M, N, K);
  return QH_OK;
}

// Deterministic column sum (bias gradient): out[n] = sum_m X[m, n].
template <typename T, typename OT>
__global__ __launch_bounds__(256) void colsum_kernel(const T* __restrict__ X, int64_t ldx, int M, int N,
                                                     OT* __restrict__ out) {
  __shared__ float part[16][17];
  const int cl = threadIdx.x & 15, sub = threadIdx.x >> 4;
  const int n = blockIdx.x * 16 + cl;
  float s = 0.f;
  if (n < N)
    for (int m = sub; m < M; m += 16) s += to_f32(X[(int64_t)m * ldx + n]);
  part[sub][cl] = s;
  __syncthreads();
  if (sub == 0 && n < N) {
    float t = 0.f;
    for (int i = 0; i < 16; ++i) t += part[i][cl];
    out[n] = from_f32<OT>(t);
  }
}

}  // namespace

extern "C" int64_t qh_gemm_workspace(int64_t M, int64_t N, int64_t K, int dtype) {
  if (dtype != QH_BF16 && dtype != QH_F16) return 0;
  const int s = qh_gemm_splitk_count(M, N, K);
  return s > 1 ? (int64_t)s * M * N * 4 : 0;
}

extern "C" int qh_gemm(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
                       const void* B, int64_t ldb, void* C, int64_t ldc, const void* bias, int dtype, int out_dtype,
                       void* stream) {
  return qh_gemm_ws(trans_a, trans_b, M, N, K, A, lda, B, ldb, C, ldc, bias, dtype, out_dtype, nullptr, 0, stream);
}

extern "C" int qh_gemm_ws(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
                          const void* B, int64_t ldb, void* C, int64_t ldc, const void* bias, int dtype, int out_dtype,
                          void* ws, int64_t ws_bytes, void* stream) {
  QH_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "qh_gemm: negative shape");
  QH_CHECK_ARG(M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31), "qh_gemm: dimension exceeds 2^31");
  QH_CHECK_ARG(ldc >= N, "qh_gemm: ldc %lld < N %lld", (long long)ldc, (long long)N);
  QH_CHECK_ARG(trans_a ? lda >= M : lda >= K, "qh_gemm: lda too small");
  QH_CHECK_ARG(trans_b ? ldb >= N : ldb >= K, "qh_gemm: ldb too small");
  if (M == 0 || N == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  if (K == 0) {
    QH_CHECK_ARG(bias == nullptr && ldc == N, "qh_gemm: K == 0 with bias or strided C is not supported");
    return qh_zero(C, M * N * (out_dtype == QH_F32 ? 4 : 2), stream);
  }
  int rc = QH_OK;
#define QH_GEMM_OUT(T)                                                                                           \
  switch (out_dtype) {                                                                                          \
    case QH_F32: rc = gemm_typed<T, float>(trans_a, trans_b, (int)M, (int)N, (int)K, A, lda, B, ldb, C, ldc, bias, ws, ws_bytes, st); break; \
    case QH_F16: rc = gemm_typed<T, f16_t>(trans_a, trans_b, (int)M, (int)N, (int)K, A, lda, B, ldb, C, ldc, bias, ws, ws_bytes, st); break; \
    case QH_BF16: rc = gemm_typed<T, bf16_t>(trans_a, trans_b, (int)M, (int)N, (int)K, A, lda, B, ldb, C, ldc, bias, ws, ws_bytes, st); break; \
    default: qh::set_error("qh_gemm: bad out dtype %d", out_dtype); return QH_E_DTYPE;                          \
  }
  QH_DISPATCH_DTYPE(dtype, T, "qh_gemm", QH_GEMM_OUT(T));
#undef QH_GEMM_OUT
  if (rc) return rc;
  QH_CHECK_LAUNCH("qh_gemm_ws");
  return QH_OK;
}

extern "C" int qh_gemm_multi_ex(int64_t M, int64_t K, const void* A, int64_t lda, int count, const void* const* B,
                                const int64_t* ldb, const int64_t* N, void* const* C, const int64_t* ldc,
                                const void* const* bias, const void* const* residual, const int64_t* ldr, int gated,
                                const void* norm_w, int norm_wdtype, float eps, int one_plus, int dtype,
                                void* stream) {
  QH_CHECK_ARG(count >= 1 && count <= kMaxProducts, "qh_gemm_multi: 1..%d products", kMaxProducts);
  QH_CHECK_ARG(M >= 0 && M <= 128 && K > 0 && K < (1ll << 31), "qh_gemm_multi: needs 0 <= M <= 128 and K > 0");
  QH_CHECK_ARG(!gated || (count == 2 && N[0] == N[1]), "qh_gemm_multi: gated needs two products of equal N");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_gemm_multi: bf16/f16 only");
  QH_CHECK_ARG(aligned16(A) && lda % 8 == 0 && lda >= K && K % 8 == 0,
               "qh_gemm_multi: A must be 16-byte aligned with K, lda multiples of 8");
  for (int i = 0; i < count; ++i) {
    QH_CHECK_ARG(N[i] > 0 && N[i] < (1ll << 31) && aligned16(B[i]) && ldb[i] % 8 == 0 && ldb[i] >= K,
                 "qh_gemm_multi: product %d: bad B or N", i);
    QH_CHECK_ARG((gated && i == 1) || (C[i] != nullptr && ldc[i] >= N[i]), "qh_gemm_multi: product %d: bad C", i);
    QH_CHECK_ARG(residual == nullptr || residual[i] == nullptr || (!gated && ldr != nullptr && ldr[i] >= N[i]),
                 "qh_gemm_multi: product %d: residual needs a non-gated product and ldr >= N", i);
  }
  QH_CHECK_ARG(norm_w == nullptr || (norm_wdtype == dtype && aligned16(norm_w)),
               "qh_gemm_multi: the norm weight must have the activation dtype and be 16-byte aligned");
  QH_CHECK_ARG(norm_w == nullptr || M == 0 || decode_norm_fits((int)M, (int)K, gated != 0, count, N),
               "qh_gemm_multi: the norm prologue does not fit M=%lld K=%lld (see qh_gemm_multi_norm_fits)",
               (long long)M, (long long)K);
  if (M == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const DecodeNorm nrm{norm_w, eps, one_plus ? 1.f : 0.f, 0};
  int rc = QH_OK;
#define QH_MULTI(T)                                                                                     \
  {                                                                                                     \
    DecodeProducts<T, T> P = {};                                                                        \
    for (int i = 0; i < count; ++i) {                                                                   \
      P.B[i] = (const T*)B[i];                                                                          \
      P.C[i] = (T*)C[i];                                                                                \
      P.bias[i] = bias ? (const T*)bias[i] : nullptr;                                                   \
      P.res[i] = residual ? (const T*)residual[i] : nullptr;                                            \
      P.ldb[i] = ldb[i];                                                                                \
      P.ldc[i] = ldc[i];                                                                                \
      P.ldr[i] = residual && residual[i] ? ldr[i] : 0;                                                  \
      P.N[i] = (int)N[i];                                                                               \
    }                                                                                                   \
    P.count = count;                                                                                    \
    rc = launch_decode_products<T, T>((const T*)A, lda, P, (int)M, (int)K, gated != 0, st, &nrm);   \
  }
  if (dtype == QH_BF16) QH_MULTI(bf16_t) else QH_MULTI(f16_t)
#undef QH_MULTI
  if (rc) {
    qh::set_error("qh_gemm_multi: the norm prologue does not fit M=%lld K=%lld", (long long)M, (long long)K);
    return rc;
  }
  QH_CHECK_LAUNCH("qh_gemm_multi");
  return QH_OK;
}

extern "C" int qh_gemm_multi_rms(int64_t M, int64_t K, const void* A, int64_t lda, int count, const void* const* B,
                                 const int64_t* ldb, const int64_t* N, void* const* C, const int64_t* ldc,
                                 const void* const* bias, int gated, float eps, int dtype, void* stream) {
  QH_CHECK_ARG(count >= 1 && count <= kMaxProducts, "qh_gemm_multi_rms: 1..%d products", kMaxProducts);
  QH_CHECK_ARG(M >= 0 && M <= 128 && K > 0 && K < (1ll << 31), "qh_gemm_multi_rms: needs 0 <= M <= 128 and K > 0");
  QH_CHECK_ARG(!gated || (count == 2 && N[0] == N[1]), "qh_gemm_multi_rms: gated needs two products of equal N");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_gemm_multi_rms: bf16/f16 only");
  QH_CHECK_ARG(aligned16(A) && lda % 8 == 0 && lda >= K && K % 8 == 0,
               "qh_gemm_multi_rms: A must be 16-byte aligned with K, lda multiples of 8");
  for (int i = 0; i < count; ++i) {
    QH_CHECK_ARG(N[i] > 0 && N[i] < (1ll << 31) && aligned16(B[i]) && ldb[i] % 8 == 0 && ldb[i] >= K,
                 "qh_gemm_multi_rms: product %d: bad B or N", i);
    QH_CHECK_ARG((gated && i == 1) || (C[i] != nullptr && ldc[i] >= N[i]), "qh_gemm_multi_rms: product %d: bad C",
                 i);
  }
  if (M == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const DecodeNorm nrm{nullptr, eps, 0.f, 1};
  int rc = QH_OK;
#define QH_MULTI(T)                                                                                     \
  {                                                                                                     \
    DecodeProducts<T, T> P = {};                                                                        \
    for (int i = 0; i < count; ++i) {                                                                   \
      P.B[i] = (const T*)B[i];                                                                          \
      P.C[i] = (T*)C[i];                                                                                \
      P.bias[i] = bias ? (const T*)bias[i] : nullptr;                                                   \
      P.ldb[i] = ldb[i];                                                                                \
      P.ldc[i] = ldc[i];                                                                                \
      P.N[i] = (int)N[i];                                                                               \
    }                                                                                                   \
    P.count = count;                                                                                    \
    rc = launch_decode_products<T, T>((const T*)A, lda, P, (int)M, (int)K, gated != 0, st, &nrm);   \
  }
  if (dtype == QH_BF16) QH_MULTI(bf16_t) else QH_MULTI(f16_t)
#undef QH_MULTI
  if (rc) {
    qh::set_error("qh_gemm_multi_rms: launch failed (M=%lld K=%lld)", (long long)M, (long long)K);
    return rc;
  }
  QH_CHECK_LAUNCH("qh_gemm_multi_rms");
  return QH_OK;
}

extern "C" int qh_gemm_multi(int64_t M, int64_t K, const void* A, int64_t lda, int count, const void* const* B,
                             const int64_t* ldb, const int64_t* N, void* const* C, const int64_t* ldc,
                             const void* const* bias, int gated, int dtype, void* stream) {
  return qh_gemm_multi_ex(M, K, A, lda, count, B, ldb, N, C, ldc, bias, nullptr, nullptr, gated, nullptr, QH_F32,
                          0.f, 0, dtype, stream);
}

extern "C" int64_t qh_gemm_multi_norm_fits(int64_t M, int64_t K, int gated, int count, const int64_t* N) {
  if (M < 0 || M > 128 || K <= 0 || K >= (1ll << 31) || count < 1 || count > kMaxProducts) return 0;
  if (M == 0) return 1;
  return decode_norm_fits((int)M, (int)K, gated != 0, count, N) ? 1 : 0;
}

extern "C" int qh_moe_gemm(int mode, const void* A, int64_t lda, const int32_t* rows, const void* const* B_table,
                           int64_t ldb, void* C, int64_t ldc, const void* wrow, const int32_t* seg_off,
                           const int32_t* tile_off, int64_t R, int64_t E, int64_t N, int64_t K, int dtype,
                           void* stream) {
  QH_CHECK_ARG(mode == MOE_GATED || mode == MOE_SCALED, "qh_moe_gemm: bad mode %d", mode);
  QH_CHECK_ARG(R >= 0 && E > 0 && E < (1 << 20) && N > 0 && K > 0 && N < (1ll << 31) && K < (1ll << 31),
               "qh_moe_gemm: bad shape");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_moe_gemm: bf16/f16 only");
  QH_CHECK_ARG(aligned16(A) && lda % 8 == 0 && K % 8 == 0 && lda >= K && ldb % 8 == 0 && ldb >= K && ldc >= N,
               "qh_moe_gemm: operands must be 16-byte aligned with K, lda, ldb multiples of 8");
  QH_CHECK_ARG(mode != MOE_GATED || rows != nullptr, "qh_moe_gemm: gated mode gathers through rows");
  QH_CHECK_ARG(mode != MOE_SCALED || wrow != nullptr, "qh_moe_gemm: scaled mode needs the row weights");
  if (R == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  // upper bound of the M-tiles: every expert may leave one partial tile
  const int64_t mt = (R + 127) / 128 + E;
  const int64_t nt = (N + (mode == MOE_GATED ? 63 : 127)) / (mode == MOE_GATED ? 64 : 128);
  QH_CHECK_ARG(mt < (1ll << 31) && nt < 65536, "qh_moe_gemm: too many tiles");
  dim3 grid((unsigned)mt, (unsigned)nt);
#define QH_MOE(T, MD)                                                                                          \
  moe_gemm_kernel<T, MD><<<grid, 256, 0, st>>>((const T*)A, lda, rows, (const T* const*)B_table, ldb, (T*)C,  \
                                                 ldc, (const T*)wrow, seg_off, tile_off, (int)E, (int)N, (int)K)
  if (dtype == QH_BF16) {
    if (mode == MOE_GATED) QH_MOE(bf16_t, MOE_GATED); else QH_MOE(bf16_t, MOE_SCALED);
  } else {
    if (mode == MOE_GATED) QH_MOE(f16_t, MOE_GATED); else QH_MOE(f16_t, MOE_SCALED);
  }
#undef QH_MOE
  QH_CHECK_LAUNCH("qh_moe_gemm");
  return QH_OK;
}

extern "C" int qh_colsum(const void* X, int64_t ldx, int64_t M, int64_t N, void* out, int dtype, int out_dtype,
                         void* stream) {
  QH_CHECK_ARG(M >= 0 && N >= 0 && ldx >= N, "qh_colsum: bad shape");
  QH_CHECK_ARG(M < (1ll << 31) && N < (1ll << 31), "qh_colsum: dimension exceeds 2^31");
  if (N == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const int grid = (int)ceil_div(N, 16);
#define QH_CS_OUT(T)                                                                                         \
  switch (out_dtype) {                                                                                      \
    case QH_F32: colsum_kernel<T, float><<<grid, 256, 0, st>>>((const T*)X, ldx, (int)M, (int)N, (float*)out); break; \
    case QH_F16: colsum_kernel<T, f16_t><<<grid, 256, 0, st>>>((const T*)X, ldx, (int)M, (int)N, (f16_t*)out); break; \
    case QH_BF16: colsum_kernel<T, bf16_t><<<grid, 256, 0, st>>>((const T*)X, ldx, (int)M, (int)N, (bf16_t*)out); break; \
    default: qh::set_error("qh_colsum: bad out dtype"); return QH_E_DTYPE;                                  \
  }
  QH_DISPATCH_DTYPE(dtype, T, "qh_colsum", QH_CS_OUT(T));
#undef QH_CS_OUT
  QH_CHECK_LAUNCH("qh_colsum");
  return QH_OK;
}
