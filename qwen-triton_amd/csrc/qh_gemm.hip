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
//  * M <= 128 (decode, short prefill) uses 1024-thread workgroups of MFMA
//    16x16x32 whose 16 wavefronts split K, so the weight matrix is requested
//    in one or two memory round trips; partials are summed through LDS in a
//    fixed order.
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
// Skinny GEMM for M <= 128 (decode), "NN" layout (both operands k-contiguous).
// MFMA 16x16x32 with operand fragments loaded straight from global memory
// (the activation rows stay cache-resident; each weight byte is read once).
// 16x16x32 layout for lane l: A row l%16 / B col l%16 with k = 8*(l/16)+e;
// C col l%16, rows 4*(l/16)+r.
// ---------------------------------------------------------------------------
// Decode GEMM for M <= 128: one 1024-thread workgroup (16 wavefronts) per
// 16*CG output columns. The 16 waves form CG column groups x KSP K slices;
// each wave streams its 16 weight columns over its K slice with every load of
// a chunk (up to CH 32-wide k-steps) in flight before the first multiply, so
// a whole layer's weight matrix is requested from memory in one or two round
// trips. The KSP partial tiles are summed through LDS in slice order
// (deterministic, no workspace, no cross-workgroup traffic).
//
// One launch can serve several products that share the activations A (the
// q/k/v or gate/up projections of a layer): workgroups are assigned to the
// products' column tiles in order, each computing exactly what a launch of
// its own product would. GATED (two products of equal N): every wave
// multiplies the same A fragments by both weight matrices and the epilogue
// writes silu(gate) * up, each product rounded to OT first, as separate GEMMs
// followed by the SiLU-mul kernel would.
//
// k mapping per 32-wide step: lane group q = lane / 16 takes k0 + 8 q .. +7,
// so the four groups of a row read 64 contiguous bytes.
//
// NORM: the rows of A are RMSNorm inputs h. The kernel multiplies h by the
// weight operand round((w + wadd) * B) (the norm weight applied to the weight
// fragments: 8 NB values per lane and step instead of 8 MT activation values,
// which every column tile would scale again) and scales each output row by
// rsqrt(mean_k(h^2) + eps) after the sum over K: RMSNorm followed by the
// product with the per-row factor moved past the (linear) sum, and one
// rounding per product term, as the separate norm's normalised operand has.
// Every workgroup holds all K columns of its rows (its waves' K slices each
// loaded in one chunk), so the row sums of squares are this lane's pairs
// (v_dot2), the four lane groups of a row, then the slices in order through
// LDS in the epilogue; the multiplies never wait for them. NORM modes 2 and 3
// are the same with the norm weight already folded into B (B = round((w + wadd)
// * W), made once per weight): the weight fragments are used as loaded and the
// results equal mode 1's bit for bit. Mode 2 keeps mode 1's one load chunk per K
// slice (a loop of a run-time chunk count holds more registers and spilled);
// mode 3 serves the shapes whose slices need several chunks.
// Residual (per product, optional): C = round(round(product) + R), the
// residual-add kernel's rounding.
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

// NORM template mode: 0 none, 1 weight applied in the kernel, 2 folded into B
// (3: folded, K slices in several chunks; chosen at launch).
__host__ __device__ constexpr int decode_norm_mode(const DecodeNorm* n) {
  return n == nullptr ? 0 : (n->folded ? 2 : (n->w != nullptr ? 1 : 0));
}

// k-steps of 32 whose loads one wave issues together (a NORM launch needs its
// whole K slice in one chunk). A chunk's activation block (16 MT rows x 32 CH k)
// is staged in the LDS slot of the wave's K slice: 128 KB / KSP, shared by the
// slice's 16 / KSP column groups, so MT x CH <= 128 / KSP, with rows of at least
// 128 bytes (CH >= 2). Weight fragments of a chunk stay in registers (CH x NB).
constexpr int kDecodeLds = 128 * 1024;
__host__ __device__ constexpr int decode_chunk(int mt, bool gated, int ksp = 16) {
  return ksp >= 16 ? (mt == 1 ? (gated ? 4 : 8) : (mt == 2 ? 4 : 2))
                   : (mt <= 2 ? (gated ? 4 : 8) : (gated ? 4 : (ksp <= 4 ? 8 : 4)));
}
// NORM launches: the same chunks.
__host__ __device__ constexpr int decode_norm_chunk(int mt, bool gated, int ksp = 16) {
  return decode_chunk(mt, gated, ksp);
}
// Longest row a NORM launch normalises.
constexpr int kDecodeNormMaxK = 8192;

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

// NTB: weights loaded non-temporally (each weight tile read by one workgroup, ms == 1); with
// several row groups per column tile the repeat reads should find the tile in the caches.
template <typename T, typename OT, int MT, int KSP, bool GATED, int NORM, bool NTB = true>
__global__ __launch_bounds__(1024) void gemm_decode_kernel(const T* __restrict__ A, int64_t lda,
                                                           const DecodeProducts<T, OT> P, const DecodeNorm nrm,
                                                           int M, int K, int kr, int ms, int tiles) {
  constexpr int CG = 16 / KSP;
  constexpr bool SCALE = NORM == 1, ROWS = NORM != 0;  // weight scaled here; row factor applied
  constexpr bool ONE = NORM == 1 || NORM == 2;         // each K slice in one load chunk
  constexpr int NB = GATED ? 2 : 1;                   // weight matrices per wave
  constexpr int CH = decode_chunk(MT, GATED, KSP);    // k-steps loaded together
  typedef typename Mfma<T>::v8 v8;
  // Activation rows of a chunk: the waves of a K slice DMA its 16 MT x (64 CH
  // bytes) block into the slice's LDS slot as whole 128-byte lines (a row-per-
  // lane fragment load would touch 16 half-used lines per instruction, measured
  // 3-4x slower from L2), 16-byte slots XOR-swizzled per row so the fragment
  // reads are conflict-free; the slice's CG column groups share the block. The
  // K-slice sums reuse the slots after a barrier.
  constexpr int SLOT = kDecodeLds / KSP;  // LDS bytes per K slice
  constexpr int RB = CH * 64;             // bytes of one activation row in a chunk
  constexpr int S16 = RB / 16;            // 16-byte slots per row
  static_assert(MT * 16 * RB <= SLOT && CH >= 2, "activation block exceeds the slice's LDS slot");
  static_assert(16 * MT * 16 * 16 * 4 <= kDecodeLds, "K-slice sums exceed the slots");
  __shared__ __align__(16) unsigned char abuf[kDecodeLds];
  // K-slice partials. MT = 4 (1024 threads for 4 rows per wave per column):
  // per wave, MT x 64 words of 4 rows (16 i + 4 q .. + 3) of column li, word
  // i * 64 + q * 16 + li, so a lane writes its 4 rows of a row tile as one
  // 16-byte word and a summing thread takes 4 outputs. MT < 4: one float per
  // output, [wave][row][column], and a summing thread takes one output (with 4
  // outputs per thread too few threads would share the sums).
  constexpr bool WORDS = MT == 4;
  f32x4* redw = reinterpret_cast<f32x4*>(abuf);
  float(*red)[MT * 16][16] = reinterpret_cast<float(*)[MT * 16][16]>(abuf);
  __shared__ float rfac[ROWS && WORDS ? MT * 16 : 1];
  __shared__ float nss[ROWS ? 16 : 1][MT * 16];
  // Workgroup -> (column tile, row group). The ms row groups of a tile get
  // workgroup ids that are equal mod 8, so they run on one XCD and read the
  // tile's weights through the same L2.
  const int bid = (int)blockIdx.x;
  const int rest = bid >> 3;
  const int mg = rest % ms;
  const int gtile = (rest / ms) * 8 + (bid & 7);
  if (gtile >= tiles) return;
  const int m0 = mg * MT * 16;
  int pi = 0;
  while (pi + 1 < P.count && gtile >= P.tile0[pi + 1]) ++pi;
  const int tile = gtile - P.tile0[pi];
  const int N = P.N[pi];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int cg = wid / KSP, ks = wid % KSP;
  const int li = lane & 15, q = lane >> 4;
  const int n = (tile * CG + cg) * 16 + li;
  const bool nok = n < N;
  const T* brow[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) brow[j] = P.B[pi + j] + (int64_t)(nok ? n : 0) * P.ldb[pi + j];
  const int kb = ks * kr, ke = min(K, kb + kr);
  f32x4 acc[NB][MT];
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  v8 zero;
#pragma unroll
  for (int e = 0; e < 8; ++e) zero[e] = (T)0.f;
  // Every wave runs the same number of chunks (with NORM modes 1 and 2 exactly
  // one; slices past K load zeros), so all of them reach the barriers.
  auto swz = [](int r) { return S16 >= 16 ? (r & 15) : ((r >> 1) & 7); };  // slot s of row r: chunk s ^ swz(r)
  unsigned char* slot = abuf + ks * SLOT;
  const uint32_t abase = lds_addr(slot);
  const int nch = ONE ? 1 : (kr + 32 * CH - 1) / (32 * CH);
  float sq[MT];  // NORM: this lane's row sums of squares (over all its chunks)
#pragma unroll
  for (int i = 0; i < MT; ++i) sq[i] = 0.f;
  for (int ci = 0; ci < nch; ++ci) {
    const int k0 = kb + ci * 32 * CH;
    v8 b[CH][NB];
    v8 wr[SCALE ? CH : 1];  // norm weights (dtype T) of this lane's 8 columns per step
    if (ci > 0) {  // the previous chunk's fragments have been read from the slot
      if constexpr (CG > 1) __syncthreads();
      else asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
#pragma unroll
    for (int j = cg; j < MT * CH; j += CG) {
      const int c = j * 64 + lane, r = c / S16;
      const int m = m0 + r, k = k0 + ((c % S16) ^ swz(r)) * 8;
      // rows past M and chunks past the slice stage A[0..7] (in bounds; zeroed below)
      lds_dma16(m < M && k < ke ? A + (int64_t)m * lda + k : A, abase + j * 1024);
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int k = k0 + u * 32 + q * 8;
      const bool kok = k < ke;
      if constexpr (SCALE) wr[u] = kok ? *reinterpret_cast<const v8*>((const T*)nrm.w + k) : zero;
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        // weights read by one workgroup per decode step: non-temporal, so they do not evict cached data
        if (nok && kok) {
          if constexpr (NTB) b[u][j] = __builtin_nontemporal_load(reinterpret_cast<const v8*>(brow[j] + k));
          else b[u][j] = *reinterpret_cast<const v8*>(brow[j] + k);
        } else {
          b[u][j] = zero;
        }
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the staged rows (untracked DMA) and the weights
    if constexpr (CG > 1) __syncthreads();             // and the slice's other column groups' rows
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const bool kok = k0 + u * 32 + q * 8 < ke;
      if constexpr (SCALE) {  // the weight operand round((w + wadd) * B): 8 NB values per lane, not 8 MT
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float wv = to_f32(wr[u][e]) + nrm.wadd;
#pragma unroll
          for (int j = 0; j < NB; ++j) b[u][j][e] = from_f32<T>(to_f32(b[u][j][e]) * wv);
        }
      }
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int r = i * 16 + li;
        v8 a;
        if (m0 + r < M && kok) a = *reinterpret_cast<const v8*>(slot + r * RB + (((u * 4 + q) ^ swz(r)) << 4));
        else a = zero;
        if constexpr (ROWS) sq[i] = sumsq8<T>(a, sq[i]);  // row sums of squares (the epilogue adds the slices)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[j][i] = mma16<T>(a, b[u][j], acc[j][i]);
      }
    }
  }
  if constexpr (ROWS) {
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      float v = sq[i];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      if (q == 0) nss[wid][i * 16 + li] = v;
    }
  }
  // Sum the K slices in order, one weight matrix at a time through the same
  // LDS buffer. C layout: column li, rows 16 i + 4 q + r.
  if constexpr (WORDS) {
    constexpr int NW4 = MT * 64;  // words per wave
    float first[(CG * NW4 + 1023) / 1024][4];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      __syncthreads();  // every wave's fragments (j = 0) or the previous matrix's sums have been read
#pragma unroll
      for (int i = 0; i < MT; ++i) redw[wid * NW4 + i * 64 + q * 16 + li] = acc[j][i];
      if constexpr (ROWS) {  // each row's RMSNorm factor, once (column group 0's slices, in order)
        if (j == 0 && threadIdx.x < MT * 16) {
          float ss = 0.f;
#pragma unroll
          for (int s2 = 0; s2 < KSP; ++s2) ss += nss[s2][threadIdx.x];
          rfac[threadIdx.x] = rsqrtf(ss / (float)K + nrm.eps);
        }
      }
      __syncthreads();
      int slot = 0;
      for (int idx = threadIdx.x; idx < CG * NW4; idx += 1024, ++slot) {
        const int g = idx / NW4, rem = idx % NW4;
        const int col = rem % 16, row0 = (rem / 64) * 16 + ((rem / 16) % 4) * 4;
        f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s2 = 0; s2 < KSP; ++s2) v += redw[(g * KSP + s2) * NW4 + rem];
        const int gn = (tile * CG + g) * 16 + col;
        if (gn >= N) continue;
        const T* bias = P.bias[pi + j];
        const float bv = bias ? to_f32(bias[gn]) : 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int grow = m0 + row0 + r;
          if (grow >= M) continue;
          float val = v[r];
          if constexpr (ROWS) val *= rfac[row0 + r];
          val += bv;
          if constexpr (GATED) {
            if (j == 0) {
              first[slot][r] = to_f32(from_f32<OT>(val));
            } else {
              const float gt = first[slot][r], up = to_f32(from_f32<OT>(val));
              P.C[pi][(int64_t)grow * P.ldc[pi] + gn] = from_f32<OT>(gt * sigmoidf_(gt) * up);
            }
          } else {
            OT o = from_f32<OT>(val);
            const T* res = P.res[pi];
            if (res != nullptr) o = from_f32<OT>(to_f32(o) + to_f32(res[(int64_t)grow * P.ldr[pi] + gn]));
            P.C[pi][(int64_t)grow * P.ldc[pi] + gn] = o;
          }
        }
      }
    }
  } else {
    float first[(CG * MT * 256 + 1023) / 1024];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      __syncthreads();  // every wave's fragments (j = 0) or the previous matrix's sums have been read
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wid][i * 16 + q * 4 + r][li] = acc[j][i][r];
      __syncthreads();
      int slot = 0;
      for (int idx = threadIdx.x; idx < CG * MT * 256; idx += 1024, ++slot) {
        const int g = idx / (MT * 256), rem = idx % (MT * 256);
        const int row = rem / 16, col = rem % 16;
        float v = 0.f;
#pragma unroll
        for (int s2 = 0; s2 < KSP; ++s2) v += red[g * KSP + s2][row][col];
        const int gn = (tile * CG + g) * 16 + col;
        const int grow = m0 + row;
        if (grow >= M || gn >= N) continue;
        const T* bias = P.bias[pi + j];
        if constexpr (ROWS) {  // the row's RMSNorm factor (slices summed in order)
          float ss = 0.f;
#pragma unroll
          for (int s2 = 0; s2 < KSP; ++s2) ss += nss[s2][row];  // column group 0's slices
          v *= rsqrtf(ss / (float)K + nrm.eps);
        }
        const float val = v + (bias ? to_f32(bias[gn]) : 0.f);
        if constexpr (GATED) {
          if (j == 0) {
            first[slot] = to_f32(from_f32<OT>(val));
          } else {
            const float gt = first[slot], up = to_f32(from_f32<OT>(val));
            P.C[pi][(int64_t)grow * P.ldc[pi] + gn] = from_f32<OT>(gt * sigmoidf_(gt) * up);
          }
        } else {
          OT o = from_f32<OT>(val);
          const T* res = P.res[pi];
          if (res != nullptr) o = from_f32<OT>(to_f32(o) + to_f32(res[(int64_t)grow * P.ldr[pi] + gn]));
          P.C[pi][(int64_t)grow * P.ldc[pi] + gn] = o;
        }
      }
    }
  }
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
                                                          int K, int ncols) {
  static_assert(RC == 1 || !GATED, "a wave takes several columns of non-gated products only");
  constexpr bool SCALE = NORM == 1, ROWS = NORM != 0;  // activation scaled here; row factor applied
  constexpr int NB = GATED ? 2 : RC;
  constexpr int CH = gemv_chunk(MR, GATED, RC);
  typedef typename Mfma<T>::v8 v8;
  const int lane = threadIdx.x & 63;
  const int col = ((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6)) * RC;
  if (col >= ncols) return;
  int pi = 0;  // P.tile0 holds the first column of each product here
  while (pi + 1 < P.count && col >= P.tile0[pi + 1]) ++pi;
  const int n = col - P.tile0[pi];
  const T* brow[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int nj = RC > 1 ? min(n + j, P.N[pi] - 1) : n;  // columns past N re-read the last row
    brow[j] = P.B[pi + (RC > 1 ? 0 : j)] + (int64_t)nj * P.ldb[pi + (RC > 1 ? 0 : j)];
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
      const T* bias = P.bias[pi + (RC > 1 ? 0 : j)];
      if (bias != nullptr) pb[j] = to_f32(bias[RC > 1 ? min(n + j, P.N[pi] - 1) : n]);
      if constexpr (!GATED) {
        const T* res = P.res[pi];
        if (res != nullptr && (RC == 1 || n + j < P.N[pi]))
          pr[j] = to_f32(res[(int64_t)lane * P.ldr[pi] + n + (RC > 1 ? j : 0)]);
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
    if constexpr (RC > 1) {
      const bool res = P.res[pi] != nullptr;
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        if (n + j >= P.N[pi]) continue;
        OT o = from_f32<OT>(v[j]);
        if (res) o = from_f32<OT>(to_f32(o) + pr[j]);
        P.C[pi][(int64_t)i * P.ldc[pi] + n + j] = o;
      }
    } else if constexpr (GATED) {
      const float gt = to_f32(from_f32<OT>(v[0])), up = to_f32(from_f32<OT>(v[1]));
      P.C[pi][(int64_t)i * P.ldc[pi] + n] = from_f32<OT>(gt * sigmoidf_(gt) * up);
    } else {
      OT o = from_f32<OT>(v[0]);
      if (P.res[pi] != nullptr) o = from_f32<OT>(to_f32(o) + pr[0]);
      P.C[pi][(int64_t)i * P.ldc[pi] + n] = o;
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
#define QH_GR(MRV, NV, RCV) gemv_decode_kernel<T, OT, MRV, false, NV, RCV><<<grid, 256, 0, st>>>(a, lda, P, nz, M, K, ncols)
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
#define QH_GV(MRV, GV, NV) gemv_decode_kernel<T, OT, MRV, GV, NV><<<grid, 256, 0, st>>>(a, lda, P, nz, M, K, ncols)
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

// Returns QH_E_ARG (nothing launched) when a norm prologue is asked for a
// shape whose K slices do not fit one load chunk (decode_norm_fits).
// Launch shape of a decode-kernel launch. K slices per column group (ksp): 4
// for wide outputs (4 column groups x 4 slices); 8 from 65 rows when 16-column
// tiles would need more than one workgroup per CU (2 column groups share each
// slice's activation block: a 128-row q/k/v launch 11.9 us instead of 14.0, gate/
// up 16.3 instead of 18.0; slower at 1024 columns and at 64 rows); else 16. Row
// groups per column tile (ms): with few column tiles, up to one workgroup per
// 16 rows, until about one workgroup per CU.
struct DecodePlan {
  int ksp, cols, tiles, kr, ms, mtw;
  bool norm_fits;
};

static DecodePlan decode_plan(int M, int K, bool gated, bool norm, int count, const int* N, int ksp_force,
                              int ms_force) {
  DecodePlan d{};
  int maxN = 0;
  for (int i = 0; i < count; ++i) maxN = N[i] > maxN ? N[i] : maxN;
  const bool wide = !gated && !norm && maxN > 8192;
  const int mt = (M + 15) / 16;
  d.ksp = wide ? 4 : 16;
  if (!wide && mt > 4) {  // 8 slices when 16-column tiles would need more than one workgroup per CU
    int t16 = 0;
    for (int i = 0; i < (gated ? 1 : count); ++i) t16 += (N[i] + 15) / 16;
    int ms16 = 1;
    while (ms16 * 4 < mt) ms16 *= 2;
    if (t16 * ms16 > 256) d.ksp = 8;
  }
  if (!wide && (ksp_force == 8 || ksp_force == 16)) d.ksp = ksp_force;
  d.cols = 16 * (16 / d.ksp);
  const int nprod = gated ? 1 : count;  // the gated pair shares its column tiles
  d.tiles = 0;
  for (int i = 0; i < nprod; ++i) d.tiles += (N[i] + d.cols - 1) / d.cols;
  d.kr = ((K + d.ksp - 1) / d.ksp + 31) / 32 * 32;
  int ms = 1;
  while (ms * 4 < mt) ms *= 2;  // at most 4 row tiles (64 rows) per workgroup
  while (ms < mt && d.tiles * ms * 2 <= 256) ms *= 2;
  if (ms > mt) ms = mt;
  if (ms_force > 0 && ms_force <= mt) ms = ms_force;
  d.ms = ms;
  d.mtw = (mt + ms - 1) / ms;
  d.norm_fits = K <= kDecodeNormMaxK && d.kr <= 32 * decode_norm_chunk(d.mtw, gated, d.ksp);
  return d;
}

// Returns QH_E_ARG (nothing launched) when a norm prologue is asked for a
// shape whose K slices do not fit one load chunk (decode_norm_fits).
template <typename T, typename OT>
int launch_decode_products(const T* a, int64_t lda, DecodeProducts<T, OT>& P, int M, int K, bool gated,
                           hipStream_t st, int ms_force = 0, const DecodeNorm* nrm = nullptr, int ksp_force = 0) {
  const int nmode = decode_norm_mode(nrm);
  const bool norm = nmode != 0;
  if (M <= kGemvMaxRows && ms_force == 0 && ksp_force == 0) {
    if (norm && !std::is_same<T, OT>::value) return QH_E_ARG;
    launch_gemv_products<T, OT>(a, lda, P, M, K, gated, norm ? *nrm : DecodeNorm{nullptr, 0.f, 0.f, 0}, st);
    return QH_OK;
  }
  // modes 1 and 2 load each K slice in one chunk; folded weights whose slices do not fit
  // one chunk take the plain plan (mode 3)
  DecodePlan d = decode_plan(M, K, gated, nmode != 0, P.count, P.N, ksp_force, ms_force);
  int kmode = nmode;
  if (nmode == 2 && !d.norm_fits) {
    d = decode_plan(M, K, gated, false, P.count, P.N, ksp_force, ms_force);
    kmode = 3;
  }
  const int nprod = gated ? 1 : P.count;
  P.tile0[0] = 0;
  for (int i = 0; i < nprod; ++i) P.tile0[i + 1] = P.tile0[i] + (P.N[i] + d.cols - 1) / d.cols;
  if (gated) P.count = 1;
  const int tiles = d.tiles, kr = d.kr, ms = d.ms, mtw = d.mtw, ksp = d.ksp;
  const int grid = (tiles + 7) / 8 * 8 * ms;
  if (nmode == 1 && !d.norm_fits) return QH_E_ARG;
  const DecodeNorm nz = norm ? *nrm : DecodeNorm{nullptr, 0.f, 0.f, 0};
  constexpr bool kNormOk = std::is_same<T, OT>::value;  // the only instantiation a norm launch reaches
  if (norm && !kNormOk) return QH_E_ARG;
#define QH_DG(MTV, KSPV, GV, NV)                                                                        \
  do {                                                                                                 \
    if (ms == 1) gemm_decode_kernel<T, OT, MTV, KSPV, GV, NV, true><<<grid, 1024, 0, st>>>(a, lda, P, nz, M, K, kr, ms, tiles); \
    else gemm_decode_kernel<T, OT, MTV, KSPV, GV, NV, false><<<grid, 1024, 0, st>>>(a, lda, P, nz, M, K, kr, ms, tiles); \
  } while (0)
#define QH_DG_K(MTV, GV, NV) \
  if (ksp == 8) QH_DG(MTV, 8, GV, NV); else QH_DG(MTV, 16, GV, NV);
#define QH_DG_W(MTV)                                           \
  if constexpr (kNormOk) {                                     \
    if (nmode == 1) {                                          \
      if (gated) { QH_DG_K(MTV, true, 1) } else { QH_DG_K(MTV, false, 1) } \
      return QH_OK;                                            \
    }                                                          \
    if (kmode == 2) {                                          \
      if (gated) { QH_DG_K(MTV, true, 2) } else { QH_DG_K(MTV, false, 2) } \
      return QH_OK;                                            \
    }                                                          \
    if (kmode == 3) {                                          \
      if (gated) { QH_DG_K(MTV, true, 3) } else { QH_DG_K(MTV, false, 3) } \
      return QH_OK;                                            \
    }                                                          \
  }                                                            \
  if (gated) { QH_DG_K(MTV, true, 0) }                         \
  else if (ksp == 4) QH_DG(MTV, 4, false, 0);                  \
  else { QH_DG_K(MTV, false, 0) }
  if (mtw == 1) { QH_DG_W(1) } else if (mtw == 2) { QH_DG_W(2) } else if (mtw == 3) { QH_DG_W(3) } else { QH_DG_W(4) }
#undef QH_DG_W
#undef QH_DG_K
#undef QH_DG
  return QH_OK;
}

// Whether a norm-prologue launch of M rows, K columns fits (all K slices of
// every workgroup loaded in one chunk); mirrors launch_decode_products.
static bool decode_norm_fits(int M, int K, bool gated, int count, const int64_t* N) {
  if (M <= kGemvMaxRows) return true;  // the one-wave-per-column kernel normalises any K
  int n32[kMaxProducts];
  for (int i = 0; i < count && i < kMaxProducts; ++i) n32[i] = (int)N[i];
  return decode_plan(M, K, gated, true, count, n32, 0, 0).norm_fits;
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
    rc = launch_decode_products<T, T>((const T*)A, lda, P, (int)M, (int)K, gated != 0, st, 0, &nrm);   \
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
    rc = launch_decode_products<T, T>((const T*)A, lda, P, (int)M, (int)K, gated != 0, st, 0, &nrm);   \
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
