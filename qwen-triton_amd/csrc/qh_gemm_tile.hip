// Large-tile MFMA GEMM core for gfx950 and the dense products that use it.
//
// C[M,N] = A(M,K) B(N,K)^T with each operand either k-contiguous ("N": element
// (i,k) at P[i*ld + k]) or k-outer ("T": element (i,k) at P[k*ld + i]), the
// same operand convention as the other GEMM kernels of the library.
//
// Workgroup: 512 threads = 8 wavefronts (two per SIMD, so one wave's memory or
// barrier stall is covered by the other's MFMAs) in a 2x4 grid over a BM x BN
// output tile (256 x 256); each wavefront owns 128 x 64 as 4x2 MFMA 32x32x16
// tiles with fp32 accumulators. k advances in tiles of 32:
//  * both operand tiles are written to LDS by direct-to-LDS loads (16 bytes
//    per lane, no staging registers) into NST = 4 LDS stages, so two to three
//    k-tiles are in flight while one feeds the matrix cores (one tile's round
//    trip from L2 is longer than its math);
//  * the loop is rotated around the barrier: a tile's first-half MFMAs run
//    while its second-half fragments are read, then (after the next tile has
//    landed and the barrier) its second-half MFMAs run while the next tile's
//    first fragments are read, so neither the barrier nor the first LDS reads
//    of a tile leave the matrix cores idle;
//  * LDS has 64 banks (256 bytes per cycle): a ds_read_b128 serves 16 lanes a
//    cycle and a ds_read_b64 32, and those lanes must hit distinct banks;
//  * "N" operands keep their natural [row][32 k] layout (64-byte rows), with
//    the 16-byte chunk c of row r stored at chunk c ^ ((r >> 2) & 3), so the 16
//    rows of a 16-lane fragment read fill all 64 banks once; a fragment is one
//    ds_read_b128 per lane;
//  * "T" operands keep their natural [k][row] layout; chunk c of k-row kr is
//    stored at c ^ 4(kr & 3), so the 4 k-rows x 4 chunks read by 32 lanes are
//    distinct banks. A fragment is two ds_read_b64_tr_b16 per lane:
//    in each 16-lane group, lane j addresses k-row kb + j/4 at rows
//    rb + 4(j % 4), and lane i receives rows rb + i of k-rows kb..kb+3, i.e.
//    exactly the lane's MFMA row with k = 8(lane/32) + 0..3 (then 4..7), the
//    k order of the "N" fragment, so any mix of layouts multiplies correctly.
// A k-tile that runs past K is zeroed in LDS after it lands; rows past M or N
// read clamped (valid) memory and their results are not stored.
//
// The core is a template over a "problem" type that places the tile (output
// coordinates, operand bases per k-tile, reduction length) and stores the
// accumulators, so grouped products reuse the same main loop.
#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

#include "qh_lds.h"
#include "qh_mfma.h"

namespace {

constexpr int NWAVE = 8; // wavefronts per workgroup (2 per SIMD)
constexpr int NTHR = 64 * NWAVE;

template <typename T>
using V8 = typename Mfma<T>::v8;

// ---------------------------------------------------------------------------
// LDS tile layouts (BK = k extent of one tile: 32 or 64)
// ---------------------------------------------------------------------------
// "N" tile: ROWS x BK elements. W = 256 / (2 BK) rows share one 256-byte bank
// window, so chunk c of row r is stored at c ^ ((r / W) mod CPR): the 16 rows
// of a 16-lane fragment read then cover every bank exactly once.
template <typename T, int ROWS, int BK>
struct NTile {
  static_assert(sizeof(T) == 2, "16-bit operands");
  static constexpr int ELEMS = ROWS * BK;
  static constexpr int CPR = BK / 8;       // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;     // rows per 1 KiB DMA instruction
  static constexpr int W = 128 / BK;       // rows per 256-byte bank window
  static constexpr int PW = ROWS / RPI / NWAVE;  // DMA instructions per wave
  static_assert(PW >= 1 && (ROWS / RPI) % NWAVE == 0, "tile height");

  static __device__ __forceinline__ int sw(int r) { return (r / W) & (CPR - 1); }
  // Rows of instruction n are RPI n + lane / CPR with n = wid + NWAVE i; RPI / W
  // is 4 and NWAVE is even, so sw(row) is fixed per lane across instructions.
  static __device__ __forceinline__ uint32_t voff(int64_t ld, int wid) {
    const int lane = threadIdx.x & 63;
    const int rin = lane / CPR, c = (lane % CPR) ^ sw(RPI * wid + rin);
    return (uint32_t)(((int64_t)rin * ld + 8 * c) * (int64_t)sizeof(T));
  }
  // g: element (tile row 0, k0). vrows: valid rows from row 0; vk: valid k from k0.
  static __device__ __forceinline__ void issue(uint32_t lds, const T* g, int64_t ld, int vrows, int vk,
                                               uint32_t vo, int wid) {
    if (vrows >= ROWS && vk >= BK) {
#pragma unroll
      for (int i = 0; i < PW; ++i) {
        const int n = wid + NWAVE * i;
        lds_dma16_s(vo, g + (int64_t)(RPI * n) * ld, lds + (uint32_t)n * 1024u);
      }
    } else {
      const int lane = threadIdx.x & 63;
      const int rin = lane / CPR;
      int kc = 8 * ((lane % CPR) ^ sw(RPI * wid + rin));
      if (kc > vk - 8) kc = vk - 8;  // vk is a positive multiple of 8
#pragma unroll
      for (int i = 0; i < PW; ++i) {
        const int n = wid + NWAVE * i;
        int r = RPI * n + rin;
        if (r > vrows - 1) r = vrows - 1;
        lds_dma16(g + (int64_t)r * ld + kc, lds + (uint32_t)n * 1024u);
      }
    }
  }
  // Zero the k chunks at or past vk (all rows).
  static __device__ __forceinline__ void zero_k_tail(T* S, int vk) {
    for (int idx = threadIdx.x; idx < ROWS * CPR; idx += NTHR) {
      const int r = idx / CPR, c = idx % CPR;
      if (8 * c >= vk) *reinterpret_cast<uint4*>(S + r * BK + 8 * (c ^ sw(r))) = make_uint4(0, 0, 0, 0);
    }
  }
  // Fragment of rows r0 .. r0+31 at k16 step kk.
  static __device__ __forceinline__ V8<T> frag(const T* S, int r0, int kk) {
    const int lane = threadIdx.x & 63;
    const int row = r0 + (lane & 31);
    const int ch = (2 * kk + (lane >> 5)) ^ sw(row);
    return *reinterpret_cast<const V8<T>*>(S + row * BK + ch * 8);
  }
};

// "T" tile: BK k-rows x COLS elements.
template <typename T, int COLS, int BK>
struct TTile {
  static_assert(sizeof(T) == 2, "16-bit operands");
  static constexpr int ELEMS = BK * COLS;
  static constexpr int CPR = COLS / 8;   // 16-byte chunks per k-row
  static constexpr int RPI = 64 / CPR;   // k-rows per 1 KiB instruction (64 lanes x 16 bytes)
  static constexpr int NI = BK / RPI;
  static constexpr int PW = NI / NWAVE;
  static_assert(CPR >= 16 && CPR <= 64 && PW >= 1 && NI % NWAVE == 0, "tile width");
  static __device__ __forceinline__ int sw(int kr) { return 4 * (kr & 3); }

  // k-row of this lane in instruction n is n*RPI + lane/CPR; n = wid + NWAVE i
  // and NWAVE*RPI is a multiple of 4, so (k-row & 3) is fixed per lane and so
  // is its swizzled chunk.
  static __device__ __forceinline__ uint32_t voff(int64_t ld, int wid) {
    const int lane = threadIdx.x & 63;
    const int kin = lane / CPR, slot = lane % CPR;
    const int c = slot ^ sw(wid * RPI + kin);
    return (uint32_t)(((int64_t)kin * ld + 8 * c) * (int64_t)sizeof(T));
  }
  // g: element (k0, tile column 0). vcols: valid columns; vk: valid k-rows.
  static __device__ __forceinline__ void issue(uint32_t lds, const T* g, int64_t ld, int vcols, int vk,
                                               uint32_t vo, int wid) {
    if (vcols >= COLS && vk >= BK) {
#pragma unroll
      for (int i = 0; i < PW; ++i) {
        const int n = wid + NWAVE * i;
        lds_dma16_s(vo, g + (int64_t)(n * RPI) * ld, lds + (uint32_t)n * 1024u);
      }
    } else {
      const int lane = threadIdx.x & 63;
      const int kin = lane / CPR, slot = lane % CPR;
#pragma unroll
      for (int i = 0; i < PW; ++i) {
        const int n = wid + NWAVE * i;
        int kr = n * RPI + kin;
        int col = 8 * (slot ^ sw(kr));
        if (col > vcols - 8) col = vcols - 8;  // vcols is a positive multiple of 8
        if (kr > vk - 1) kr = vk - 1;
        lds_dma16(g + (int64_t)kr * ld + col, lds + (uint32_t)n * 1024u);
      }
    }
  }
  static __device__ __forceinline__ void zero_k_tail(T* S, int vk) {
    for (int idx = threadIdx.x; idx < BK * CPR; idx += NTHR) {
      const int kr = idx / CPR;
      if (kr >= vk) *reinterpret_cast<uint4*>(S + idx * 8) = make_uint4(0, 0, 0, 0);
    }
  }
  // Fragment of rows (tile columns) r0 .. r0+31 at k16 step kk.
  static __device__ __forceinline__ V8<T> frag(const T* S, int r0, int kk) {
    const int lane = threadIdx.x & 63;
    const int grp = lane >> 4, j = lane & 15;
    const int m = r0 + 16 * (grp & 1) + 4 * (j & 3);
    const int kr0 = 16 * kk + 8 * (grp >> 1) + (j >> 2);
    const int kr1 = kr0 + 4;
    const T* s0 = S + kr0 * COLS + 8 * ((m >> 3) ^ sw(kr0)) + (m & 7);
    const T* s1 = S + kr1 * COLS + 8 * ((m >> 3) ^ sw(kr1)) + (m & 7);
    const qh_v4i16 w0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) qh_v4i16*)(s0));
    const qh_v4i16 w1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) qh_v4i16*)(s1));
    const qh_v8i16 w = __builtin_shufflevector(w0, w1, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(V8<T>, w);
  }
};

template <typename T, int ROWS, int BK, bool TR>
using OpTile = typename std::conditional<TR, TTile<T, ROWS, BK>, NTile<T, ROWS, BK>>::type;

// ---------------------------------------------------------------------------
// Tile context filled by the problem type.
// ---------------------------------------------------------------------------
template <typename T>
struct TileCtx {
  int m0, n0;        // output tile origin
  int K;             // reduction length of this tile
  int vm, vn;        // valid output rows / columns from (m0, n0)
  int64_t lda, ldb;  // operand strides
  int aux;           // problem-defined (e.g. expert index)
};

// ---------------------------------------------------------------------------
// Main loop
// ---------------------------------------------------------------------------
// Instruction schedule of one basic block of NM MFMAs and ND LDS reads: the
// reads are spread over the first SPAN MFMAs, so the last NM - SPAN MFMAs
// cover the latency of the last reads.
template <int ND, int SPAN, int M>
__device__ __forceinline__ void mma_schedule_slot() {
  constexpr int nd = M < SPAN ? ((M + 1) * ND) / SPAN - (M * ND) / SPAN : 0;
  if constexpr (nd > 0) __builtin_amdgcn_sched_group_barrier(0x100, nd, 0);
  __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
}
template <int ND, int SPAN, int... Ms>
__device__ __forceinline__ void mma_schedule(std::integer_sequence<int, Ms...>) {
  (mma_schedule_slot<ND, SPAN, Ms>(), ...);
}

template <typename T, int BM, int BN, int BK, int NS, bool AT, bool BT, class P>
__global__ __launch_bounds__(NTHR) void gemm_tile_kernel(P p) {
  using TA = OpTile<T, BM, BK, AT>;
  using TB = OpTile<T, BN, BK, BT>;
  constexpr int WGM = 2, WGN = NWAVE / 2;  // wavefront grid over the tile
  constexpr int WTM = BM / WGM, WTN = BN / WGN, TM = WTM / 32, TN = WTN / 32;
  constexpr int STAGE = TA::ELEMS + TB::ELEMS;
  constexpr int KS = BK / 16;  // MFMA k steps per tile
  static_assert(KS % 2 == 0 && NS >= 2 && NS <= 4, "pipeline shape");
  extern __shared__ __attribute__((aligned(1024))) unsigned char qh_tile_smem[];
  T* smem = reinterpret_cast<T*>(qh_tile_smem);

  TileCtx<T> c;
  if (!p.tile(c)) return;
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wid / WGN, wn = wid % WGN;
  const uint32_t lds0 = lds_addr(smem);
  const uint32_t voa = TA::voff(c.lda, wid);
  const uint32_t vob = TB::voff(c.ldb, wid);

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = zero16();

  constexpr int NPT = TA::PW + TB::PW;  // DMA instructions per wave and k-tile
  constexpr int ND = TM * (AT ? 2 : 1) + TN * (BT ? 2 : 1);  // LDS reads per k16 step
  constexpr int NM = TM * TN;
  const int nk = (c.K + BK - 1) / BK;
  auto stage = [&](int kt) { return smem + (kt % NS) * STAGE; };
  auto issue = [&](int kt) {
    const int k0 = kt * BK;
    const int vk = c.K - k0;
    const uint32_t base = lds0 + (uint32_t)((kt % NS) * STAGE * (int)sizeof(T));
    TA::issue(base, p.a_tile(c, k0), c.lda, c.vm, vk, voa, wid);
    TB::issue(base + (uint32_t)(TA::ELEMS * sizeof(T)), p.b_tile(c, k0), c.ldb, c.vn, vk, vob, wid);
  };
  // Make k-tile kt visible to every wave, with `after` later tiles still in flight.
  auto land = [&](int kt, int after) {
    if (after <= 0) __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    else if (after == 1) __builtin_amdgcn_s_waitcnt(waitcnt_vm(NPT));
    else if (after == 2) __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * NPT));
    else __builtin_amdgcn_s_waitcnt(waitcnt_vm(3 * NPT));
    __syncthreads();
    const int vk = c.K - kt * BK;
    if (vk < BK) {
      T* S = stage(kt);
      TA::zero_k_tail(S, vk);
      TB::zero_k_tail(S + TA::ELEMS, vk);
      __syncthreads();
    }
  };
  V8<T> af[2][TM], bf[2][TN];
  auto read = [&](const T* S, int kk, int b) {
#pragma unroll
    for (int i = 0; i < TM; ++i) af[b][i] = TA::frag(S, wm * WTM + 32 * i, kk);
#pragma unroll
    for (int j = 0; j < TN; ++j) bf[b][j] = TB::frag(S + TA::ELEMS, wn * WTN + 32 * j, kk);
  };
  auto mma = [&](int b) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = Mfma<T>::mma(af[b][i], bf[b][j], acc[i][j]);
  };
  // Tiles 0 .. NS-1 fill every stage. After the barrier that lands tile kt+1,
  // every wave has finished reading tile kt (its last fragments were read
  // before that barrier), so tile kt+NS can go into tile kt's stage.
  if (nk > 0) {
    const int pro = nk < NS ? nk : NS;
    for (int t = 0; t < pro; ++t) issue(t);
    land(0, pro - 1);
    read(stage(0), 0, 0);
  }
  for (int kt = 0; kt < nk; ++kt) {
    // steps 0 .. KS-2 of tile kt, each overlapping the next step's reads
#pragma unroll
    for (int st = 0; st + 1 < KS; ++st) {
      read(stage(kt), st + 1, (st + 1) & 1);
      mma(st & 1);
      mma_schedule<ND, NM * 3 / 4>(std::make_integer_sequence<int, NM>{});
    }
    if (kt + 1 < nk) {
      // tiles issued so far: 0 .. min(kt + NS - 1, nk - 1)
      const int issued = kt + NS - 1 < nk - 1 ? kt + NS - 1 : nk - 1;
      land(kt + 1, issued - (kt + 1));
      if (kt + NS < nk) issue(kt + NS);  // into the stage tile kt used
    }
    // last step of tile kt; the next tile's first fragments are read meanwhile
    // (after the last tile this reads an unused stage, harmlessly)
    read(stage(kt + 1), 0, 0);
    mma((KS - 1) & 1);
    mma_schedule<ND, NM * 3 / 4>(std::make_integer_sequence<int, NM>{});
  }
  p.template epilogue<TM, TN>(c, acc, wm * WTM, wn * WTN, lane);
}

// ---------------------------------------------------------------------------
// Dense problem: C = A B^T (+ bias), OT output.
// ---------------------------------------------------------------------------
template <typename T, typename OT, int BM, int BN, bool AT, bool BT>
struct DenseProblem {
  const T* A;
  const T* B;
  OT* C;
  const T* bias;
  int64_t lda, ldb, ldc;
  int M, N, K, tiles_m, tiles_n;

  __device__ __forceinline__ bool tile(TileCtx<T>& c) const {
    int tm, tn;
    tile_order(tiles_m, tiles_n, tm, tn);
    c.m0 = tm * BM;
    c.n0 = tn * BN;
    c.K = K;
    c.vm = M - c.m0;
    c.vn = N - c.n0;
    c.lda = lda;
    c.ldb = ldb;
    c.aux = 0;
    return true;
  }
  __device__ __forceinline__ const T* a_tile(const TileCtx<T>& c, int k0) const {
    return AT ? A + (int64_t)k0 * lda + c.m0 : A + (int64_t)c.m0 * lda + k0;
  }
  __device__ __forceinline__ const T* b_tile(const TileCtx<T>& c, int k0) const {
    return BT ? B + (int64_t)k0 * ldb + c.n0 : B + (int64_t)c.n0 * ldb + k0;
  }
  // C layout of a 32x32 tile: column lane % 32, rows 8g + 4(lane/32) + r. One
  // base pointer per 32x32 block; rows are constant offsets from it.
  template <int TM, int TN>
  __device__ __forceinline__ void epilogue(const TileCtx<T>& c, const f32x16 (&acc)[TM][TN], int wr, int wc,
                                           int lane) const {
    const bool full = c.vm >= BM && c.vn >= BN;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = c.n0 + wc + 32 * j + (lane & 31);
      if (!full && col >= N) continue;
      const float bv = bias ? to_f32(bias[col]) : 0.f;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int rb = c.m0 + wr + 32 * i + 4 * (lane >> 5);
        OT* base = C + (int64_t)rb * ldc + col;
        if (full) {
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int r = 0; r < 4; ++r) base[(8 * g + r) * ldc] = from_f32<OT>(acc[i][j][4 * g + r] + bv);
        } else {
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (rb + 8 * g + r < M) base[(8 * g + r) * ldc] = from_f32<OT>(acc[i][j][4 * g + r] + bv);
        }
      }
    }
  }
};

template <int BM, int BN, int BK, int NS, typename T>
constexpr int tile_lds_bytes() {
  return NS * (BM + BN) * BK * (int)sizeof(T);
}

template <typename T, int BM, int BN, int BK, int NS, bool AT, bool BT, class P>
int launch_tile(const P& p, int grid, hipStream_t st, const char* name) {
  constexpr int lds = tile_lds_bytes<BM, BN, BK, NS, T>();
  auto kern = gemm_tile_kernel<T, BM, BN, BK, NS, AT, BT, P>;
  // The dynamic-LDS limit is raised once per instantiation and device.
  static uint64_t attr_set = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    qh::set_error("%s: no current device", name);
    return QH_E_HIP;
  }
  if (!(attr_set >> dev & 1)) {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) {
      qh::set_error("%s: cannot raise the LDS limit to %d bytes: %s", name, lds, hipGetErrorString(e));
      return QH_E_HIP;
    }
    attr_set |= 1ull << dev;
  }
  kern<<<grid, NTHR, lds, st>>>(p);
  return QH_OK;
}

// Pipeline shape of the dense tile kernel.
constexpr int kDenseBK = 64, kDenseNS = 2;

template <typename T, typename OT, int BM, int BN, bool AT, bool BT>
int dense_tile(const T* A, int64_t lda, const T* B, int64_t ldb, OT* C, int64_t ldc, const T* bias, int M, int N,
               int K, hipStream_t st) {
  DenseProblem<T, OT, BM, BN, AT, BT> p;
  p.A = A;
  p.B = B;
  p.C = C;
  p.bias = bias;
  p.lda = lda;
  p.ldb = ldb;
  p.ldc = ldc;
  p.M = M;
  p.N = N;
  p.K = K;
  p.tiles_m = (M + BM - 1) / BM;
  p.tiles_n = (N + BN - 1) / BN;
  return launch_tile<T, BM, BN, kDenseBK, kDenseNS, AT, BT>(p, p.tiles_m * p.tiles_n, st, "qh_gemm_tile");
}

template <typename T, typename OT>
int dense_tile_layout(int ta, int tb, const T* A, int64_t lda, const T* B, int64_t ldb, OT* C, int64_t ldc,
                      const T* bias, int M, int N, int K, hipStream_t st) {
  if (!ta && !tb) return dense_tile<T, OT, 256, 256, false, false>(A, lda, B, ldb, C, ldc, bias, M, N, K, st);
  if (!ta && tb) return dense_tile<T, OT, 256, 256, false, true>(A, lda, B, ldb, C, ldc, bias, M, N, K, st);
  if (ta && tb) return dense_tile<T, OT, 256, 256, true, true>(A, lda, B, ldb, C, ldc, bias, M, N, K, st);
  return dense_tile<T, OT, 256, 256, true, false>(A, lda, B, ldb, C, ldc, bias, M, N, K, st);
}

}  // namespace

// Large-tile path of qh_gemm (called by its dispatcher; not part of the C ABI).
// Requirements, checked by the caller: 16-bit operands, 16-byte aligned bases,
// strides and the contiguous extent of each operand (K for "N", M or N for "T")
// multiples of 8.
int qh_gemm_tile_dispatch(int ta, int tb, int M, int N, int K, const void* A, int64_t lda, const void* B,
                          int64_t ldb, void* C, int64_t ldc, const void* bias, int dtype, int out_dtype,
                          hipStream_t st) {
#define QH_TILE_OUT(T)                                                                                        \
  switch (out_dtype) {                                                                                       \
    case QH_F32:                                                                                             \
      return dense_tile_layout<T, float>(ta, tb, (const T*)A, lda, (const T*)B, ldb, (float*)C, ldc,          \
                                         (const T*)bias, M, N, K, st);                                       \
    case QH_F16:                                                                                             \
      return dense_tile_layout<T, f16_t>(ta, tb, (const T*)A, lda, (const T*)B, ldb, (f16_t*)C, ldc,          \
                                         (const T*)bias, M, N, K, st);                                       \
    case QH_BF16:                                                                                            \
      return dense_tile_layout<T, bf16_t>(ta, tb, (const T*)A, lda, (const T*)B, ldb, (bf16_t*)C, ldc,        \
                                          (const T*)bias, M, N, K, st);                                      \
    default: qh::set_error("qh_gemm: bad out dtype %d", out_dtype); return QH_E_DTYPE;                       \
  }
  if (dtype == QH_BF16) QH_TILE_OUT(bf16_t)
  if (dtype == QH_F16) QH_TILE_OUT(f16_t)
#undef QH_TILE_OUT
  qh::set_error("qh_gemm: the tile path takes bf16/f16 operands");
  return QH_E_DTYPE;
}
