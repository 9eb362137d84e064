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
// coordinates, reduction length), gives the address of any operand element
// (a_at / b_at; the loaders call it once per 1 KiB instruction, or per lane on
// partial tiles, so operands may be split over several matrices at 8-row or
// 8-k boundaries) and stores the accumulators, so grouped products reuse the
// same main loop.
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
  // at(i, k): address of element (tile row i, k). Rows RPI n .. RPI n + RPI-1
  // must share one stride ld. vrows: valid rows; vk: valid k from k0.
  template <class AT>
  static __device__ __forceinline__ void issue(uint32_t lds, const AT& at, int k0, int vrows, int vk, uint32_t vo,
                                               int wid) {
    if (vrows >= ROWS && vk >= BK) {
#pragma unroll
      for (int i = 0; i < PW; ++i) {
        const int n = wid + NWAVE * i;
        lds_dma16_s(vo, at(RPI * n, k0), lds + (uint32_t)n * 1024u);
      }
    } else {
      // (the empty asm keeps the lane's clamped addresses inside this rarely taken
      // branch: hoisted out of the k-loop they stay live in registers through it)
      int lane = threadIdx.x & 63;
      asm volatile("" : "+v"(lane));
      const int rin = lane / CPR;
      int kc = 8 * ((lane % CPR) ^ sw(RPI * wid + rin));
      if (kc > vk - 8) kc = vk - 8;  // vk is a positive multiple of 8
#pragma unroll
      for (int i = 0; i < PW; ++i) {
        const int n = wid + NWAVE * i;
        int r = RPI * n + rin;
        if (r > vrows - 1) r = vrows - 1;
        lds_dma16(at(r, k0 + kc), lds + (uint32_t)n * 1024u);
      }
    }
  }
  // Split roles: wave wid also issues the instructions of wave wid + NWAVE/2, whose
  // rows lie NWAVE/2 RPI rows further on at the same swizzle, so they take the same
  // scalar row address with the lane offset vo2 = vo + shift(ld) (at() linear in the
  // row with stride ld).
  static __device__ __forceinline__ uint32_t shift(int64_t ld) {
    return (uint32_t)((int64_t)(NWAVE / 2) * RPI * ld * (int64_t)sizeof(T));
  }
  template <class AT>
  static __device__ __forceinline__ void issue2(uint32_t lds, const AT& at, int k0, int vrows, int vk, uint32_t vo,
                                                uint32_t vo2, int wid) {
    if (vrows >= ROWS && vk >= BK) {
#pragma unroll
      for (int i = 0; i < PW; ++i) {
        const int n = wid + NWAVE * i;
        const T* base = at(RPI * n, k0);
        lds_dma16_s(vo, base, lds + (uint32_t)n * 1024u);
        lds_dma16_s(vo2, base, lds + (uint32_t)(n + NWAVE / 2) * 1024u);
      }
    } else {
      issue(lds, at, k0, vrows, vk, vo, wid);
      issue(lds, at, k0, vrows, vk, vo2, wid + NWAVE / 2);
    }
  }
  // Row of the tile that this lane loads in DMA instruction i (its row pointer
  // is fixed for the whole tile when rows are gathered).
  static __device__ __forceinline__ int lane_row(int wid, int i) {
    return RPI * (wid + NWAVE * i) + (int)(threadIdx.x & 63) / CPR;
  }
  // Rows reached through per-lane row pointers (gathered operands): rowp[i] is
  // the lane's row lane_row(wid, i), already clamped to a valid row.
  static __device__ __forceinline__ void issue_rows(uint32_t lds, const T* const (&rowp)[PW], int k0, int vk, int wid) {
    const int lane = threadIdx.x & 63;
    int kc = 8 * ((lane % CPR) ^ sw(RPI * wid + lane / CPR));
    if (kc > vk - 8) kc = vk - 8;  // vk is a positive multiple of 8
#pragma unroll
    for (int i = 0; i < PW; ++i) lds_dma16(rowp[i] + k0 + kc, lds + (uint32_t)(wid + NWAVE * i) * 1024u);
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
  // at(i, k): address of element (tile column i, k). k-rows RPI n .. RPI n +
  // RPI-1 must share one stride ld. vcols: valid columns; vk: valid k-rows.
  template <class AT>
  static __device__ __forceinline__ void issue(uint32_t lds, const AT& at, int k0, int vcols, int vk, uint32_t vo,
                                               int wid) {
    if (vcols >= COLS && vk >= BK) {
#pragma unroll
      for (int i = 0; i < PW; ++i) {
        const int n = wid + NWAVE * i;
        lds_dma16_s(vo, at(0, k0 + n * RPI), lds + (uint32_t)n * 1024u);
      }
    } else {
      int lane = threadIdx.x & 63;
      asm volatile("" : "+v"(lane));  // (as in NTile::issue)
      const int kin = lane / CPR, slot = lane % CPR;
#pragma unroll
      for (int i = 0; i < PW; ++i) {
        const int n = wid + NWAVE * i;
        int kr = n * RPI + kin;
        int col = 8 * (slot ^ sw(kr));
        if (col > vcols - 8) col = vcols - 8;  // vcols is a positive multiple of 8
        if (kr > vk - 1) kr = vk - 1;
        lds_dma16(at(col, k0 + kr), lds + (uint32_t)n * 1024u);
      }
    }
  }
  // Split roles (as NTile::issue2): the instructions of wave wid + NWAVE/2 read the
  // k-rows NWAVE/2 RPI further on at the same swizzle.
  static __device__ __forceinline__ uint32_t shift(int64_t ld) {
    return (uint32_t)((int64_t)(NWAVE / 2) * RPI * ld * (int64_t)sizeof(T));
  }
  template <class AT>
  static __device__ __forceinline__ void issue2(uint32_t lds, const AT& at, int k0, int vcols, int vk, uint32_t vo,
                                                uint32_t vo2, int wid) {
    if (vcols >= COLS && vk >= BK) {
#pragma unroll
      for (int i = 0; i < PW; ++i) {
        const int n = wid + NWAVE * i;
        const T* base = at(0, k0 + n * RPI);
        lds_dma16_s(vo, base, lds + (uint32_t)n * 1024u);
        lds_dma16_s(vo2, base, lds + (uint32_t)(n + NWAVE / 2) * 1024u);
      }
    } else {
      issue(lds, at, k0, vcols, vk, vo, wid);
      issue(lds, at, k0, vcols, vk, vo2, wid + NWAVE / 2);
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
  int aux, aux2;     // problem-defined (expert index, segment start)
  const T* w0;       // problem-defined operand bases (expert weights)
  const T* w1;
  T* out;            // problem-defined output base
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

// A wavefront's output tile (ROWS x COLS, rounded to T) staged in LDS for a
// vectorised epilogue. 16-byte chunk c of row r is stored at chunk
// c ^ 4((r >> 2) & 1): the staging writes (32 columns of rows r and r + 4 per
// instruction) and the 16-byte row reads are both conflict-free.
template <typename T, int ROWS, int COLS>
struct EpiTile {
  static_assert(COLS == 64, "64-column wavefront tiles");
  T* base;
  static __device__ __forceinline__ int at(int r, int col) {
    return r * COLS + 8 * ((col >> 3) ^ (((r >> 2) & 1) << 2)) + (col & 7);
  }
  __device__ __forceinline__ void put(int r, int col, T v) const { base[at(r, col)] = v; }
  // 8 consecutive columns 8 c8 .. 8 c8 + 7 of row r.
  __device__ __forceinline__ Vec16<T> row8(int r, int c8) const { return ld16(base + at(r, 8 * c8)); }
};

// Problems that define kPersistent = true place their tiles through tile_at()
// on a logical index (see the schedule in gemm_tile_kernel).
template <class P, class = void>
struct TilePersistent : std::false_type {};
template <class P>
struct TilePersistent<P, std::void_t<decltype(P::kPersistent)>> : std::integral_constant<bool, P::kPersistent> {};

// Problems that define kGatherA = true give the A tile's rows through
// a_row(ctx, i) (a pointer to row i's k = 0), so the rows may lie anywhere.
template <class P, class = void>
struct TileGatherA : std::false_type {};
template <class P>
struct TileGatherA<P, std::void_t<decltype(P::kGatherA)>> : std::integral_constant<bool, P::kGatherA> {};

// Problems that define kSkipRows = true (grouped products whose segments leave
// partial M-tiles) skip the fragment reads and MFMAs of a wavefront's 32-row
// blocks that hold no valid row: a nearly empty tail tile of an expert then
// costs its loads, not a full tile's products.
template <class P, class = void>
struct TileSkipRows : std::false_type {};
template <class P>
struct TileSkipRows<P, std::void_t<decltype(P::kSkipRows)>> : std::integral_constant<bool, P::kSkipRows> {};

// Persistent problems with 16-byte row epilogues that define kSplitStores = true
// split the wavefronts by role: waves 0 .. NWAVE/2-1 issue every operand load
// (their own share of each k-tile and that of wave w + NWAVE/2), waves
// NWAVE/2 .. NWAVE-1 every output store (their own staged rows and those of
// wave w - NWAVE/2). vmcnt counts both loads and stores, so a wave that waits
// for a k-tile also waits for its own earlier stores; with the split no wave
// does both, and a tile's stores drain while the next tile computes.
// The store waves call the problem's epilogue_store(); problems that also define
// kSplitReduce = true give the loading waves epilogue_reduce() on the same two
// staged half-tiles (row reductions beside the stores).
template <class P, class = void>
struct TileSplitStores : std::false_type {};
template <class P>
struct TileSplitStores<P, std::void_t<decltype(P::kSplitStores)>> : std::integral_constant<bool, P::kSplitStores> {};
template <class P, class = void>
struct TileSplitReduce : std::false_type {};
template <class P>
struct TileSplitReduce<P, std::void_t<decltype(P::kSplitReduce)>> : std::integral_constant<bool, P::kSplitReduce> {};

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

  // Tile schedule. Problems with kPersistent take logical tiles by XCD: the
  // workgroups of XCD x = blockIdx % 8 walk the range [x * per, (x + 1) * per)
  // of logical tiles (per = the tile count padded to a multiple of 8, over 8)
  // in steps of gridDim / 8 from blockIdx / 8, so the tiles an XCD runs at once
  // are consecutive; a grid of the padded tile count gives each workgroup one
  // tile, a smaller grid (one workgroup per CU) makes the workgroups persistent
  // (their operand strides must be the same for every tile). The other
  // problems place one tile per workgroup themselves.
  TileCtx<T> c;
  int t_local = 0, t_step = 0, t_end = 0, t_base = 0;
  constexpr bool kPersist = TilePersistent<P>::value;
  constexpr bool kGather = TileGatherA<P>::value;
  constexpr bool kSplit = TileSplitStores<P>::value && kPersist && P::kVecEpilogue;
  static_assert(!(kSplit && kGather), "split roles: k-contiguous row loads");
  static_assert(!(kGather && (kPersist || AT)), "gathered A rows: k-contiguous A, one tile per workgroup");
  if constexpr (kPersist) {
    t_end = (p.tiles_total() + 7) / 8;
    t_base = (int)(blockIdx.x & 7) * t_end;
    t_local = (int)(blockIdx.x >> 3);
    t_step = (int)(gridDim.x >> 3);
    if (t_local >= t_end || !p.tile_at(t_base + t_local, c)) return;
  } else {
    if (!p.tile(c)) return;
  }
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wid / WGN, wn = wid % WGN;
  const uint32_t lds0 = lds_addr(smem);

  f32x16 acc[TM][TN];

  constexpr int NPT = TA::PW + TB::PW;  // DMA instructions per wave and k-tile
  constexpr int ND = TM * (AT ? 2 : 1) + TN * (BT ? 2 : 1);  // LDS reads per k16 step
  constexpr int NM = TM * TN;
  auto stage = [&](int kt) { return smem + (kt % NS) * STAGE; };
  const uint32_t voa = TA::voff(c.lda, wid), vob = TB::voff(c.ldb, wid);
  const bool storer = kSplit && wid >= NWAVE / 2;  // wave-uniform
  // kSplit: lane offsets of the load share of wave wid + NWAVE/2, issued by this (loading) wave
  const uint32_t voa2 = kSplit ? voa + TA::shift(c.lda) : 0u;
  const uint32_t vob2 = kSplit ? vob + TB::shift(c.ldb) : 0u;
  // Gathered A: the lane's row pointers, taken once for the tile (rows past
  // the valid ones repeat the last valid row; the epilogue drops them).
  const T* arow[kGather ? TA::PW : 1];
  if constexpr (kGather) {
#pragma unroll
    for (int i = 0; i < TA::PW; ++i) {
      const int r = TA::lane_row(wid, i);
      arow[i] = p.a_row(c, r < c.vm ? r : c.vm - 1);
    }
  }
  // the load share of wave w (lane offsets va, vb) of k-tile kt of tile cc
  auto issue_share = [&](const TileCtx<T>& cc, int kt, uint32_t va, uint32_t vb, int w) {
    const int k0 = kt * BK;
    const int vk = cc.K - k0;
    const uint32_t base = lds0 + (uint32_t)((kt % NS) * STAGE * (int)sizeof(T));
    if constexpr (kGather) TA::issue_rows(base, arow, k0, vk, w);
    else TA::issue(base, [&](int i, int k) { return p.a_at(cc, i, k); }, k0, cc.vm, vk, va, w);
    TB::issue(base + (uint32_t)(TA::ELEMS * sizeof(T)), [&](int i, int k) { return p.b_at(cc, i, k); }, k0, cc.vn, vk,
              vb, w);
  };
  auto issue_for = [&](const TileCtx<T>& cc, int kt) {
    if constexpr (kSplit) {
      if (!storer) {
        const int k0 = kt * BK;
        const int vk = cc.K - k0;
        const uint32_t base = lds0 + (uint32_t)((kt % NS) * STAGE * (int)sizeof(T));
        TA::issue2(base, [&](int i, int k) { return p.a_at(cc, i, k); }, k0, cc.vm, vk, voa, voa2, wid);
        TB::issue2(base + (uint32_t)(TA::ELEMS * sizeof(T)), [&](int i, int k) { return p.b_at(cc, i, k); }, k0,
                   cc.vn, vk, vob, vob2, wid);
      }
    } else {
      issue_share(cc, kt, voa, vob, wid);
    }
  };
  auto issue = [&](int kt) { issue_for(c, kt); };
  // Make k-tile kt visible to every wave, with `after` later tiles still in flight.
  // (kSplit: loader waves issue two shares per k-tile; store waves issue no load, so they
  // do not wait on vmcnt, which counts their stores)
  constexpr int NPW = kSplit ? 2 * NPT : NPT;
  static_assert(3 * NPW <= 63, "vmcnt");
  auto land = [&](int kt, int after) {
    if (!storer) {
      if (after <= 0) __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
      else if (after == 1) __builtin_amdgcn_s_waitcnt(waitcnt_vm(NPW));
      else if (after == 2) __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * NPW));
      else __builtin_amdgcn_s_waitcnt(waitcnt_vm(3 * NPW));
    }
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
  constexpr bool kSkip = TileSkipRows<P>::value;
  int live = TM;  // kSkip: this wavefront's 32-row blocks with a valid row (set per tile)
  // sk: std::true_type for the copy of the k-loop that runs partial tiles
  // (branches on live), std::false_type for the branch-free full-tile copy
  auto read = [&](auto sk, const T* S, int kk, int b) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
      if (!decltype(sk)::value || i < live) af[b][i] = TA::frag(S, wm * WTM + 32 * i, kk);
#pragma unroll
    for (int j = 0; j < TN; ++j) bf[b][j] = TB::frag(S + TA::ELEMS, wn * WTN + 32 * j, kk);
  };
  auto mma = [&](auto sk, int b) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
      if (!decltype(sk)::value || i < live)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = Mfma<T>::mma(af[b][i], bf[b][j], acc[i][j]);
  };
  bool warm = false;  // k-tile 0 of c was issued during the previous tile's epilogue
  for (;;) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = zero16();
    if constexpr (kSkip) {
      const int lr = c.vm - wm * WTM;  // valid rows from this wavefront's first row
      live = __builtin_amdgcn_readfirstlane(lr <= 0 ? 0 : (lr >= WTM ? TM : (lr + 31) / 32));
    }
    const int nk = (c.K + BK - 1) / BK;
    // Tiles 0 .. NS-1 fill every stage. After the barrier that lands tile kt+1,
    // every wave has finished reading tile kt (its last fragments were read
    // before that barrier), so tile kt+NS can go into tile kt's stage.
    if (nk > 0) {
      const int pro = nk < NS ? nk : NS;
      if (warm) {
        // k-tile 0 is in flight with the previous tile's epilogue stores (vmcnt
        // counts both; with split roles the loading waves store nothing): wait
        // for all of them, then fill the other stages (stage 1 held the staged
        // rows until this barrier)
        land(0, 0);
        for (int t = 1; t < pro; ++t) issue(t);
      } else {
        for (int t = 0; t < pro; ++t) issue(t);
        land(0, pro - 1);
      }
    }
    auto kloop = [&](auto sk) {
      if (nk > 0) read(sk, stage(0), 0, 0);
      for (int kt = 0; kt < nk; ++kt) {
        // steps 0 .. KS-2 of tile kt, each overlapping the next step's reads
#pragma unroll
        for (int st = 0; st + 1 < KS; ++st) {
          read(sk, stage(kt), st + 1, (st + 1) & 1);
          mma(sk, st & 1);
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
        read(sk, stage(kt + 1), 0, 0);
        mma(sk, (KS - 1) & 1);
        mma_schedule<ND, NM * 3 / 4>(std::make_integer_sequence<int, NM>{});
      }
    };
    if (kSkip && live < TM) kloop(std::integral_constant<bool, kSkip>{});
    else kloop(std::false_type{});
    if constexpr (!kPersist) {
      break;
    } else {
      TileCtx<T> cn;
      t_local += t_step;
      if (!(t_local < t_end && p.tile_at(t_base + t_local, cn))) break;
      // Hand-over: the next tile's k-tile 0 goes into stage 0 while this tile's
      // epilogue stages its rows through stage 1 (two halves of 64 rows per wave)
      // or stores straight from registers.
      __syncthreads();  // every wave is done with the operand stages
      if ((cn.K + BK - 1) / BK > 0) issue_for(cn, 0);  // strides are the same for every tile
      bool staged = false;
      if constexpr (kSplit) {
        if (p.vec_ok()) {
          // every wave stages its rows, then the store waves write the rows of two waves each
          static_assert(TM % 2 == 0 && NWAVE * (WTM / 2) * WTN <= (NS - 1) * STAGE, "half tiles fit past stage 0");
          EpiTile<T, WTM / 2, WTN> et{smem + STAGE + wid * ((WTM / 2) * WTN)};
#pragma unroll
          for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < TM / 2; ++i)
#pragma unroll
              for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g)
#pragma unroll
                  for (int r = 0; r < 4; ++r)
                    et.put(32 * i + 4 * (lane >> 5) + 8 * g + r, 32 * j + (lane & 31),
                           from_f32<T>(acc[h * (TM / 2) + i][j][4 * g + r]));
            __syncthreads();  // (waits for this wave's LDS writes) every wave's half is staged
            if (storer) {
#pragma unroll
              for (int o = 0; o < 2; ++o) {
                const int src = o == 0 ? wid : wid - NWAVE / 2;
                EpiTile<T, WTM / 2, WTN> es{smem + STAGE + src * ((WTM / 2) * WTN)};
                p.template epilogue_store<WTM / 2>(c, es, (src / WGN) * WTM + h * (WTM / 2), (src % WGN) * WTN,
                                                   lane);
              }
              __builtin_amdgcn_s_waitcnt(kWaitLgkm0);  // the staged rows are read
            } else if constexpr (TileSplitReduce<P>::value) {
#pragma unroll
              for (int o = 0; o < 2; ++o) {
                const int src = o == 0 ? wid : wid + NWAVE / 2;
                EpiTile<T, WTM / 2, WTN> es{smem + STAGE + src * ((WTM / 2) * WTN)};
                p.template epilogue_reduce<WTM / 2>(c, es, (src / WGN) * WTM + h * (WTM / 2), (src % WGN) * WTN,
                                                    lane);
              }
              __builtin_amdgcn_s_waitcnt(kWaitLgkm0);  // the staged rows are read
            }
            // the first half is read before the second is staged; the second before the next
            // tile's k-tile 1 is loaded into this stage (after the barrier of its k-tile 0)
            if (h == 0) __syncthreads();
          }
          staged = true;
        }
      } else if constexpr (P::kVecEpilogue) {
        if (p.vec_ok()) {
          static_assert(TM % 2 == 0 && NWAVE * (WTM / 2) * WTN <= (NS - 1) * STAGE, "half tiles fit past stage 0");
          EpiTile<T, WTM / 2, WTN> et{smem + STAGE + wid * ((WTM / 2) * WTN)};
#pragma unroll
          for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < TM / 2; ++i)
#pragma unroll
              for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g)
#pragma unroll
                  for (int r = 0; r < 4; ++r)
                    et.put(32 * i + 4 * (lane >> 5) + 8 * g + r, 32 * j + (lane & 31),
                           from_f32<T>(acc[h * (TM / 2) + i][j][4 * g + r]));
            __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
            __builtin_amdgcn_wave_barrier();
            p.template epilogue_vec<WTM / 2>(c, et, wm * WTM + h * (WTM / 2), wn * WTN, lane);
            __builtin_amdgcn_s_waitcnt(kWaitLgkm0);  // this half's rows are read before the next is staged
            __builtin_amdgcn_wave_barrier();
          }
          staged = true;
        }
      }
      if (!staged) p.template epilogue<TM, TN>(c, acc, wm * WTM, wn * WTN, lane);
      c = cn;
      warm = true;
    }
  }
  if constexpr (P::kVecEpilogue) {
    if (p.vec_ok()) {
      // Stage the wavefront's tile (rounded to T) in LDS, then hand it to the
      // problem as 16-byte row vectors.
      __syncthreads();  // every wave is done with the operand stages
      EpiTile<T, WTM, WTN> et{smem + wid * (WTM * WTN)};
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              et.put(32 * i + 4 * (lane >> 5) + 8 * g + r, 32 * j + (lane & 31), from_f32<T>(acc[i][j][4 * g + r]));
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      __builtin_amdgcn_wave_barrier();
      p.epilogue_vec(c, et, wm * WTM, wn * WTN, lane);
      return;
    }
  }
  p.template epilogue<TM, TN>(c, acc, wm * WTM, wn * WTN, lane);
}

// ---------------------------------------------------------------------------
// Dense problem: C = A B^T (+ bias), OT output.
// ---------------------------------------------------------------------------
// ACC (fp32 C only): C += A B^T instead of C = A B^T (+ bias).
template <typename T, typename OT, int BM, int BN, bool AT, bool BT, bool ACC = false>
struct DenseProblem {
  static_assert(!ACC || std::is_same<OT, float>::value, "accumulation into fp32 outputs only");
  const T* A;
  const T* B;
  OT* C;
  const T* bias;
  int64_t lda, ldb, ldc;
  int M, N, K, tiles_m, tiles_n;

  static constexpr bool kVecEpilogue = std::is_same<OT, T>::value && !ACC;
  static constexpr bool kPersistent = true;
  static constexpr bool kSplitStores = true;
  // 16-byte row stores write 8 columns at once: only without bias, with N and ldc multiples of 8
  // and C 16-byte aligned (else a row's last chunk would run into the next row)
  __device__ __forceinline__ bool vec_ok() const {
    return bias == nullptr && (N & 7) == 0 && (ldc & 7) == 0 && ((uintptr_t)C & 15) == 0;
  }
  // ROWS rows of 64 columns staged in et, written at tile rows wr.., columns wc..
  template <int ROWS, class ET>
  __device__ __forceinline__ void epilogue_store(const TileCtx<T>& c, const ET& et, int wr, int wc, int lane) const {
    epilogue_vec<ROWS>(c, et, wr, wc, lane);
  }
  // All of the lane's staged rows are read before its first store: one LDS round trip per call,
  // not one per 16-byte store.
  template <int ROWS = 128, class ET>
  __device__ __forceinline__ void epilogue_vec(const TileCtx<T>& c, const ET& et, int wr, int wc, int lane) const {
    constexpr int NQ = ROWS / 8;  // lane rows lane / 8 + 8 u, columns 8 (lane % 8) ..
    const int r0 = lane >> 3, c8 = lane & 7;
    const int col = c.n0 + wc + 8 * c8;
    Vec16<T> v[NQ];
#pragma unroll
    for (int u = 0; u < NQ; ++u) v[u] = et.row8(r0 + 8 * u, c8);
    T* p0 = reinterpret_cast<T*>(C) + (int64_t)(c.m0 + wr + r0) * ldc + col;
#pragma unroll
    for (int u = 0; u < NQ; ++u)
      if (c.m0 + wr + r0 + 8 * u < M && col < N) st16(p0 + (int64_t)(8 * u) * ldc, v[u]);
  }
  __device__ __forceinline__ int tiles_total() const { return tiles_m * tiles_n; }
  // Logical tile t (grouped by 8 M-tiles) of the output; false past the last.
  __device__ __forceinline__ bool tile_at(int t, TileCtx<T>& c) const {
    if (t >= tiles_m * tiles_n) return false;
    int tm, tn;
    tile_group_order(t, tiles_m, tiles_n, tm, tn);
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
  __device__ __forceinline__ const T* a_at(const TileCtx<T>& c, int i, int k) const {
    return AT ? A + (int64_t)k * lda + (c.m0 + i) : A + (int64_t)(c.m0 + i) * lda + k;
  }
  __device__ __forceinline__ const T* b_at(const TileCtx<T>& c, int i, int k) const {
    return BT ? B + (int64_t)k * ldb + (c.n0 + i) : B + (int64_t)(c.n0 + i) * ldb + k;
  }
  // C layout of a 32x32 tile: column lane % 32, rows 8g + 4(lane/32) + r. One
  // base pointer per 32x32 block; rows are constant offsets from it.
  template <int TM, int TN>
  __device__ __forceinline__ void epilogue(const TileCtx<T>& c, const f32x16 (&acc)[TM][TN], int wr, int wc,
                                           int lane) const {
    const bool full = c.vm >= BM && c.vn >= BN;
    if constexpr (ACC) {
      if (full) {
        // C += acc: all of a 32-row block's C values are loaded before the first store (a store
        // to C may alias a later load of C for the compiler, which otherwise waits out one load
        // round trip per element: +0.5 ms on the 151936 x 1024 fp32 weight gradient)
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          float cv[TN][16];
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int col = c.n0 + wc + 32 * j + (lane & 31);
            const OT* base = C + (int64_t)(c.m0 + wr + 32 * i + 4 * (lane >> 5)) * ldc + col;
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
              for (int r = 0; r < 4; ++r) cv[j][4 * g + r] = base[(8 * g + r) * ldc];
          }
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int col = c.n0 + wc + 32 * j + (lane & 31);
            OT* base = C + (int64_t)(c.m0 + wr + 32 * i + 4 * (lane >> 5)) * ldc + col;
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
              for (int r = 0; r < 4; ++r) base[(8 * g + r) * ldc] = cv[j][4 * g + r] + acc[i][j][4 * g + r];
          }
        }
        return;
      }
    }
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
            for (int r = 0; r < 4; ++r) {
              if constexpr (ACC) base[(8 * g + r) * ldc] += acc[i][j][4 * g + r];
              else base[(8 * g + r) * ldc] = from_f32<OT>(acc[i][j][4 * g + r] + bv);
            }
        } else {
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (rb + 8 * g + r < M) {
                if constexpr (ACC) base[(8 * g + r) * ldc] += acc[i][j][4 * g + r];
                else base[(8 * g + r) * ldc] = from_f32<OT>(acc[i][j][4 * g + r] + bv);
              }
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
  if (TilePersistent<P>::value && (grid <= 0 || grid % 8 != 0)) {  // the XCD schedule covers every tile only then
    qh::set_error("%s: grid %d is not a positive multiple of 8", name, grid);
    return QH_E_ARG;
  }
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
constexpr int TBKS = kDenseBK;  // split-K ranges are whole k-tiles

// Workgroups of a dense tile launch: the tile count padded to a multiple of 8
// (one tile each), or, from two rounds of tiles on, one persistent workgroup
// per CU (a multiple of 8: each XCD walks its range of tiles), which hands each
// tile's first k-tile load over to the previous tile's epilogue.
static int dense_grid(int tiles) {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 8) n = 8;
    cus[dev] = n / 8 * 8;
  }
  const int padded = (tiles + 7) / 8 * 8;
  return tiles >= 2 * cus[dev] ? cus[dev] : padded;
}

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
  return launch_tile<T, BM, BN, kDenseBK, kDenseNS, AT, BT>(p, dense_grid(p.tiles_m * p.tiles_n), st,
                                                            "qh_gemm_tile");
}

template <typename T, typename OT>
int dense_tile_layout(int ta, int tb, const T* A, int64_t lda, const T* B, int64_t ldb, OT* C, int64_t ldc,
                      const T* bias, int M, int N, int K, hipStream_t st) {
  if (!ta && !tb) return dense_tile<T, OT, 256, 256, false, false>(A, lda, B, ldb, C, ldc, bias, M, N, K, st);
  if (!ta && tb) return dense_tile<T, OT, 256, 256, false, true>(A, lda, B, ldb, C, ldc, bias, M, N, K, st);
  if (ta && tb) return dense_tile<T, OT, 256, 256, true, true>(A, lda, B, ldb, C, ldc, bias, M, N, K, st);
  return dense_tile<T, OT, 256, 256, true, false>(A, lda, B, ldb, C, ldc, bias, M, N, K, st);
}

// ===========================================================================
// Grouped expert products (MoE) over the segments of an expert-sorted row list
// ===========================================================================
// Rows of the activation operands are sorted by expert: expert e owns rows
// [seg[e], seg[e+1]). Row-tiled products place one 256-row M-tile of one
// expert per workgroup (toff[e] = first M-tile of expert e, the prefix sum of
// ceil(n_e / 256); surplus workgroups exit). Weight-gradient products reduce
// over an expert's rows (K = n_e) and place (expert, part, M-tile, N-tile).
// Expert weights are separate tensors reached through device pointer tables.
constexpr int kMoeTileM = 256;

// Workgroup id remapped so each XCD takes a contiguous run of logical tiles
// (grids are padded to a multiple of 8).
__device__ __forceinline__ int xcd_logical_tile() {
  const int pid = blockIdx.x, nblk = gridDim.x;
  return (nblk & 7) == 0 ? (pid & 7) * (nblk >> 3) + (pid >> 3) : pid;
}

// As xcd_logical_tile, over the first `total` logical tiles of a grid sized for
// an upper bound of the tile count: each XCD takes a run of ceil(total / 8), so
// the surplus workgroups (which exit, -1) do not all fall on the last XCDs.
__device__ __forceinline__ int xcd_logical_tile_of(int total) {
  const int pid = blockIdx.x, nblk = gridDim.x;
  if ((nblk & 7) != 0) return pid < total ? pid : -1;
  const int per = (total + 7) >> 3;  // nblk / 8 >= per: the grid covers the bound
  const int local = pid >> 3, t = (pid & 7) * per + local;
  return local < per && t < total ? t : -1;
}

// M-tile tm of the expert-sorted rows: expert e, first row, valid rows.
__device__ __forceinline__ bool seg_tile(const int32_t* seg, const int32_t* toff, int E, int tm, int& e, int& row0,
                                         int& rows) {
  if (tm >= toff[E]) return false;
  int lo = 0, hi = E;  // largest e with toff[e] <= tm
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (toff[mid] <= tm) lo = mid;
    else hi = mid;
  }
  e = lo;
  row0 = seg[e] + (tm - toff[e]) * kMoeTileM;
  rows = min(kMoeTileM, seg[e + 1] - row0);
  return true;
}

// Gate/up: [G | U](rows of e) = Xs(rows) [Wg_e ; Wu_e]^T, H = silu(G) * U.
// An N-tile holds 128 features: its 256 B-rows alternate 32-row blocks of
// gate and up rows, so each wavefront's two 32-column MFMA tiles hold the
// same features of gate and up and the epilogue forms H directly (G and U are
// rounded to T first, as the expert MLP's two GEMMs would). With GA the A rows
// are gathered: sorted row i is token row rows[i] of X, so no sorted copy of
// the routed rows is written first.
template <typename T, bool GA = false>
struct MoeUpProblem {
  static constexpr bool kGatherA = GA;
  static constexpr bool kSkipRows = true;
  const T* X;
  const int32_t* rows;  // GA: token row of each sorted row
  const T* const* Wt;  // 2E pointers: gate_e, up_e
  T *G, *U, *H;        // G and U may be null
  const int32_t *seg, *toff;
  int64_t ldx, ldw, ldo;
  int E, I, Kdim, tiles_n;
  __device__ __forceinline__ bool tile(TileCtx<T>& c) const {
    const int t = xcd_logical_tile_of(toff[E] * tiles_n);
    int e, row0, rows;
    if (t < 0 || !seg_tile(seg, toff, E, t / tiles_n, e, row0, rows)) return false;
    c.m0 = row0;
    c.n0 = (t % tiles_n) * 128;
    c.K = Kdim;
    c.vm = rows;
    c.vn = 256;  // I is a multiple of 128
    c.lda = ldx;
    c.ldb = ldw;
    c.aux = e;
    c.w0 = Wt[2 * e];
    c.w1 = Wt[2 * e + 1];
    return true;
  }
  __device__ __forceinline__ const T* a_at(const TileCtx<T>& c, int i, int k) const {
    return X + (int64_t)(c.m0 + i) * ldx + k;
  }
  __device__ __forceinline__ const T* a_row(const TileCtx<T>& c, int i) const {
    return X + (int64_t)rows[c.m0 + i] * ldx;
  }
  __device__ __forceinline__ const T* b_at(const TileCtx<T>& c, int i, int k) const {
    const int b = i >> 5;
    const T* W = (b & 1) ? c.w1 : c.w0;
    return W + (int64_t)(c.n0 + (b >> 1) * 32 + (i & 31)) * ldw + k;
  }
  static constexpr bool kVecEpilogue = true;
  __device__ __forceinline__ bool vec_ok() const { return true; }
  // Wavefront tile columns 0..31 hold gate and 32..63 up values of the same 32
  // features.
  // (all of the lane's staged pieces are read before its first store: one LDS round trip)
  template <class ET>
  __device__ __forceinline__ void epilogue_vec(const TileCtx<T>& c, const ET& et, int wr, int wc, int lane) const {
    const int row_end = c.m0 + c.vm;
    const int r0 = lane >> 2, c8 = lane & 3;  // lane rows r0 + 16 u
    Vec16<T> gvs[8], uvs[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      gvs[u] = et.row8(r0 + 16 * u, c8);
      uvs[u] = et.row8(r0 + 16 * u, c8 + 4);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int row = c.m0 + wr + r0 + 16 * u;
      if (row >= row_end) continue;
      const Vec16<T> gv = gvs[u], uv = uvs[u];
      Vec16<T> hv;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float gf = to_f32(gv.v[e]);
        hv.v[e] = from_f32<T>(gf * sigmoidf_(gf) * to_f32(uv.v[e]));
      }
      const int64_t o = (int64_t)row * ldo + c.n0 + (wc >> 1) + 8 * c8;
      st16(H + o, hv);
      if (G != nullptr) {
        st16(G + o, gv);
        st16(U + o, uv);
      }
    }
  }
  template <int TM, int TN>
  __device__ __forceinline__ void epilogue(const TileCtx<T>& c, const f32x16 (&acc)[TM][TN], int wr, int wc,
                                           int lane) const {
    static_assert(TN == 2, "one gate and one up MFMA tile per wavefront");
    const int f = c.n0 + (wc >> 1) + (lane & 31);  // wavefront wc/64 holds features 32 (wc/64) ..
    const int row_end = c.m0 + c.vm;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int rb = c.m0 + wr + 32 * i + 4 * (lane >> 5);
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = rb + 8 * g + r;
          if (row >= row_end) continue;
          const T gt = (T)acc[i][0][4 * g + r], up = (T)acc[i][1][4 * g + r];
          const float gf = to_f32(gt);
          const int64_t o = (int64_t)row * ldo + f;
          H[o] = from_f32<T>(gf * sigmoidf_(gf) * to_f32(up));
          if (G != nullptr) {
            G[o] = gt;
            U[o] = up;
          }
        }
    }
  }
};

// Row-tiled product with one expert matrix per segment: C(rows of e) =
// A(rows) op(W_e), W_e either [N, K] ("N", the down projection) or [K, N]
// ("T", the down projection's input gradient). Epilogues:
//   0: C = round(acc)
//   1: C = round(round(acc) * w[row])  (routing-weight scaling)
//   2: SiLU-mul backward: go = round(acc), with g = G[row, col], u = U[row, col]
//      and s = sigmoid(g): C = go u s (1 + g (1 - s)), C2 = go g s
template <typename T, bool BT, int EPI>
struct MoeRowProblem {
  static constexpr bool kSkipRows = true;
  const T* A;
  const T* const* Wt;  // E pointers
  T* C;
  T* C2;
  const T* wrow;
  const T *G, *U;
  const int32_t *seg, *toff;
  int64_t lda, ldw, ldc, ldg;
  int E, N, Kdim, tiles_n;
  __device__ __forceinline__ bool tile(TileCtx<T>& c) const {
    const int t = xcd_logical_tile_of(toff[E] * tiles_n);
    int e, row0, rows;
    if (t < 0 || !seg_tile(seg, toff, E, t / tiles_n, e, row0, rows)) return false;
    c.m0 = row0;
    c.n0 = (t % tiles_n) * 256;
    c.K = Kdim;
    c.vm = rows;
    c.vn = N - c.n0;
    c.lda = lda;
    c.ldb = ldw;
    c.aux = e;
    c.w0 = Wt[e];
    c.w1 = nullptr;
    return true;
  }
  __device__ __forceinline__ const T* a_at(const TileCtx<T>& c, int i, int k) const {
    return A + (int64_t)(c.m0 + i) * lda + k;
  }
  __device__ __forceinline__ const T* b_at(const TileCtx<T>& c, int i, int k) const {
    return BT ? c.w0 + (int64_t)k * ldw + (c.n0 + i) : c.w0 + (int64_t)(c.n0 + i) * ldw + k;
  }
  static constexpr bool kVecEpilogue = true;
  __device__ __forceinline__ bool vec_ok() const { return true; }
  // The lane's staged pieces are read 8 at a time, and their rows' routing weights or SiLU
  // inputs loaded (from clamped rows, unconditionally), before the first of their stores: a
  // store may alias a later load for the compiler, which would otherwise wait out one round
  // trip per row.
  template <class ET>
  __device__ __forceinline__ void epilogue_vec(const TileCtx<T>& c, const ET& et, int wr, int wc, int lane) const {
    const int row_end = c.m0 + c.vm;
    const int r0 = lane >> 3, c8 = lane & 7;  // lane rows r0 + 8 u
    const int col = c.n0 + wc + 8 * c8;
    const int colc = col < N ? col : N - 8;  // N is a multiple of 8
#pragma unroll
    for (int u0 = 0; u0 < 16; u0 += 8) {
      Vec16<T> vs[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) vs[u] = et.row8(r0 + 8 * (u0 + u), c8);
      if constexpr (EPI == 0) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int row = c.m0 + wr + r0 + 8 * (u0 + u);
          if (row < row_end && col < N) st16(C + (int64_t)row * ldc + col, vs[u]);
        }
      } else if constexpr (EPI == 1) {
        float w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int row = c.m0 + wr + r0 + 8 * (u0 + u);
          w[u] = to_f32(wrow[row < row_end ? row : row_end - 1]);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int row = c.m0 + wr + r0 + 8 * (u0 + u);
          if (row >= row_end || col >= N) continue;
          Vec16<T> out;
#pragma unroll
          for (int e = 0; e < 8; ++e) out.v[e] = from_f32<T>(to_f32(vs[u].v[e]) * w[u]);
          st16(C + (int64_t)row * ldc + col, out);
        }
      } else {
        Vec16<T> gv[8], uv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int row = c.m0 + wr + r0 + 8 * (u0 + u);
          const int64_t og = (int64_t)(row < row_end ? row : row_end - 1) * ldg + colc;
          gv[u] = ld16(G + og);
          uv[u] = ld16(U + og);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int row = c.m0 + wr + r0 + 8 * (u0 + u);
          if (row >= row_end || col >= N) continue;
          Vec16<T> dg, du;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float go = to_f32(vs[u].v[e]), gf = to_f32(gv[u].v[e]), uf = to_f32(uv[u].v[e]);
            const float sg = sigmoidf_(gf);
            dg.v[e] = from_f32<T>(go * uf * sg * (1.f + gf * (1.f - sg)));
            du.v[e] = from_f32<T>(go * gf * sg);
          }
          const int64_t o = (int64_t)row * ldc + col;
          st16(C + o, dg);
          st16(C2 + o, du);
        }
      }
    }
  }
  template <int TM, int TN>
  __device__ __forceinline__ void epilogue(const TileCtx<T>& c, const f32x16 (&acc)[TM][TN], int wr, int wc,
                                           int lane) const {
    const int row_end = c.m0 + c.vm;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = c.n0 + wc + 32 * j + (lane & 31);
      if (col >= N) continue;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int rb = c.m0 + wr + 32 * i + 4 * (lane >> 5);
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = rb + 8 * g + r;
            if (row >= row_end) continue;
            const int64_t o = (int64_t)row * ldc + col;
            const float v = to_f32((T)acc[i][j][4 * g + r]);
            if constexpr (EPI == 0) {
              C[o] = from_f32<T>(v);
            } else if constexpr (EPI == 1) {
              C[o] = from_f32<T>(v * to_f32(wrow[row]));
            } else {
              const int64_t og = (int64_t)row * ldg + col;
              const float gf = to_f32(G[og]), uf = to_f32(U[og]);
              const float sg = sigmoidf_(gf);
              C[o] = from_f32<T>(v * uf * sg * (1.f + gf * (1.f - sg)));
              C2[o] = from_f32<T>(v * gf * sg);
            }
          }
      }
    }
  }
};

// Input gradient of the gate/up projections: dX(rows of e) = [dG | dU] (rows)
// [Wg_e ; Wu_e] (K = 2I; I is a multiple of 64 so no k-tile straddles).
template <typename T>
struct MoeDxProblem {
  static constexpr bool kSkipRows = true;
  const T *dG, *dU;
  const T* const* Wt;  // 2E pointers: gate_e, up_e ([I, H] each)
  T* C;
  const int32_t *seg, *toff;
  int64_t ldg, ldw, ldc;
  int E, I, N, tiles_n;
  __device__ __forceinline__ bool tile(TileCtx<T>& c) const {
    const int t = xcd_logical_tile_of(toff[E] * tiles_n);
    int e, row0, rows;
    if (t < 0 || !seg_tile(seg, toff, E, t / tiles_n, e, row0, rows)) return false;
    c.m0 = row0;
    c.n0 = (t % tiles_n) * 256;
    c.K = 2 * I;
    c.vm = rows;
    c.vn = N - c.n0;
    c.lda = ldg;
    c.ldb = ldw;
    c.aux = e;
    c.w0 = Wt[2 * e];
    c.w1 = Wt[2 * e + 1];
    return true;
  }
  __device__ __forceinline__ const T* a_at(const TileCtx<T>& c, int i, int k) const {
    return k < I ? dG + (int64_t)(c.m0 + i) * ldg + k : dU + (int64_t)(c.m0 + i) * ldg + (k - I);
  }
  __device__ __forceinline__ const T* b_at(const TileCtx<T>& c, int i, int k) const {
    return k < I ? c.w0 + (int64_t)k * ldw + (c.n0 + i) : c.w1 + (int64_t)(k - I) * ldw + (c.n0 + i);
  }
  static constexpr bool kVecEpilogue = true;
  __device__ __forceinline__ bool vec_ok() const { return true; }
  // (all of the lane's staged pieces are read before its first store: one LDS round trip)
  template <class ET>
  __device__ __forceinline__ void epilogue_vec(const TileCtx<T>& c, const ET& et, int wr, int wc, int lane) const {
    const int row_end = c.m0 + c.vm;
    const int r0 = lane >> 3, c8 = lane & 7;  // lane rows r0 + 8 u
    const int col = c.n0 + wc + 8 * c8;
    Vec16<T> v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = et.row8(r0 + 8 * u, c8);
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int row = c.m0 + wr + r0 + 8 * u;
      if (row < row_end && col < N) st16(C + (int64_t)row * ldc + col, v[u]);
    }
  }
  template <int TM, int TN>
  __device__ __forceinline__ void epilogue(const TileCtx<T>& c, const f32x16 (&acc)[TM][TN], int wr, int wc,
                                           int lane) const {
    const int row_end = c.m0 + c.vm;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = c.n0 + wc + 32 * j + (lane & 31);
      if (col >= N) continue;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int rb = c.m0 + wr + 32 * i + 4 * (lane >> 5);
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = rb + 8 * g + r;
            if (row < row_end) C[(int64_t)row * ldc + col] = from_f32<T>(acc[i][j][4 * g + r]);
          }
      }
    }
  }
};

// Weight gradients: C_e[m, n] = sum over rows r of expert e of A[r, m] B[r, n]
// (both operands k-outer, K = n_e). NP parts share the B operand and have
// their own A and output (gate and up: NP = 2; down: NP = 1). Output e of part
// q is Out[q] + e * out_stride, row-major with row stride ldo.
template <typename T, int NP>
struct MoeWgradProblem {
  const T* A[NP];
  const T* B;
  T* Out[NP];
  const int32_t* seg;
  int64_t lda, ldb, ldo, out_stride;
  int E, M, N, tiles_m, tiles_n;
  __device__ __forceinline__ bool tile(TileCtx<T>& c) const {
    const int t = xcd_logical_tile();
    const int per_part = tiles_m * tiles_n;
    const int per_e = NP * per_part;
    const int e = t / per_e;
    if (e >= E) return false;
    const int q = (t % per_e) / per_part, rest = t % per_part;
    c.m0 = (rest / tiles_n) * 256;
    c.n0 = (rest % tiles_n) * 256;
    const int s0 = seg[e];
    c.K = seg[e + 1] - s0;
    c.vm = M - c.m0;
    c.vn = N - c.n0;
    c.lda = lda;
    c.ldb = ldb;
    c.aux = e;
    c.aux2 = s0;
    c.w0 = A[0];
    c.out = Out[0];
    if constexpr (NP > 1) {
      if (q == 1) {
        c.w0 = A[1];
        c.out = Out[1];
      }
    }
    return true;
  }
  __device__ __forceinline__ const T* a_at(const TileCtx<T>& c, int i, int k) const {
    return c.w0 + (int64_t)(c.aux2 + k) * lda + (c.m0 + i);
  }
  __device__ __forceinline__ const T* b_at(const TileCtx<T>& c, int i, int k) const {
    return B + (int64_t)(c.aux2 + k) * ldb + (c.n0 + i);
  }
  static constexpr bool kVecEpilogue = true;
  __device__ __forceinline__ bool vec_ok() const { return true; }
  template <class ET>
  __device__ __forceinline__ void epilogue_vec(const TileCtx<T>& c, const ET& et, int wr, int wc, int lane) const {
    T* out = c.out + (int64_t)c.aux * out_stride;
    // (all of the lane's staged pieces are read before its first store: one LDS round trip)
    const int r0 = lane >> 3, c8 = lane & 7;  // lane rows r0 + 8 u
    const int col = c.n0 + wc + 8 * c8;
    Vec16<T> v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = et.row8(r0 + 8 * u, c8);
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int row = c.m0 + wr + r0 + 8 * u;
      if (row < M && col < N) st16(out + (int64_t)row * ldo + col, v[u]);
    }
  }
  template <int TM, int TN>
  __device__ __forceinline__ void epilogue(const TileCtx<T>& c, const f32x16 (&acc)[TM][TN], int wr, int wc,
                                           int lane) const {
    T* out = c.out + (int64_t)c.aux * out_stride;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = c.n0 + wc + 32 * j + (lane & 31);
      if (col >= N) continue;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int rb = c.m0 + wr + 32 * i + 4 * (lane >> 5);
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = rb + 8 * g + r;
            if (row < M) out[(int64_t)row * ldo + col] = from_f32<T>(acc[i][j][4 * g + r]);
          }
      }
    }
  }
};

// Grid of a row-tiled grouped product: every possible M-tile (an upper bound:
// ceil(R / 256) + E) times the N-tiles, padded to a multiple of 8.
inline int moe_row_grid(int64_t R, int64_t E, int tiles_n) {
  const int64_t g = ((R + kMoeTileM - 1) / kMoeTileM + E) * tiles_n;
  return (int)((g + 7) / 8 * 8);
}

template <typename T, bool AT, bool BT, class P>
int launch_moe(const P& p, int64_t grid, hipStream_t st, const char* name) {
  if (grid >= (1ll << 31)) {
    qh::set_error("%s: too many tiles", name);
    return QH_E_ARG;
  }
  return launch_tile<T, 256, 256, kDenseBK, kDenseNS, AT, BT>(p, (int)grid, st, name);
}

// ---------------------------------------------------------------------------
// Split-K dense product: few output tiles, long K. Split s of S computes the
// K range [s Ks, (s+1) Ks) of every tile into an fp32 partial; a reduction
// then adds the S partials in order (deterministic), adds the bias and
// converts.
// ---------------------------------------------------------------------------
template <typename T, bool AT, bool BT>
struct SplitKProblem {
  const T* A;
  const T* B;
  float* P;  // S partials of [M, N]
  int64_t lda, ldb;
  int M, N, K, Ks, S, tiles_m, tiles_n;
  static constexpr bool kVecEpilogue = false;
  __device__ __forceinline__ bool vec_ok() const { return false; }
  __device__ __forceinline__ bool tile(TileCtx<T>& c) const {
    const int t = xcd_logical_tile();
    const int per = tiles_m * tiles_n;
    const int sp = t / per;
    if (sp >= S) return false;
    // N-tiles fastest: the N-tiles of an M-tile run at once on one XCD and walk their K range
    // together, so each A k-tile comes from HBM once for all of them (with M-tiles fastest, the
    // 5632 x 151936 logit-gradient block of the fused LM head's input gradient was fetched ~3x)
    const int rest = t % per;
    c.m0 = (rest / tiles_n) * 256;
    c.n0 = (rest % tiles_n) * 256;
    c.aux = sp * Ks;
    c.K = min(Ks, K - c.aux);
    c.vm = M - c.m0;
    c.vn = N - c.n0;
    c.lda = lda;
    c.ldb = ldb;
    c.aux2 = sp;
    return true;
  }
  __device__ __forceinline__ const T* a_at(const TileCtx<T>& c, int i, int k) const {
    const int kk = c.aux + k;
    return AT ? A + (int64_t)kk * lda + (c.m0 + i) : A + (int64_t)(c.m0 + i) * lda + kk;
  }
  __device__ __forceinline__ const T* b_at(const TileCtx<T>& c, int i, int k) const {
    const int kk = c.aux + k;
    return BT ? B + (int64_t)kk * ldb + (c.n0 + i) : B + (int64_t)(c.n0 + i) * ldb + kk;
  }
  template <class ET>
  __device__ __forceinline__ void epilogue_vec(const TileCtx<T>&, const ET&, int, int, int) const {}
  template <int TM, int TN>
  __device__ __forceinline__ void epilogue(const TileCtx<T>& c, const f32x16 (&acc)[TM][TN], int wr, int wc,
                                           int lane) const {
    float* out = P + (int64_t)c.aux2 * M * N;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = c.n0 + wc + 32 * j + (lane & 31);
      if (col >= N) continue;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int rb = c.m0 + wr + 32 * i + 4 * (lane >> 5);
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = rb + 8 * g + r;
            if (row < M) out[(int64_t)row * N + col] = acc[i][j][4 * g + r];
          }
      }
    }
  }
};

template <typename T, typename OT>
__global__ __launch_bounds__(256) void splitk_reduce(const float* __restrict__ P, int S, int64_t M, int64_t N,
                                                     const T* __restrict__ bias, OT* __restrict__ C, int64_t ldc) {
  const int64_t total = M * N;
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    float s = 0.f;
    for (int sp = 0; sp < S; ++sp) s += P[sp * total + i];
    const int64_t row = i / N, col = i - row * N;
    if (bias) s += to_f32(bias[col]);
    C[row * ldc + col] = from_f32<OT>(s);
  }
}

// Splits for a dense product (1 = no split): fewer 256x256 tiles than one round of workgroups
// (256) and long K. Each split's K range is at least 1024; the count is the smallest that fills
// the rounds it needs within 10% of the best fill up to 16 splits (a 128-tile product with
// K = 151936, the LM head's input gradient for 8192 rows, ran on half the CUs unsplit: 3.26 ms).
inline int splitk_count(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + 255) / 256) * ((N + 255) / 256);
  if (M < 256 || N < 256 || tiles >= 256 || K < 2048) return 1;
  const int64_t smax = K / 1024 < 16 ? K / 1024 : 16;
  auto fill = [&](int64_t s) {
    const int64_t w = s * tiles;
    return (double)w / (double)(((w + 255) / 256) * 256);
  };
  double best = 0.0;
  for (int64_t s = 1; s <= smax; ++s) best = fill(s) > best ? fill(s) : best;
  for (int64_t s = 1; s <= smax; ++s)
    if (fill(s) >= 0.9 * best && s * tiles >= 192) return (int)s;
  return (int)smax;
}

template <typename T, typename OT, bool AT, bool BT>
int splitk_run(const T* A, int64_t lda, const T* B, int64_t ldb, OT* C, int64_t ldc, const T* bias, int M, int N,
               int K, int S, float* ws, hipStream_t st) {
  SplitKProblem<T, AT, BT> p;
  p.A = A;
  p.B = B;
  p.P = ws;
  p.lda = lda;
  p.ldb = ldb;
  p.M = M;
  p.N = N;
  p.K = K;
  p.Ks = ((K + S - 1) / S + TBKS - 1) / TBKS * TBKS;
  p.S = (K + p.Ks - 1) / p.Ks;
  p.tiles_m = (M + 255) / 256;
  p.tiles_n = (N + 255) / 256;
  const int64_t grid = ((int64_t)p.S * p.tiles_m * p.tiles_n + 7) / 8 * 8;
  int rc = launch_tile<T, 256, 256, kDenseBK, kDenseNS, AT, BT>(p, (int)grid, st, "qh_gemm (split-K)");
  if (rc) return rc;
  const int64_t total = (int64_t)M * N;
  const int g = (int)((total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192);
  splitk_reduce<T, OT><<<g, 256, 0, st>>>(ws, p.S, M, N, bias, C, ldc);
  return QH_OK;
}

template <typename T, typename OT>
int splitk_layout(int ta, int tb, const T* A, int64_t lda, const T* B, int64_t ldb, OT* C, int64_t ldc,
                  const T* bias, int M, int N, int K, int S, float* ws, hipStream_t st) {
  if (!ta && !tb) return splitk_run<T, OT, false, false>(A, lda, B, ldb, C, ldc, bias, M, N, K, S, ws, st);
  if (!ta && tb) return splitk_run<T, OT, false, true>(A, lda, B, ldb, C, ldc, bias, M, N, K, S, ws, st);
  if (ta && tb) return splitk_run<T, OT, true, true>(A, lda, B, ldb, C, ldc, bias, M, N, K, S, ws, st);
  return splitk_run<T, OT, true, false>(A, lda, B, ldb, C, ldc, bias, M, N, K, S, ws, st);
}

// ===========================================================================
// Fused LM head + cross-entropy over vocabulary tiles
// ===========================================================================
// Logits S = X W^T (X [N, H] token rows, W [V, H] vocabulary rows, both
// k-contiguous) are produced tile by tile by the main loop and consumed by
// the epilogue, rounded to T first (the dtype the unfused LM head writes its
// logits in), so no [N, V] logits tensor exists.
//
// Forward: each 256-column tile of a row becomes one partial (max, sum of
// exp(s - max)) in a fixed layout part[row][tile]; the tile holding a row's
// target also stores that logit. Each wavefront stages its 128 x 64 tile; lane
// l folds rows l and l + 64 (max pass, then sum pass over the 64 values in
// LDS); the four column waves of a row half then fold their partials through
// LDS in column order, so a row's partial does not depend on timing.
__device__ __forceinline__ void lmce_merge(float& m, float& s, float m2, float s2) {
  const float M = fmaxf(m, m2);
  if (M == -INFINITY) return;
  s = (m == -INFINITY ? 0.f : s * __expf(m - M)) + (m2 == -INFINITY ? 0.f : s2 * __expf(m2 - M));
  m = M;
}

template <typename T>
struct LmceFwdProblem {
  const T* X;
  const T* W;
  const int64_t* tgt;
  float* part;    // [M][tiles_n][2]
  float* tlogit;  // [M]
  int64_t ldx, ldw;
  int M, N, K, tiles_m, tiles_n;

  static constexpr bool kVecEpilogue = true;
  __device__ __forceinline__ bool vec_ok() const { return true; }
  __device__ __forceinline__ bool tile(TileCtx<T>& c) const {
    int tm, tn;
    tile_order(tiles_m, tiles_n, tm, tn);
    c.m0 = tm * 256;
    c.n0 = tn * 256;
    c.K = K;
    c.vm = M - c.m0;
    c.vn = N - c.n0;
    c.lda = ldx;
    c.ldb = ldw;
    c.aux = tn;
    return true;
  }
  __device__ __forceinline__ const T* a_at(const TileCtx<T>& c, int i, int k) const {
    return X + (int64_t)(c.m0 + i) * ldx + k;
  }
  __device__ __forceinline__ const T* b_at(const TileCtx<T>& c, int i, int k) const {
    return W + (int64_t)(c.n0 + i) * ldw + k;
  }
  template <class ET>
  __device__ __forceinline__ void epilogue_vec(const TileCtx<T>& c, const ET& et, int wr, int wc, int lane) const {
    const int ncol = max(0, min(64, c.vn - wc));  // valid columns of this wave's tile
    float pm[2], ps[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = lane + 64 * h;
      const int row = c.m0 + wr + r;
      float m = -INFINITY, sum = 0.f;
      if (row < M && ncol > 0) {
#pragma unroll
        for (int c8 = 0; c8 < 8; ++c8) {
          const Vec16<T> v = et.row8(r, c8);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (8 * c8 + e < ncol) m = fmaxf(m, to_f32(v.v[e]));
        }
#pragma unroll
        for (int c8 = 0; c8 < 8; ++c8) {
          const Vec16<T> v = et.row8(r, c8);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (8 * c8 + e < ncol) sum += __expf(to_f32(v.v[e]) - m);
        }
        const int64_t t = tgt[row];
        const int64_t tc = t - (int64_t)(c.n0 + wc);
        if (tc >= 0 && tc < ncol) tlogit[row] = to_f32(et.row8(r, (int)(tc >> 3)).v[tc & 7]);
      }
      pm[h] = m;
      ps[h] = sum;
    }
    // fold the four column waves of this row half in column order
    const int wm = wr / 128, wn = wc / 64;
    float* mine = reinterpret_cast<float*>(et.base);  // this wave's staging area, reads above are done
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      mine[2 * (lane + 64 * h)] = pm[h];
      mine[2 * (lane + 64 * h) + 1] = ps[h];
    }
    __syncthreads();
    if (wn != 0) return;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = lane + 64 * h;
      const int row = c.m0 + wr + r;
      float m = -INFINITY, sum = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float* other = reinterpret_cast<const float*>(et.base + w * 128 * 64);  // wave (wm, w)
        lmce_merge(m, sum, other[2 * r], other[2 * r + 1]);
      }
      if (row < M) {
        float* o = part + ((int64_t)row * tiles_n + c.aux) * 2;
        o[0] = m;
        o[1] = sum;
      }
    }
    (void)wm;
  }
  template <int TM, int TN>
  __device__ __forceinline__ void epilogue(const TileCtx<T>&, const f32x16 (&)[TM][TN], int, int, int) const {}
};

// Logits of a block of rows for the fused LM head + cross-entropy with
// gradients: Z = X W^T rounded to T and written out (the caller turns Z into
// the logit gradient in place), and per row the (max, sum of exp) of every
// 64-column block of the rounded logits, so the row's logsumexp needs no
// further pass over Z (the combine reads the target logits from Z). The
// epilogue issues no global load: on gfx9 vmcnt also counts stores, so a load
// waited for in the epilogue would wait for the tile's Z stores and for the
// next tile's first operand loads. Persistent like the dense problem; each
// wavefront reduces its own 64 columns, so no cross-wave step is needed in the
// epilogue.
template <typename T>
struct LmceLogitsProblem {
  const T* X;
  const T* W;
  T* Z;
  float2* part;   // [nblk][M] (max, sum of exp): a wave's rows are consecutive, stores coalesce
  int64_t ldx, ldw, ldz;
  int M, N, K, tiles_m, tiles_n, nblk;

  static constexpr bool kVecEpilogue = true;
  static constexpr bool kPersistent = true;
  // persistent hand-over: store waves write the logits, loading waves form the row partials
  static constexpr bool kSplitStores = true;
  static constexpr bool kSplitReduce = true;
  __device__ __forceinline__ bool vec_ok() const { return true; }
  __device__ __forceinline__ int tiles_total() const { return tiles_m * tiles_n; }
  __device__ __forceinline__ bool tile_at(int t, TileCtx<T>& c) const {
    if (t >= tiles_m * tiles_n) return false;
    int tm, tn;
    tile_group_order(t, tiles_m, tiles_n, tm, tn);
    c.m0 = tm * 256;
    c.n0 = tn * 256;
    c.K = K;
    c.vm = M - c.m0;
    c.vn = N - c.n0;
    c.lda = ldx;
    c.ldb = ldw;
    c.aux = 0;
    return true;
  }
  __device__ __forceinline__ const T* a_at(const TileCtx<T>& c, int i, int k) const {
    return X + (int64_t)(c.m0 + i) * ldx + k;
  }
  __device__ __forceinline__ const T* b_at(const TileCtx<T>& c, int i, int k) const {
    return W + (int64_t)(c.n0 + i) * ldw + k;
  }
  template <int ROWS = 128, class ET>
  __device__ __forceinline__ void epilogue_vec(const TileCtx<T>& c, const ET& et, int wr, int wc, int lane) const {
    epilogue_store<ROWS>(c, et, wr, wc, lane);
    epilogue_reduce<ROWS>(c, et, wr, wc, lane);
  }
  template <int ROWS, class ET>
  __device__ __forceinline__ void epilogue_store(const TileCtx<T>& c, const ET& et, int wr, int wc, int lane) const {
    {
      // the rounded logits, 8 lanes per 128-byte row piece; all of the lane's staged pieces
      // are read before its first store (one LDS round trip, not one per store)
      constexpr int NQ = ROWS / 8;
      const int r0 = lane >> 3, c8 = lane & 7;
      const int col = c.n0 + wc + 8 * c8;
      Vec16<T> v[NQ];
#pragma unroll
      for (int u = 0; u < NQ; ++u) v[u] = et.row8(r0 + 8 * u, c8);
      T* p0 = Z + (int64_t)(c.m0 + wr + r0) * ldz + col;
#pragma unroll
      for (int u = 0; u < NQ; ++u)
        if (c.m0 + wr + r0 + 8 * u < M && col < N) st16(p0 + (int64_t)(8 * u) * ldz, v[u]);
    }
  }
  // (max, sum of exp) of each staged row's piece of up to 64 columns, one row per lane
  template <int ROWS, class ET>
  __device__ __forceinline__ void epilogue_reduce(const TileCtx<T>& c, const ET& et, int wr, int wc, int lane) const {
    const int ncol = max(0, min(64, c.vn - wc));
    const int blk = (c.n0 + wc) >> 6;
    for (int r = lane; r < ROWS; r += 64) {
      const int row = c.m0 + wr + r;
      if (row >= M || ncol == 0) continue;
      float m = -INFINITY, sum = 0.f;
      if (ncol == 64) {
        // a whole 64-column piece: the row's 8 pieces read at once, its max first, then one
        // exp per value
        Vec16<T> v[8];
#pragma unroll
        for (int c8 = 0; c8 < 8; ++c8) v[c8] = et.row8(r, c8);
#pragma unroll
        for (int c8 = 0; c8 < 8; ++c8)
#pragma unroll
          for (int e = 0; e < 8; ++e) m = fmaxf(m, to_f32(v[c8].v[e]));
        if (m != -INFINITY) {
#pragma unroll
          for (int c8 = 0; c8 < 8; ++c8)
#pragma unroll
            for (int e = 0; e < 8; ++e) sum += __expf(to_f32(v[c8].v[e]) - m);
        }
        part[(int64_t)blk * M + row] = make_float2(m, sum);
        continue;
      }
#pragma unroll
      for (int c8 = 0; c8 < 8; ++c8) {
        if (8 * c8 >= ncol) break;
        const Vec16<T> v = et.row8(r, c8);
        float lm = -INFINITY;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (8 * c8 + e < ncol) lm = fmaxf(lm, to_f32(v.v[e]));
        if (lm > m) {
          sum = m == -INFINITY ? 0.f : sum * __expf(m - lm);
          m = lm;
        }
        if (m != -INFINITY) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (8 * c8 + e < ncol) sum += __expf(to_f32(v.v[e]) - m);
        }
      }
      part[(int64_t)blk * M + row] = make_float2(m, sum);
    }
  }
  template <int TM, int TN>
  __device__ __forceinline__ void epilogue(const TileCtx<T>&, const f32x16 (&)[TM][TN], int, int, int) const {}
};

// lse and loss_rows of the row block from LmceLogitsProblem's [nblk][M]
// partials: 64 consecutive rows per workgroup; wave w folds the blocks
// b = w, w + 16, ... of its lane's row in order, eight loads in flight at a time
// (lanes read consecutive rows: coalesced), then the 16 wave results are folded
// in wave order. The target logit is read from Z (the rounded logits).
constexpr int kCombWaves = 16;
template <typename T>
__global__ __launch_bounds__(64 * kCombWaves) void lmce_combine_cols_kernel(
    const float2* __restrict__ part, const T* __restrict__ Z, int64_t ldz, const int64_t* __restrict__ tgt, int64_t N,
    int nblk, int64_t V, int64_t ignore, float* __restrict__ lse, float* __restrict__ loss_rows) {
  __shared__ float sm[kCombWaves][64], ss[kCombWaves][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * 64 + lane;
  float m = -INFINITY, s = 0.f;
  if (row < N) {
    constexpr int U = 8;
    for (int b0 = w; b0 < nblk; b0 += kCombWaves * U) {
      float2 p[U];
#pragma unroll
      for (int j = 0; j < U; ++j) {
        const int b = b0 + kCombWaves * j;
        p[j] = b < nblk ? part[(int64_t)b * N + row] : make_float2(-INFINITY, 0.f);
      }
#pragma unroll
      for (int j = 0; j < U; ++j) lmce_merge(m, s, p[j].x, p[j].y);
    }
  }
  sm[w][lane] = m;
  ss[w][lane] = s;
  __syncthreads();
  if (w != 0 || row >= N) return;
  m = sm[0][lane];
  s = ss[0][lane];
#pragma unroll
  for (int i = 1; i < kCombWaves; ++i) lmce_merge(m, s, sm[i][lane], ss[i][lane]);
  const int64_t t = tgt[row];
  const float l = m + __logf(s);
  if (t == ignore) {
    lse[row] = 0.f;
    loss_rows[row] = 0.f;
  } else {
    lse[row] = l;
    loss_rows[row] = (t >= 0 && t < V) ? l - to_f32(Z[row * ldz + t]) : __int_as_float(0x7fc00000);
  }
}

// n_valid = number of targets != ignore (fp32, exact below 2^24 rows).
__global__ __launch_bounds__(1024) void lmce_count_kernel(const int64_t* __restrict__ tgt, int64_t N, int64_t ignore,
                                                          float* __restrict__ nvalid_out) {
  __shared__ float red[16];
  float n = 0.f;
  for (int64_t i = threadIdx.x; i < N; i += 1024) n += (tgt[i] != ignore) ? 1.f : 0.f;
  n = block_sum(n, red);
  if (threadIdx.x == 0) nvalid_out[0] = n;
}

// lse[row] from the row's tile partials (tile order), loss_rows[row] =
// lse - target logit (0 for ignored rows, NaN for targets outside [0, V)).
__global__ __launch_bounds__(256) void lmce_combine_kernel(const float* __restrict__ part,
                                                           const float* __restrict__ tlogit,
                                                           const int64_t* __restrict__ tgt, int64_t N, int tiles,
                                                           int64_t V, int64_t ignore, float* __restrict__ lse,
                                                           float* __restrict__ loss_rows) {
  const int64_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= N) return;
  // lanes fold interleaved tiles, then a fixed xor tree
  float m = -INFINITY, s = 0.f;
  for (int t = lane; t < tiles; t += 64) lmce_merge(m, s, part[(row * tiles + t) * 2], part[(row * tiles + t) * 2 + 1]);
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(s, o);
    lmce_merge(m, s, m2, s2);
  }
  if (lane == 0) {
    const int64_t t = tgt[row];
    const float l = m + __logf(s);
    if (t == ignore) {
      lse[row] = 0.f;
      loss_rows[row] = 0.f;
    } else {
      lse[row] = l;
      loss_rows[row] = (t >= 0 && t < V) ? l - tlogit[row] : __int_as_float(0x7fc00000);
    }
  }
}

// loss_out = sum(loss_rows) / max(1, n_valid) (fixed order), nvalid_out = n_valid.
__global__ __launch_bounds__(1024) void lmce_finalize_kernel(const float* __restrict__ loss_rows,
                                                             const int64_t* __restrict__ tgt, int64_t N,
                                                             int64_t ignore, float* __restrict__ loss_out,
                                                             float* __restrict__ nvalid_out) {
  __shared__ float red[16];
  float s = 0.f, n = 0.f;
  for (int64_t i = threadIdx.x; i < N; i += 1024) {
    s += loss_rows[i];
    n += (tgt[i] != ignore) ? 1.f : 0.f;
  }
  s = block_sum(s, red);
  n = block_sum(n, red);
  if (threadIdx.x == 0) {
    loss_out[0] = s / fmaxf(n, 1.f);
    nvalid_out[0] = n;
  }
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

// ===========================================================================
// C ABI: grouped expert products
// ===========================================================================
namespace {
bool moe_ok(const void* p, int64_t ld) { return aligned16(p) && ld % 8 == 0; }
}  // namespace

extern "C" int qh_moe_up(const void* X, int64_t ldx, const int32_t* rows, int64_t R, int64_t K,
                         const void* const* gu_table, int64_t ldw, int64_t I, const int32_t* seg_off,
                         const int32_t* tile_off, int64_t E, void* G, void* U, void* H, int64_t ldo, int dtype,
                         void* stream) {
  QH_CHECK_ARG(R >= 0 && K > 0 && I > 0 && E > 0 && E <= 65536, "qh_moe_up: bad shape");
  QH_CHECK_ARG(I % 128 == 0 && K % 8 == 0 && ldo >= I, "qh_moe_up: needs I %% 128 == 0, K %% 8 == 0");
  QH_CHECK_ARG(moe_ok(X, ldx) && ldw % 8 == 0 && moe_ok(H, ldo) && (G == nullptr) == (U == nullptr),
               "qh_moe_up: operands must be 16-byte aligned with strides multiples of 8");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_moe_up: bf16/f16 only");
  if (R == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const int tn = (int)(I / 128);
  int rc = QH_OK;
#define QH_UP(T, GA)                                                                                    \
  {                                                                                                     \
    MoeUpProblem<T, GA> p;                                                                              \
    p.X = (const T*)X;                                                                                  \
    p.rows = rows;                                                                                      \
    p.Wt = (const T* const*)gu_table;                                                                   \
    p.G = (T*)G;                                                                                        \
    p.U = (T*)U;                                                                                        \
    p.H = (T*)H;                                                                                        \
    p.seg = seg_off;                                                                                    \
    p.toff = tile_off;                                                                                  \
    p.ldx = ldx;                                                                                        \
    p.ldw = ldw;                                                                                        \
    p.ldo = ldo;                                                                                        \
    p.E = (int)E;                                                                                       \
    p.I = (int)I;                                                                                       \
    p.Kdim = (int)K;                                                                                    \
    p.tiles_n = tn;                                                                                     \
    rc = launch_moe<T, false, false>(p, moe_row_grid(R, E, tn), st, "qh_moe_up");                       \
  }
  if (rows != nullptr) {
    if (dtype == QH_BF16) QH_UP(bf16_t, true) else QH_UP(f16_t, true)
  } else {
    if (dtype == QH_BF16) QH_UP(bf16_t, false) else QH_UP(f16_t, false)
  }
#undef QH_UP
  if (rc) return rc;
  QH_CHECK_LAUNCH("qh_moe_up");
  return QH_OK;
}

namespace {
template <typename T, bool BT, int EPI>
int moe_row_launch(const void* A, int64_t lda, int64_t R, int64_t K, const void* const* table, int64_t ldw, int64_t N,
                   const int32_t* seg, const int32_t* toff, int64_t E, void* C, void* C2, int64_t ldc,
                   const void* wrow, const void* G, const void* U, int64_t ldg, hipStream_t st, const char* name) {
  MoeRowProblem<T, BT, EPI> p;
  p.A = (const T*)A;
  p.Wt = (const T* const*)table;
  p.C = (T*)C;
  p.C2 = (T*)C2;
  p.wrow = (const T*)wrow;
  p.G = (const T*)G;
  p.U = (const T*)U;
  p.seg = seg;
  p.toff = toff;
  p.lda = lda;
  p.ldw = ldw;
  p.ldc = ldc;
  p.ldg = ldg;
  p.E = (int)E;
  p.N = (int)N;
  p.Kdim = (int)K;
  p.tiles_n = (int)((N + 255) / 256);
  return launch_moe<T, false, BT>(p, moe_row_grid(R, E, p.tiles_n), st, name);
}
}  // namespace

extern "C" int qh_moe_down(const void* A, int64_t lda, int64_t R, int64_t K, const void* const* d_table, int64_t ldw,
                           int64_t N, const int32_t* seg_off, const int32_t* tile_off, int64_t E, void* C,
                           int64_t ldc, const void* wrow, int dtype, void* stream) {
  QH_CHECK_ARG(R >= 0 && K > 0 && N > 0 && E > 0 && E <= 65536 && K % 8 == 0 && ldc >= N,
               "qh_moe_down: bad shape");
  QH_CHECK_ARG(moe_ok(A, lda) && ldw % 8 == 0, "qh_moe_down: A must be 16-byte aligned with strides multiples of 8");
  QH_CHECK_ARG(N % 8 == 0 && moe_ok(C, ldc),  // the epilogue stores 16-byte rows of 8 columns
               "qh_moe_down: C must be 16-byte aligned with N and ldc multiples of 8");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_moe_down: bf16/f16 only");
  if (R == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  int rc;
  if (dtype == QH_BF16)
    rc = wrow ? moe_row_launch<bf16_t, false, 1>(A, lda, R, K, d_table, ldw, N, seg_off, tile_off, E, C, nullptr, ldc,
                                                 wrow, nullptr, nullptr, 0, st, "qh_moe_down")
              : moe_row_launch<bf16_t, false, 0>(A, lda, R, K, d_table, ldw, N, seg_off, tile_off, E, C, nullptr, ldc,
                                                 nullptr, nullptr, nullptr, 0, st, "qh_moe_down");
  else
    rc = wrow ? moe_row_launch<f16_t, false, 1>(A, lda, R, K, d_table, ldw, N, seg_off, tile_off, E, C, nullptr, ldc,
                                                wrow, nullptr, nullptr, 0, st, "qh_moe_down")
              : moe_row_launch<f16_t, false, 0>(A, lda, R, K, d_table, ldw, N, seg_off, tile_off, E, C, nullptr, ldc,
                                                nullptr, nullptr, nullptr, 0, st, "qh_moe_down");
  if (rc) return rc;
  QH_CHECK_LAUNCH("qh_moe_down");
  return QH_OK;
}

extern "C" int qh_moe_down_dgrad(const void* dD, int64_t ldd, int64_t R, int64_t K, const void* const* d_table,
                                 int64_t ldw, int64_t I, const int32_t* seg_off, const int32_t* tile_off, int64_t E,
                                 const void* G, const void* U, int64_t ldg, void* dG, void* dU, int64_t ldo,
                                 int dtype, void* stream) {
  QH_CHECK_ARG(R >= 0 && K > 0 && I > 0 && E > 0 && E <= 65536 && K % 8 == 0 && I % 8 == 0,
               "qh_moe_down_dgrad: bad shape");
  QH_CHECK_ARG(moe_ok(dD, ldd) && ldw % 8 == 0 && ldo >= I && ldg >= I,
               "qh_moe_down_dgrad: operands must be 16-byte aligned with strides multiples of 8");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_moe_down_dgrad: bf16/f16 only");
  if (R == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const int rc = dtype == QH_BF16
                     ? moe_row_launch<bf16_t, true, 2>(dD, ldd, R, K, d_table, ldw, I, seg_off, tile_off, E, dG, dU,
                                                       ldo, nullptr, G, U, ldg, st, "qh_moe_down_dgrad")
                     : moe_row_launch<f16_t, true, 2>(dD, ldd, R, K, d_table, ldw, I, seg_off, tile_off, E, dG, dU,
                                                      ldo, nullptr, G, U, ldg, st, "qh_moe_down_dgrad");
  if (rc) return rc;
  QH_CHECK_LAUNCH("qh_moe_down_dgrad");
  return QH_OK;
}

extern "C" int qh_moe_up_dgrad(const void* dG, const void* dU, int64_t ldg, int64_t R, int64_t I,
                               const void* const* gu_table, int64_t ldw, int64_t N, const int32_t* seg_off,
                               const int32_t* tile_off, int64_t E, void* dX, int64_t ldx, int dtype, void* stream) {
  QH_CHECK_ARG(R >= 0 && I > 0 && N > 0 && E > 0 && E <= 65536 && I % 64 == 0 && N % 8 == 0 && ldx >= N,
               "qh_moe_up_dgrad: bad shape (I must be a multiple of 64)");
  QH_CHECK_ARG(moe_ok(dG, ldg) && moe_ok(dU, ldg) && ldw % 8 == 0,
               "qh_moe_up_dgrad: operands must be 16-byte aligned with strides multiples of 8");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_moe_up_dgrad: bf16/f16 only");
  if (R == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const int tn = (int)((N + 255) / 256);
  int rc = QH_OK;
#define QH_DX(T)                                                              \
  {                                                                           \
    MoeDxProblem<T> p;                                                        \
    p.dG = (const T*)dG;                                                      \
    p.dU = (const T*)dU;                                                      \
    p.Wt = (const T* const*)gu_table;                                         \
    p.C = (T*)dX;                                                             \
    p.seg = seg_off;                                                          \
    p.toff = tile_off;                                                        \
    p.ldg = ldg;                                                              \
    p.ldw = ldw;                                                              \
    p.ldc = ldx;                                                              \
    p.E = (int)E;                                                             \
    p.I = (int)I;                                                             \
    p.N = (int)N;                                                             \
    p.tiles_n = tn;                                                           \
    rc = launch_moe<T, false, true>(p, moe_row_grid(R, E, tn), st, "qh_moe_up_dgrad"); \
  }
  if (dtype == QH_BF16) QH_DX(bf16_t) else QH_DX(f16_t)
#undef QH_DX
  if (rc) return rc;
  QH_CHECK_LAUNCH("qh_moe_up_dgrad");
  return QH_OK;
}

extern "C" int qh_moe_wgrad(int parts, const void* A0, const void* A1, int64_t lda, int64_t M, const void* B,
                            int64_t ldb, int64_t N, const int32_t* seg_off, int64_t E, void* out0, void* out1,
                            int64_t ldo, int64_t out_stride, int dtype, void* stream) {
  QH_CHECK_ARG(parts == 1 || parts == 2, "qh_moe_wgrad: 1 or 2 parts");
  QH_CHECK_ARG(M > 0 && N > 0 && E > 0 && E <= 65536 && M % 8 == 0 && N % 8 == 0 && ldo >= N,
               "qh_moe_wgrad: bad shape (M, N multiples of 8)");
  QH_CHECK_ARG(moe_ok(A0, lda) && moe_ok(B, ldb) && (parts == 1 || moe_ok(A1, lda)) && out0 != nullptr &&
                   (parts == 1 || out1 != nullptr),
               "qh_moe_wgrad: operands must be 16-byte aligned with strides multiples of 8");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_moe_wgrad: bf16/f16 only");
  hipStream_t st = (hipStream_t)stream;
  const int tm = (int)((M + 255) / 256), tn = (int)((N + 255) / 256);
  const int64_t grid = ((int64_t)E * parts * tm * tn + 7) / 8 * 8;
  int rc = QH_OK;
#define QH_WG(T, NP)                                              \
  {                                                               \
    MoeWgradProblem<T, NP> p;                                     \
    p.A[0] = (const T*)A0;                                        \
    p.Out[0] = (T*)out0;                                          \
    if constexpr (NP > 1) {                                       \
      p.A[NP - 1] = (const T*)A1;                                 \
      p.Out[NP - 1] = (T*)out1;                                   \
    }                                                             \
    p.B = (const T*)B;                                            \
    p.seg = seg_off;                                              \
    p.lda = lda;                                                  \
    p.ldb = ldb;                                                  \
    p.ldo = ldo;                                                  \
    p.out_stride = out_stride;                                    \
    p.E = (int)E;                                                 \
    p.M = (int)M;                                                 \
    p.N = (int)N;                                                 \
    p.tiles_m = tm;                                               \
    p.tiles_n = tn;                                               \
    rc = launch_moe<T, true, true>(p, grid, st, "qh_moe_wgrad");  \
  }
  if (dtype == QH_BF16) {
    if (parts == 2) QH_WG(bf16_t, 2) else QH_WG(bf16_t, 1)
  } else {
    if (parts == 2) QH_WG(f16_t, 2) else QH_WG(f16_t, 1)
  }
#undef QH_WG
  if (rc) return rc;
  QH_CHECK_LAUNCH("qh_moe_wgrad");
  return QH_OK;
}

// Split-K path of qh_gemm_ws (not part of the C ABI): splits for (M, N, K), or 1.
int qh_gemm_splitk_count(int64_t M, int64_t N, int64_t K) { return splitk_count(M, N, K); }

int qh_gemm_splitk_dispatch(int ta, int tb, int M, int N, int K, const void* A, int64_t lda, const void* B,
                            int64_t ldb, void* C, int64_t ldc, const void* bias, int dtype, int out_dtype, int S,
                            void* ws, hipStream_t st) {
#define QH_SK_OUT(T)                                                                                             \
  switch (out_dtype) {                                                                                          \
    case QH_F32:                                                                                                \
      return splitk_layout<T, float>(ta, tb, (const T*)A, lda, (const T*)B, ldb, (float*)C, ldc, (const T*)bias, \
                                     M, N, K, S, (float*)ws, st);                                               \
    case QH_F16:                                                                                                \
      return splitk_layout<T, f16_t>(ta, tb, (const T*)A, lda, (const T*)B, ldb, (f16_t*)C, ldc, (const T*)bias, \
                                     M, N, K, S, (float*)ws, st);                                               \
    case QH_BF16:                                                                                               \
      return splitk_layout<T, bf16_t>(ta, tb, (const T*)A, lda, (const T*)B, ldb, (bf16_t*)C, ldc,              \
                                      (const T*)bias, M, N, K, S, (float*)ws, st);                              \
    default: qh::set_error("qh_gemm: bad out dtype %d", out_dtype); return QH_E_DTYPE;                          \
  }
  if (dtype == QH_BF16) QH_SK_OUT(bf16_t)
  if (dtype == QH_F16) QH_SK_OUT(f16_t)
#undef QH_SK_OUT
  qh::set_error("qh_gemm: the split-K path takes bf16/f16 operands");
  return QH_E_DTYPE;
}

// ===========================================================================
// C ABI: fused LM head + cross-entropy, fp32 accumulating GEMM
// ===========================================================================
namespace {
constexpr int kLmceTile = 256;
int64_t lmce_tiles(int64_t V) { return (V + kLmceTile - 1) / kLmceTile; }
}  // namespace

extern "C" int64_t qh_lmce_workspace(int64_t N, int64_t V) {
  if (N <= 0 || V <= 0) return 0;
  return N * lmce_tiles(V) * 2 * 4 + 2 * N * 4;  // tile partials, target logits, per-row losses
}

extern "C" int qh_lmce_fwd(const void* X, int64_t ldx, const void* W, int64_t ldw, const int64_t* targets, int64_t N,
                           int64_t V, int64_t H, int64_t ignore_index, float* lse, float* loss_rows, float* loss_out,
                           float* nvalid_out, void* ws, int64_t ws_bytes, int dtype, void* stream) {
  QH_CHECK_ARG(N >= 0 && V > 0 && H > 0 && N < (1ll << 31) && V < (1ll << 31) && H < (1ll << 31),
               "qh_lmce_fwd: bad shape N=%lld V=%lld H=%lld", (long long)N, (long long)V, (long long)H);
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_lmce_fwd: bf16/f16 only");
  QH_CHECK_ARG(aligned16(X) && aligned16(W) && ldx % 8 == 0 && ldw % 8 == 0 && H % 8 == 0 && ldx >= H && ldw >= H,
               "qh_lmce_fwd: X and W must be 16-byte aligned k-contiguous rows with H, ldx, ldw multiples of 8");
  QH_CHECK_ARG(ws_bytes >= qh_lmce_workspace(N, V), "qh_lmce_fwd: workspace %lld < %lld", (long long)ws_bytes,
               (long long)qh_lmce_workspace(N, V));
  if (N == 0) return qh_zero(loss_out, 4, stream) || qh_zero(nvalid_out, 4, stream);
  hipStream_t st = (hipStream_t)stream;
  const int tiles_n = (int)lmce_tiles(V);
  float* part = (float*)ws;
  float* tlog = part + N * tiles_n * 2;
  float* rows = loss_rows ? loss_rows : tlog + N;
  int rc = QH_OK;
#define QH_LMCE(TT)                                                                              \
  {                                                                                              \
    LmceFwdProblem<TT> p;                                                                        \
    p.X = (const TT*)X;                                                                          \
    p.W = (const TT*)W;                                                                          \
    p.tgt = targets;                                                                             \
    p.part = part;                                                                               \
    p.tlogit = tlog;                                                                             \
    p.ldx = ldx;                                                                                 \
    p.ldw = ldw;                                                                                 \
    p.M = (int)N;                                                                                \
    p.N = (int)V;                                                                                \
    p.K = (int)H;                                                                                \
    p.tiles_m = (int)((N + 255) / 256);                                                          \
    p.tiles_n = tiles_n;                                                                         \
    rc = launch_tile<TT, 256, 256, kDenseBK, kDenseNS, false, false>(p, p.tiles_m * p.tiles_n, st, "qh_lmce_fwd"); \
  }
  if (dtype == QH_BF16) QH_LMCE(bf16_t) else QH_LMCE(f16_t)
#undef QH_LMCE
  if (rc) return rc;
  lmce_combine_kernel<<<(unsigned)((N + 3) / 4), 256, 0, st>>>(part, tlog, targets, N, tiles_n, V, ignore_index, lse,
                                                               rows);
  lmce_finalize_kernel<<<1, 1024, 0, st>>>(rows, targets, N, ignore_index, loss_out, nvalid_out);
  QH_CHECK_LAUNCH("qh_lmce_fwd");
  return QH_OK;
}

extern "C" int64_t qh_lmce_rows_workspace(int64_t N, int64_t V) {
  if (N <= 0 || V <= 0) return 0;
  return N * ((V + 63) / 64) * 2 * 4;  // 64-column (max, sum of exp) partials
}

extern "C" int qh_lmce_rows_fwd(const void* X, int64_t ldx, const void* W, int64_t ldw, const int64_t* targets,
                                int64_t N, int64_t V, int64_t H, int64_t ignore_index, void* Z, int64_t ldz, float* lse,
                                float* loss_rows, void* ws, int64_t ws_bytes, int dtype, void* stream) {
  QH_CHECK_ARG(N >= 0 && V > 0 && H > 0 && N < (1ll << 31) && V < (1ll << 31) && H < (1ll << 31),
               "qh_lmce_rows_fwd: bad shape N=%lld V=%lld H=%lld", (long long)N, (long long)V, (long long)H);
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_lmce_rows_fwd: bf16/f16 only");
  QH_CHECK_ARG(aligned16(X) && aligned16(W) && aligned16(Z) && ldx % 8 == 0 && ldw % 8 == 0 && ldz % 8 == 0 &&
                   H % 8 == 0 && V % 8 == 0 && ldx >= H && ldw >= H && ldz >= V,
               "qh_lmce_rows_fwd: 16-byte aligned rows with H, V, ldx, ldw, ldz multiples of 8 required");
  QH_CHECK_ARG(ws_bytes >= qh_lmce_rows_workspace(N, V), "qh_lmce_rows_fwd: workspace %lld < %lld",
               (long long)ws_bytes, (long long)qh_lmce_rows_workspace(N, V));
  QH_CHECK_ARG(lse != nullptr && loss_rows != nullptr, "qh_lmce_rows_fwd: lse and loss_rows are required");
  if (N == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const int nblk = (int)((V + 63) / 64);
  float2* part = (float2*)ws;
  int rc = QH_OK;
#define QH_LMCER(TT)                                                                               \
  {                                                                                                \
    LmceLogitsProblem<TT> p;                                                                       \
    p.X = (const TT*)X;                                                                            \
    p.W = (const TT*)W;                                                                            \
    p.Z = (TT*)Z;                                                                                  \
    p.part = part;                                                                                 \
    p.ldx = ldx;                                                                                   \
    p.ldw = ldw;                                                                                   \
    p.ldz = ldz;                                                                                   \
    p.M = (int)N;                                                                                  \
    p.N = (int)V;                                                                                  \
    p.K = (int)H;                                                                                  \
    p.tiles_m = (int)((N + 255) / 256);                                                            \
    p.tiles_n = (int)((V + 255) / 256);                                                            \
    p.nblk = nblk;                                                                                 \
    rc = launch_tile<TT, 256, 256, kDenseBK, kDenseNS, false, false>(p, dense_grid(p.tiles_m * p.tiles_n), st, \
                                                                     "qh_lmce_rows_fwd");          \
    if (rc == QH_OK)                                                                               \
      lmce_combine_cols_kernel<TT><<<(unsigned)((N + 63) / 64), 64 * kCombWaves, 0, st>>>(        \
          part, (const TT*)Z, ldz, targets, N, nblk, V, ignore_index, lse, loss_rows);             \
  }
  if (dtype == QH_BF16) QH_LMCER(bf16_t) else QH_LMCER(f16_t)
#undef QH_LMCER
  if (rc) return rc;
  QH_CHECK_LAUNCH("qh_lmce_rows_fwd");
  return QH_OK;
}

extern "C" int qh_lmce_count(const int64_t* targets, int64_t N, int64_t ignore_index, float* nvalid_out,
                             void* stream) {
  QH_CHECK_ARG(N >= 0 && N < (1ll << 31) && nvalid_out != nullptr, "qh_lmce_count: bad arguments");
  lmce_count_kernel<<<1, 1024, 0, (hipStream_t)stream>>>(targets, N, ignore_index, nvalid_out);
  QH_CHECK_LAUNCH("qh_lmce_count");
  return QH_OK;
}

extern "C" int qh_lmce_finish(const float* loss_rows, const int64_t* targets, int64_t N, int64_t ignore_index,
                              float* loss_out, float* nvalid_out, void* stream) {
  QH_CHECK_ARG(N >= 0 && N < (1ll << 31) && loss_out != nullptr && nvalid_out != nullptr,
               "qh_lmce_finish: bad arguments");
  lmce_finalize_kernel<<<1, 1024, 0, (hipStream_t)stream>>>(loss_rows, targets, N, ignore_index, loss_out,
                                                            nvalid_out);
  QH_CHECK_LAUNCH("qh_lmce_finish");
  return QH_OK;
}

extern "C" int qh_gemm_acc(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
                           const void* B, int64_t ldb, float* C, int64_t ldc, int dtype, void* stream) {
  QH_CHECK_ARG(M >= 0 && N >= 0 && K >= 0 && M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31),
               "qh_gemm_acc: bad shape");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_gemm_acc: bf16/f16 operands only");
  QH_CHECK_ARG(ldc >= N && (trans_a ? lda >= M : lda >= K) && (trans_b ? ldb >= N : ldb >= K),
               "qh_gemm_acc: leading dimensions too small");
  QH_CHECK_ARG(aligned16(A) && aligned16(B) && lda % 8 == 0 && ldb % 8 == 0 && (trans_a ? M % 8 == 0 : K % 8 == 0) &&
                   (trans_b ? N % 8 == 0 : K % 8 == 0),
               "qh_gemm_acc: 16-byte aligned operands with contiguous extents and strides multiples of 8 required");
  if (M == 0 || N == 0 || K == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  int rc = QH_OK;
#define QH_ACC_L(TT, ATV, BTV)                                                                        \
  {                                                                                                   \
    DenseProblem<TT, float, 256, 256, ATV, BTV, true> p;                                              \
    p.A = (const TT*)A;                                                                               \
    p.B = (const TT*)B;                                                                               \
    p.C = C;                                                                                          \
    p.bias = nullptr;                                                                                 \
    p.lda = lda;                                                                                      \
    p.ldb = ldb;                                                                                      \
    p.ldc = ldc;                                                                                      \
    p.M = (int)M;                                                                                     \
    p.N = (int)N;                                                                                     \
    p.K = (int)K;                                                                                     \
    p.tiles_m = (int)((M + 255) / 256);                                                               \
    p.tiles_n = (int)((N + 255) / 256);                                                               \
    rc = launch_tile<TT, 256, 256, kDenseBK, kDenseNS, ATV, BTV>(p, dense_grid(p.tiles_m * p.tiles_n), st,   \
                                                                 "qh_gemm_acc");                             \
  }
#define QH_ACC(TT)                                               \
  if (!trans_a && !trans_b) QH_ACC_L(TT, false, false)           \
  else if (!trans_a && trans_b) QH_ACC_L(TT, false, true)        \
  else if (trans_a && trans_b) QH_ACC_L(TT, true, true)          \
  else QH_ACC_L(TT, true, false)
  if (dtype == QH_BF16) { QH_ACC(bf16_t) } else { QH_ACC(f16_t) }
#undef QH_ACC
#undef QH_ACC_L
  if (rc) return rc;
  QH_CHECK_LAUNCH("qh_gemm_acc");
  return QH_OK;
}
