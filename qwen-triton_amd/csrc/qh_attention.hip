// Flash attention (forward, deterministic backward, split-KV decode) for gfx950.
//
// Layouts: q [B,Hq,Sq,D], k/v [B,Hkv,Sk,D] with arbitrary batch/head/seq strides
// and unit stride on D; outputs are contiguous. GQA maps q-head h to kv-head
// h / (Hq / Hkv) inside the kernels (no repeated K/V). D is padded to DP in
// {32, 64, 128} with zeros, so any D <= 128 that is a multiple of 8 works.
//
// Causal masking: key j is visible to query i iff j <= i + causal_offset
// (offset 0 = top-left alignment of the reference kernel; Sk - Sq =
// bottom-right alignment for chunked prefill).
//
// Forward (per workgroup: 4 wavefronts x 32*QT queries of one (b, h)):
//   S^T = K Q^T on MFMA 32x32x16 with Q kept in registers and K tiles in LDS;
//   the C layout puts one query per lane, so the online-softmax max/sum are
//   in-lane reductions plus one cross-half swap. P^T (bf16) is then used
//   directly as the B operand of O^T += V^T P^T, with V staged transposed in
//   LDS and the k index permuted to match the C layout (no LDS round trip for
//   P). Softmax runs in base 2 with the scale folded into one multiply.
//   LSE (natural log) is saved for the backward.
//
// Backward: Delta = rowsum(O * dO); a dK/dV kernel per (b, kv-head, 128 keys)
// that loops over the group's q-heads and all visible q-tiles (no atomics);
// and a separate dQ kernel per (b, q-head, 128 queries) that loops over key
// tiles. Both recompute P from the saved LSE. Results are bitwise
// reproducible.
//
// Decode (Sq == 1): split-KV over the cache, one wavefront per (split, b,
// kv-head) streaming K/V tiles through LDS on the matrix cores (the pass is
// HBM-bound on K/V), partial (m, l, o) per split in the workspace, then a
// fixed-order combine.
#include <mutex>

#include "qh_lds.h"
#include "qh_mfma.h"
#include "qh_prep.h"

// fp32 inputs (qh_attention_f32.hip): same arguments, after the shape checks.
int qh_flash_fwd_f32(const float* q, int64_t sqb, int64_t sqh, int64_t sqs, const float* k, int64_t skb, int64_t skh,
                     int64_t sks, const float* v, int64_t svb, int64_t svh, int64_t svs, float* o, int64_t sob,
                     int64_t soh, int64_t sos, float* lse, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk,
                     int64_t D, float scale, int causal, int64_t coff, hipStream_t st);
int qh_flash_bwd_f32(const float* q, int64_t sqb, int64_t sqh, int64_t sqs, const float* k, int64_t skb, int64_t skh,
                     int64_t sks, const float* v, int64_t svb, int64_t svh, int64_t svs, const float* o,
                     const float* dout, const float* lse, float* dq, float* dk, float* dv, float* delta, float* lse2,
                     int64_t sqp, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D, float scale,
                     int causal, int64_t coff, hipStream_t st);

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float exp2_(float x) { return __builtin_amdgcn_exp2f(x); }

// Combine lane l with lane l ^ 32 in registers: v_permlane32_swap exchanges the
// upper half of its first operand with the lower half of its second, so with x
// in both the two results hold x[l] and x[l ^ 32] (in low-half, high-half
// order on every lane, so sums round identically on both halves).
__device__ __forceinline__ float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Block order of the (blocks x rows) attention grids: the grid is walked as
// one sequence in dispatch order (x fastest) and position L runs block rank
// L / rows of row L % rows. Every row's rank-0 block is dispatched before any
// row's rank-1 block, so with the heaviest blocks at rank 0 (the most visible
// keys or queries under a causal mask) the long blocks start first and the
// short ones fill the tail. A row keeps L mod 8, i.e. one XCD and its L2,
// when rows is a multiple of 8.
__device__ __forceinline__ void block_rank_row(int& rank, int& row) {
  const int L = (int)(blockIdx.y * gridDim.x + blockIdx.x);
  rank = L / (int)gridDim.y;
  row = L - rank * (int)gridDim.y;
}

// A pointer computed from kernel arguments and block indices only, stated
// wave-uniform so that address arithmetic on it stays in scalar registers.
template <typename P>
__device__ __forceinline__ P* uniform_ptr(P* p) {
  const uint64_t b = (uint64_t)(uintptr_t)p;
  const uint64_t u = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b) |
                     ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32);
  return (P*)(uintptr_t)u;
}

template <typename T>
__device__ __forceinline__ typename Mfma<T>::v8 load_frag16(const T* p) {
  return *reinterpret_cast<const typename Mfma<T>::v8*>(p);
}

// Two 8-byte LDS reads forming one 8-element fragment (permuted-k operand).
template <typename T>
__device__ __forceinline__ typename Mfma<T>::v8 load_frag_split(const T* p0, const T* p1) {
  typedef typename Mfma<T>::v4 v4;
  typedef typename Mfma<T>::v8 v8;
  const v4 a = *reinterpret_cast<const v4*>(p0);
  const v4 b = *reinterpret_cast<const v4*>(p1);
  v8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

// Pack accumulator groups g0 and g0+1 (8 values) of a C-layout tile as bf16/f16.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::v8 pack_pair(const f32x16& c, int g0) {
  typename Mfma<T>::v8 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    r[e] = (T)c[g0 * 4 + e];
    r[4 + e] = (T)c[(g0 + 1) * 4 + e];
  }
  return r;
}

// Stage ROWS rows x DP columns (row-major, rows along seq) into LDS with row
// stride LD; rows >= nrows or columns >= D are zero.
template <typename T, int ROWS, int DP, int LD>
__device__ __forceinline__ void stage_rows(T* __restrict__ S, const T* __restrict__ G, int64_t gstride, int row0,
                                           int nrows, int D) {
  constexpr int CPR = DP / 8;  // 16-byte chunks per row
  const uint4 z = make_uint4(0, 0, 0, 0);
  for (int c = threadIdx.x; c < ROWS * CPR; c += 256) {
    const int r = c / CPR, d0 = (c % CPR) * 8;
    const int gr = row0 + r;
    uint4 v = z;
    if (gr < nrows && d0 < D) v = *reinterpret_cast<const uint4*>(G + (int64_t)gr * gstride + d0);
    *reinterpret_cast<uint4*>(S + r * LD + d0) = v;
  }
}

// Stage the transpose: S[d][r] = G[row0 + r][d] for ROWS rows, DP columns;
// LDS row stride LD (>= ROWS). Zero outside the valid range.
template <typename T, int ROWS, int DP, int LD>
__device__ __forceinline__ void stage_rows_t(T* __restrict__ S, const T* __restrict__ G, int64_t gstride, int row0,
                                             int nrows, int D) {
  constexpr int RB = ROWS / 8, DB = DP / 8;
  const uint4 z = make_uint4(0, 0, 0, 0);
  for (int sb = threadIdx.x; sb < RB * DB; sb += 256) {
    const int rb = sb % RB, db = sb / RB;
    const int d0 = db * 8;
    uint4 in[8], out[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int gr = row0 + rb * 8 + j;
      if (gr < nrows && d0 < D) in[j] = *reinterpret_cast<const uint4*>(G + (int64_t)gr * gstride + d0);
      else in[j] = z;
    }
    transpose8x8(in, out);
#pragma unroll
    for (int c = 0; c < 8; ++c) *reinterpret_cast<uint4*>(S + (d0 + c) * LD + rb * 8) = out[c];
  }
}

// ===========================================================================
// Forward
// ===========================================================================
// LDS tiles of K and V are stored in their natural [key][d] layout with DP*2
// byte rows and no padding; the 16-byte chunks of row r are XOR-swizzled
// (swz() below) so that both fragment reads below
// spread over all 32 banks. Tiles are written straight from global memory by
// global_load_lds (16 bytes per lane, lane l -> base + 16*l), so staging needs
// neither registers nor VALU work and overlaps the previous tile's math.
//
//  * K is the A operand of S^T = K Q^T: one 16-byte read per fragment.
//  * V^T is the A operand of O^T += V^T P^T: gfx950's ds_read_b64_tr_b16
//    returns, in each 16-lane group, element (i % 4) of the 8-byte words
//    addressed by lanes i/4 + 4e (e = 0..3); lanes that address 4 consecutive
//    keys x 4 d-quads therefore receive 4 consecutive keys of one d each.


// Physical 16-byte chunk of logical chunk `chunk` in tile row `row` (cpr
// chunks per row). With 256-byte rows (DP = 128) every row starts on the same
// LDS banks, so the XOR pattern must (a) give 16 consecutive rows 16 distinct
// chunk positions for one logical chunk (the 16-byte fragment reads) and
// (b) place 4 consecutive rows x 4 adjacent chunks in 16 distinct positions
// (the 8-byte transpose reads): XOR with the row's low 4 bits rotated by two.
// Narrower rows XOR with (row mod cpr).
__device__ __forceinline__ int swz(int row, int chunk, int cpr) {
  if (cpr >= 16) return chunk ^ (((row & 3) << 2) | ((row >> 2) & 3));
  return chunk ^ (row & (cpr - 1));
}

// One V^T A-operand fragment: two transpose reads at keys key and key + 8 of
// column d, joined as whole vectors (element-wise short -> bf16 inserts are
// lowered incorrectly by the current compiler: they broadcast element 0).
template <typename T, int DP>
__device__ __forceinline__ typename Mfma<T>::v8 read_vt_frag(const T* Vt, int key, int d) {
  constexpr int CPR = DP / 8;
  const T* s0 = Vt + key * DP + swz(key, d >> 3, CPR) * 8 + (d & 7);
  const T* s1 = Vt + (key + 8) * DP + swz(key + 8, d >> 3, CPR) * 8 + (d & 7);
  const qh_v4i16 w0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) qh_v4i16*)(s0));
  const qh_v4i16 w1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) qh_v4i16*)(s1));
  const qh_v8i16 w = __builtin_shufflevector(w0, w1, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(typename Mfma<T>::v8, w);
}

// Loader of ROWS x DP tiles (rows along seq, DP columns) into the swizzled
// LDS layout. Each of the 4 waves issues ROWS / RPI / 4 instructions of 1 KiB
// (RPI rows each). A lane's byte offset inside its rows is the same for every
// instruction and every tile, so full tiles cost no per-lane address math;
// a tile that runs past nrows clamps its rows (and d-chunks past D) onto valid
// memory, whose finite contents are masked or multiplied by zero downstream.
template <typename T, int ROWS, int DP>
struct TileLoader {
  static constexpr int CPR = DP / 8;     // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;   // rows per wave instruction
  static constexpr int NI = ROWS / RPI;  // instructions per tile
  static_assert(NI % 4 == 0, "tile must split evenly over 4 waves");
  int wid, rl, d0;
  uint32_t voff;
  __device__ __forceinline__ TileLoader(int64_t gstride, int D) {
    const int lane = threadIdx.x & 63;
    wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    rl = lane / CPR;
    // the row's swizzle depends only on (n * RPI + rl) % min(CPR, 16), which is
    // the same for every instruction n of this wave (n = 4 i + wid, and 4 RPI
    // is a multiple of 16)
    const int c = swz(wid * RPI + rl, lane % CPR, CPR);
    d0 = c * 8 < D ? c * 8 : D - 8;
    voff = (uint32_t)(((int64_t)rl * gstride + d0) * (int64_t)sizeof(T));
  }
  __device__ __forceinline__ void load(T* lds_tile, const T* __restrict__ G, int64_t gstride, int row0,
                                       int nrows) const {
    const uint32_t base = lds_addr(lds_tile);
    if (row0 + ROWS <= nrows) {
#pragma unroll
      for (int i = 0; i < NI / 4; ++i) {
        const int n = i * 4 + wid;
        lds_dma16_s(voff, G + (int64_t)(row0 + n * RPI) * gstride, base + (uint32_t)(n * RPI * DP * sizeof(T)));
      }
    } else {
#pragma unroll
      for (int i = 0; i < NI / 4; ++i) {
        const int n = i * 4 + wid;
        int gr = row0 + n * RPI + rl;
        gr = gr < nrows ? gr : nrows - 1;
        lds_dma16(G + (int64_t)gr * gstride + d0, base + (uint32_t)(n * RPI * DP * sizeof(T)));
      }
    }
  }
};

// MASKED adds a lower key bound `lo` per query (a sliding window) and a
// per-key validity word `bits` for the tile (bit j: key kv0 + j may be seen).
template <typename T, int DP, bool MASKED = false>
__device__ __forceinline__ void fa_fwd_tile(const T* Kt, const T* Vt, const typename Mfma<T>::v8 (&qf)[DP / 16],
                                            f32x16 (&acc)[DP / 32], float& m, float& l, int kv0, bool need_mask,
                                            int lim, float scale_log2, int lane, int lo = 0, uint64_t bits = 0) {
  constexpr int CPR = DP / 8, DT = DP / 32, KD = DP / 16;
  typedef typename Mfma<T>::v8 v8;
  const int ql = lane & 31, hf = lane >> 5;
  f32x16 s[2];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    s[kt] = zero16();
    const int row = kt * 32 + ql;
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
      const int c = swz(row, kd * 2 + hf, CPR);
      s[kt] = Mfma<T>::mma(load_frag16<T>(Kt + row * DP + c * 8), qf[kd], s[kt]);
    }
  }
  // Issue order of the 2 KD fragment reads (R) and MFMAs (M): KD reads, then
  // (M R) x KD, then the last KD MFMAs, so that KD reads are in flight when
  // the first product needs its operand (LDS latency is several MFMAs long).
  __builtin_amdgcn_sched_group_barrier(0x100, KD, 0);
#pragma unroll
  for (int i = 0; i < KD; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, KD, 0);
  if (need_mask) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = kv0 + kt * 32 + g * 8 + hf * 4 + r;
          bool off = key > lim;
          if constexpr (MASKED) off = off || key < lo || !((bits >> (key - kv0)) & 1);
          s[kt][g * 4 + r] = off ? -INFINITY : s[kt][g * 4 + r];
        }
  }
  float mx = fmaxf(s[0][0], s[1][0]);
#pragma unroll
  for (int e = 1; e < 16; ++e) mx = fmaxf(mx, fmaxf(s[0][e], s[1][e]));
  mx = halves_max(mx);
  // Rescale only when some lane's running max grew by more than 2^8 in
  // probability terms: until then P = exp2((s - m) scale_log2) <= 256 stays
  // well inside bf16/fp32 range, and O / l and the LSE use the same m, so the
  // result is unchanged while most tiles skip the 64 multiplies.
  if (__any((mx - m) * scale_log2 > 8.f)) {
    const float mnew = fmaxf(m, mx);
    const float alpha = (m == -INFINITY) ? 0.f : exp2_((m - mnew) * scale_log2);
    l *= alpha;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[dt][e] *= alpha;
    m = mnew;
  }
  const float mb = (m == -INFINITY) ? 0.f : m * scale_log2;
  float ps = 0.f;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float p = exp2_(__builtin_fmaf(s[kt][e], scale_log2, -mb));
      s[kt][e] = p;
      ps += p;
    }
  l += ps;  // this half's keys only: the halves' sums are joined once, after the last tile
  // V^T fragments through the LDS transpose read (see the note above).
  const int grp = lane >> 4, j = lane & 15;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const v8 pf = pack_pair<T>(s[ks >> 1], (ks & 1) * 2);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int d = dt * 32 + 16 * (grp & 1) + 4 * (j & 3);
      const v8 a = read_vt_frag<T, DP>(Vt, ks * 16 + 4 * (grp >> 1) + (j >> 2), d);
      acc[dt] = Mfma<T>::mma(a, pf, acc[dt]);
    }
  }
}

// MASKED: key j is also hidden from query i when j <= i + coff - window
// (window > 0) or bit j of the batch row's validity words is clear
// (kbits non-null; word t covers keys 64t .. 64t + 63).
// PACK (Sq == 1, grid (1, B * Hkv)): the block's rows are the `groups` q-heads
// of one kv-head, all at query position 0, so the kv-head's keys are read once
// for all of them.
template <typename T, int DP, bool MASKED = false, bool PACK = false>
__global__ __launch_bounds__(256) void fa_fwd_kernel(const T* __restrict__ Q, int64_t sqb, int64_t sqh, int64_t sqs,
                                                     const T* __restrict__ K, int64_t skb, int64_t skh, int64_t sks,
                                                     const T* __restrict__ V, int64_t svb, int64_t svh, int64_t svs,
                                                     T* __restrict__ O, int64_t sob, int64_t soh, int64_t sos,
                                                     float* __restrict__ LSE, int Hq, int groups, int Sq, int Sk, int D,
                                                     float scale_log2, int causal, int coff,
                                                     const uint64_t* __restrict__ kbits = nullptr, int64_t kbits_b = 0,
                                                     int window = 0) {
  constexpr int BN = 64, BMQ = 128;
  constexpr int DT = DP / 32, KD = DP / 16;
  typedef typename Mfma<T>::v8 v8;
  __shared__ __attribute__((aligned(1024))) T Ks[2][BN * DP];
  __shared__ __attribute__((aligned(1024))) T Vs[2][BN * DP];

  const int nqb = (Sq + BMQ - 1) / BMQ;
  int rank, bh;
  block_rank_row(rank, bh);
  const int qb = nqb - 1 - rank;  // last query blocks see the most keys
  const int hkv = Hq / groups;
  const int b = PACK ? bh / hkv : bh / Hq;
  const int hk = PACK ? bh % hkv : (bh % Hq) / groups;
  const int hq = PACK ? hk * groups : bh % Hq;  // PACK: the group's first q-head
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: keeps tile branches scalar
  const int ql = lane & 31, hf = lane >> 5;
  const T* Qb = Q + b * sqb + hq * sqh;
  const T* Kb = uniform_ptr(K + b * skb + hk * skh);
  const T* Vb = uniform_ptr(V + b * svb + hk * svh);
  const int qw0 = PACK ? 0 : qb * BMQ + wid * 32;  // query position of the wave's first row
  const int qi = PACK ? 0 : qw0 + ql;              // this lane's query position
  const int prow = wid * 32 + ql;                   // PACK: this lane's q-head within the group
  const bool qvalid = PACK ? prow < groups : qi < Sq;
  const int64_t qoff = PACK ? (int64_t)prow * sqh : (int64_t)qi * sqs;

  v8 qf[KD];
#pragma unroll
  for (int kd = 0; kd < KD; ++kd) {
    const int d0 = kd * 16 + hf * 8;
    if (qvalid && d0 < D) qf[kd] = load_frag16<T>(Qb + qoff + d0);
    else
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[kd][e] = (T)0.f;
  }
  float m = -INFINITY, l = 0.f;
  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = zero16();

  int kv_end = Sk;
  if (causal) kv_end = min(Sk, qb * BMQ + BMQ + coff);
  const int ntiles = kv_end > 0 ? (kv_end + BN - 1) / BN : 0;
  // last key visible to this lane's query (causal and/or Sk bound)
  const int lim = causal ? min(Sk - 1, qi + coff) : Sk - 1;

  // first tile: with a window, the block's first query sees no key below
  // qb * BMQ + coff - window + 1
  int it0 = 0, lo = 0;
  if constexpr (MASKED) {
    if (window > 0) {
      lo = qi + coff - window + 1;
      const int blo = qb * BMQ + coff - window + 1;
      it0 = blo > 0 ? blo / BN : 0;
    }
    // leading tiles with no visible key (left padding) are not even loaded
    if (kbits)
      while (it0 < ntiles && kbits[b * kbits_b + it0] == 0) ++it0;
  }

  const TileLoader<T, BN, DP> kload(sks, D), vload(svs, D);
  if (ntiles > it0) {
    kload.load(Ks[it0 & 1], Kb, sks, it0 * BN, Sk);
    vload.load(Vs[it0 & 1], Vb, svs, it0 * BN, Sk);
  }
  for (int it = it0; it < ntiles; ++it) {
    const int kv0 = it * BN;
    const int buf = it & 1;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's loads of tile `it` have landed
    __syncthreads();                // ... and everyone else's; tile it-1 is fully consumed
    if (it + 1 < ntiles) {
      kload.load(Ks[buf ^ 1], Kb, sks, kv0 + BN, Sk);
      vload.load(Vs[buf ^ 1], Vb, svs, kv0 + BN, Sk);
    }
    // wave-uniform: does any key of this tile lie past a query's limit?
    // (one code path for both: two inlined copies of the tile would hold the
    // accumulators in different registers on each side)
    const bool need_mask = (kv0 + BN > Sk) || (causal && kv0 + BN - 1 > qw0 + coff);
    if constexpr (MASKED) {
      const uint64_t w = kbits ? kbits[b * kbits_b + it] : ~0ull;  // block-uniform
      if (w == 0) continue;  // no visible key in the tile
      const bool cut = window > 0 && kv0 < qw0 + 31 + coff - window + 1;
      fa_fwd_tile<T, DP, true>(Ks[buf], Vs[buf], qf, acc, m, l, kv0, need_mask || cut || w != ~0ull, lim,
                               scale_log2, lane, lo, w);
    } else {
      fa_fwd_tile<T, DP>(Ks[buf], Vs[buf], qf, acc, m, l, kv0, need_mask, lim, scale_log2, lane);
    }
  }

  l = halves_sum(l);
  if (qvalid) {
    T* Ob = O + b * sob + hq * soh + (PACK ? (int64_t)prow * soh : (int64_t)qi * sos);
    const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = dt * 32 + g * 8 + hf * 4;
        if (d < D) {
          typename Mfma<T>::v4 o4;
#pragma unroll
          for (int r = 0; r < 4; ++r) o4[r] = (T)(acc[dt][g * 4 + r] * inv);
          *reinterpret_cast<typename Mfma<T>::v4*>(Ob + d) = o4;
        }
      }
    if (hf == 0 && LSE) {
      const int64_t li = PACK ? (int64_t)b * Hq + hq + prow : (int64_t)bh * Sq + qi;
      LSE[li] = l > 0.f ? (m * scale_log2 + __log2f(l)) * kLn2 : -INFINITY;
    }
  }
}

// ===========================================================================
// Backward
// ===========================================================================
// Per query row: Delta = rowsum(O * dO) and the saved LSE in log2 units, in
// rows of sqp >= Sq + 64 floats per (b, q-head) whose tail is zero, so that
// the backward kernels read whole 64-query tiles (as float4) without bounds
// checks. 16 lanes per row, 8 elements per lane per step.
template <typename T>
__global__ __launch_bounds__(256) void fa_bwd_prep_kernel(const T* __restrict__ O, const T* __restrict__ dO,
                                                          const float* __restrict__ LSE, float* __restrict__ delta,
                                                          float* __restrict__ lse2, int64_t padded_rows, int Sq,
                                                          int64_t sqp, int D) {
  const int64_t prow = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int li = threadIdx.x & 15;
  const int64_t bh = prow / sqp;
  const int q = (int)(prow - bh * sqp);
  const bool real = prow < padded_rows && q < Sq;
  const int64_t row = bh * Sq + q;
  float s = 0.f;
  if (real) {
    for (int d = li * 8; d < D; d += 128) {
      Vec16<T> a = ld16(O + row * D + d), b = ld16(dO + row * D + d);
#pragma unroll
      for (int e = 0; e < 8; ++e) s += to_f32(a.v[e]) * to_f32(b.v[e]);
    }
  }
  s = wave_sum(s, 16);
  if (prow < padded_rows && li == 0) {
    delta[prow] = s;
    lse2[prow] = real ? LSE[row] * kLog2e : 0.f;
  }
}

// dK, dV for 128 keys (4 wavefronts x 32 keys) of one (b, kv-head). The
// wave's K and V fragments stay in registers (B operands); Q and dO tiles of
// 64 queries stream through double-buffered swizzled LDS (direct-to-LDS
// loads), over every q-head of the group and every visible q-tile. Per 32
// queries:
//   S = Q K^T, dP = dO V^T           (C layout: column = key, rows = queries)
//   P = exp2(S scale_log2 - lse2), dS = P (dP - Delta)
//   dV^T += dO^T P, dK^T += Q^T dS   (A operands read transposed from the
//                                     row-major Q / dO tiles; P and dS are the
//                                     B operands straight from the C layout)
template <typename T, int DP, bool MASK>
__device__ __forceinline__ void fa_bwd_dkdv_tile(const T* Qt, const T* Ot, const typename Mfma<T>::v8 (&kf)[DP / 16],
                                                 const typename Mfma<T>::v8 (&vf)[DP / 16], f32x16 (&dk)[DP / 32],
                                                 f32x16 (&dv)[DP / 32], const float* __restrict__ lse_row,
                                                 const float* __restrict__ dl_row, int q0, int kj, int Sq, int Sk,
                                                 int causal, int coff, float scale_log2, int lane) {
  constexpr int CPR = DP / 8, DT = DP / 32, KD = DP / 16;
  typedef typename Mfma<T>::v8 v8;
  const int ql = lane & 31, hf = lane >> 5;
  const int grp = lane >> 4, j = lane & 15;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    // lse (log2 units) and Delta of this lane's 16 queries q0 + qt*32 + 8 g + 4 hf + r
    float4 ls[4], dl[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int il = qt * 32 + g * 8 + hf * 4;
      ls[g] = *reinterpret_cast<const float4*>(lse_row + il);
      dl[g] = *reinterpret_cast<const float4*>(dl_row + il);
    }
    f32x16 sc = zero16(), dp = zero16();
    const int row = qt * 32 + ql;
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
      const int c = swz(row, kd * 2 + hf, CPR);
      sc = Mfma<T>::mma(load_frag16<T>(Qt + row * DP + c * 8), kf[kd], sc);
      dp = Mfma<T>::mma(load_frag16<T>(Ot + row * DP + c * 8), vf[kd], dp);
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float lv[4] = {ls[g].x, ls[g].y, ls[g].z, ls[g].w};
      const float dv4[4] = {dl[g].x, dl[g].y, dl[g].z, dl[g].w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float p = exp2_(__builtin_fmaf(sc[g * 4 + r], scale_log2, -lv[r]));
        if constexpr (MASK) {
          const int qi = q0 + qt * 32 + g * 8 + hf * 4 + r;
          const bool ok = qi < Sq && kj < Sk && !(causal && kj > qi + coff);
          p = ok ? p : 0.f;
        }
        sc[g * 4 + r] = p;
        dp[g * 4 + r] = p * (dp[g * 4 + r] - dv4[r]);
      }
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const v8 pf = pack_pair<T>(sc, ks * 2);
      const v8 df = pack_pair<T>(dp, ks * 2);
      const int qrow = qt * 32 + ks * 16 + 4 * (grp >> 1) + (j >> 2);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d = dt * 32 + 16 * (grp & 1) + 4 * (j & 3);
        dv[dt] = Mfma<T>::mma(read_vt_frag<T, DP>(Ot, qrow, d), pf, dv[dt]);
        dk[dt] = Mfma<T>::mma(read_vt_frag<T, DP>(Qt, qrow, d), df, dk[dt]);
      }
    }
  }
}

template <typename T, int DP>
__global__ __launch_bounds__(256) void fa_bwd_dkdv_kernel(
    const T* __restrict__ Q, int64_t sqb, int64_t sqh, int64_t sqs, const T* __restrict__ K, int64_t skb, int64_t skh,
    int64_t sks, const T* __restrict__ V, int64_t svb, int64_t svh, int64_t svs, const T* __restrict__ dO,
    const float* __restrict__ LSE2, const float* __restrict__ Delta, int64_t sqp, T* __restrict__ dK,
    T* __restrict__ dV, int Hq, int Hkv, int groups, int Sq, int Sk, int D, float scale_log2, float scale, int causal,
    int coff) {
  constexpr int BQ = 64;
  constexpr int DT = DP / 32, KD = DP / 16;
  typedef typename Mfma<T>::v8 v8;
  __shared__ __attribute__((aligned(1024))) T Qs[2][BQ * DP];
  __shared__ __attribute__((aligned(1024))) T Os[2][BQ * DP];

  int rank, bk;
  block_rank_row(rank, bk);  // first key blocks see the most queries
  const int b = bk / Hkv, hk = bk % Hkv;
  const int k0 = rank * 128;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int ql = lane & 31, hf = lane >> 5;
  const int kj = k0 + wid * 32 + ql;  // this lane's key (C-layout column)
  const int kw0 = k0 + wid * 32;      // first key of this wave
  const T* Kb = K + b * skb + hk * skh;
  const T* Vb = V + b * svb + hk * svh;

  v8 kf[KD], vf[KD];
#pragma unroll
  for (int kd = 0; kd < KD; ++kd) {
    const int d0 = kd * 16 + hf * 8;
    if (kj < Sk && d0 < D) {
      kf[kd] = load_frag16<T>(Kb + (int64_t)kj * sks + d0);
      vf[kd] = load_frag16<T>(Vb + (int64_t)kj * svs + d0);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) kf[kd][e] = vf[kd][e] = (T)0.f;
    }
  }
  f32x16 dk[DT], dv[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dk[dt] = dv[dt] = zero16();

  // visible q-tiles: queries q with q + coff >= k0 (causal), all otherwise
  int q_start = 0;
  if (causal) {
    q_start = k0 - coff;
    if (q_start < 0) q_start = 0;
    q_start = (q_start / BQ) * BQ;
  }
  const int nqt = q_start < Sq ? (Sq - q_start + BQ - 1) / BQ : 0;
  const int ntiles = groups * nqt;
  const TileLoader<T, BQ, DP> qload(sqs, D), oload(D, D);
  auto issue = [&](int it, int buf) {
    const int g = it / nqt, q0 = q_start + (it % nqt) * BQ;
    const int hq = hk * groups + g;
    qload.load(Qs[buf], Q + b * sqb + hq * sqh, sqs, q0, Sq);
    oload.load(Os[buf], dO + ((int64_t)b * Hq + hq) * Sq * D, D, q0, Sq);
  };
  if (ntiles > 0) issue(0, 0);
  for (int it = 0; it < ntiles; ++it) {
    const int buf = it & 1;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's loads of tile `it` have landed
    __syncthreads();                // ... and everyone else's; tile it-1 is fully consumed
    if (it + 1 < ntiles) issue(it + 1, buf ^ 1);
    const int g = it / nqt, q0 = q_start + (it % nqt) * BQ;
    const int64_t bh = (int64_t)b * Hq + hk * groups + g;
    // wave-uniform: does any (query, key) pair of the tile need masking?
    const bool need_mask = (q0 + BQ > Sq) || (kw0 + 32 > Sk) || (causal && kw0 + 31 > q0 + coff);
    const float* lse_row = LSE2 + bh * sqp + q0;
    const float* dl_row = Delta + bh * sqp + q0;
    if (need_mask)
      fa_bwd_dkdv_tile<T, DP, true>(Qs[buf], Os[buf], kf, vf, dk, dv, lse_row, dl_row, q0, kj, Sq, Sk, causal, coff,
                                    scale_log2, lane);
    else
      fa_bwd_dkdv_tile<T, DP, false>(Qs[buf], Os[buf], kf, vf, dk, dv, lse_row, dl_row, q0, kj, Sq, Sk, causal,
                                     coff, scale_log2, lane);
  }
  if (kj < Sk) {
    T* dKr = dK + ((int64_t)bk * Sk + kj) * D;
    T* dVr = dV + ((int64_t)bk * Sk + kj) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) {
        const int d = dt * 32 + gg * 8 + hf * 4;
        if (d < D) {
          typename Mfma<T>::v4 a, c;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            a[r] = (T)(dk[dt][gg * 4 + r] * scale);
            c[r] = (T)dv[dt][gg * 4 + r];
          }
          *reinterpret_cast<typename Mfma<T>::v4*>(dKr + d) = a;
          *reinterpret_cast<typename Mfma<T>::v4*>(dVr + d) = c;
        }
      }
  }
}

// LDS layout of the 8-wave dK/dV kernel (bytes): K and V of the block, two
// stages of Q and of dO, two stages of the tile's lse2 | Delta rows. A stage
// is selected by one address bit (each region is aligned to twice its stage
// size), so the per-lane fragment offsets switch stage with one XOR per tile.
template <int DP>
struct DkdvLds {
  static constexpr int BQ = 64, KB = 128;
  static constexpr uint32_t K = 0, V = KB * DP * 2, Q = 2 * V, QSTAGE = BQ * DP * 2, O = Q + 2 * QSTAGE,
                            L = O + 2 * QSTAGE, LSTAGE = 2 * BQ * 4, DELTA = BQ * 4, BYTES = L + 2 * LSTAGE;
  static_assert((QSTAGE & (QSTAGE - 1)) == 0 && Q % (2 * QSTAGE) == 0 && O % (2 * QSTAGE) == 0,
                "Q/dO stages must differ in one address bit");
  static_assert((LSTAGE & (LSTAGE - 1)) == 0 && L % (2 * LSTAGE) == 0, "lse stages must differ in one address bit");
  static_assert(O - Q < 65536 && V - K < 65536, "partner operands must be an immediate offset apart");
};

// Per-lane LDS addresses of one wavefront's fragment reads (loop-invariant
// apart from the stage bit; the dynamic LDS block's own address included, so
// that every read is a register plus an immediate): K fragments of each k16 step (V = +V-K), Q rows of
// each k16 step in the current stage (dO = +O-Q), the transposed Q/dO reads of
// each 32-column block at query rows r and r + 8 (the second 16-query step is
// +16 rows), and the lane's first lse value.
template <int DP>
struct DkdvOffsets {
  static constexpr int KD = DP / 16, DT = DP / 32;
  uint32_t kv[KD], qo[KD], tr[DT][2], ls;
};

template <int DP>
__device__ __forceinline__ DkdvOffsets<DP> dkdv_offsets(const unsigned char* lds, int ks, int qt, int lane) {
  typedef DkdvLds<DP> L;
  constexpr int CPR = DP / 8;
  const uint32_t base = lds_addr(lds);
  const int ql = lane & 31, hf = lane >> 5, grp = lane >> 4, j = lane & 15;
  const int row = qt * 32 + ql, key = ks * 32 + ql;
  DkdvOffsets<DP> o;
#pragma unroll
  for (int kd = 0; kd < DkdvOffsets<DP>::KD; ++kd) {
    o.kv[kd] = base + L::K + (key * CPR + swz(key, kd * 2 + hf, CPR)) * 16;
    o.qo[kd] = base + L::Q + (row * CPR + swz(row, kd * 2 + hf, CPR)) * 16;
  }
  const int qrow = qt * 32 + 4 * (grp >> 1) + (j >> 2);
#pragma unroll
  for (int dt = 0; dt < DkdvOffsets<DP>::DT; ++dt) {
    const int d = dt * 32 + 16 * (grp & 1) + 4 * (j & 3);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = qrow + 8 * h;
      o.tr[dt][h] = base + L::Q + (r * CPR + swz(r, d >> 3, CPR)) * 16 + (d & 7) * 2;
    }
  }
  o.ls = base + L::L + (qt * 32 + hf * 4) * 4;
  return o;
}

template <int DP>
__device__ __forceinline__ void dkdv_next_stage(DkdvOffsets<DP>& o) {
  typedef DkdvLds<DP> L;
#pragma unroll
  for (int kd = 0; kd < DkdvOffsets<DP>::KD; ++kd) o.qo[kd] ^= L::QSTAGE;
#pragma unroll
  for (int dt = 0; dt < DkdvOffsets<DP>::DT; ++dt) o.tr[dt][0] ^= L::QSTAGE, o.tr[dt][1] ^= L::QSTAGE;
  o.ls ^= L::LSTAGE;
}

typedef const __attribute__((address_space(3))) unsigned char lds_u8;
typedef float lds_f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ lds_u8* lds_at(uint32_t a) { return (lds_u8*)(uintptr_t)a; }

template <typename T>
__device__ __forceinline__ typename Mfma<T>::v8 lds_frag16(uint32_t a, uint32_t imm = 0) {
  return *reinterpret_cast<const __attribute__((address_space(3))) typename Mfma<T>::v8*>(lds_at(a) + imm);
}

// One transposed A-operand fragment from two 8-byte transpose reads (rows r and
// r + 8 of a 4-row x 4-column block per 16 lanes), joined as whole vectors.
template <typename T>
__device__ __forceinline__ typename Mfma<T>::v8 lds_tr_frag(uint32_t a0, uint32_t a1, uint32_t imm) {
  typedef __attribute__((address_space(3))) qh_v4i16 lv4;
  const qh_v4i16 w0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lv4*)(lds_at(a0) + imm));
  const qh_v4i16 w1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lv4*)(lds_at(a1) + imm));
  const qh_v8i16 w = __builtin_shufflevector(w0, w1, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(typename Mfma<T>::v8, w);
}

// dK/dV for 128 keys of one (b, kv-head) with 8 wavefronts, two per SIMD:
// wavefront w owns keys k0 + 32 (w & 3) .. + 31 and, of every 64-query tile,
// the 32 queries of half w >> 2. K and V of the workgroup's keys are staged in
// LDS once and their fragments are read per use (holding them in registers
// would not fit two waves per SIMD); Q and dO tiles stream through two LDS
// stages, all loaded by wavefronts 0-3, together with the tile's 64 lse and
// Delta values (a global load inside the loop would make the compiler's
// vmcnt wait also cover the next tile's untracked LDS fill). At the end the two
// query halves' dK/dV partials are added in a fixed order (half 0 + half 1)
// through LDS. Same per-tile arithmetic as fa_bwd_dkdv_tile. Every fragment
// read is a per-lane offset (DkdvOffsets) plus an immediate.
template <typename T, int DP>
__device__ __forceinline__ void fa_bwd_dkdv_half(const DkdvOffsets<DP>& o,
                                                 f32x16 (&dk)[DP / 32], f32x16 (&dv)[DP / 32], int q0, int qt,
                                                 bool need_mask, int q_lo, int q_hi, float scale_log2, int lane) {
  typedef DkdvLds<DP> L;
  constexpr int DT = DP / 32, KD = DP / 16;
  typedef typename Mfma<T>::v8 v8;
  const int hf = lane >> 5;
  // S and dP: each k16 step's four fragments are read one step ahead; the
  // scheduling barriers keep the reads from being hoisted further (registers
  // for two wavefronts per SIMD), the other wavefront covers the latency.
  f32x16 sc = zero16(), dp = zero16();
  v8 fq[2], fk[2], fo[2], fv[2];
  auto rd_s = [&](int kd, int b) {
    fq[b] = lds_frag16<T>(o.qo[kd]);
    fk[b] = lds_frag16<T>(o.kv[kd]);
    fo[b] = lds_frag16<T>(o.qo[kd], L::O - L::Q);
    fv[b] = lds_frag16<T>(o.kv[kd], L::V - L::K);
  };
  rd_s(0, 0);
#pragma unroll
  for (int kd = 0; kd < KD; ++kd) {
    if (kd + 1 < KD) rd_s(kd + 1, (kd + 1) & 1);
    sc = Mfma<T>::mma(fq[kd & 1], fk[kd & 1], sc);
    dp = Mfma<T>::mma(fo[kd & 1], fv[kd & 1], dp);
    __builtin_amdgcn_sched_barrier(0);
  }
  // lse (log2 units) and Delta of this lane's 16 queries, from the tile's LDS
  // copy (read here: holding them across the products would cost 32 registers)
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const lds_f32x4 lv = *reinterpret_cast<const __attribute__((address_space(3))) lds_f32x4*>(lds_at(o.ls) + g * 32);
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[g * 4 + r] = exp2_(__builtin_fmaf(sc[g * 4 + r], scale_log2, -lv[r]));
  }
  // masked scores (diagonal and tail tiles only: the flag is wave-uniform, so
  // the other tiles branch past the compares and selects)
  if (__builtin_amdgcn_readfirstlane((int)need_mask)) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int qi = q0 + qt * 32 + (e >> 2) * 8 + hf * 4 + (e & 3);
      sc[e] = (qi >= q_lo && qi < q_hi) ? sc[e] : 0.f;
    }
  }
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const lds_f32x4 dv4 =
        *reinterpret_cast<const __attribute__((address_space(3))) lds_f32x4*>(lds_at(o.ls) + L::DELTA + g * 32);
#pragma unroll
    for (int r = 0; r < 4; ++r) dp[g * 4 + r] = sc[g * 4 + r] * (dp[g * 4 + r] - dv4[r]);
  }
  // dV += dO^T P, dK += Q^T dS with the transposed operands read one step ahead.
  const v8 pf[2] = {pack_pair<T>(sc, 0), pack_pair<T>(sc, 2)};
  const v8 df[2] = {pack_pair<T>(dp, 0), pack_pair<T>(dp, 2)};
  v8 ta[2], tb[2];
  auto rd_t = [&](int st, int b) {
    const int ks = st / DT, dt = st % DT;
    const uint32_t rs = ks * 16 * DP * 2;  // second 16-query step: 16 rows on
    ta[b] = lds_tr_frag<T>(o.tr[dt][0], o.tr[dt][1], rs + (L::O - L::Q));
    tb[b] = lds_tr_frag<T>(o.tr[dt][0], o.tr[dt][1], rs);
  };
  rd_t(0, 0);
#pragma unroll
  for (int st = 0; st < 2 * DT; ++st) {
    if (st + 1 < 2 * DT) rd_t(st + 1, (st + 1) & 1);
    const int ks = st / DT, dt = st % DT;
    dv[dt] = Mfma<T>::mma(ta[st & 1], pf[ks], dv[dt]);
    dk[dt] = Mfma<T>::mma(tb[st & 1], df[ks], dk[dt]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <typename T, int DP>
__global__ __launch_bounds__(512) void fa_bwd_dkdv8_kernel(
    const T* __restrict__ Q, int64_t sqb, int64_t sqh, int64_t sqs, const T* __restrict__ K, int64_t skb, int64_t skh,
    int64_t sks, const T* __restrict__ V, int64_t svb, int64_t svh, int64_t svs, const T* __restrict__ dO,
    const float* __restrict__ LSE2, const float* __restrict__ Delta, int64_t sqp, T* __restrict__ dK,
    T* __restrict__ dV, int Hq, int Hkv, int groups, int Sq, int Sk, int D, float scale_log2, float scale, int causal,
    int coff) {
  typedef DkdvLds<DP> L;
  constexpr int BQ = L::BQ, KB = L::KB;
  constexpr int DT = DP / 32;
  extern __shared__ __attribute__((aligned(1024))) unsigned char qh_dkdv_smem[];
  T* Ks = reinterpret_cast<T*>(qh_dkdv_smem + L::K);      // [KB][DP]
  T* Vs = reinterpret_cast<T*>(qh_dkdv_smem + L::V);      // [KB][DP]
  T* Qs = reinterpret_cast<T*>(qh_dkdv_smem + L::Q);      // [2][BQ][DP]
  T* Os = reinterpret_cast<T*>(qh_dkdv_smem + L::O);      // [2][BQ][DP]
  float* Ls = reinterpret_cast<float*>(qh_dkdv_smem + L::L);  // [2][lse2 BQ | Delta BQ]

  int rank, bk;
  block_rank_row(rank, bk);  // first key blocks see the most queries
  const int b = bk / Hkv, hk = bk % Hkv;
  const int k0 = rank * KB;
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ks = wid & 3, qt = wid >> 2;
  const int ql = lane & 31, hf = lane >> 5;
  const int kj = k0 + ks * 32 + ql;  // this lane's key (C-layout column)
  const int kw0 = k0 + ks * 32;      // first key of this wavefront
  // queries [q_lo, q_hi) see key kj: below Sq, at or after kj - coff when
  // causal, none when kj is past Sk
  const int q_lo = causal ? kj - coff : INT_MIN;
  const int q_hi = kj < Sk ? Sq : INT_MIN;
  const T* Kb = K + b * skb + hk * skh;
  const T* Vb = V + b * svb + hk * svh;

  f32x16 dk[DT], dv[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dk[dt] = dv[dt] = zero16();

  int q_start = 0;
  if (causal) {
    q_start = k0 - coff;
    if (q_start < 0) q_start = 0;
    q_start = (q_start / BQ) * BQ;
  }
  const int nqt = q_start < Sq ? (Sq - q_start + BQ - 1) / BQ : 0;
  const int ntiles = groups * nqt;
  const bool loader = wid < 4;  // wavefronts 0-3 issue every LDS fill
  if (loader) {
    // K and V of the workgroup's 128 keys (rows past Sk are clamped; their
    // scores are masked and their dK/dV rows are not stored)
    const TileLoader<T, KB, DP> kload(sks, D), vload(svs, D);
    kload.load(Ks, Kb, sks, k0, Sk);
    vload.load(Vs, Vb, svs, k0, Sk);
  }
  auto issue = [&](int it, int buf) {
    const TileLoader<T, BQ, DP> qload(sqs, D), oload(D, D);
    const int g = it / nqt, q0 = q_start + (it % nqt) * BQ;
    const int hq = hk * groups + g;
    qload.load(Qs + buf * BQ * DP, Q + b * sqb + hq * sqh, sqs, q0, Sq);
    oload.load(Os + buf * BQ * DP, dO + ((int64_t)b * Hq + hq) * Sq * D, D, q0, Sq);
    // rows are sqp >= q0 + BQ floats long, 16-byte aligned: lanes 0-15 copy
    // lse2[q0 .. q0 + 63], lanes 16-31 Delta[q0 .. q0 + 63]
    if (wid == 0 && lane < 32) {
      const int64_t bhq = (int64_t)b * Hq + hq;
      const float* src = (lane < 16 ? LSE2 : Delta) + bhq * sqp + q0 + 4 * (lane & 15);
      lds_dma16(src, lds_addr(Ls + buf * 2 * BQ));
    }
  };
  if (ntiles > 0 && loader) issue(0, 0);
  DkdvOffsets<DP> off = dkdv_offsets<DP>(qh_dkdv_smem, ks, qt, lane);
  for (int it = 0; it < ntiles; ++it) {
    const int buf = it & 1;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's loads of tile `it` (and of V) have landed
    __syncthreads();                // ... and everyone else's; tile it-1 is fully consumed
    if (it + 1 < ntiles && loader) issue(it + 1, buf ^ 1);
    const int q0 = q_start + (it % nqt) * BQ;
    const int qh0 = q0 + qt * 32;
    const bool need_mask = (qh0 + 32 > Sq) || (kw0 + 32 > Sk) || (causal && kw0 + 31 > qh0 + coff);
    // one code path for masked and unmasked tiles (the mask is a wave-uniform
    // branch inside): two inlined copies would keep the dK/dV accumulators in
    // different registers on each side
    fa_bwd_dkdv_half<T, DP>(off, dk, dv, q0, qt, need_mask, q_lo, q_hi, scale_log2, lane);
    dkdv_next_stage<DP>(off);
  }
  // half 1 hands its partials to half 0 through LDS (dV, then dK)
  float* red = reinterpret_cast<float*>(qh_dkdv_smem);
  const int slot = ks * DT * 16 * 64 + lane;
  auto combine = [&](f32x16(&a)[DT]) {
    __syncthreads();
    if (qt == 1) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) red[slot + (dt * 16 + e) * 64] = a[dt][e];
    }
    __syncthreads();
    if (qt == 0) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) a[dt][e] += red[slot + (dt * 16 + e) * 64];
    }
  };
  combine(dv);
  combine(dk);
  if (qt == 0 && kj < Sk) {
    T* dKr = dK + ((int64_t)bk * Sk + kj) * D;
    T* dVr = dV + ((int64_t)bk * Sk + kj) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) {
        const int d = dt * 32 + gg * 8 + hf * 4;
        if (d < D) {
          typename Mfma<T>::v4 a, c;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            a[r] = (T)(dk[dt][gg * 4 + r] * scale);
            c[r] = (T)dv[dt][gg * 4 + r];
          }
          *reinterpret_cast<typename Mfma<T>::v4*>(dKr + d) = a;
          *reinterpret_cast<typename Mfma<T>::v4*>(dVr + d) = c;
        }
      }
  }
}

// dQ for 128 queries (4 wavefronts x 32 queries) of one (b, q-head): the
// forward kernel's structure with dP computed beside S. K and V tiles of 64
// keys stream through double-buffered swizzled LDS; per tile
//   S^T = K Q^T, dP^T = V dO^T      (C layout: column = query, rows = keys)
//   dS^T = P^T (dP^T - Delta)
//   dQ^T += K^T dS^T                (K^T read transposed from the K tile)
// Per-lane LDS addresses of the dQ kernel's fragment reads in the current K/V
// stage: K rows of each k16 step (V = +KV_OFF, the second 32-key half = +32
// rows) and the transposed K reads of each 32-column block at key rows r and
// r + 8 (the other 16-key steps: +16 rows). The row swizzle depends on a row's
// low 4 bits only, so those steps are immediates.
template <int DP>
struct DqOffsets {
  static constexpr int KD = DP / 16, DT = DP / 32;
  uint32_t kf[KD], tr[DT][2];
};

template <int DP>
__device__ __forceinline__ DqOffsets<DP> dq_offsets(uint32_t kbase, int lane) {
  constexpr int CPR = DP / 8;
  const int ql = lane & 31, hf = lane >> 5, grp = lane >> 4, j = lane & 15;
  DqOffsets<DP> o;
#pragma unroll
  for (int kd = 0; kd < DqOffsets<DP>::KD; ++kd) o.kf[kd] = kbase + (ql * CPR + swz(ql, kd * 2 + hf, CPR)) * 16;
  const int krow = 4 * (grp >> 1) + (j >> 2);
#pragma unroll
  for (int dt = 0; dt < DqOffsets<DP>::DT; ++dt) {
    const int d = dt * 32 + 16 * (grp & 1) + 4 * (j & 3);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = krow + 8 * h;
      o.tr[dt][h] = kbase + (r * CPR + swz(r, d >> 3, CPR)) * 16 + (d & 7) * 2;
    }
  }
  return o;
}

template <int DP>
__device__ __forceinline__ void dq_shift(DqOffsets<DP>& o, int delta) {
#pragma unroll
  for (int kd = 0; kd < DqOffsets<DP>::KD; ++kd) o.kf[kd] += delta;
#pragma unroll
  for (int dt = 0; dt < DqOffsets<DP>::DT; ++dt) o.tr[dt][0] += delta, o.tr[dt][1] += delta;
}

// dQ for 128 queries (4 wavefronts x 32 queries) of one (b, q-head): the
// forward kernel's structure with dP computed beside S. K and V tiles of 64
// keys stream through double-buffered swizzled LDS; per tile
//   S^T = K Q^T, dP^T = V dO^T      (C layout: column = query, rows = keys)
//   dS^T = P^T (dP^T - Delta)
//   dQ^T += K^T dS^T                (K^T read transposed from the K tile)
// KV_OFF: bytes from a K tile to the V tile of the same stage.
template <typename T, int DP, bool MASK, uint32_t KV_OFF>
__device__ __forceinline__ void fa_bwd_dq_tile(const DqOffsets<DP>& o, const typename Mfma<T>::v8 (&qf)[DP / 16],
                                               const typename Mfma<T>::v8 (&of)[DP / 16], f32x16 (&dq)[DP / 32],
                                               float lse2, float dl, int kv0, int lim, float scale_log2, int lane) {
  constexpr int DT = DP / 32, KD = DP / 16;
  typedef typename Mfma<T>::v8 v8;
  const int hf = lane >> 5;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    f32x16 sc = zero16(), dp = zero16();
    constexpr uint32_t kt_rows = 32 * DP * 2;
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
      sc = Mfma<T>::mma(lds_frag16<T>(o.kf[kd], kt * kt_rows), qf[kd], sc);
      dp = Mfma<T>::mma(lds_frag16<T>(o.kf[kd], KV_OFF + kt * kt_rows), of[kd], dp);
    }
    // Issue order of the 2 KD fragment reads (R) and MFMAs (M): 4 R, then
    // (M R) x (2 KD - 4), then 4 M: four reads in flight ahead of their
    // products instead of one. The fence keeps the later dQ reads out.
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 2 * KD - 4; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float p = exp2_(__builtin_fmaf(sc[g * 4 + r], scale_log2, -lse2));
        if constexpr (MASK) {
          const int key = kv0 + kt * 32 + g * 8 + hf * 4 + r;
          p = key > lim ? 0.f : p;
        }
        dp[g * 4 + r] = p * (dp[g * 4 + r] - dl);
      }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const v8 df = pack_pair<T>(dp, ks * 2);
      const uint32_t rows = (kt * 32 + ks * 16) * DP * 2;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) dq[dt] = Mfma<T>::mma(lds_tr_frag<T>(o.tr[dt][0], o.tr[dt][1], rows), df, dq[dt]);
    }
  }
}

template <typename T, int DP>
__global__ __launch_bounds__(256) void fa_bwd_dq_kernel(
    const T* __restrict__ Q, int64_t sqb, int64_t sqh, int64_t sqs, const T* __restrict__ K, int64_t skb, int64_t skh,
    int64_t sks, const T* __restrict__ V, int64_t svb, int64_t svh, int64_t svs, const T* __restrict__ dO,
    const float* __restrict__ LSE2, const float* __restrict__ Delta, int64_t sqp, T* __restrict__ dQ, int Hq,
    int groups, int Sq, int Sk, int D, float scale_log2, float scale, int causal, int coff) {
  constexpr int BN = 64, BMQ = 128;
  constexpr int DT = DP / 32, KD = DP / 16;
  typedef typename Mfma<T>::v8 v8;
  // K stage 0, K stage 1, V stage 0, V stage 1
  __shared__ __attribute__((aligned(1024))) T KVs[4][BN * DP];
  constexpr uint32_t kStage = BN * DP * 2, kKv = 2 * kStage;

  const int nqb = (Sq + BMQ - 1) / BMQ;
  int rank, bhi;
  block_rank_row(rank, bhi);
  const int qb = nqb - 1 - rank;  // last query blocks see the most keys
  const int64_t bh = bhi;
  const int b = (int)(bh / Hq), hq = (int)(bh % Hq), hk = hq / groups;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int ql = lane & 31, hf = lane >> 5;
  const int qw0 = qb * BMQ + wid * 32;
  const int qi = qw0 + ql;
  const T* Qb = Q + b * sqb + hq * sqh;
  const T* Kb = K + b * skb + hk * skh;
  const T* Vb = V + b * svb + hk * svh;
  const T* dOb = dO + bh * Sq * D;

  v8 qf[KD], of[KD];
#pragma unroll
  for (int kd = 0; kd < KD; ++kd) {
    const int d0 = kd * 16 + hf * 8;
    if (qi < Sq && d0 < D) {
      qf[kd] = load_frag16<T>(Qb + (int64_t)qi * sqs + d0);
      of[kd] = load_frag16<T>(dOb + (int64_t)qi * D + d0);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[kd][e] = of[kd][e] = (T)0.f;
    }
  }
  // queries past Sq read the zero tail of the padded lse / Delta rows
  const float lse2 = LSE2[bh * sqp + (qi < Sq ? qi : Sq)];
  const float dl = Delta[bh * sqp + (qi < Sq ? qi : Sq)];
  f32x16 dq[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dq[dt] = zero16();

  int kv_end = Sk;
  if (causal) kv_end = min(Sk, qb * BMQ + BMQ + coff);
  const int ntiles = kv_end > 0 ? (kv_end + BN - 1) / BN : 0;
  // last key visible to this lane's query (causal and/or Sk bound); none for padding lanes
  const int lim = qi < Sq ? (causal ? min(Sk - 1, qi + coff) : Sk - 1) : -1;
  const TileLoader<T, BN, DP> kload(sks, D), vload(svs, D);
  if (ntiles > 0) {
    kload.load(KVs[0], Kb, sks, 0, Sk);
    vload.load(KVs[2], Vb, svs, 0, Sk);
  }
  DqOffsets<DP> off = dq_offsets<DP>(lds_addr(KVs[0]), lane);
  int shift = (int)kStage;  // to the other stage: +kStage after even tiles, -kStage after odd ones
  for (int it = 0; it < ntiles; ++it) {
    const int kv0 = it * BN;
    const int buf = it & 1;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (it + 1 < ntiles) {
      kload.load(KVs[buf ^ 1], Kb, sks, kv0 + BN, Sk);
      vload.load(KVs[2 + (buf ^ 1)], Vb, svs, kv0 + BN, Sk);
    }
    const bool need_mask = (kv0 + BN > Sk) || (qw0 + 32 > Sq) || (causal && kv0 + BN - 1 > qw0 + coff);
    if (need_mask)
      fa_bwd_dq_tile<T, DP, true, kKv>(off, qf, of, dq, lse2, dl, kv0, lim, scale_log2, lane);
    else
      fa_bwd_dq_tile<T, DP, false, kKv>(off, qf, of, dq, lse2, dl, kv0, lim, scale_log2, lane);
    dq_shift<DP>(off, shift);
    shift = -shift;
  }
  if (qi < Sq) {
    T* dQr = dQ + (bh * Sq + qi) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) {
        const int d = dt * 32 + gg * 8 + hf * 4;
        if (d < D) {
          typename Mfma<T>::v4 a;
#pragma unroll
          for (int r = 0; r < 4; ++r) a[r] = (T)(dq[dt][gg * 4 + r] * scale);
          *reinterpret_cast<typename Mfma<T>::v4*>(dQr + d) = a;
        }
      }
  }
}

// ===========================================================================
// Decode: Sq == 1, split-KV.
// ===========================================================================

// Split-KV decode on the matrix cores. One wavefront per (split, b, kv-head)
// streams the split's keys in tiles of 32 through NS LDS stages filled by
// direct-to-LDS loads (NS - 1 tiles are in flight while one is used; only this
// wave touches its LDS, so s_waitcnt replaces barriers).
// Per tile:
//   S^T = K Q^T  on MFMA 16x16x32 (keys x queries; the G query heads of the
//                kv-head are the columns, the rest of the 16 are zero),
//   online softmax on the C layout (a lane holds 8 keys of one query; the
//                running max is shared by the 4 lanes of a query),
//   O^T += V^T P^T with V^T read by ds_read_b64_tr_b16 and P^T taken from the
//                C layout with the key index permuted to match.
// K/V rows use the same XOR-swizzled layout as the forward kernel.
template <typename T, int DP, int G, int NS, bool IL = false>
__global__ __launch_bounds__(64) void fa_decode_kernel(const T* __restrict__ Q, int64_t sqb, int64_t sqh,
                                                       const T* __restrict__ K, int64_t skb, int64_t skh, int64_t sks,
                                                       const T* __restrict__ V, int64_t svb, int64_t svh, int64_t svs,
                                                       float* __restrict__ ws_o, float* __restrict__ ws_ml,
                                                       const int* __restrict__ seqlens, int Hkv, int Sk, int D,
                                                       int kps, float scale_log2) {
  static_assert(G >= 1 && G <= 16, "query heads per kv-head");
  static_assert(NS >= 2 && NS <= 5, "LDS stages");
  constexpr int BN = 32;            // keys per tile
  constexpr int CPR = DP / 8;       // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;     // rows per 1 KiB load instruction
  constexpr int NI = BN / RPI;      // load instructions per tile and tensor
  constexpr int KD = DP / 32;       // 32-wide d steps of S
  constexpr int DT = DP / 16;       // 16-row d tiles of O^T
  typedef typename Mfma<T>::v8 v8;
  __shared__ __attribute__((aligned(1024))) T Ks[NS][BN * DP];
  __shared__ __attribute__((aligned(1024))) T Vs[NS][BN * DP];

  const int split = blockIdx.x, nsplit = gridDim.x;
  const int bk = blockIdx.y;
  const int b = bk / Hkv, hk = bk % Hkv;
  const int lane = threadIdx.x;
  const int li = lane & 15, lg = lane >> 4;

  // Q^T fragments (B operand): column = query li, k = d = 32 kd + 8 lg + e.
  v8 qf[KD];
#pragma unroll
  for (int kd = 0; kd < KD; ++kd) {
    const int d = kd * 32 + lg * 8;
    if (li < G && d < D) qf[kd] = *reinterpret_cast<const v8*>(Q + b * sqb + (int64_t)(hk * G + li) * sqh + d);
    else
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[kd][e] = (T)0.f;
  }

  const T* Kb = K + b * skb + hk * skh;
  const T* Vb = V + b * svb + hk * svh;
  const int sk_b = seqlens ? min(seqlens[b], Sk) : Sk;
  // IL: split s takes tiles s, s + nsplit, ... of the sequence, so the splits of
  // one (b, kv-head) stream neighbouring tiles at the same time; otherwise split
  // s takes the kps keys from s * kps.
  const int rbase = IL ? split * BN : split * kps;
  const int rstep = IL ? nsplit * BN : BN;
  const int ke = IL ? sk_b : min(sk_b, rbase + kps);
  const int ntiles = IL ? (split * BN < sk_b ? ((sk_b + BN - 1) / BN - split + nsplit - 1) / nsplit : 0)
                        : (ke > rbase ? (ke - rbase + BN - 1) / BN : 0);

  // DMA lane geometry: row rl of each RPI-row group, physical chunk p.
  const int rl = lane / CPR, p = lane % CPR;
  // The swizzle of row n * RPI + rl repeats every NPAT instructions.
  constexpr int NPAT = (CPR < 16 ? CPR : 16) / RPI > 1 ? (CPR < 16 ? CPR : 16) / RPI : 1;
  int dsw[NPAT];
  uint32_t koff[NPAT], voff[NPAT];
#pragma unroll
  for (int par = 0; par < NPAT; ++par) {
    const int c = swz(par * RPI + rl, p, CPR);
    dsw[par] = c * 8 < D ? c * 8 : D - 8;
    koff[par] = (uint32_t)(((int64_t)rl * sks + dsw[par]) * (int64_t)sizeof(T));
    voff[par] = (uint32_t)(((int64_t)rl * svs + dsw[par]) * (int64_t)sizeof(T));
  }
  auto tile_row = [&](int t) { return rbase + t * rstep; };
  auto issue = [&](int t) {
    const int row0 = tile_row(t);
    const int st = t % NS;
    const uint32_t kl = lds_addr(Ks[st]), vl = lds_addr(Vs[st]);
    if (row0 + BN <= ke) {
#pragma unroll
      for (int n = 0; n < NI; ++n) {
        lds_dma16_s_nt(koff[n % NPAT], Kb + (int64_t)(row0 + n * RPI) * sks, kl + (uint32_t)(n * RPI * DP * sizeof(T)));
        lds_dma16_s_nt(voff[n % NPAT], Vb + (int64_t)(row0 + n * RPI) * svs, vl + (uint32_t)(n * RPI * DP * sizeof(T)));
      }
    } else {
#pragma unroll
      for (int n = 0; n < NI; ++n) {
        int gr = row0 + n * RPI + rl;
        gr = gr < ke ? gr : ke - 1;
        lds_dma16_nt(Kb + (int64_t)gr * sks + dsw[n % NPAT], kl + (uint32_t)(n * RPI * DP * sizeof(T)));
        lds_dma16_nt(Vb + (int64_t)gr * svs + dsw[n % NPAT], vl + (uint32_t)(n * RPI * DP * sizeof(T)));
      }
    }
  };

  float m = -INFINITY, l = 0.f;  // running max (log2 units) / this lane's partial sum, query li
  f32x4 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int t = 0; t < NS - 1; ++t)
    if (t < ntiles) issue(t);
  for (int t = 0; t < ntiles; ++t) {
    // refill the stage of tile t - 1 (its LDS reads completed last iteration),
    // so NS - 1 tiles stay in flight while tile t is waited for
    if (t + NS - 1 < ntiles) issue(t + NS - 1);
    // tile t has landed once only the tiles issued after it (at most NS - 1)
    // have loads outstanding, 2 NI instructions each
    const int after = min(ntiles - 1 - t, NS - 1);
    if (after <= 0) __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    else if (after == 1) __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * NI));
    else if (after == 2) __builtin_amdgcn_s_waitcnt(waitcnt_vm(4 * NI));
    else if (after == 3) __builtin_amdgcn_s_waitcnt(waitcnt_vm(6 * NI));
    else __builtin_amdgcn_s_waitcnt(waitcnt_vm(8 * NI));
    const T* Kt = Ks[t % NS];
    const T* Vt = Vs[t % NS];
    f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
      const int ch = kd * 4 + lg;
      const v8 a0 = *reinterpret_cast<const v8*>(Kt + li * DP + swz(li, ch, CPR) * 8);
      const v8 a1 = *reinterpret_cast<const v8*>(Kt + (16 + li) * DP + swz(16 + li, ch, CPR) * 8);
      s0 = mma16<T>(a0, qf[kd], s0);
      s1 = mma16<T>(a1, qf[kd], s1);
    }
    // scores of keys 4 lg + r (s0) and 16 + 4 lg + r (s1), in log2 units
    const int kbase = tile_row(t) + 4 * lg;
    float x[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = kbase + r < ke ? s0[r] * scale_log2 : -INFINITY;
      x[4 + r] = kbase + 16 + r < ke ? s1[r] * scale_log2 : -INFINITY;
    }
    float mx = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    if (mx > m) {
      const float a = exp2_(m - mx);  // 0 while m is still -inf
      l *= a;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] *= a;
      m = mx;
    }
    const float mr = m == -INFINITY ? 0.f : m;
    v8 pf;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float pe = exp2_(x[e] - mr);
      l += pe;
      pf[e] = (T)pe;
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      // A = V^T: row d = 16 dt + li; keys 4 lg + e and 16 + 4 lg + e (e < 4)
      const int key = 4 * lg + (li >> 2);
      const int d = dt * 16 + 4 * (li & 3);
      const T* s0p = Vt + key * DP + swz(key, d >> 3, CPR) * 8 + (d & 7);
      const T* s1p = Vt + (key + 16) * DP + swz(key + 16, d >> 3, CPR) * 8 + (d & 7);
      const qh_v4i16 w0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) qh_v4i16*)(s0p));
      const qh_v4i16 w1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) qh_v4i16*)(s1p));
      const v8 av = __builtin_bit_cast(v8, qh_v8i16(__builtin_shufflevector(w0, w1, 0, 1, 2, 3, 4, 5, 6, 7)));
      o[dt] = mma16<T>(av, pf, o[dt]);
    }
    // the LDS reads of this stage are complete before the stage is refilled
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  }
  // l: sum the 4 lanes of each query; o: lane holds d = 16 dt + 4 lg + r of query li
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (li < G) {
    const int64_t slot = ((int64_t)bk * G + li) * nsplit + split;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = dt * 16 + 4 * lg + r;
        if (d < D) ws_o[slot * DP + d] = o[dt][r];
      }
    if (lg == 0) {
      ws_ml[slot * 2] = m;
      ws_ml[slot * 2 + 1] = l;
    }
  }
}

template <typename T, int DP>
__global__ __launch_bounds__(256) void fa_decode_combine(const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
                                                         T* __restrict__ O, float* __restrict__ LSE, int rows,
                                                         int nsplit, int D) {
  const int row = blockIdx.x * (256 / DP) + threadIdx.x / DP;  // one (b, q-head) per DP threads
  const int d = threadIdx.x % DP;
  if (row >= rows) return;
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, ws_ml[((int64_t)row * nsplit + s) * 2]);
  const float Mr = (M == -INFINITY) ? 0.f : M;
  float L = 0.f, acc = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const int64_t slot = (int64_t)row * nsplit + s;
    const float w = exp2_(ws_ml[slot * 2] - Mr);
    L += ws_ml[slot * 2 + 1] * w;
    if (d < D) acc += ws_o[slot * DP + d] * w;
  }
  if (d < D) O[(int64_t)row * D + d] = from_f32<T>(L > 0.f ? acc / L : 0.f);
  if (d == 0 && LSE) LSE[row] = L > 0.f ? (M + __log2f(L)) * kLn2 : -INFINITY;
}

// Decode for many sequences: one 256-thread workgroup per (b, kv-head) whose
// wavefront w takes key tiles w, w + 4, w + 8, ... -- the key partition of
// fa_decode_kernel with 4 interleaved splits, and the same per-tile arithmetic.
// K fragments go from global memory straight into registers in the MFMA
// operand layout (no LDS); V tiles go through two LDS stages per wavefront (the
// transposed operand reads need LDS), so two workgroups fit on a CU. The four
// partial (m, l, o) are combined in LDS in wavefront order with
// fa_decode_combine's arithmetic: no workspace and no second launch, and the
// same results as the split kernel plus combine at 4 splits.
//
// K and V are __restrict__ except with PREP, where the kernel writes the new
// cache rows and later reads them through the same pointers.
//
// PREP (one new token per sequence): the kernel also prepares its own rows,
// replacing the separate prepare pass. Each wavefront loads its rows, issues
// its first two K/V tiles, then normalises and rotates the group's G query
// rows itself (norm_rope_row, the prepare pass's arithmetic) and regroups them
// into its MFMA operand through a private LDS slot, so no wavefront waits for
// another. The wavefront that will read the key tile holding the new position
// p also writes the new key row (normalised, rotated) and value row into the
// caches at p, and keeps both in LDS: when that tile has landed, the lanes
// holding key p take the key row from LDS and the value rows from p to the
// tile's end (key p, and the rows past the last key that the tile load clamps
// to it) are rewritten in the V stage. So no load waits for the stores, whose
// bytes are those the patch supplies.
template <typename T, bool PREP>
using kv_ptr = typename std::conditional<PREP, const T*, const T* __restrict__>::type;

template <typename T, typename C>
struct DecodePrepArgs {
  const T* q;  // projected rows of the step: q [B, Hq * D], k and v [B, Hkv * D] (row strides sq, sk, sv)
  const T* k;
  const T* v;
  int64_t sq, sk, sv;
  const void* qw;  // q_norm / k_norm weights (wdtype), + wadd
  const void* kw;
  int wdtype;
  float eps, wadd;
  const C* cs;  // cos / sin of the step, [cos_batch, 1, rot] (batch stride scb)
  const C* sn;
  int64_t scb;
  int cos_batch, half, rot;
  const int64_t* pos;  // the step's cache position (one for every sequence)
  int64_t cap;         // rows allocated in the caches (positions outside [0, cap) are not written)
};

// NTKV: K/V tiles read non-temporally (a large cache streamed once per step past the
// last-level cache); short caches, read again at the next step, keep the default policy.
// NW wavefronts per workgroup (8 for short caches of more than 4 tiles, so that no
// wave computes two tiles one after the other).
template <typename T, int DP, int G, bool PREP = false, typename C = float, bool NTKV = true, int NW = 4>
__global__ __launch_bounds__(64 * NW) void fa_decode_wg_kernel(const T* __restrict__ Q, int64_t sqb, int64_t sqh,
                                                          kv_ptr<T, PREP> K, int64_t skb, int64_t skh,
                                                          int64_t sks, kv_ptr<T, PREP> V, int64_t svb,
                                                          int64_t svh, int64_t svs, T* __restrict__ O,
                                                          float* __restrict__ LSE, const int* __restrict__ seqlens,
                                                          int Hkv, int Sk, int D, float scale_log2,
                                                          const DecodePrepArgs<T, C> pa) {
  static_assert(G >= 1 && G <= 8, "query heads per kv-head");
  constexpr int BN = 32, NS = 2;
  constexpr int CPR = DP / 8;    // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;  // rows per 1 KiB load instruction
  constexpr int NI = BN / RPI;   // V load instructions per tile
  constexpr int KD = DP / 32;    // 32-wide d steps of S
  constexpr int DT = DP / 16;    // 16-row d tiles of O^T
  constexpr int NPAT = (CPR < 16 ? CPR : 16) / RPI > 1 ? (CPR < 16 ? CPR : 16) / RPI : 1;
  constexpr int KLD = 2 * KD;    // K load instructions per tile
  typedef typename Mfma<T>::v8 v8;
  __shared__ __attribute__((aligned(1024))) T Vs[NW][NS][BN * DP];
  __shared__ float cml[NW][G][2];
  __shared__ float co[NW][G][DP];
  __shared__ __attribute__((aligned(16))) T qs[PREP ? NW : 1][PREP ? G : 1][DP];
  __shared__ __attribute__((aligned(16))) T kvp[PREP ? NW : 1][2][PREP ? DP : 8];  // PREP: new key / value row

  const int bk = blockIdx.x;
  const int b = bk / Hkv, hk = bk % Hkv;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, lg = lane >> 4;

  const T* Kb = K + b * skb + hk * skh;
  const T* Vb = V + b * svb + hk * svh;
  const int sk_b = seqlens ? min(seqlens[b], Sk) : Sk;
  const int ntiles = w * BN < sk_b ? ((sk_b + BN - 1) / BN - w + NW - 1) / NW : 0;

  // K operand lanes: key 16 h + li of the tile, chunk d = 32 kd + 8 lg (clamped
  // into the row when D < DP; those products meet zero Q entries).
  int kdo[KD];
#pragma unroll
  for (int kd = 0; kd < KD; ++kd) {
    const int d = kd * 32 + lg * 8;
    kdo[kd] = d < D ? d : D - 8;
  }
  // V DMA lanes: row rl of each RPI-row group, physical chunk p (swizzled).
  const int rl = lane / CPR, p = lane % CPR;
  int dsw[NPAT];
  uint32_t voff[NPAT];
#pragma unroll
  for (int par = 0; par < NPAT; ++par) {
    const int c = swz(par * RPI + rl, p, CPR);
    dsw[par] = c * 8 < D ? c * 8 : D - 8;
    voff[par] = (uint32_t)(((int64_t)rl * svs + dsw[par]) * (int64_t)sizeof(T));
  }
  // PREP: this wave's tile holding the new position p, p's row in it, and the end of the V
  // rows to rewrite (past p only when p is the last key: the tile load clamps later rows to it)
  int tp = -1, kp = 0, kpe = 0;
  auto issue = [&](int t, v8 (&kf)[2][KD]) {
    const int row0 = (w + t * NW) * BN;
    const uint32_t vl = lds_addr(Vs[w][t % NS]);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      int key = row0 + 16 * h + li;
      key = key < sk_b ? key : sk_b - 1;
      const T* kr = Kb + (int64_t)key * sks;
#pragma unroll
      for (int kd = 0; kd < KD; ++kd)
        kf[h][kd] = NTKV ? __builtin_nontemporal_load(reinterpret_cast<const v8*>(kr + kdo[kd]))
                         : *reinterpret_cast<const v8*>(kr + kdo[kd]);
    }
    if (row0 + BN <= sk_b) {
#pragma unroll
      for (int n = 0; n < NI; ++n) {
        const T* vb = Vb + (int64_t)(row0 + n * RPI) * svs;
        const uint32_t dst = vl + (uint32_t)(n * RPI * DP * sizeof(T));
        if constexpr (NTKV) lds_dma16_s_nt(voff[n % NPAT], vb, dst);
        else lds_dma16_s(voff[n % NPAT], vb, dst);
      }
    } else {
#pragma unroll
      for (int n = 0; n < NI; ++n) {
        int gr = row0 + n * RPI + rl;
        gr = gr < sk_b ? gr : sk_b - 1;
        const T* src = Vb + (int64_t)gr * svs + dsw[n % NPAT];
        const uint32_t dst = vl + (uint32_t)(n * RPI * DP * sizeof(T));
        if constexpr (NTKV) lds_dma16_nt(src, dst);
        else lds_dma16(src, dst);
      }
    }
  };

  // Two register sets for K (one tile ahead); the loop below is unrolled by
  // two so each set is named statically.
  v8 ka[2][KD], kb[2][KD];
  v8 qf[KD];
  bool pre1 = false;  // tile 1 already requested before the loop
  if constexpr (PREP) {
    const int64_t p = pa.pos[0];
    const bool pin = p >= 0 && p < sk_b && p < pa.cap;  // the new row is one of the keys read here
    const int wp = pin ? (int)((p / BN) % NW) : 0;
    if (pin && w == wp) {
      tp = (int)(p / BN - w) / NW;
      kp = (int)(p % BN);
      kpe = p == sk_b - 1 ? BN : kp + 1;
    }
    // 16-lane group gi takes rows gi, gi + 4, ...: the G query rows, then (wave
    // wp) the key row and the value row; one 16-byte load per lane and pass.
    constexpr int NPASS = (G + 2 + 3) / 4;
    const int gi = lane >> 4, g = lane & 15, d0 = 8 * g;
    const bool act = d0 < D, pok = w == wp && p >= 0 && p < pa.cap;
    const int dl = act ? d0 : D - 8;
    // Rows and their parameters (norm scales, cos/sin) are requested before the
    // tiles, so waiting for them never waits for a tile.
    const int64_t co_row = (pa.cos_batch == 1 ? 0 : b) * pa.scb;
    Vec16<T> xv[NPASS];
    RowRaw rr[NPASS];
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int r = gi + 4 * ps;
      const T* src = r < G ? pa.q + b * pa.sq + (int64_t)(hk * G + r) * D
                           : (r == G ? pa.k + b * pa.sk : pa.v + b * pa.sv) + (int64_t)hk * D;
      xv[ps] = ld16((r < G + 2 ? src : pa.q + b * pa.sq) + dl);
      rr[ps] = load_row_raw<C>(r < G ? pa.qw : pa.kw, pa.wdtype, d0, act, pa.half, pa.rot, pa.cs, pa.sn, co_row);
    }
    if (ntiles > 0) {
      issue(0, ka);
      if (ntiles > 1) issue(1, kb), pre1 = true;
    }
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int r = gi + 4 * ps;
      const bool isq = r < G, isk = r == G && pok, isv = r == G + 1 && pok;
      Vec16<T> x = xv[ps];
      if (!act) x.raw = make_uint4(0, 0, 0, 0);
      const RowParams rp = row_params_from<C>(rr[ps], pa.wdtype, pa.wadd, d0, act, pa.rot);
      const Vec16<T> y = norm_rope_apply<T>(x, act, rp, pa.eps, D, d0, pa.half / 8, pa.half, pa.rot);
      if (act) {
        if (isq) {
          *reinterpret_cast<uint4*>(&qs[w][r][d0]) = y.raw;
        } else if (isk) {
          st16(const_cast<T*>(Kb) + p * sks + d0, y);
          *reinterpret_cast<uint4*>(&kvp[w][0][d0]) = y.raw;
        } else if (isv) {
          st16(const_cast<T*>(Vb) + p * svs + d0, x);
          *reinterpret_cast<uint4*>(&kvp[w][1][d0]) = x.raw;
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);  // this wave's qs (and kvp) rows are written
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
      const int d = kd * 32 + lg * 8;
      if (li < G && d < D) qf[kd] = *reinterpret_cast<const v8*>(&qs[w][li][d]);
      else
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[kd][e] = (T)0.f;
    }
  } else {
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
      const int d = kd * 32 + lg * 8;
      if (li < G && d < D) qf[kd] = *reinterpret_cast<const v8*>(Q + b * sqb + (int64_t)(hk * G + li) * sqh + d);
      else
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[kd][e] = (T)0.f;
    }
    if (ntiles > 0) issue(0, ka);
  }

  float m = -INFINITY, l = 0.f;
  f32x4 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int t, const v8 (&kf)[2][KD]) {
    const T* Vt = Vs[w][t % NS];
    f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
      s0 = mma16<T>(kf[0][kd], qf[kd], s0);
      s1 = mma16<T>(kf[1][kd], qf[kd], s1);
    }
    const int kbase = (w + t * NW) * BN + 4 * lg;
    float x[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = kbase + r < sk_b ? s0[r] * scale_log2 : -INFINITY;
      x[4 + r] = kbase + 16 + r < sk_b ? s1[r] * scale_log2 : -INFINITY;
    }
    float mx = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    if (mx > m) {
      const float a = exp2_(m - mx);
      l *= a;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] *= a;
      m = mx;
    }
    const float mr = m == -INFINITY ? 0.f : m;
    v8 pf;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float pe = exp2_(x[e] - mr);
      l += pe;
      pf[e] = (T)pe;
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int key = 4 * lg + (li >> 2);
      const int d = dt * 16 + 4 * (li & 3);
      const T* s0p = Vt + key * DP + swz(key, d >> 3, CPR) * 8 + (d & 7);
      const T* s1p = Vt + (key + 16) * DP + swz(key + 16, d >> 3, CPR) * 8 + (d & 7);
      const qh_v4i16 w0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) qh_v4i16*)(s0p));
      const qh_v4i16 w1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) qh_v4i16*)(s1p));
      const v8 av = __builtin_bit_cast(v8, qh_v8i16(__builtin_shufflevector(w0, w1, 0, 1, 2, 3, 4, 5, 6, 7)));
      o[dt] = mma16<T>(av, pf, o[dt]);
    }
    // this stage's LDS reads are complete before it is refilled
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  };

  // PREP, tile tp (landed): key p's fragments from the kept row; V rows kp..kpe-1
  // (key p, and when p is the last key the clamped rows past it) rewritten with the new value row.
  auto patch = [&](int t, v8 (&kf)[2][KD]) {
    if (!PREP || t != tp) return;
    if (li == (kp & 15)) {
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) {
        const v8 kv = *reinterpret_cast<const v8*>(&kvp[w][0][kdo[kd]]);
        if (kp < 16) kf[0][kd] = kv;
        else kf[1][kd] = kv;
      }
    }
    T* Vt = Vs[w][t % NS];
    for (int i = lane; i < (kpe - kp) * CPR; i += 64) {
      const int r = kp + i / CPR, c = i % CPR;
      const int dsrc = c * 8 < D ? c * 8 : D - 8;
      *reinterpret_cast<uint4*>(Vt + r * DP + swz(r, c, CPR) * 8) = *reinterpret_cast<const uint4*>(&kvp[w][1][dsrc]);
    }
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  };

  // Tile t has landed once only tile t + 1's KLD + NI instructions are
  // outstanding (tile 0 was issued above).
  for (int t = 0; t < ntiles; t += 2) {
    if (t + 1 < ntiles) {
      if (!(pre1 && t == 0)) issue(t + 1, kb);
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(KLD + NI));
    } else {
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    }
    patch(t, ka);
    compute(t, ka);
    if (t + 1 < ntiles) {
      if (t + 2 < ntiles) {
        issue(t + 2, ka);
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(KLD + NI));
      } else {
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
      }
      patch(t + 1, kb);
      compute(t + 1, kb);
    }
  }
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (li < G) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) co[w][li][dt * 16 + 4 * lg + r] = o[dt][r];
    if (lg == 0) {
      cml[w][li][0] = m;
      cml[w][li][1] = l;
    }
  }
  __syncthreads();
  // combine the four wavefronts in order (fa_decode_combine's arithmetic)
  for (int idx = threadIdx.x; idx < G * DP; idx += 64 * NW) {
    const int g = idx / DP, d = idx % DP;
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < NW; ++s) M = fmaxf(M, cml[s][g][0]);
    const float Mr = (M == -INFINITY) ? 0.f : M;
    float L = 0.f, acc = 0.f;
#pragma unroll
    for (int s = 0; s < NW; ++s) {
      const float wgt = exp2_(cml[s][g][0] - Mr);
      L += cml[s][g][1] * wgt;
      acc += co[s][g][d] * wgt;
    }
    const int64_t row = (int64_t)bk * G + g;
    if (d < D) O[row * D + d] = from_f32<T>(L > 0.f ? acc / L : 0.f);
    if (d == 0 && LSE) LSE[row] = L > 0.f ? (M + __log2f(L)) * kLn2 : -INFINITY;
  }
}

static int pick_dp(int64_t D) {
  if (D <= 32) return 32;
  if (D <= 64) return 64;
  if (D <= 128) return 128;
  return 0;
}

// Splits per (b, kv-head): about 2048 single-wave workgroups in total (a few
// per SIMD, so one wave's tile math overlaps the others' loads), each with at
// least 8 tiles of 32 keys. Two LDS stages: more stages cost occupancy and
// measured slower. The splits take interleaved tiles (split s: tiles s,
// s + nsplit, ...): the waves of one sequence then read neighbouring rows at
// the same time, which measured 3% faster at 4 splits than contiguous ranges
// (and 10% at 8).
// From this many (b, kv-head) pairs on (two workgroups per CU), head dim 128
// decodes with fa_decode_wg_kernel.
constexpr int64_t kDecodeWgMinSeqs = 512;

static int decode_splits(int64_t B, int64_t Hkv, int64_t Sk) {
  const int64_t tiles = (Sk + 31) / 32;
  int64_t s = (2048 + B * Hkv - 1) / (B * Hkv);
  const int64_t cap = (tiles + 7) / 8;
  if (s > cap) s = cap;
  if (s < 1) s = 1;
  return (int)s;
}

template <typename T, int DP, int G>
void launch_decode(const void* q, int64_t sqb, int64_t sqh, const void* k, int64_t skb, int64_t skh, int64_t sks,
                   const void* v, int64_t svb, int64_t svh, int64_t svs, float* ws_o, float* ws_ml,
                   const int* seqlens, int B, int Hkv, int Sk, int D, int nsplit, float scale_log2, hipStream_t st) {
  const int kps = (Sk + nsplit - 1) / nsplit;
  dim3 grid(nsplit, B * Hkv);
  fa_decode_kernel<T, DP, G, 2, true><<<grid, 64, 0, st>>>((const T*)q, sqb, sqh, (const T*)k, skb, skh, sks, (const T*)v, svb,
                                                   svh, svs, ws_o, ws_ml, seqlens, Hkv, Sk, D, kps,
                                                   scale_log2);
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" int qh_flash_fwd(const void* q, int64_t sqb, int64_t sqh, int64_t sqs, const void* k, int64_t skb,
                            int64_t skh, int64_t sks, const void* v, int64_t svb, int64_t svh, int64_t svs, void* o,
                            int64_t sob, int64_t soh, int64_t sos, float* lse, int64_t B, int64_t Hq, int64_t Hkv,
                            int64_t Sq, int64_t Sk, int64_t D, float scale, int causal, int64_t causal_offset, int dtype,
                            void* stream) {
  QH_CHECK_ARG(B >= 0 && Hq > 0 && Hkv > 0 && Sq >= 0 && Sk >= 0, "qh_flash_fwd: bad shape");
  QH_CHECK_ARG(Hq % Hkv == 0, "qh_flash_fwd: Hq=%lld not a multiple of Hkv=%lld", (long long)Hq, (long long)Hkv);
  if (dtype == QH_F32) {
    QH_CHECK_ARG(pick_dp(D) && D % 4 == 0, "qh_flash_fwd: fp32 head dim %lld must be a multiple of 4 and <= 128",
                 (long long)D);
    QH_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o), "qh_flash_fwd: pointers must be 16-byte aligned");
    QH_CHECK_ARG(sqs % 4 == 0 && sks % 4 == 0 && svs % 4 == 0 && sqh % 4 == 0 && skh % 4 == 0 && svh % 4 == 0 &&
                     sqb % 4 == 0 && skb % 4 == 0 && svb % 4 == 0 && sob % 4 == 0 && soh % 4 == 0 && sos % 4 == 0,
                 "qh_flash_fwd: fp32 strides must be multiples of 4 elements");
    QH_CHECK_ARG(B * Hq < 65536 && Sq < (1 << 30) && Sk < (1 << 30), "qh_flash_fwd: too large");
    if (B * Hq * Sq == 0) return QH_OK;
    qh_flash_fwd_f32((const float*)q, sqb, sqh, sqs, (const float*)k, skb, skh, sks, (const float*)v, svb, svh, svs,
                     (float*)o, sob, soh, sos, lse, B, Hq, Hkv, Sq, Sk, D, scale, causal, causal_offset,
                     (hipStream_t)stream);
    QH_CHECK_LAUNCH("qh_flash_fwd");
    return QH_OK;
  }
  const int dp = pick_dp(D);
  QH_CHECK_ARG(dp && D % 8 == 0, "qh_flash_fwd: head dim %lld must be a multiple of 8 and <= 128", (long long)D);
  QH_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o), "qh_flash_fwd: pointers must be 16-byte aligned");
  QH_CHECK_ARG(sqs % 8 == 0 && sks % 8 == 0 && svs % 8 == 0 && sqh % 8 == 0 && skh % 8 == 0 && svh % 8 == 0 &&
                   sqb % 8 == 0 && skb % 8 == 0 && svb % 8 == 0 && sob % 8 == 0 && soh % 8 == 0 && sos % 8 == 0,
               "qh_flash_fwd: strides must be multiples of 8 elements");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_flash_fwd: bf16/f16 only");
  QH_CHECK_ARG(B * Hq < 65536 && Sq < (1 << 30) && Sk < (1 << 30), "qh_flash_fwd: too large");
  QH_CHECK_ARG((Sq + 127) / 128 * B * Hq < (1ll << 31), "qh_flash_fwd: too many query blocks");
  if (B * Hq * Sq == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const float sl2 = scale * kLog2e;
  const int groups = (int)(Hq / Hkv);
  dim3 grid((unsigned)ceil_div(Sq, 128), (unsigned)(B * Hq));
#define QH_FWD(T, DPV)                                                                                          \
  fa_fwd_kernel<T, DPV><<<grid, 256, 0, st>>>((const T*)q, sqb, sqh, sqs, (const T*)k, skb, skh, sks,       \
                                                 (const T*)v, svb, svh, svs, (T*)o, sob, soh, sos, lse, (int)Hq,   \
                                                 groups, (int)Sq, (int)Sk, (int)D, sl2, causal, (int)causal_offset)
#define QH_FWD_D(T) \
  if (dp == 32) QH_FWD(T, 32); else if (dp == 64) QH_FWD(T, 64); else QH_FWD(T, 128);
  if (dtype == QH_BF16) { QH_FWD_D(bf16_t) } else { QH_FWD_D(f16_t) }
#undef QH_FWD_D
#undef QH_FWD
  QH_CHECK_LAUNCH("qh_flash_fwd");
  return QH_OK;
}

extern "C" int qh_flash_fwd_masked(const void* q, int64_t sqb, int64_t sqh, int64_t sqs, const void* k, int64_t skb,
                                   int64_t skh, int64_t sks, const void* v, int64_t svb, int64_t svh, int64_t svs,
                                   void* o, int64_t sob, int64_t soh, int64_t sos, float* lse, int64_t B, int64_t Hq,
                                   int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D, float scale, int causal,
                                   int64_t causal_offset, const uint64_t* key_bits, int64_t bits_stride,
                                   int64_t window, int dtype, void* stream) {
  QH_CHECK_ARG(B >= 0 && Hq > 0 && Hkv > 0 && Sq >= 0 && Sk >= 0, "qh_flash_fwd_masked: bad shape");
  QH_CHECK_ARG(Hq % Hkv == 0, "qh_flash_fwd_masked: Hq=%lld not a multiple of Hkv=%lld", (long long)Hq,
               (long long)Hkv);
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_flash_fwd_masked: bf16/f16 only");
  const int dp = pick_dp(D);
  QH_CHECK_ARG(dp && D % 8 == 0, "qh_flash_fwd_masked: head dim %lld must be a multiple of 8 and <= 128",
               (long long)D);
  QH_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o),
               "qh_flash_fwd_masked: pointers must be 16-byte aligned");
  QH_CHECK_ARG(sqs % 8 == 0 && sks % 8 == 0 && svs % 8 == 0 && sqh % 8 == 0 && skh % 8 == 0 && svh % 8 == 0 &&
                   sqb % 8 == 0 && skb % 8 == 0 && svb % 8 == 0 && sob % 8 == 0 && soh % 8 == 0 && sos % 8 == 0,
               "qh_flash_fwd_masked: strides must be multiples of 8 elements");
  QH_CHECK_ARG(B * Hq < 65536 && Sq < (1 << 30) && Sk < (1 << 30), "qh_flash_fwd_masked: too large");
  QH_CHECK_ARG((Sq + 127) / 128 * B * Hq < (1ll << 31), "qh_flash_fwd_masked: too many query blocks");
  QH_CHECK_ARG(window >= 0 && window < (1 << 30), "qh_flash_fwd_masked: bad window %lld", (long long)window);
  QH_CHECK_ARG(causal_offset > -(1ll << 30) && causal_offset < (1ll << 30), "qh_flash_fwd_masked: bad causal offset");
  QH_CHECK_ARG(key_bits == nullptr || (((uintptr_t)key_bits & 7) == 0 && bits_stride >= (Sk + 63) / 64),
               "qh_flash_fwd_masked: key_bits must be 8-byte aligned with >= ceil(Sk / 64) words per batch row");
  if (B * Hq * Sq == 0) return QH_OK;
  hipStream_t st = (hipStream_t)stream;
  const float sl2 = scale * kLog2e;
  const int groups = (int)(Hq / Hkv);
  // one query per sequence: the q-heads of a kv-head share a block (its keys are read once)
  const bool pack = Sq == 1 && groups > 1 && groups <= 128;
  dim3 grid((unsigned)ceil_div(Sq, 128), (unsigned)(pack ? B * Hkv : B * Hq));
#define QH_FWD(T, DPV)                                                                                            \
  do {                                                                                                            \
    if (pack)                                                                                                     \
      fa_fwd_kernel<T, DPV, true, true><<<grid, 256, 0, st>>>(                                                    \
          (const T*)q, sqb, sqh, sqs, (const T*)k, skb, skh, sks, (const T*)v, svb, svh, svs, (T*)o, sob, soh,    \
          sos, lse, (int)Hq, groups, (int)Sq, (int)Sk, (int)D, sl2, causal, (int)causal_offset, key_bits,         \
          bits_stride, (int)window);                                                                              \
    else                                                                                                          \
      fa_fwd_kernel<T, DPV, true><<<grid, 256, 0, st>>>(                                                          \
          (const T*)q, sqb, sqh, sqs, (const T*)k, skb, skh, sks, (const T*)v, svb, svh, svs, (T*)o, sob, soh,    \
          sos, lse, (int)Hq, groups, (int)Sq, (int)Sk, (int)D, sl2, causal, (int)causal_offset, key_bits,         \
          bits_stride, (int)window);                                                                              \
  } while (0)
#define QH_FWD_D(T) \
  if (dp == 32) QH_FWD(T, 32); else if (dp == 64) QH_FWD(T, 64); else QH_FWD(T, 128);
  if (dtype == QH_BF16) { QH_FWD_D(bf16_t) } else { QH_FWD_D(f16_t) }
#undef QH_FWD_D
#undef QH_FWD
  QH_CHECK_LAUNCH("qh_flash_fwd_masked");
  return QH_OK;
}

// Padded row length of the per-query Delta / LSE2 arrays of the backward.
static int64_t bwd_row_pad(int64_t Sq) { return (Sq + 63) / 64 * 64 + 64; }

extern "C" int64_t qh_flash_bwd_workspace(int64_t B, int64_t Hq, int64_t Sq) {
  return 2 * B * Hq * bwd_row_pad(Sq) * 4;
}

namespace {
// LDS of fa_bwd_dkdv8_kernel: K and V of 128 keys plus two Q and two dO tiles of 64 rows,
// and two (lse2, Delta) pairs of 64 floats.
constexpr int kDkdv8Lds = DkdvLds<128>::BYTES;

// Raise the dynamic-LDS limit of fa_bwd_dkdv8_kernel once per device.
template <typename T>
int dkdv8_lds_ready() {
  static uint64_t done = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    qh::set_error("qh_flash_bwd: no current device");
    return QH_E_HIP;
  }
  if (done >> dev & 1) return QH_OK;
  const hipError_t e = hipFuncSetAttribute((const void*)fa_bwd_dkdv8_kernel<T, 128>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kDkdv8Lds);
  if (e != hipSuccess) {
    qh::set_error("qh_flash_bwd: cannot raise the LDS limit: %s", hipGetErrorString(e));
    return QH_E_HIP;
  }
  done |= 1ull << dev;
  return QH_OK;
}
}  // namespace

extern "C" int qh_flash_bwd(const void* q, int64_t sqb, int64_t sqh, int64_t sqs, const void* k, int64_t skb,
                            int64_t skh, int64_t sks, const void* v, int64_t svb, int64_t svh, int64_t svs,
                            const void* o, const void* dout, const float* lse, void* dq, void* dk, void* dv, void* ws,
                            int64_t ws_bytes, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
                            float scale, int causal, int64_t causal_offset, int dtype, void* stream) {
  QH_CHECK_ARG(B >= 0 && Hq > 0 && Hkv > 0 && Sq >= 0 && Sk >= 0, "qh_flash_bwd: bad shape");
  QH_CHECK_ARG(Hq % Hkv == 0, "qh_flash_bwd: Hq not a multiple of Hkv");
  if (dtype == QH_F32) {
    QH_CHECK_ARG(pick_dp(D) && D % 4 == 0, "qh_flash_bwd: fp32 head dim must be a multiple of 4 and <= 128");
    QH_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o) && aligned16(dout) && aligned16(dq) &&
                     aligned16(dk) && aligned16(dv),
                 "qh_flash_bwd: pointers must be 16-byte aligned");
    QH_CHECK_ARG(sqs % 4 == 0 && sks % 4 == 0 && svs % 4 == 0 && sqh % 4 == 0 && skh % 4 == 0 && svh % 4 == 0 &&
                     sqb % 4 == 0 && skb % 4 == 0 && svb % 4 == 0,
                 "qh_flash_bwd: fp32 strides must be multiples of 4 elements");
    QH_CHECK_ARG(B * Hq < 65536 && Sq < (1 << 30) && Sk < (1 << 30), "qh_flash_bwd: too large");
    const int64_t need32 = qh_flash_bwd_workspace(B, Hq, Sq);
    if (ws_bytes < need32) {
      qh::set_error("qh_flash_bwd: workspace %lld < %lld", (long long)ws_bytes, (long long)need32);
      return QH_E_WORKSPACE;
    }
    if (Sq == 0 || B == 0) {
      int rc = qh_zero(dk, B * Hkv * Sk * D * 4, stream);
      if (rc) return rc;
      return qh_zero(dv, B * Hkv * Sk * D * 4, stream);
    }
    const int64_t sqp32 = bwd_row_pad(Sq);
    float* delta32 = (float*)ws;
    qh_flash_bwd_f32((const float*)q, sqb, sqh, sqs, (const float*)k, skb, skh, sks, (const float*)v, svb, svh, svs,
                     (const float*)o, (const float*)dout, lse, (float*)dq, (float*)dk, (float*)dv, delta32,
                     delta32 + B * Hq * sqp32, sqp32, B, Hq, Hkv, Sq, Sk, D, scale, causal, causal_offset,
                     (hipStream_t)stream);
    QH_CHECK_LAUNCH("qh_flash_bwd");
    return QH_OK;
  }
  const int dp = pick_dp(D);
  QH_CHECK_ARG(dp && D % 8 == 0, "qh_flash_bwd: head dim must be a multiple of 8 and <= 128");
  QH_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o) && aligned16(dout) && aligned16(dq) &&
                   aligned16(dk) && aligned16(dv),
               "qh_flash_bwd: pointers must be 16-byte aligned");
  QH_CHECK_ARG(sqs % 8 == 0 && sks % 8 == 0 && svs % 8 == 0 && sqh % 8 == 0 && skh % 8 == 0 && svh % 8 == 0 &&
                   sqb % 8 == 0 && skb % 8 == 0 && svb % 8 == 0,
               "qh_flash_bwd: strides must be multiples of 8 elements");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_flash_bwd: bf16/f16 only");
  QH_CHECK_ARG(B * Hq < 65536 && Sq < (1 << 30) && Sk < (1 << 30), "qh_flash_bwd: too large");
  QH_CHECK_ARG((Sq + 127) / 128 * B * Hq < (1ll << 31) && (Sk + 127) / 128 * B * Hkv < (1ll << 31),
               "qh_flash_bwd: too many query or key blocks");
  const int64_t need = qh_flash_bwd_workspace(B, Hq, Sq);
  if (ws_bytes < need) {
    qh::set_error("qh_flash_bwd: workspace %lld < %lld", (long long)ws_bytes, (long long)need);
    return QH_E_WORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  const int esz = 2;
  if (Sq == 0 || B == 0) {
    int rc = qh_zero(dk, B * Hkv * Sk * D * esz, stream);
    if (rc) return rc;
    return qh_zero(dv, B * Hkv * Sk * D * esz, stream);
  }
  const int64_t sqp = bwd_row_pad(Sq);
  const int64_t prow = B * Hq * sqp;
  float* delta = (float*)ws;
  float* lse2 = delta + prow;
  const float sl2 = scale * kLog2e;
  const int groups = (int)(Hq / Hkv);
  dim3 gkv((unsigned)ceil_div(Sk, 128), (unsigned)(B * Hkv));
  dim3 gq((unsigned)ceil_div(Sq, 128), (unsigned)(B * Hq));
#define QH_BWD(T, DPV)                                                                                              \
  do {                                                                                                              \
    fa_bwd_prep_kernel<T><<<(unsigned)ceil_div(prow, 16), 256, 0, st>>>((const T*)o, (const T*)dout, lse, delta,   \
                                                                        lse2, prow, (int)Sq, sqp, (int)D);          \
    if (Sk > 0 && DPV == 128) {                                                                                     \
      const int rc8 = dkdv8_lds_ready<T>();                                                                         \
      if (rc8) return rc8;                                                                                          \
      fa_bwd_dkdv8_kernel<T, 128><<<gkv, 512, kDkdv8Lds, st>>>(                                                     \
          (const T*)q, sqb, sqh, sqs, (const T*)k, skb, skh, sks, (const T*)v, svb, svh, svs, (const T*)dout, lse2,  \
          delta, sqp, (T*)dk, (T*)dv, (int)Hq, (int)Hkv, groups, (int)Sq, (int)Sk, (int)D, sl2, scale, causal,       \
          (int)causal_offset);                                                                                      \
    } else if (Sk > 0)                                                                                              \
      fa_bwd_dkdv_kernel<T, DPV><<<gkv, 256, 0, st>>>((const T*)q, sqb, sqh, sqs, (const T*)k, skb, skh, sks,       \
                                                      (const T*)v, svb, svh, svs, (const T*)dout, lse2, delta, sqp,   \
                                                      (T*)dk,                                                         \
                                                      (T*)dv, (int)Hq, (int)Hkv, groups, (int)Sq, (int)Sk, (int)D,  \
                                                      sl2, scale, causal, (int)causal_offset);                      \
    fa_bwd_dq_kernel<T, DPV><<<gq, 256, 0, st>>>((const T*)q, sqb, sqh, sqs, (const T*)k, skb, skh, sks,            \
                                                 (const T*)v, svb, svh, svs, (const T*)dout, lse2, delta, sqp,      \
                                                 (T*)dq,                                                            \
                                                 (int)Hq, groups, (int)Sq, (int)Sk, (int)D, sl2, scale, causal,     \
                                                 (int)causal_offset);                                               \
  } while (0)
#define QH_BWD_D(T) \
  if (dp == 32) QH_BWD(T, 32); else if (dp == 64) QH_BWD(T, 64); else QH_BWD(T, 128);
  if (dtype == QH_BF16) { QH_BWD_D(bf16_t) } else { QH_BWD_D(f16_t) }
#undef QH_BWD_D
#undef QH_BWD
  QH_CHECK_LAUNCH("qh_flash_bwd");
  return QH_OK;
}

// The workgroup kernel (head dim 128, at least kDecodeWgMinSeqs (sequence,
// kv-head) pairs) combines its partials in LDS and needs no workspace; the
// split kernel keeps [B*Hq, splits, D+2] fp32 partials.
static bool decode_on_chip(int64_t B, int64_t Hkv, int dp) { return dp == 128 && B * Hkv >= kDecodeWgMinSeqs; }

extern "C" int64_t qh_flash_decode_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sk, int64_t D) {
  const int dp = pick_dp(D);
  if (!dp || Hkv <= 0 || B <= 0 || decode_on_chip(B, Hkv, dp)) return 0;
  const int ns = decode_splits(B, Hkv, Sk);
  return B * Hq * ns * (dp + 2) * 4;
}

extern "C" int qh_flash_decode(const void* q, int64_t sqb, int64_t sqh, const void* k, int64_t skb, int64_t skh,
                               int64_t sks, const void* v, int64_t svb, int64_t svh, int64_t svs, void* o, float* lse,
                               const int32_t* seqlens, void* ws, int64_t ws_bytes, int64_t B, int64_t Hq, int64_t Hkv,
                               int64_t Sk, int64_t D, float scale, int dtype, void* stream) {
  QH_CHECK_ARG(B >= 0 && Hq > 0 && Hkv > 0 && Sk >= 0, "qh_flash_decode: bad shape");
  QH_CHECK_ARG(Hq % Hkv == 0, "qh_flash_decode: Hq not a multiple of Hkv");
  const int dp = pick_dp(D);
  QH_CHECK_ARG(dp && D % 8 == 0, "qh_flash_decode: head dim must be a multiple of 8 and <= 128");
  QH_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v), "qh_flash_decode: pointers must be 16-byte aligned");
  QH_CHECK_ARG(sqb % 8 == 0 && sqh % 8 == 0 && skb % 8 == 0 && skh % 8 == 0 && sks % 8 == 0 && svb % 8 == 0 &&
                   svh % 8 == 0 && svs % 8 == 0,
               "qh_flash_decode: strides must be multiples of 8 elements");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_flash_decode: bf16/f16 only");
  const int groups = (int)(Hq / Hkv);
  QH_CHECK_ARG(groups == 1 || groups == 2 || groups == 4 || groups == 8, "qh_flash_decode: group size %d unsupported",
               groups);
  QH_CHECK_ARG(B * Hkv < 65536, "qh_flash_decode: too many sequences");
  QH_CHECK_ARG(sks < (1 << 24) && svs < (1 << 24), "qh_flash_decode: key/value row stride too large");
  if (B == 0) return QH_OK;
  const int64_t need = qh_flash_decode_workspace(B, Hq, Hkv, Sk, D);
  if (ws_bytes < need) {
    qh::set_error("qh_flash_decode: workspace %lld < %lld", (long long)ws_bytes, (long long)need);
    return QH_E_WORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  const float sl2 = scale * kLog2e;
  if (decode_on_chip(B, Hkv, dp)) {
    // many sequences: one workgroup per (b, kv-head), combined in LDS
#define QH_WG(T, GV)                                                                                              \
  fa_decode_wg_kernel<T, 128, GV><<<(unsigned)(B * Hkv), 256, 0, st>>>(                                         \
      (const T*)q, sqb, sqh, (const T*)k, skb, skh, sks, (const T*)v, svb, svh, svs, (T*)o, lse, seqlens, (int)Hkv, \
      (int)Sk, (int)D, sl2, DecodePrepArgs<T, float>{})
#define QH_WG_G(T) \
  if (groups == 1) QH_WG(T, 1); else if (groups == 2) QH_WG(T, 2); else if (groups == 4) QH_WG(T, 4); else QH_WG(T, 8);
    if (dtype == QH_BF16) { QH_WG_G(bf16_t) } else { QH_WG_G(f16_t) }
#undef QH_WG_G
#undef QH_WG
    QH_CHECK_LAUNCH("qh_flash_decode");
    return QH_OK;
  }
  const int ns = decode_splits(B, Hkv, Sk);
  float* ws_o = (float*)ws;
  float* ws_ml = ws_o + B * Hq * ns * dp;
#define QH_DEC(T, DPV, GV)                                                                                   \
  launch_decode<T, DPV, GV>(q, sqb, sqh, k, skb, skh, sks, v, svb, svh, svs, ws_o, ws_ml, seqlens, (int)B,  \
                            (int)Hkv, (int)Sk, (int)D, ns, sl2, st)
#define QH_DEC_G(T, DPV) \
  if (groups == 1) QH_DEC(T, DPV, 1); else if (groups == 2) QH_DEC(T, DPV, 2); else if (groups == 4) QH_DEC(T, DPV, 4); else QH_DEC(T, DPV, 8);
#define QH_DEC_D(T) \
  if (dp == 32) { QH_DEC_G(T, 32) } else if (dp == 64) { QH_DEC_G(T, 64) } else { QH_DEC_G(T, 128) }
  const int rows = (int)(B * Hq);
  if (dtype == QH_BF16) {
    QH_DEC_D(bf16_t)
    if (dp == 32) fa_decode_combine<bf16_t, 32><<<(unsigned)ceil_div(rows, 8), 256, 0, st>>>(ws_o, ws_ml, (bf16_t*)o, lse, rows, ns, (int)D);
    else if (dp == 64) fa_decode_combine<bf16_t, 64><<<(unsigned)ceil_div(rows, 4), 256, 0, st>>>(ws_o, ws_ml, (bf16_t*)o, lse, rows, ns, (int)D);
    else fa_decode_combine<bf16_t, 128><<<(unsigned)ceil_div(rows, 2), 256, 0, st>>>(ws_o, ws_ml, (bf16_t*)o, lse, rows, ns, (int)D);
  } else {
    QH_DEC_D(f16_t)
    if (dp == 32) fa_decode_combine<f16_t, 32><<<(unsigned)ceil_div(rows, 8), 256, 0, st>>>(ws_o, ws_ml, (f16_t*)o, lse, rows, ns, (int)D);
    else if (dp == 64) fa_decode_combine<f16_t, 64><<<(unsigned)ceil_div(rows, 4), 256, 0, st>>>(ws_o, ws_ml, (f16_t*)o, lse, rows, ns, (int)D);
    else fa_decode_combine<f16_t, 128><<<(unsigned)ceil_div(rows, 2), 256, 0, st>>>(ws_o, ws_ml, (f16_t*)o, lse, rows, ns, (int)D);
  }
#undef QH_DEC_D
#undef QH_DEC_G
#undef QH_DEC
  QH_CHECK_LAUNCH("qh_flash_decode");
  return QH_OK;
}

// ---------------------------------------------------------------------------
// Allocation-free decode: qh_flash_decode with its split partials in a
// file-scope device array instead of a caller workspace, for callers that
// cannot allocate (code under HIP graph capture, serving loops that forbid
// hipMalloc). Each GPU holds its own copy of the array from the first call on
// it until the process ends. The array keeps the last call's contents; nothing
// needs clearing, because every split of a call writes all of its partials
// (m, l and o, also for a split with no keys) before the combine reads them.
// Calls that overlap on one GPU (two streams, or two host threads) share the
// array and race.
constexpr int64_t kDecodeScratchBytes = 16ll << 20;
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

namespace {
constexpr int kScratchMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchMaxDevices] = {};

// Device address of `scratch` on the device of `st` (hipGetSymbolAddress once
// per device, with that device current). Host code uses only this address:
// the array's name on the host side is a stand-in, not a device pointer.
int decode_scratch(hipStream_t st, void** out) {
  int cur = 0;
  QH_CHECK_HIP(hipGetDevice(&cur), "qh_flash_decode_noalloc: hipGetDevice");
  int dev = cur;
  if (st != nullptr) QH_CHECK_HIP(hipStreamGetDevice(st, &dev), "qh_flash_decode_noalloc: hipStreamGetDevice");
  QH_CHECK_ARG(dev >= 0 && dev < kScratchMaxDevices, "qh_flash_decode_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    if (dev != cur) QH_CHECK_HIP(hipSetDevice(dev), "qh_flash_decode_noalloc: hipSetDevice");
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) QH_CHECK_HIP(hipSetDevice(cur), "qh_flash_decode_noalloc: hipSetDevice");
    if (e != hipSuccess || p == nullptr) {
      qh::set_error("qh_flash_decode_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                    hipGetErrorString(e));
      return QH_E_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return QH_OK;
}
}  // namespace

extern "C" int qh_flash_decode_noalloc(const void* q, int64_t sqb, int64_t sqh, const void* k, int64_t skb,
                                       int64_t skh, int64_t sks, const void* v, int64_t svb, int64_t svh,
                                       int64_t svs, void* o, float* lse, const int32_t* seqlens, int64_t B,
                                       int64_t Hq, int64_t Hkv, int64_t Sk, int64_t D, float scale, int dtype,
                                       void* stream) {
  QH_CHECK_ARG(B >= 0 && Hq > 0 && Hkv > 0 && Sk >= 0, "qh_flash_decode_noalloc: bad shape");
  // 0 for the workgroup kernel (head dim 128, many sequences), which keeps its partials on chip
  const int64_t need = qh_flash_decode_workspace(B, Hq, Hkv, Sk, D);
  if (need > kDecodeScratchBytes) {
    qh::set_error("qh_flash_decode_noalloc: this shape needs %lld bytes of split partials, more than the %lld-byte "
                  "static scratch; use qh_flash_decode with a workspace",
                  (long long)need, (long long)kDecodeScratchBytes);
    return QH_E_WORKSPACE;
  }
  void* ws = nullptr;
  if (need > 0) {
    const int rc = decode_scratch((hipStream_t)stream, &ws);
    if (rc != QH_OK) return rc;
  }
  return qh_flash_decode(q, sqb, sqh, k, skb, skh, sks, v, svb, svh, svs, o, lse, seqlens, ws, need, B, Hq, Hkv, Sk,
                         D, scale, dtype, stream);
}

// Keys a few workgroups stream fast enough on their own: short caches take the
// one-workgroup-per-(sequence, kv-head) kernel whatever the batch.
constexpr int64_t kDecodeWgShortKeys = 512;

extern "C" int64_t qh_flash_decode_prepare_ok(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sk, int64_t D) {
  if (B <= 0 || Hkv <= 0 || Hq % Hkv != 0 || D != 128 || Sk < 0) return 0;
  const int64_t g = Hq / Hkv;
  return (g == 1 || g == 2 || g == 4 || g == 8) && (B * Hkv >= kDecodeWgMinSeqs || Sk <= kDecodeWgShortKeys) &&
                 B * Hkv < 65536
             ? 1
             : 0;
}

extern "C" int qh_flash_decode_prepare(const void* q, int64_t sq, const void* k, int64_t sk, const void* v, int64_t sv,
                                       const void* qw, const void* kw, float eps, int one_plus, const void* cos,
                                       const void* sin, int64_t scb, int64_t cos_batch, int64_t rot, void* k_cache,
                                       int64_t kcb, int64_t kch, int64_t kcs, void* v_cache, int64_t vcb, int64_t vch,
                                       int64_t vcs, int64_t cap, const int64_t* positions, void* o, float* lse,
                                       const int32_t* seqlens, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sk,
                                       int64_t D, float scale, int dtype, int wdtype, int cdtype, void* stream) {
  QH_CHECK_ARG(qh_flash_decode_prepare_ok(B, Hq, Hkv, Sk, D), "qh_flash_decode_prepare: shape not served (B=%lld "
               "Hq=%lld Hkv=%lld Sk=%lld D=%lld; see qh_flash_decode_prepare_ok)", (long long)B, (long long)Hq,
               (long long)Hkv, (long long)Sk, (long long)D);
  QH_CHECK_ARG(Sk >= 0 && Sk <= cap && cap < (1ll << 31), "qh_flash_decode_prepare: need 0 <= Sk <= cap < 2^31");
  const int64_t half = rot / 2;
  QH_CHECK_ARG(rot >= 16 && rot <= D && rot % 16 == 0 && ((half / 8) & (half / 8 - 1)) == 0,
               "qh_flash_decode_prepare: rotary dim %lld must be 16 * 2^k <= D", (long long)rot);
  QH_CHECK_ARG(cos_batch == 1 || cos_batch == B, "qh_flash_decode_prepare: cos/sin batch must be 1 or B");
  QH_CHECK_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o) && aligned16(k_cache) &&
                   aligned16(v_cache),
               "qh_flash_decode_prepare: pointers must be 16-byte aligned");
  QH_CHECK_ARG(sq % 8 == 0 && sk % 8 == 0 && sv % 8 == 0 && kcb % 8 == 0 && kch % 8 == 0 && kcs % 8 == 0 &&
                   vcb % 8 == 0 && vch % 8 == 0 && vcs % 8 == 0,
               "qh_flash_decode_prepare: strides must be multiples of 8 elements");
  QH_CHECK_ARG(kcs < (1 << 24) && vcs < (1 << 24), "qh_flash_decode_prepare: key/value row stride too large");
  QH_CHECK_ARG(dtype == QH_BF16 || dtype == QH_F16, "qh_flash_decode_prepare: bf16/f16 only");
  QH_CHECK_ARG(wdtype == QH_F32 || wdtype == dtype, "qh_flash_decode_prepare: norm weights must be fp32 or the dtype");
  // cos/sin in the activation dtype: every product of the norm and the rotation is then a product of
  // two 16-bit values, exact in fp32, so the result cannot depend on how the compiler contracts
  // multiply-adds and equals qh_attn_prepare's bit for bit.
  QH_CHECK_ARG(cdtype == dtype, "qh_flash_decode_prepare: cos/sin must have the activation dtype");
  QH_CHECK_ARG(aligned16(qw) && aligned16(kw) && aligned16(cos) && aligned16(sin) && scb % 8 == 0,
               "qh_flash_decode_prepare: norm weights and cos/sin must be 16-byte aligned (batch stride multiple of 8)");
  hipStream_t st = (hipStream_t)stream;
  const float sl2 = scale * kLog2e;
  const int groups = (int)(Hq / Hkv);
#define QH_WGP(T, C, GV)                                                                                           \
  {                                                                                                                \
    DecodePrepArgs<T, C> pa{(const T*)q, (const T*)k, (const T*)v, sq, sk, sv, qw, kw, wdtype, eps,               \
                            one_plus ? 1.f : 0.f, (const C*)cos, (const C*)sin, scb, (int)cos_batch, (int)half,    \
                            (int)rot, positions, cap};                                                            \
    if (B * Hkv >= kDecodeWgMinSeqs)                                                                              \
      fa_decode_wg_kernel<T, 128, GV, true, C><<<(unsigned)(B * Hkv), 256, 0, st>>>(                             \
          (const T*)o, 0, 0, (const T*)k_cache, kcb, kch, kcs, (const T*)v_cache, vcb, vch, vcs, (T*)o, lse,      \
          seqlens, (int)Hkv, (int)Sk, (int)D, sl2, pa);                                                           \
    else if (GV <= 4 && Sk > 4 * 32)                                                                               \
      fa_decode_wg_kernel<T, 128, GV, true, C, false, (GV <= 4 ? 8 : 4)><<<(unsigned)(B * Hkv), 64 * (GV <= 4 ? 8 : 4), 0, st>>>( \
          (const T*)o, 0, 0, (const T*)k_cache, kcb, kch, kcs, (const T*)v_cache, vcb, vch, vcs, (T*)o, lse,      \
          seqlens, (int)Hkv, (int)Sk, (int)D, sl2, pa);                                                           \
    else                                                                                                           \
      fa_decode_wg_kernel<T, 128, GV, true, C, false><<<(unsigned)(B * Hkv), 256, 0, st>>>(                      \
          (const T*)o, 0, 0, (const T*)k_cache, kcb, kch, kcs, (const T*)v_cache, vcb, vch, vcs, (T*)o, lse,      \
          seqlens, (int)Hkv, (int)Sk, (int)D, sl2, pa);                                                           \
  }
#define QH_WGP_G(T, C) \
  if (groups == 1) QH_WGP(T, C, 1) else if (groups == 2) QH_WGP(T, C, 2) else if (groups == 4) QH_WGP(T, C, 4) else QH_WGP(T, C, 8)
  if (dtype == QH_BF16) {
    QH_WGP_G(bf16_t, bf16_t)
  } else {
    QH_WGP_G(f16_t, f16_t)
  }
#undef QH_WGP_G
#undef QH_WGP
  QH_CHECK_LAUNCH("qh_flash_decode_prepare");
  return QH_OK;
}
