/*
 * qwen_hip.h — C ABI of the MI355X (gfx950) operator library `libqwen_hip.so`.
 *
 * Every entry point:
 *   - takes plain device pointers, int64 sizes/strides (in elements), a dtype
 *     code and a hipStream_t passed as `void*` (the caller's current stream);
 *   - enqueues work on that stream and never allocates device memory; buffers
 *     beyond inputs and outputs come in as a caller-allocated `ws` workspace
 *     whose size is given by the matching `*_workspace` query;
 *   - returns QH_OK (0) or a QH_E_* code; qh_last_error() then holds a
 *     thread-local message.
 *
 * Each declaration cites the reference (luozoupi/Qwen-Triton) interface it
 * replaces as `path:line`.
 */
#ifndef QWEN_HIP_H_
#define QWEN_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { QH_F32 = 0, QH_F16 = 1, QH_BF16 = 2 };
enum { QH_OK = 0, QH_E_ARG = 1, QH_E_DTYPE = 2, QH_E_HIP = 3, QH_E_WORKSPACE = 4 };

/* ---- library ------------------------------------------------------------ */
const char* qh_last_error(void);
const char* qh_version(void);
/* Zero `nbytes` of device memory with a kernel (graph-capture safe). */
int qh_zero(void* ptr, int64_t nbytes, void* stream);

/* ---- elementwise -------------------------------------------------------- */
/* dst[i] = round(src[i] * scale[0]) in dtype (fp32 src 16-byte aligned, scale a
 * device pointer). No counterpart in the reference: it applies the upstream
 * gradient of the fused LM head + cross-entropy (known only in the backward)
 * to the gradients the forward formed unscaled. */
int qh_scale_cast(const float* src, void* dst, int64_t n, const float* scale, int dtype, void* stream);
/* out = x + r over n contiguous elements.
 * Replaces qwen_triton/kernels/residual_add.py:50-60 (_residual_add_kernel), :86-101. */
int qh_add(const void* x, const void* r, void* out, int64_t n, int dtype, void* stream);

/* out = silu(gate) * up, fp32 math, one rounding.
 * Replaces qwen_triton/kernels/swiglu.py:84-92 (_silu_mul_kernel), :175-190. */
int qh_silu_mul_fwd(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream);
/* dgate = g*u*s*(1+gate*(1-s)), dup = g*gate*s with s = sigmoid(gate).
 * Replaces qwen_triton/kernels/swiglu.py:106-132 (_silu_mul_backward_kernel), :39-51. */
int qh_silu_mul_bwd(const void* gate, const void* up, const void* gout, void* dgate, void* dup,
                    int64_t n, int dtype, void* stream);

/* out = x * sigmoid(gate).
 * Replaces qwen_triton/kernels/sigmoid_mul.py:66-83 (_sigmoid_mul_kernel), :180-195. */
int qh_sigmoid_mul_fwd(const void* x, const void* gate, void* out, int64_t n, int dtype, void* stream);
/* dx = g*s, dgate = g*x*s*(1-s).
 * Replaces qwen_triton/kernels/sigmoid_mul.py:97-120 (_sigmoid_mul_backward_kernel), :39-50. */
int qh_sigmoid_mul_bwd(const void* x, const void* gate, const void* gout, void* dx, void* dgate,
                       int64_t n, int dtype, void* stream);

/* ---- RMSNorm ------------------------------------------------------------ */
/* y = x * rsqrt(mean(x^2) + eps) * (w or 1+w), rows x cols contiguous, fp32 math.
 * `wdtype` is the weight's dtype. Replaces qwen_triton/kernels/rmsnorm.py:101-133, :64-82. */
int qh_rmsnorm_fwd(const void* x, const void* w, void* y, int64_t rows, int64_t cols, float eps,
                   int one_plus, int dtype, int wdtype, void* stream);
/* sum = x + r (rounded to the dtype) and y = RMSNorm(sum) * (w or 1 + w) in
 * one pass over rows x cols; both outputs equal qh_add followed by
 * qh_rmsnorm_fwd. bf16/f16. Replaces, fused, the residual add and the
 * following norm of qwen_triton/models/core.py:95-153 (QwenDecoderLayer:
 * residual_add, qwen_triton/kernels/residual_add.py:86-101, then rmsnorm,
 * qwen_triton/kernels/rmsnorm.py:101-196). */
int qh_add_rmsnorm(const void* x, const void* r, const void* w, void* sum, void* y, int64_t rows, int64_t cols,
                   float eps, int one_plus, int dtype, int wdtype, void* stream);
/* Workspace bytes for qh_rmsnorm_bwd (deterministic two-stage dW). */
int64_t qh_rmsnorm_bwd_workspace(int64_t rows, int64_t cols, int dtype);
/* gx (dtype) and gw (wdtype, summed over rows in a fixed order, no atomics).
 * Replaces qwen_triton/kernels/rmsnorm.py:148-196 (_rmsnorm_backward_kernel), :213-240. */
int qh_rmsnorm_bwd(const void* x, const void* w, const void* gy, void* gx, void* gw, void* ws,
                   int64_t ws_bytes, int64_t rows, int64_t cols, float eps, int one_plus, int dtype,
                   int wdtype, void* stream);

/* ---- RoPE --------------------------------------------------------------- */
/* Rotate-half RoPE of x[B,H,S,D] (any strides) into contiguous out[B,H,S,D]:
 * for d < rot/2: o[d] = x[d]c - x[d+h]s, o[d+h] = x[d+h]c + x[d]s with c,s =
 * cos/sin[b', s, d] (only the first rot/2 entries are read); dims >= rot are
 * copied. cos/sin are [cos_batch, S, >=rot/2] with strides (scb, scs, scd);
 * cos_batch == 1 broadcasts over B. neg_sin != 0 uses -sin (the exact
 * transpose, i.e. the backward).
 * Replaces qwen_triton/kernels/rope.py:78-120 (_rope_tensor_kernel), :131-162, :165-203 and
 * qwen_triton/csrc/rope_op_kernel.cu:12-39 (rope_tensor_forward_kernel). */
int qh_rope(const void* x, int64_t sxb, int64_t sxh, int64_t sxs, int64_t sxd, const void* cos,
            const void* sin, int64_t scb, int64_t scs, int64_t scd, int64_t cos_batch, void* out,
            int64_t B, int64_t H, int64_t S, int64_t D, int64_t rot, int neg_sin, int dtype,
            int cdtype, void* stream);

/* ---- KV cache ----------------------------------------------------------- */
/* cache[b,h,pos[s],:] = values[b,h,s,:] (strided). Positions outside [0,cap)
 * are skipped. Replaces qwen_triton/kernels/cache.py:72-98 (_write_kv_kernel), :142-181. */
int qh_kv_write(void* cache, int64_t scb, int64_t sch, int64_t scs, int64_t scd, const void* values,
                int64_t svb, int64_t svh, int64_t svs, int64_t svd, const int64_t* positions,
                int64_t B, int64_t H, int64_t S, int64_t D, int64_t cap, int dtype, void* stream);
/* out[B,H,So+Sn,D] = cat(prefix[B,H,So,D], suffix[B,H,Sn,D]) along S (contiguous).
 * Replaces qwen_triton/kernels/cache.py:37-69 (_append_kv_kernel), :101-139. */
int qh_kv_append(const void* prefix, const void* suffix, void* out, int64_t B, int64_t H,
                 int64_t s_old, int64_t s_new, int64_t D, int dtype, void* stream);

/* ---- embedding ---------------------------------------------------------- */
/* out[t,:] = w[ids[t],:]; rows of ids outside [0,V) produce zeros.
 * Replaces qwen_triton/kernels/embedding.py:50-60 (_embedding_kernel), :97-112. */
int qh_embedding_fwd(const int64_t* ids, const void* w, int64_t stride_w, void* out, int64_t n_tokens,
                     int64_t V, int64_t Hd, int dtype, void* stream);
/* Workspace bytes of qh_embedding_bwd: id sort space for n_tokens. */
int64_t qh_embedding_bwd_workspace(int64_t n_tokens, int64_t V);
/* gw[v,:] = sum_{t: ids[t]==v} gout[t,:] (fp32 sum in token order, stored as
 * wdtype), gw[padding_idx] = 0; rows never referenced are zero; ids outside
 * [0, V) contribute nothing. Deterministic: every row is written once. Up to
 * 32768 tokens (with Hd a multiple of 8 and 16-byte aligned buffers) in one
 * launch without a sort: workgroup g of G owns the rows v = g mod G and keeps
 * the position-ordered list of its hits in LDS; above that, a radix sort by id
 * first. The workspace is the sort's (unused by the single launch).
 * Replaces qwen_triton/kernels/embedding.py:78-94 (_embedding_backward_kernel), :124-145. */
int qh_embedding_bwd(const int64_t* ids, const void* gout, void* gw, void* ws, int64_t ws_bytes,
                     int64_t n_tokens, int64_t V, int64_t Hd, int64_t padding_idx, int gdtype,
                     int wdtype, void* stream);

/* ---- softmax ------------------------------------------------------------ */
/* Row softmax over the last dim. Replaces qwen_triton/kernels/softmax.py:56-88, :130-135. */
int qh_softmax_fwd(const void* x, void* y, int64_t rows, int64_t cols, int dtype, void* stream);
/* gx = y * (gy - sum(gy*y)). Replaces qwen_triton/kernels/softmax.py:100-127. */
int qh_softmax_bwd(const void* y, const void* gy, void* gx, int64_t rows, int64_t cols, int dtype,
                   void* stream);

/* ---- cross-entropy ------------------------------------------------------ */
/* Per row: lse = logsumexp(logits[row,:V]) (single-pass online), loss_row =
 * lse - logits[row, t]; rows with t == ignore_index give 0; rows with t
 * outside [0,V) give NaN. *loss_out = sum(loss_row) / max(1, n_valid), *nvalid_out
 * = n_valid (fp32, fixed-order sum). Replaces qwen_triton/kernels/cross_entropy.py:55-95, :142-161. */
int qh_ce_fwd(const void* logits, int64_t stride, const int64_t* targets, float* lse, float* loss_rows,
              float* loss_out, float* nvalid_out, int64_t N, int64_t V, int64_t ignore_index, int dtype,
              void* stream);
/* glogits = (softmax - onehot(t)) * grad_loss[0] / max(1, nvalid[0]); ignored rows 0.
 * grad_loss and nvalid are device pointers (no host sync). glogits may be logits
 * itself (in place, gstride == stride).
 * Replaces qwen_triton/kernels/cross_entropy.py:108-139, :180-192. */
int qh_ce_bwd(const void* logits, int64_t stride, const int64_t* targets, const float* lse,
              const float* grad_loss, const float* nvalid, void* glogits, int64_t gstride, int64_t N,
              int64_t V, int64_t ignore_index, int dtype, void* stream);

/* ---- Greedy decoding --------------------------------------------------- */
/* One greedy step on device state: per row b of logits [B, V] (row stride ld) the
 * argmax (torch.argmax: NaN is the largest value, ties -> lowest column), then
 * ids[b] = tokens[b * ldt + col] = argmax (the token is stored only when
 * 0 <= col < ncols), seqlens[b] += 1, col += 1, positions += 1. Every output
 * pointer may be NULL. B <= 64; ws of at least qh_greedy_step_workspace(B, V)
 * bytes. Two launches, no host synchronisation (graph-capturable).
 * Replaces the argmax and bookkeeping of qwen_triton/models/core.py:405-408. */
int64_t qh_greedy_step_workspace(int64_t B, int64_t V);
int qh_greedy_step(const void* logits, int64_t ld, int64_t B, int64_t V, int64_t* ids, int64_t* tokens,
                   int64_t ldt, int64_t ncols, int64_t* col, int64_t* positions, int32_t* seqlens, void* ws,
                   int64_t ws_bytes, int dtype, void* stream);

/* ---- MoE routing primitives --------------------------------------------- */
/* Top-k per row, values sorted descending, ties -> lowest index.
 * Replaces qwen_triton/kernels/moe_routing.py:45-144 (_topk_k2_kernel, _topk_general_kernel). */
int qh_topk(const void* x, void* vals, int64_t* idx, int64_t N, int64_t C, int64_t k, int dtype,
            void* stream);
/* out[n,c] = (idx[n] == c) as int64. Replaces qwen_triton/kernels/moe_routing.py:175-200. */
int qh_one_hot(const int64_t* idx, int64_t* out, int64_t N, int64_t C, void* stream);
int64_t qh_index_add_workspace(int64_t n_src);
/* target[index[r],:] += src[r,:] (rows with index outside [0,n_target) are
 * skipped). Each touched row gets target + (fp32 sum of its sources in source
 * order), rounded once; deterministic.
 * Replaces qwen_triton/kernels/moe_routing.py:218-255 (_index_add_kernel, _triton_index_add). */
int qh_index_add(void* target, int64_t stride_t, const void* src, int64_t stride_s, const int64_t* index,
                 int64_t n_src, int64_t n_target, int64_t D, void* ws, int64_t ws_bytes, int dtype,
                 void* stream);

/* ---- MoE experts: dispatch, grouped GEMM, combine ------------------------ */
/* Sort/segment dispatch of the n_tokens*top_k routed (token, slot) pairs by
 * expert (stable radix sort; selected is int64 [n_tokens, top_k], ids outside
 * [0, n_experts) are dropped). Outputs, for the R = n_tokens*top_k sorted rows:
 * rows[r] (token), wsorted[r] (routing weight, dtype), inv[token*top_k + slot]
 * = r; and seg_off[e] (first row of expert e, e = 0..n_experts) and
 * tile_off[e] (first M-tile of expert e for tiles of tile_m rows, prefix sum).
 * Replaces the expert_mask / nonzero / where bookkeeping of
 * qwen_triton/modules/moe.py:45-51 (triton_one_hot, qwen_triton/kernels/moe_routing.py:175-200). */
int64_t qh_moe_dispatch_workspace(int64_t n_tokens, int64_t top_k, int64_t n_experts);
int qh_moe_dispatch(const int64_t* selected, const void* weights, int64_t n_tokens, int64_t top_k,
                    int64_t n_experts, int64_t tile_m, void* ws, int64_t ws_bytes, int32_t* rows, void* wsorted,
                    int32_t* inv, int32_t* seg_off, int32_t* tile_off, int dtype, void* stream);
/* Grouped expert GEMM over the dispatch segments (tile_off for tile_m = 128).
 * B_table is a DEVICE array of weight pointers ([out, in] row-major, row stride
 * ldb): mode 0 (gated): 2*E entries (gate_e, up_e), A = X gathered through
 * rows[], C[r] = silu(X[rows[r]] Wg^T) * (X[rows[r]] Wu^T), N = intermediate;
 * mode 1 (scaled): E entries, A rows contiguous, C[r] = (A[r] Wd^T) * wrow[r].
 * Each product is rounded to the dtype before the SiLU-mul / scaling, as the
 * reference's per-expert TritonLinear, silu_mul and multiply do.
 * Replaces the per-expert QwenMLP calls of qwen_triton/modules/moe.py:47-50
 * (qwen_triton/modules/mlp.py:19-22, kernels/matmul.py:130-155, kernels/swiglu.py:175-190). */
int qh_moe_gemm(int mode, const void* A, int64_t lda, const int32_t* rows, const void* const* B_table,
                int64_t ldb, void* C, int64_t ldc, const void* wrow, const int32_t* seg_off,
                const int32_t* tile_off, int64_t R, int64_t E, int64_t N, int64_t K, int dtype, void* stream);
/* out[t] = sum of the token's expert rows Y[inv[t*top_k + j]] in ascending
 * expert order, rounded to the dtype after every add (the reference's
 * per-expert index_add into zeros). With weights ([n_tokens, top_k], dtype),
 * row j contributes round(Y[.] * weights[t, j]) (the routing-weight multiply
 * of the expert output); weights may be NULL. Deterministic; out fully written.
 * Replaces qwen_triton/modules/moe.py:49-51 (the routing-weight multiply and
 * triton_index_add, kernels/moe_routing.py:322-343). */
int qh_moe_combine(const void* Y, int64_t ldy, const int32_t* inv, const int64_t* selected, const void* weights,
                   int64_t n_tokens, int64_t top_k, int64_t n_experts, void* out, int64_t H, int dtype, void* stream);
/* Xs[r] = X[rows[r]] for the R expert-sorted rows (the flat[tok] gather of
 * qwen_triton/modules/moe.py:48, done once for all experts). */
int qh_moe_gather(const void* X, int64_t ldx, const int32_t* rows, int64_t R, int64_t H, void* Xs, int64_t lds,
                  int dtype, void* stream);

/* ---- Grouped expert GEMMs on the 256x256 tile kernel (training path) -----
 * Rows are the expert-sorted dispatch rows; seg_off from qh_moe_dispatch and
 * tile_off from it with tile_m = 256. Weight tables are DEVICE arrays of
 * pointers to the experts' [out, in] row-major weights (row stride ldw);
 * gu_table holds 2E entries (gate_e, up_e), d_table E entries (down_e).
 * Together with qh_moe_gather, qh_moe_combine and qh_moe_scale_bwd these
 * replace the forward and the autograd backward of the per-expert loop of
 * qwen_triton/modules/moe.py:45-51 (QwenMLP = modules/mlp.py:19-22 over
 * TritonLinear, kernels/matmul.py:130-155, and silu_mul, kernels/swiglu.py). */
/* G = Xs Wg_e^T, U = Xs Wu_e^T (each rounded), H = round(silu(G) * U) per
 * expert segment; G and U (both or neither) may be NULL. I % 128 == 0.
 * rows == NULL: X holds the R sorted rows (Xs = X, e.g. from qh_moe_gather).
 * rows != NULL: X holds the tokens and sorted row r is X[rows[r]] (rows from
 * qh_moe_dispatch, each a valid row of X), gathered by the product itself. */
int qh_moe_up(const void* X, int64_t ldx, const int32_t* rows, int64_t R, int64_t K, const void* const* gu_table,
              int64_t ldw, int64_t I, const int32_t* seg_off, const int32_t* tile_off, int64_t E, void* G, void* U,
              void* H, int64_t ldo, int dtype, void* stream);
/* C = A Wd_e^T per segment, rounded; with wrow (per-row weights) C =
 * round(round(A Wd_e^T) * wrow[r]). C is written as 16-byte rows: N and ldc
 * multiples of 8, C 16-byte aligned (else QH_E_ARG). */
int qh_moe_down(const void* A, int64_t lda, int64_t R, int64_t K, const void* const* d_table, int64_t ldw, int64_t N,
                const int32_t* seg_off, const int32_t* tile_off, int64_t E, void* C, int64_t ldc, const void* wrow,
                int dtype, void* stream);
/* Gradient through the down projection and SiLU-mul: dH = round(dD Wd_e),
 * s = sigmoid(G): dG = round(dH U s (1 + G (1 - s))), dU = round(dH G s). */
int qh_moe_down_dgrad(const void* dD, int64_t ldd, int64_t R, int64_t K, const void* const* d_table, int64_t ldw,
                      int64_t I, const int32_t* seg_off, const int32_t* tile_off, int64_t E, const void* G,
                      const void* U, int64_t ldg, void* dG, void* dU, int64_t ldo, int dtype, void* stream);
/* dXs = dG Wg_e + dU Wu_e per segment (one fp32 accumulation, rounded once).
 * I % 64 == 0. */
int qh_moe_up_dgrad(const void* dG, const void* dU, int64_t ldg, int64_t R, int64_t I, const void* const* gu_table,
                    int64_t ldw, int64_t N, const int32_t* seg_off, const int32_t* tile_off, int64_t E, void* dX,
                    int64_t ldx, int dtype, void* stream);
/* Expert weight gradients: out_q + e*out_stride = A_q(rows of e)^T B(rows of e)
 * ([M, N], row stride ldo, rounded), for parts q < parts (1 or 2) sharing B:
 * gate/up: A = dG, dU, B = Xs; down: A = dD, B = H. Experts without rows get
 * zeros. */
int qh_moe_wgrad(int parts, const void* A0, const void* A1, int64_t lda, int64_t M, const void* B, int64_t ldb,
                 int64_t N, const int32_t* seg_off, int64_t E, void* out0, void* out1, int64_t ldo,
                 int64_t out_stride, int dtype, void* stream);
/* Backward of the routing-weight multiply, per token t and slot j (row p =
 * inv[t*top_k + j]): dD[p] = round(dout[t] * weights[t, j]) and
 * dw[t, j] = round(sum_c dout[t, c] * D[p, c]) (fp32, fixed order); slots with
 * an out-of-range expert get dw = 0. */
int qh_moe_scale_bwd(const void* dout, int64_t ldo, const void* D, int64_t ldd, const void* weights,
                     const int32_t* inv, const int64_t* selected, int64_t n_tokens, int64_t top_k, int64_t n_experts,
                     int64_t H, void* dD, int64_t ldg, void* dw, int dtype, void* stream);

/* ---- GEMM (Linear) ------------------------------------------------------ */
/* C[M,N] = A(M,K) . B(N,K)^T (+ bias[N]) with operand views
 *   A(m,k) = trans_a ? A[k*lda + m] : A[m*lda + k]
 *   B(n,k) = trans_b ? B[k*ldb + n] : B[n*ldb + k]
 * so forward x W^T (0,0), dX = dY W (0,1) and dW = dY^T X (1,1) need no copies.
 * bf16/f16 run on MFMA (32x32x16 tiles; 16x16x32 with a 16-way K split in one
 * workgroup for M <= 128) with fp32 accumulation; f32 runs on VALU.
 * bias has the input dtype; C has out_dtype.
 * Replaces qwen_triton/kernels/matmul.py:64-97 (_matmul_kernel), :100-111 (_bias_add_kernel),
 * :130-200 (forward/backward launchers incl. the per-call transposes at :140, :184). */
int qh_gemm(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
            const void* B, int64_t ldb, void* C, int64_t ldc, const void* bias, int dtype, int out_dtype,
            void* stream);
/* Workspace bytes with which qh_gemm_ws splits K for (M, N, K) (0: no split).
 * Products with few 256x256 output tiles and long K (weight gradients) are
 * computed as fp32 partials over K ranges, then summed in a fixed order. */
int64_t qh_gemm_workspace(int64_t M, int64_t N, int64_t K, int dtype);
/* qh_gemm with a workspace (ws may be NULL: then as qh_gemm). Same results
 * run to run; the split-K sum order differs from the unsplit product's. */
int qh_gemm_ws(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
               const void* B, int64_t ldb, void* C, int64_t ldc, const void* bias, int dtype, int out_dtype,
               void* ws, int64_t ws_bytes, void* stream);
/* Several decode-sized products sharing the activations, in one launch:
 * C_i[M, N_i] = A(M,K) . B_i(N_i,K)^T (+ bias_i) for i < count (<= 4), M <= 128,
 * all operands k-contiguous, C in the input dtype (bf16/f16). B, ldb, N, C,
 * ldc and bias are host arrays of count entries (bias may be NULL, or hold NULL
 * entries). Each product is computed exactly as qh_gemm would. gated = 1 (two
 * products of equal N, e.g. gate and up) writes C_0 = silu(C_gate) * C_up with
 * each product rounded to the dtype first, as qh_gemm twice followed by
 * qh_silu_mul_fwd would (C_1 is not written).
 * Replaces, fused, the separate TritonLinear calls of
 * qwen_triton/modules/attention.py:55-66 (q/k/v) and qwen_triton/modules/mlp.py:19-22
 * (gate/up, silu_mul), each via qwen_triton/kernels/matmul.py:130-155. */
int qh_gemm_multi(int64_t M, int64_t K, const void* A, int64_t lda, int count, const void* const* B,
                  const int64_t* ldb, const int64_t* N, void* const* C, const int64_t* ldc,
                  const void* const* bias, int gated, int dtype, void* stream);
/* qh_gemm_multi with two fusions of the decoder layer's inference chain:
 * - norm_w != NULL: A holds RMSNorm inputs h and the products are those of
 *   RMSNorm(h): operand round(h * (norm_w + one_plus)), each output row scaled
 *   by rsqrt(mean_k(h^2) + eps) (fp32, fixed order) after the sum over K. The
 *   single rounding of the normalised operand is taken before the row factor
 *   instead of after it (qh_rmsnorm_fwd then a product). norm_w [K] has the
 *   activation dtype (norm_wdtype == dtype), 16-byte aligned. Needs
 *   qh_gemm_multi_norm_fits(M, K, gated, count, N).
 * - residual (host array of count entries, or NULL; entries may be NULL):
 *   C_i = round(round(product_i) + R_i) with R_i [M, N_i] of row stride ldr[i],
 *   as qh_gemm followed by qh_add; not with gated.
 * Replaces, fused, the norms of qwen_triton/models/core.py:127 and :146 (via
 * qwen_triton/kernels/rmsnorm.py:101-196) with the projections that follow
 * them (qwen_triton/modules/attention.py:55-66, qwen_triton/modules/mlp.py:19-22),
 * and the residual adds of qwen_triton/models/core.py:144 and :152 (via
 * qwen_triton/kernels/residual_add.py:86-101) with the o_proj and down_proj
 * products before them (qwen_triton/modules/attention.py:128, mlp.py:22). */
int qh_gemm_multi_ex(int64_t M, int64_t K, const void* A, int64_t lda, int count, const void* const* B,
                     const int64_t* ldb, const int64_t* N, void* const* C, const int64_t* ldc,
                     const void* const* bias, const void* const* residual, const int64_t* ldr, int gated,
                     const void* norm_w, int norm_wdtype, float eps, int one_plus, int dtype, void* stream);
/* 1 when a qh_gemm_multi_ex launch of these shapes can take the norm prologue
 * (every workgroup holds all K columns of its rows in one load chunk), else 0.
 * No counterpart in the reference: a capability query for the fusion above. */
int64_t qh_gemm_multi_norm_fits(int64_t M, int64_t K, int gated, int count, const int64_t* N);
/* qh_gemm_multi_ex's norm fusion for weights that already carry the norm weight:
 * B_i[n][k] = round(W_i[n][k] * (norm_w[k] + one_plus)) (fp32 product, one
 * rounding to the dtype; prepared once per weight). A holds the RMSNorm inputs
 * h; each output row is scaled by rsqrt(mean_k(h^2) + eps) (fp32, fixed order)
 * after the sum over K, then bias. For M > 4 the results equal qh_gemm_multi_ex
 * with norm_w bit for bit; for M <= 4 the normalised operand is rounded on the
 * weight side too (qh_gemm_multi_ex rounds round(h * w) there). Any shape
 * qh_gemm_multi takes (no qh_gemm_multi_norm_fits condition).
 * Replaces, fused, the same reference calls as qh_gemm_multi_ex's norm fusion
 * (qwen_triton/models/core.py:127 and :146 with the projections after them);
 * the folded-weight form has no counterpart in the reference. */
int qh_gemm_multi_rms(int64_t M, int64_t K, const void* A, int64_t lda, int count, const void* const* B,
                      const int64_t* ldb, const int64_t* N, void* const* C, const int64_t* ldc,
                      const void* const* bias, int gated, float eps, int dtype, void* stream);
/* out[n] = sum_m X[m*ldx + n] in a fixed order (bias gradient).
 * Replaces qwen_triton/kernels/matmul.py:114-127 (_row_sum_kernel). */
int qh_colsum(const void* X, int64_t ldx, int64_t M, int64_t N, void* out, int dtype, int out_dtype,
              void* stream);

/* ---- gated delta rule (Qwen3-Next / Qwen3.5 linear attention) ------------ */
/* Whole-sequence recurrence per (b, head): with the fp32 state S [K, Vd]
 * (state_in, or zeros when NULL), for t = 0..S-1: S *= exp(g[b,t,h]);
 * d = (v_t - S^T k_t) * beta[b,t,h]; S += k_t d^T; out[b,t,h,:] = S^T q'_t
 * with q'_t = q_t * scale rounded to the dtype (output rounded to the dtype). q/k [B,S,H,K] share strides (sqb, sqs, sqh),
 * v [B,S,H,Vd] (svb, svs, svh), out (sob, sos, soh), all with unit last
 * stride; g and beta fp32 [B,S,H] with strides (sgb, sgs, sgh); state_out
 * (may be NULL) receives the final fp32 state [B,H,K,Vd] (contiguous, as
 * state_in). K <= 128. One launch for the whole sequence.
 * Replaces qwen_triton/kernels/linear_attention.py:54-101
 * (_gated_delta_rule_step_kernel, one launch per token) and the token loop of
 * :130-189 (gated_delta_rule_sequence). */
int qh_gated_delta_rule(const void* q, const void* k, int64_t sqb, int64_t sqs, int64_t sqh, const void* v,
                        int64_t svb, int64_t svs, int64_t svh, const float* g, const float* beta, int64_t sgb,
                        int64_t sgs, int64_t sgh, const float* state_in, float* state_out, void* out, int64_t sob,
                        int64_t sos, int64_t soh, int64_t B, int64_t S, int64_t H, int64_t K, int64_t Vd,
                        float scale, int dtype, void* stream);

/* ---- fused LM head + cross-entropy ---------------------------------------- */
/* The reference computes logits = TritonLinear(hidden) ([N, V], written to
 * memory) and then triton_cross_entropy(logits, targets) (README.md:370 of the
 * reference lists the fused form as its next step). These entry points produce
 * the same loss and gradients without any [N, V] tensor: the logits exist only
 * as GEMM tiles, rounded to the activation dtype as the unfused LM head rounds
 * them.
 * Replaces, fused, qwen_triton/kernels/matmul.py:130-200 (the LM head product of
 * qwen_triton/models/core.py:333, tied weights) with
 * qwen_triton/kernels/cross_entropy.py:55-202 (forward and backward). */
/* Workspace bytes of qh_lmce_fwd: per-row partials of every 256-column tile,
 * target logits and per-row losses. */
int64_t qh_lmce_workspace(int64_t N, int64_t V);
/* X [N, H] (row stride ldx), W [V, H] (row stride ldw), targets [N] int64.
 * lse[row] = logsumexp of the row's logits, loss_rows[row] (may be NULL) =
 * lse - logit[target] (0 for ignore_index rows, NaN for targets outside
 * [0, V)); *loss_out = sum / max(1, n_valid), *nvalid_out = n_valid (fp32,
 * fixed-order sums, as qh_ce_fwd). bf16/f16. */
int qh_lmce_fwd(const void* X, int64_t ldx, const void* W, int64_t ldw, const int64_t* targets, int64_t N,
                int64_t V, int64_t H, int64_t ignore_index, float* lse, float* loss_rows, float* loss_out,
                float* nvalid_out, void* ws, int64_t ws_bytes, int dtype, void* stream);
/* The fused LM head + cross-entropy with gradients, one block of rows at a
 * time, with no recomputed logits: Z = X W^T for a block of rows (the only
 * [rows, V] buffer), the row's logsumexp from per-64-column partials formed in
 * the same GEMM's epilogue, then the logit gradient formed in Z in place
 * (qh_ce_bwd) and multiplied into dX (these rows) and dW (accumulated over the
 * blocks, qh_gemm_acc). No counterpart in the reference; it replaces, fused,
 * the same calls as qh_lmce_fwd above, with gradients. */
/* Workspace bytes of qh_lmce_rows_fwd: per-64-column (max, sum of exp) partials. */
int64_t qh_lmce_rows_workspace(int64_t N, int64_t V);
/* Z [N, V] (row stride ldz) = X W^T rounded to the dtype; lse[row] and
 * loss_rows[row] = lse - logit[target] (0 for ignore_index rows, NaN for
 * targets outside [0, V)) as qh_lmce_fwd gives them. bf16/f16, V % 8 == 0. */
int qh_lmce_rows_fwd(const void* X, int64_t ldx, const void* W, int64_t ldw, const int64_t* targets, int64_t N,
                     int64_t V, int64_t H, int64_t ignore_index, void* Z, int64_t ldz, float* lse, float* loss_rows,
                     void* ws, int64_t ws_bytes, int dtype, void* stream);
/* *nvalid_out = number of targets != ignore_index (fp32, exact below 2^24). */
int qh_lmce_count(const int64_t* targets, int64_t N, int64_t ignore_index, float* nvalid_out, void* stream);
/* *loss_out = sum(loss_rows) / max(1, n_valid), *nvalid_out = n_valid (fixed-order
 * fp32 sums, as qh_ce_fwd's finish). */
int qh_lmce_finish(const float* loss_rows, const int64_t* targets, int64_t N, int64_t ignore_index,
                   float* loss_out, float* nvalid_out, void* stream);
/* C[M,N] += A(M,K) . B(N,K)^T with fp32 C and bf16/f16 operands in the operand
 * views of qh_gemm (256x256 tile kernel). No counterpart in the reference: the
 * fixed-order accumulation of the fused cross-entropy's weight gradient over
 * row blocks. */
int qh_gemm_acc(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, const void* B,
                int64_t ldb, float* C, int64_t ldc, int dtype, void* stream);

/* ---- fused attention input preparation (inference) ---------------------- */
/* One pass over the projected q/k/v rows of B*S tokens (token-major views
 * [B*S, H*D] with row strides sq, sk, sv): per-head RMSNorm of q and k with
 * weights qw, kw (dtype wdtype, +1 when one_plus), rotate-half RoPE of both
 * with cos/sin [cos_batch, S, rot] (strides scb, scs, unit last; only the first
 * rot/2 columns are read), q written to q_out [B,Hq,S,D] (contiguous), k and v
 * written into the caches at positions[s] (same positions for every batch row;
 * positions outside [0, cap) are skipped). Matches the unfused kernels exactly.
 * D <= 128, D % 8 == 0, rot = 16 * 2^k <= D.
 * Replaces, fused, the chain at qwen_triton/modules/attention.py:104-114
 * (q_norm/k_norm via qwen_triton/kernels/rmsnorm.py:101-196, apply_rope via
 * qwen_triton/kernels/rope.py:78-120, update_attention via
 * qwen_triton/kernels/cache.py:72-98). */
int qh_attn_prepare(const void* q, int64_t sq, const void* k, int64_t sk, const void* v, int64_t sv,
                    const void* qw, const void* kw, float eps, int one_plus, const void* cos, const void* sin,
                    int64_t scb, int64_t scs, int64_t cos_batch, int64_t rot, void* q_out, void* k_cache,
                    int64_t kcb, int64_t kch, int64_t kcs, void* v_cache, int64_t vcb, int64_t vch, int64_t vcs,
                    const int64_t* positions, int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int64_t D,
                    int64_t cap, int dtype, int wdtype, int cdtype, void* stream);

/* ---- flash attention ---------------------------------------------------- */
/* O = softmax(scale * Q K^T + causal mask) V, LSE = logsumexp per query (fp32,
 * natural log, [B,Hq,Sq]). q [B,Hq,Sq,D], k/v [B,Hkv,Sk,D] with the given
 * batch/head/seq strides (unit stride on D); o [B,Hq,Sq,D] with its own batch/head/
 * seq strides (sob, soh, sos; contiguous: Hq*Sq*D, Sq*D, D; [B,Sq,Hq*D] rows for the
 * output projection: Sq*Hq*D, D, Hq*D). GQA
 * maps q-head h to kv-head h/(Hq/Hkv). Causal: key j visible to query i iff
 * j <= i + causal_offset (0 = the reference's top-left alignment). bf16/f16
 * (D % 8 == 0, strides multiples of 8) or fp32 (fp32 matrix cores; D % 4 == 0,
 * strides multiples of 4), D <= 128. lse may be NULL.
 * Replaces qwen_triton/kernels/flash_attention.py:54-152 (_flash_attn_fwd_kernel), :280-314. */
int qh_flash_fwd(const void* q, int64_t sqb, int64_t sqh, int64_t sqs, const void* k, int64_t skb,
                 int64_t skh, int64_t sks, const void* v, int64_t svb, int64_t svh, int64_t svs, void* o,
                 int64_t sob, int64_t soh, int64_t sos, float* lse, int64_t B, int64_t Hq, int64_t Hkv,
                 int64_t Sq, int64_t Sk, int64_t D, float scale, int causal, int64_t causal_offset, int dtype,
                 void* stream);
/* qh_flash_fwd (bf16/f16 only) with the model's padding and sliding-window
 * masks applied in the kernel: key j is also hidden from query i when
 * window > 0 and j <= i + causal_offset - window, or when key_bits (may be
 * NULL; 8-byte aligned, bits_stride >= ceil(Sk / 64) words per batch row) has
 * bit j % 64 of word b * bits_stride + j / 64 clear. A query that sees no key
 * gets a zero row and LSE = -inf. Tiles with no visible key are skipped; with
 * Sq == 1 the q-heads of a kv-head share one workgroup (its keys read once).
 * Replaces the masked fp32 SDPA call of qwen_triton/modules/attention.py:114-119
 * with the mask of qwen_triton/models/core.py:47-75 (_build_causal_mask). */
int qh_flash_fwd_masked(const void* q, int64_t sqb, int64_t sqh, int64_t sqs, const void* k, int64_t skb,
                        int64_t skh, int64_t sks, const void* v, int64_t svb, int64_t svh, int64_t svs, void* o,
                        int64_t sob, int64_t soh, int64_t sos, float* lse, int64_t B, int64_t Hq, int64_t Hkv,
                        int64_t Sq, int64_t Sk, int64_t D, float scale, int causal, int64_t causal_offset,
                        const uint64_t* key_bits, int64_t bits_stride, int64_t window, int dtype, void* stream);
/* Workspace bytes of qh_flash_bwd: Delta = rowsum(O dO) and the LSE in log2 units,
 * per (b, q-head) in rows of Sq rounded up to 64 plus one 64-query tile. */
int64_t qh_flash_bwd_workspace(int64_t B, int64_t Hq, int64_t Sq);
/* dq [B,Hq,Sq,D], dk/dv [B,Hkv,Sk,D] (contiguous, fully written) from o and
 * dout (contiguous [B,Hq,Sq,D]) and the forward's lse. Deterministic: a dK/dV
 * pass over key blocks (looping over the GQA group's q-heads) and a separate
 * dQ pass over query blocks; no atomics.
 * Replaces qwen_triton/kernels/flash_attention.py:155-277 (_flash_attn_bwd_preprocess,
 * _flash_attn_bwd_kernel), :317-367. */
int qh_flash_bwd(const void* q, int64_t sqb, int64_t sqh, int64_t sqs, const void* k, int64_t skb,
                 int64_t skh, int64_t sks, const void* v, int64_t svb, int64_t svh, int64_t svs,
                 const void* o, const void* dout, const float* lse, void* dq, void* dk, void* dv, void* ws,
                 int64_t ws_bytes, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
                 float scale, int causal, int64_t causal_offset, int dtype, void* stream);
/* Bytes of split-KV partials qh_flash_decode needs: 0 where head dim 128 meets
 * at least 512 (sequence, kv-head) pairs (one workgroup per pair, partials
 * combined on chip), else B * Hq * splits * (D + 2) * 4. */
int64_t qh_flash_decode_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sk, int64_t D);
/* Single-query attention (Sq == 1, no mask) over a KV cache: split-KV partials
 * + fixed-order combine. q strides (batch, head); o contiguous [B,Hq,1,D].
 * seqlens (device int32[B], may be NULL) gives each sequence's valid key count
 * (clamped to Sk); with it the launch does not depend on the current length, so
 * a captured decode step can be replayed as the cache grows. Sk then only
 * bounds the keys read and plans the split count.
 * Replaces the q_len == 1 use of qwen_triton/kernels/flash_attention.py:54-152 made by
 * qwen_triton/modules/attention.py:100-109. */
int qh_flash_decode(const void* q, int64_t sqb, int64_t sqh, const void* k, int64_t skb, int64_t skh,
                    int64_t sks, const void* v, int64_t svb, int64_t svh, int64_t svs, void* o, float* lse,
                    const int32_t* seqlens, void* ws, int64_t ws_bytes, int64_t B, int64_t Hq, int64_t Hkv,
                    int64_t Sk, int64_t D, float scale, int dtype, void* stream);
/* qh_flash_decode without a workspace argument and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops or harnesses that
 * forbid hipMalloc). The split partials live in a static 16 MiB device array
 * per GPU (held from the first call on that GPU until the process ends);
 * shapes whose partials need more (qh_flash_decode_workspace; 0 where head
 * dim 128 meets at least 512 (sequence, kv-head) pairs, which then touch no
 * scratch) return QH_E_WORKSPACE.
 * Results equal qh_flash_decode's bit for bit. Calls that overlap on one GPU
 * share the array and race; serialise them (one stream). */
int qh_flash_decode_noalloc(const void* q, int64_t sqb, int64_t sqh, const void* k, int64_t skb, int64_t skh,
                            int64_t sks, const void* v, int64_t svb, int64_t svh, int64_t svs, void* o, float* lse,
                            const int32_t* seqlens, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sk, int64_t D,
                            float scale, int dtype, void* stream);
/* 1 when qh_flash_decode_prepare serves these shapes (D == 128, Hq / Hkv in
 * {1, 2, 4, 8}, and at least 512 (sequence, kv-head) pairs or at most 512 keys
 * Sk), else 0. No counterpart in the reference: a capability query for the
 * fused decode step below. */
int64_t qh_flash_decode_prepare_ok(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sk, int64_t D);
/* One decode step of attention (one new token per sequence) with its input
 * preparation: q_norm/k_norm, RoPE and the K/V cache writes of qh_attn_prepare
 * (same arithmetic, bitwise equal) fused into the decode kernel, so the
 * prepared q never leaves the chip. q, k, v are the step's projected rows
 * ([B, H*D], row strides sq, sk, sv), cos/sin [cos_batch, 1, rot] (batch stride
 * scb; the activation dtype, so every product is exact in fp32 and the result
 * is independent of multiply-add contraction), positions[0] the step's cache
 * position (rows outside [0, cap) are not
 * written), k_cache/v_cache [B, Hkv, cap, D] with the given strides. The
 * attention reads keys [0, min(seqlens[b], Sk)) (seqlens may be NULL: Sk) and
 * writes o [B, Hq, D] and, if lse is not NULL, the log-sum-exp as qh_flash_decode.
 * Replaces, fused, qwen_triton/modules/attention.py:68-82 (q/k norm, RoPE, the
 * cache update) and the q_len == 1 attention of :100-109 (via
 * qwen_triton/kernels/flash_attention.py:54-152). */
int qh_flash_decode_prepare(const void* q, int64_t sq, const void* k, int64_t sk, const void* v, int64_t sv,
                            const void* qw, const void* kw, float eps, int one_plus, const void* cos,
                            const void* sin, int64_t scb, int64_t cos_batch, int64_t rot, void* k_cache,
                            int64_t kcb, int64_t kch, int64_t kcs, void* v_cache, int64_t vcb, int64_t vch,
                            int64_t vcs, int64_t cap, const int64_t* positions, void* o, float* lse,
                            const int32_t* seqlens, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sk,
                            int64_t D, float scale, int dtype, int wdtype, int cdtype, void* stream);


#ifdef __cplusplus
}
#endif

#endif /* QWEN_HIP_H_ */
