/* pragnosia_hip.h -- C ABI of libpragnosia_hip.so, the MI355X (gfx950) kernels of Pragnosia's carrier hot path.
 *
 * Every entry point is stream-ordered and allocation-free: the caller owns every buffer (device pointers,
 * dense row-major, the layouts stated per function), nothing synchronises the host, and nothing is captured
 * that a hipGraph could not replay. `stream` is a hipStream_t passed as void* (NULL = the null stream).
 * Return value: 0 on success; a hipError_t value (> 0) if a launch failed; a negative PRAGNOSIA_ERR_* code if
 * the arguments were rejected before anything was launched. pragnosia_error_string() names any code.
 *
 * Each declaration cites the reference interface it replaces (paths relative to the reference repository). */
#ifndef PRAGNOSIA_HIP_H
#define PRAGNOSIA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PRAGNOSIA_OK 0
#define PRAGNOSIA_ERR_INVALID_ARGUMENT (-1)
#define PRAGNOSIA_ERR_UNSUPPORTED (-2)
#define PRAGNOSIA_ERR_TOO_LARGE (-3)

/* Bytes of device scratch the allocation-free entry point pragnosia_aspin_chunk_fwd_seg_noalloc holds per GPU. */
#define PRAGNOSIA_SEG_SCRATCH_BYTES (32u << 20)

/* Operand types of the exact (fp32 / fp64) scan. */
#define PRAGNOSIA_F32 0
#define PRAGNOSIA_F64 1

/* Tokens per checkpointed state of the exact scan's forward. */
#define PRAGNOSIA_EXACT_CKPT_TOKENS 8

/* ABI version of this header (22); bumped on any change of the entry points. */
int pragnosia_abi_version(void);

/* Human-readable name of a return code (static storage). */
const char* pragnosia_error_string(int code);

/* ---------------------------------------------------------------------------------------------------------
 * Complex diagonal recurrence with per-token lambda (fspin):
 *     h_t = exp(logmag_t + i ang_t) h_{t-1} + u_t,   h_{-1} = h0r + i h0i (zero when h0r/h0i are NULL).
 * Forward: writes hr = Re h and hi = Im h for every t (both (B, T, D) fp32; hr is the output y, hi is saved for
 * the backward) and, when hr_last/hi_last are non-NULL, the final state (Re h_{T-1}, Im h_{T-1}) as two (B, D) fp32
 * arrays. Replaces `_Scan.forward` / `_fwd` of src/scan_kernel.py:24-50, :105-119.
 * u, logmag, ang: (B, T, D) fp32. h0r, h0i: (B, D) fp32 or NULL (both or neither). T = 0 is allowed: the final
 * state is then h0 (zero when NULL), as the reference's scan returns it. */
int pragnosia_diag_scan_fwd(const float* u, const float* logmag, const float* ang,
                            const float* h0r, const float* h0i,
                            float* hr, float* hi, float* hr_last, float* hi_last,
                            int64_t B, int64_t T, int64_t D, void* stream);

/* Backward of pragnosia_diag_scan_fwd (the adjoint recurrence run in reverse). Replaces `_Scan.backward` /
 * `_bwd` of src/scan_kernel.py:53-99, :121-140, including the folding of the final-state gradients:
 * g_last_r adds to g at t = T-1 and g_last_i seeds the imaginary adjoint (either may be NULL = zero).
 * g, hr, hi, logmag, ang: (B, T, D) fp32; du, dlogmag, dang: (B, T, D) fp32 outputs.
 * h0r/h0i: the forward's initial state or NULL; dh0r/dh0i: (B, D) outputs or NULL (written only if non-NULL).
 * T = 0: dh0 = the final state's gradient (g_last_r, g_last_i). */
int pragnosia_diag_scan_bwd(const float* g, const float* g_last_r, const float* g_last_i,
                            const float* logmag, const float* ang, const float* hr, const float* hi,
                            const float* h0r, const float* h0i,
                            float* du, float* dlogmag, float* dang, float* dh0r, float* dh0i,
                            int64_t B, int64_t T, int64_t D, void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * Associative carrier (aspin), plain write rule, chunked scan (chunk = 64, head dim D = 64), per (batch, head):
 *     S_t = exp(la_t) S_{t-1} + k_t v_t^T,   o_t = S_t^T q_t,   S_{-1} = S0 (zero when NULL).
 * q, k, v: (B, H, T, D) bf16; la: (B, H, T) fp32 (<= 0); S0: (B, H, D, D) fp32, keys on dim 2, or NULL.
 * Writes o: (B, H, T, D) bf16; S_final: (B, H, D, D) fp32; sent (if non-NULL): the state entering every chunk,
 * (B, H, ceil(T/64), D, D) bf16 -- required by the backward. T need not be a multiple of 64.
 * Replaces `assoc_scan_kernel` and the ops under it (`prefix_scan`, `assoc_out`) of src/assoc_kernel.py:128-323.
 * Returns PRAGNOSIA_ERR_UNSUPPORTED for D != 64 or chunk != 64. */
int pragnosia_aspin_chunk_fwd(const void* q, const void* k, const void* v, const float* la, const float* S0,
                              void* o, float* S_final, void* sent,
                              int64_t B, int64_t H, int64_t T, int64_t D, int64_t chunk, void* stream);

/* Backward of pragnosia_aspin_chunk_fwd. dO: (B, H, T, D) bf16; dS_final: (B, H, D, D) fp32 or NULL (zero);
 * sent: the forward's entering states. Writes dq, dk, dv (bf16, (B, H, T, D)), dla (fp32, (B, H, T)) and, if
 * non-NULL, dS0 (fp32, (B, H, D, D)). Replaces the registered backward of the same ops
 * (`assoc_out_bwd`, `prefix_scan_bwd` and the glue of src/assoc_kernel.py:146-299). */
int pragnosia_aspin_chunk_bwd(const void* q, const void* k, const void* v, const float* la, const void* sent,
                              const void* dO, const float* dS_final,
                              void* dq, void* dk, void* dv, float* dla, float* dS0,
                              int64_t B, int64_t H, int64_t T, int64_t D, int64_t chunk, void* stream);

/* Bytes of device workspace pragnosia_aspin_chunk_fwd_seg and pragnosia_aspin_chunk_bwd_seg need (-1 if the shape
 * is rejected). */
int64_t pragnosia_aspin_chunk_seg_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D, int64_t chunk,
                                                  int64_t seg_chunks);

/* The forward of pragnosia_aspin_chunk_fwd, segment-parallel: every head's chunks are split into segments of
 * `seg_chunks` chunks that run concurrently once their entering states are known (per-segment state sums, a prefix
 * over segments, then the chunked forward per segment), for few heads over long sequences. Same inputs and
 * outputs as pragnosia_aspin_chunk_fwd (sent may be NULL).
 * window = 0: one continuous sequence, the same function as pragnosia_aspin_chunk_fwd.
 * window > 0 (a multiple of 64 and of 64 * seg_chunks): the sequence is a run of windows of `window` tokens whose
 * q and k were rotated with positions restarting at 0 in every window; between windows the carried state's key
 * rows (2i, 2i + 1) are rotated by -window * theta[h, i] (theta: (H, D / 2) fp32). This is what successive calls of
 * the reference's carrier over consecutive windows compute, each rebasing the state it is handed
 * (`AssocCarrier.forward`, src/assoc.py:391-405, driven by `LM.forward_carried`, src/model.py:842-864); S_final is
 * the state after the last window, in that window's positions. S0 is the state entering the first window.
 * `workspace`: caller-allocated device memory of at least pragnosia_aspin_chunk_seg_workspace_bytes(...) bytes. */
int pragnosia_aspin_chunk_fwd_seg(const void* q, const void* k, const void* v, const float* la, const float* S0,
                                  const float* theta, int64_t window, void* o, float* S_final, void* sent,
                                  void* workspace, int64_t workspace_bytes, int64_t B, int64_t H, int64_t T,
                                  int64_t D, int64_t chunk, int64_t seg_chunks, void* stream);

/* pragnosia_aspin_chunk_fwd_seg without a workspace argument: the same kernels and the same results, their workspace
 * taken from a fixed array of PRAGNOSIA_SEG_SCRATCH_BYTES of device memory that the library holds on every GPU it
 * runs on until the process ends. It allocates nothing (no hipMalloc, no hipFree, no allocating library call) and
 * writes no memset, so it suits callers that cannot allocate: code under HIP graph capture, serving loops that
 * prefill long contexts, harnesses that forbid allocation. Returns PRAGNOSIA_ERR_TOO_LARGE when the shape needs more
 * than the array holds (pragnosia_aspin_chunk_seg_workspace_bytes(...) > PRAGNOSIA_SEG_SCRATCH_BYTES; e.g. B2 H12
 * T8192 in segments of 8 chunks needs 6 MiB). Every call on one GPU shares that GPU's array: calls that overlap in
 * time on one GPU (concurrent streams, or threads) race and must be serialised by the caller. Nothing in the array
 * needs to start at zero (every byte read is written first by the same call).
 * This entry point has no counterpart in the reference; it exists for the callers above. */
int pragnosia_aspin_chunk_fwd_seg_noalloc(const void* q, const void* k, const void* v, const float* la,
                                          const float* S0, const float* theta, int64_t window, void* o,
                                          float* S_final, void* sent, int64_t B, int64_t H, int64_t T, int64_t D,
                                          int64_t chunk, int64_t seg_chunks, void* stream);

/* The backward of pragnosia_aspin_chunk_bwd, segment-parallel (segments of `seg_chunks` chunks: per-segment sums of
 * q and dO, a reverse prefix over segments for the state gradient entering each segment from later ones, then the
 * chunked backward per segment). Same inputs and outputs as pragnosia_aspin_chunk_bwd (continuous sequences only);
 * `sent` from either forward. `workspace`: at least pragnosia_aspin_chunk_seg_workspace_bytes(...) bytes.
 * Replaces the same registered backward (src/assoc_kernel.py:146-299) for few heads over long sequences. */
int pragnosia_aspin_chunk_bwd_seg(const void* q, const void* k, const void* v, const float* la, const void* sent,
                                  const void* dO, const float* dS_final, void* dq, void* dk, void* dv, float* dla,
                                  float* dS0, void* workspace, int64_t workspace_bytes, int64_t B, int64_t H,
                                  int64_t T, int64_t D, int64_t chunk, int64_t seg_chunks, void* stream);

/* The plain rule at head dim D = 128 (the reference's assoc_scan_kernel at D = 128, src/assoc_kernel.py:21,302-323,
 * which the carrier takes for 128-wide heads, src/assoc.py:411, and its registered backward, :146-299). The state's
 * key rows evolve independently and o_t = S_t^T q_t sums over them, so each head runs as four 64 x 64 scans, one per
 * (key half kh, value half vh) block of its state, reading q and k at columns 64 kh and v and dO at columns 64 vh of
 * the 128-wide rows (no copies); o, dv (summed over key halves) and dq, dk (over value halves) are written as two
 * bf16 partials each, the second into the workspace, and added (fp32 sum rounded once to bf16) by one more kernel.
 * q, k, v, dO: (B, H, T, 128) bf16; la, dla: (B, H, T) fp32; S0, S_final, dS_final, dS0: (B, H, 128, 128) fp32
 * (S0, dS_final, dS0 may be NULL); sent: the entering states per scan, (B, H, 4, NC, 64, 64) bf16 (scan 2 kh + vh
 * holds block rows 64 kh.., columns 64 vh..; NC = ceil(T / 64)), written by the forward when not NULL and read by the
 * backward. seg_chunks: the segment length of the segment-parallel passes (as pragnosia_aspin_chunk_fwd_seg, no
 * windows); at least NC runs one workgroup per scan: the forward then as one workgroup per (head, value half) over
 * all 128 keys (o written once, no partial; the workspace unused), the backward as two launches of two scans per head,
 * the second adding the first's partial outputs (dla with fp32 atomics: not the same bits run to run). `workspace`: caller-allocated device memory of at least
 * pragnosia_aspin_chunk_wide_workspace_bytes(..., backward) bytes. */
int64_t pragnosia_aspin_chunk_wide_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D, int64_t chunk,
                                                   int64_t seg_chunks, int32_t backward);
int pragnosia_aspin_chunk_fwd_wide(const void* q, const void* k, const void* v, const float* la, const float* S0,
                                   void* o, float* S_final, void* sent, void* workspace, int64_t workspace_bytes,
                                   int64_t B, int64_t H, int64_t T, int64_t D, int64_t chunk, int64_t seg_chunks,
                                   void* stream);
int pragnosia_aspin_chunk_bwd_wide(const void* q, const void* k, const void* v, const float* la, const void* sent,
                                   const void* dO, const float* dS_final, void* dq, void* dk, void* dv, float* dla,
                                   float* dS0, void* workspace, int64_t workspace_bytes, int64_t B, int64_t H,
                                   int64_t T, int64_t D, int64_t chunk, int64_t seg_chunks, void* stream);

/* The carrier's output epilogue (head dim D = 64): per (batch, head, token) row x of the scan output o
 * ((B, H, T, D) bf16), r = 1 / sqrt(mean(x^2) + eps) and y[b, t, h D + d] = (x_d r) w_d, rounded once to y's dtype
 * (bf16 if y_bf16, else fp32) and written token-major, (B, T, H D); r is written to rstd ((B, H, T) fp32) for the
 * backward. weight: (D) fp32. Replaces `self.on(o).transpose(1, 2).reshape(B, T, D)` of src/assoc.py:505
 * (nn.RMSNorm(dk) with eps=None, i.e. fp32 epsilon, computed in fp32). */
int pragnosia_aspin_out_fwd(const void* o, const float* weight, float eps, void* y, int y_bf16, float* rstd,
                            int64_t B, int64_t H, int64_t T, int64_t D, void* stream);

/* LayerNorm over the last dimension (D a multiple of 4, at most 2048; rows = the product of the leading dims),
 * fp32 statistics: mu = mean(x), var = mean((x - mu)^2), y = (x - mu) / sqrt(var + eps) * weight + bias, written as
 * bf16 when y_bf16 (the dtype the matmul after it computes in under autocast) or fp32; mean and rstd ((rows) fp32)
 * are kept for the backward. x, weight, bias fp32. Replaces `self.ln(x)` of the carrier (`nn.LayerNorm(d)`,
 * src/assoc.py:323,388) and of the MLP (src/model.py:555) with the cast to bf16 that autocast's matmul applies to
 * its fp32 output. PRAGNOSIA_ERR_UNSUPPORTED for other D. */
int pragnosia_layer_norm_fwd(const float* x, const float* weight, const float* bias, float eps, void* y, int y_bf16,
                             float* mean, float* rstd, int64_t rows, int64_t D, void* stream);

/* Rows of D fp32 partial sums pragnosia_layer_norm_bwd writes for each of dweight and dbias (-1 if rejected). */
int64_t pragnosia_layer_norm_partials(int64_t rows, int64_t D);

/* Backward of pragnosia_layer_norm_fwd from dy ((rows, D), bf16 when dy_bf16, else fp32): dx (rows, D) fp32 and the
 * weight and bias gradients as partial rows (pragnosia_layer_norm_partials(rows, D) rows of D fp32 each; the
 * gradients are their sums over rows). Replaces the autograd backward of the same lines. */
int pragnosia_layer_norm_bwd(const void* dy, int dy_bf16, const float* x, const float* weight, const float* mean,
                             const float* rstd, float* dx, float* dw_partials, float* db_partials, int64_t rows,
                             int64_t D, void* stream);

/* Column sums of a row-major fp32 matrix x (rows, cols): out[c] = sum over r of x[r][c], in an order fixed by the
 * shape (deterministic). Sums the per-workgroup partial rows of the parameter gradients above (LayerNorm weight and
 * bias, the RMSNorm weight, the rotation frequencies, the decay and gate biases), the reduction the reference's
 * autograd applies to a broadcast parameter's gradient (e.g. the bias of nn.LayerNorm, src/assoc.py:388). Records no
 * memset, so a captured backward can hold it. */
int pragnosia_colsum_f32(const float* x, int64_t rows, int64_t cols, float* out, void* stream);

/* Bytes of workspace pragnosia_wgrad_bf16 needs for (M, N, K) (0: none; -1 if the shape is rejected). */
int64_t pragnosia_wgrad_workspace_bytes(int64_t M, int64_t N, int64_t K);

/* The weight gradient of a linear layer over its token rows: C (M x N fp32, row pitch ldc) = A^T B, or C += A^T B
 * when accumulate, with A (K x M) and B (K x N) bf16, row-major with row pitches lda, ldb (K = tokens; A the output
 * gradient, B the layer input). M and N multiples of 8, lda and ldb multiples of 8, ldc of 4, pointers 16-byte
 * aligned. K is split over workgroups whose fp32 partials (in the caller's workspace) are summed in a fixed order,
 * so the result is deterministic. Replaces the weight-gradient GEMM autograd forms for the F.linear / nn.Linear
 * calls around the carrier (src/assoc.py:384-512: the q/k/v/decay/gate projections and the gated o-projection) and
 * the MLP (src/model.py:552-560), there a bf16 GEMM cast to the fp32 parameter. */
int pragnosia_wgrad_bf16(const void* A, int64_t lda, const void* B, int64_t ldb, float* C, int64_t ldc, int accumulate,
                         void* workspace, int64_t workspace_bytes, int64_t M, int64_t N, int64_t K, void* stream);

/* Rows of 64 fp32 partial weight gradients pragnosia_aspin_out_bwd writes (-1 if the shape is rejected). */
int64_t pragnosia_aspin_out_weight_partials(int64_t B, int64_t H, int64_t T);

/* Backward of pragnosia_aspin_out_fwd: gy (B, T, H D), bf16 if gy_bf16 else fp32; o, weight, rstd as the forward.
 * Writes dO ((B, H, T, D) bf16, the scan's output gradient) and dw_partials (pragnosia_aspin_out_weight_partials(...)
 * rows of D fp32; the weight gradient is their sum over rows). Replaces the autograd backward of the same lines. */
int pragnosia_aspin_out_bwd(const void* gy, int gy_bf16, const void* o, const float* weight, const float* rstd,
                            void* dO, float* dw_partials, int64_t B, int64_t H, int64_t T, int64_t D, void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * Associative carrier scan with fp32 or fp64 operands (no bf16 rounding), plain rule (beta NULL) or delta rule,
 * per (batch, head), head dims 1 <= Dk <= 384, 1 <= Dv <= 128:
 *     plain: S_t = a_t S_{t-1} + k_t v_t^T;   delta: S_t = P + beta_t k_t (v_t - P^T k_t)^T, P = a_t S_{t-1};
 *     o_t = S_t^T q_t,   a_t = exp(la_t),   S_{-1} = S0 (zero when NULL).
 * Every tensor has the operand type `dtype` (PRAGNOSIA_F32 or PRAGNOSIA_F64): q, k (B, H, T, Dk); v (B, H, T, Dv);
 * la, beta (B, H, T); S0, S_final (B, H, Dk, Dv) keys on dim 2; o (B, H, T, Dv). For a backward the forward also
 * writes ckpt, the state entering every block of PRAGNOSIA_EXACT_CKPT_TOKENS tokens, (B, H, ceil(T / 8), Dk, Dv),
 * and with the delta rule resid, the residuals v_t - P^T k_t, (B, H, T, Dv) (both NULL when no backward follows).
 * Replaces `assoc_scan` of src/assoc.py:254-269 (fp32, or fp64 for fp64 inputs: `_scan_twopass`,
 * `_scan_twopass_delta`, src/assoc.py:118-165, :207-251) and its autograd backward. */
int pragnosia_aspin_exact_fwd(const void* q, const void* k, const void* v, const void* la, const void* beta,
                              const void* S0, void* o, void* S_final, void* ckpt, void* resid, int64_t B, int64_t H,
                              int64_t T, int64_t Dk, int64_t Dv, int dtype, void* stream);

/* Backward of pragnosia_aspin_exact_fwd from dO (B, H, T, Dv) and dS_final (or NULL = zero), with the forward's ckpt
 * and resid: writes dq, dk (B, H, T, Dk), dv (B, H, T, Dv), dla (B, H, T), dbeta (B, H, T; delta rule) and, if
 * non-NULL, dS0 (B, H, Dk, Dv), all of type `dtype`. PRAGNOSIA_ERR_UNSUPPORTED when its block buffers exceed the
 * 160 KiB of LDS: they grow with Dk times Dv (fp32 fits Dv 128 up to Dk 128, 80 up to 384; fp64 112 up to 128, 80 up
 * to 192, 32 up to 384). Value columns are independent recurrences: a caller splits wider ones into blocks. */
int pragnosia_aspin_exact_bwd(const void* q, const void* k, const void* v, const void* la, const void* beta,
                              const void* ckpt, const void* resid, const void* dO, const void* dS_final, void* dq,
                              void* dk, void* dv, void* dla, void* dbeta, void* dS0, int64_t B, int64_t H, int64_t T,
                              int64_t Dk, int64_t Dv, int dtype, void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * Associative carrier, DELTA write rule, chunked scan (chunk = 64, head dim D = 64 or 128), per (batch, head):
 *     S_t = a_t S_{t-1} + beta_t k_t (v_t - (a_t S_{t-1})^T k_t)^T,   o_t = S_t^T q_t,   a_t = exp(la_t).
 * Layouts as pragnosia_aspin_chunk_fwd (q, k, v, o (B, H, T, D); S0, S_final (B, H, D, D)); beta: (B, H, T) fp32 in
 * (0, 1). Writes o (bf16), S_final (fp32), sent (bf16 entering states, each chunk's transposed: sent[b, h, c, j, d] =
 * S[d, j], (B, H, ceil(T/64), D, D); required by the backward; may be NULL when no backward follows), and the two
 * saved intermediates of the backward: W, the residuals actually written, (B, H, T, D) bf16, and X, the per-chunk
 * inverse (I + diag(beta) strictly_lower((K K^T) o dec))^-1, (B, H, ceil(T/64), 64, 64) bf16, computed in fp32. At
 * D = 64 the forward is one kernel that forms each chunk's inverse on chip, and o, W, sent and X are each written only
 * when non-NULL (S_final always): with only o the call keeps nothing for a backward, with no o it is the state pass
 * that a backward recomputing the intermediates runs (the output products skipped). At D = 128 o, W and X are
 * required; the rule is independent per value column once X is known, so each head runs as two scans over its value
 * halves, each carrying a 128 x 64 state slice and sharing X.
 * Replaces `delta_scan_kernel` and the ops under it (`delta_inv`, `delta_loop_fwd`, `assoc_out`) of
 * src/assoc_kernel.py:332-386, :512-704 (head dims 64 and 128, src/assoc_kernel.py:21); the rule is
 * `_scan_twopass_delta` of src/assoc.py:207-251. */
int pragnosia_aspin_delta_fwd(const void* q, const void* k, const void* v, const float* la, const float* beta,
                              const float* S0, void* o, float* S_final, void* sent, void* W, void* X,
                              int64_t B, int64_t H, int64_t T, int64_t D, int64_t chunk, void* stream);

/* Bytes of device workspace pragnosia_aspin_delta_bwd needs at this shape (-1 if the shape is rejected). */
int64_t pragnosia_aspin_delta_bwd_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D, int64_t chunk);

/* Backward of pragnosia_aspin_delta_fwd. dO (B, H, T, D) bf16; dS_final fp32 or NULL (zero). Writes dq, dk, dv
 * (bf16), dla and dbeta (fp32, (B, H, T)) and, if non-NULL, dS0 (fp32). `workspace` is caller-allocated device
 * memory of at least pragnosia_aspin_delta_bwd_workspace_bytes(...) bytes (no alignment beyond 256 B needed). At
 * D = 64 the backward is one kernel that passes the per-chunk state gradients and drhs between its waves on chip (the
 * workspace is a token 256 bytes); at D = 128 the workspace holds them between two kernels, and the second value-half
 * scan's parts of dq, dk, dla and dbeta, which one more kernel adds.
 * Replaces the registered backward of `delta_loop_fwd`, `delta_inv` and `assoc_out`
 * (`_delta_loop_bwd`, `_inv_bwd`, `_bwd_chunk` of src/assoc_kernel.py:73-116, :389-509, :625-704). */
int pragnosia_aspin_delta_bwd(const void* q, const void* k, const void* v, const float* la, const float* beta,
                              const void* sent, const void* W, const void* X, const void* dO,
                              const float* dS_final, void* dq, void* dk, void* dv, float* dla, float* dbeta,
                              float* dS0, void* workspace, int64_t workspace_bytes,
                              int64_t B, int64_t H, int64_t T, int64_t D, int64_t chunk, void* stream);

/* The carried windows of the delta rule in one pass (with pragnosia_aspin_delta_fwd over all windows at once): the
 * entering state of every window from the windows' affine maps. A window maps its entering state as S_out = M S_in + R
 * (keys on rows; M acts on the key rows, the same for every value column): R = its final state from a zero entering
 * state, M = its final state from the identity with zero values. Between windows the state is rebased by -shift theta
 * (key-row pairs (2i, 2i+1) rotated by -shift theta[h][i]): S_in[0] = S0, S_in[w + 1] = Rot(M[w] S_in[w] + R[w]).
 * M, R, S_in: (BH, NW, 64, 64) fp32 (BH = B H, window w of sequence bh at index bh NW + w); S0: (BH, 64, 64) fp32 or
 * NULL (zero); theta (H, 32) fp32, head h = bh mod H. fp32 throughout. Replaces the window-by-window loop of
 * `LM.forward_carried` (src/model.py:842-864) over the carried-state rebase (src/assoc.py:391-405) for delta
 * carriers. */
int pragnosia_aspin_delta_window_prefix(const float* M, const float* R, const float* S0, const float* theta,
                                        float shift, float* S_in, int64_t BH, int64_t H, int64_t NW, void* stream);

/* The R and M state passes above in one launch, head dim 64, chunk 64: N sequences (N = BH NW windows, each a
 * sequence of its own) of T tokens with q, k, v (N, T, 64) bf16, la and beta (N, T) fp32 as for
 * pragnosia_aspin_delta_fwd. RM (2N, 64, 64) fp32 receives R (entries 0 .. N - 1: each sequence's final state from a
 * zero entering state) then M (entries N .. 2N - 1: its final state from the identity with zero values), the inputs
 * pragnosia_aspin_delta_window_prefix takes as R = RM and M = RM + N 64 64. One launch of 2N workgroups instead of
 * two of N (the workgroups fill the compute units' rounds better), and neither zero values nor identity states are
 * read from memory. Part of the same replacement of `LM.forward_carried`'s window loop (src/model.py:842-864). */
int pragnosia_aspin_delta_window_maps(const void* q, const void* k, const void* v, const float* la,
                                      const float* beta, float* RM, int64_t N, int64_t T, void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * The plumbing between the carrier's projections and the scan (head dim D = 64): per (b, t, h) row, unit-normalise
 * q, k, v (x / max(|x|, 1e-12)), scale k by sigmoid(gate) when `gate` is non-NULL (plain rule), rotate q and k on
 * interleaved channel pairs (2i, 2i+1) by pos[t] * theta[h, i], cast to bf16 and transpose to the scan layout.
 * qp, kp, vp: (B, T, H, D) with consecutive tokens `in_stride` elements apart (H * D when dense; larger when they are
 * column slices of one wider row, e.g. one GEMM's output holding all projections), fp32 (in_bf16 = 0) or bf16
 * (in_bf16 = 1); gate: (B, T, H) fp32 or NULL; theta: (H, D/2) fp32; pos: (T,) int64. Writes q, k, v: (B, H, T, D)
 * bf16. Replaces `prep_kernel` / `_prep_fwd` of src/assoc_kernel.py:740-769, :828-891 (torch form
 * src/assoc.py:453-460). */
int pragnosia_aspin_prep_fwd(const void* qp, const void* kp, const void* vp, const float* gate, const float* theta,
                             const int64_t* pos, void* q, void* k, void* v, int64_t B, int64_t T, int64_t H,
                             int64_t D, int64_t in_stride, int in_bf16, void* stream);

/* Rows of the theta-gradient partial buffer of pragnosia_aspin_prep_bwd: (rows, H, D/2) fp32, summed by the caller. */
int64_t pragnosia_aspin_prep_theta_partials(int64_t B, int64_t T);

/* Backward of pragnosia_aspin_prep_fwd: from dq, dk, dv ((B, H, T, D) bf16) writes dqp, dkp, dvp in the projections'
 * layout, stride and dtype, dgate ((B, T, H) fp32, required iff gate is non-NULL) and dtheta_partial
 * ((pragnosia_aspin_prep_theta_partials(B, T), H, D/2) fp32; theta's gradient is its sum over the first dim).
 * Replaces `_prep_bwd` of src/assoc_kernel.py:772-822, :848-885. */
int pragnosia_aspin_prep_bwd(const void* qp, const void* kp, const void* vp, const float* gate, const float* theta,
                             const int64_t* pos, const void* dq, const void* dk, const void* dv, void* dqp,
                             void* dkp, void* dvp, float* dgate, float* dtheta_partial, int64_t B, int64_t T,
                             int64_t H, int64_t D, int64_t in_stride, int in_bf16, void* stream);

/* The same plumbing fed by ONE GEMM's output P (B, T, stride) (fp32, or bf16 if in_bf16) holding, per token, the q,
 * k and v projections in columns [0, H D), [H D, 2 H D), [2 H D, 3 H D), the decay logits (before bias) in columns
 * [la_col, la_col + H) and at most one of: the plain rule's write-gate logits in [gate_col, gate_col + H)
 * (gate_col >= 0), or the delta rule's write-strength logits in [beta_col, beta_col + H) (beta_col >= 0); -1 = absent.
 * Besides q, k, v (as pragnosia_aspin_prep_fwd, gate = sigmoid(logit + gate_bias[h])), writes the decay in the scan's
 * layout, la (B, H, T) fp32: la = -softplus(logit + la_bias[h]) exp(A[h]), floored at la_floor[h] when la_floor is
 * non-NULL, and with beta_col >= 0 the strength beta (B, H, T) fp32 = max(sigmoid(logit + beta_bias[h]), beta_min).
 * la_bias, A, la_floor, gate_bias, beta_bias: (H) fp32 (the biases may be NULL: none). Replaces the carrier's
 * separate projections' consumers: `logalpha` (src/assoc.py:355-359), the write gate (src/assoc.py:458-459), beta
 * (src/assoc.py:468, the write_all floor 0.75 included) and `prep_kernel` (src/assoc_kernel.py:740-769), with the
 * transposes of la and beta for the scan. */
int pragnosia_aspin_prep_proj_fwd(const void* P, int64_t stride, int64_t la_col, int64_t gate_col, int64_t beta_col,
                                  const float* la_bias, const float* A, const float* la_floor,
                                  const float* gate_bias, const float* beta_bias, float beta_min,
                                  const float* theta, const int64_t* pos, void* q, void* k, void* v, float* la,
                                  float* beta, int64_t B, int64_t T, int64_t H, int64_t D, int in_bf16,
                                  void* stream);

/* Rows of 3 fp32 per-head partial sums pragnosia_aspin_prep_proj_bwd writes (-1 if the shape is rejected). */
int64_t pragnosia_aspin_prep_proj_partials(int64_t B, int64_t T, int64_t H);

/* Backward of pragnosia_aspin_prep_proj_fwd: from dq, dk, dv ((B, H, T, D) bf16), dla and (with beta_col >= 0) dbeta
 * ((B, H, T) fp32) writes the q, k, v, decay and gate or strength columns of dP (P's layout, stride and dtype; other
 * columns untouched), theta's partials (as pragnosia_aspin_prep_bwd) and `part`:
 * pragnosia_aspin_prep_proj_partials(B, T, H) rows, row (b H + h) ntb + j holding (d gate_bias[h] or
 * d beta_bias[h], d la_bias[h], dA[h]) partial sums (ntb = ceil(T / 64)); the caller sums them per head. */
int pragnosia_aspin_prep_proj_bwd(const void* P, int64_t stride, int64_t la_col, int64_t gate_col, int64_t beta_col,
                                  const float* la_bias, const float* A, const float* la_floor,
                                  const float* gate_bias, const float* beta_bias, float beta_min,
                                  const float* theta, const int64_t* pos, const void* dq, const void* dk,
                                  const void* dv, const float* dla, const float* dbeta, void* dP,
                                  float* dtheta_partial, float* part, int64_t B, int64_t T, int64_t H, int64_t D,
                                  int in_bf16, void* stream);

/* The carried-state rebase of src/assoc.py:399-402: S (B, H, D, D) fp32 with keys on dim 2; key rows (2i, 2i+1) are
 * rotated by -p0 * theta[h, i], p0 = *p0_dev when p0_dev is non-NULL (a device fp32 scalar, as the graphed decode
 * keeps it), else the host value p0. S_out must not alias S. */
int pragnosia_aspin_rebase_fwd(const float* S, const float* theta, const float* p0_dev, float p0, float* S_out,
                               int64_t B, int64_t H, int64_t D, void* stream);

/* Backward of the rebase: dS = R^T dS_out (if dS is non-NULL) and the theta-gradient partials (B, H, D/2) fp32
 * (if dtheta_partial is non-NULL; theta's gradient is their sum over B). */
int pragnosia_aspin_rebase_bwd(const float* S, const float* theta, const float* p0_dev, float p0,
                               const float* dS_out, float* dS, float* dtheta_partial, int64_t B, int64_t H,
                               int64_t D, void* stream);

/* The single-token recurrent step of one carrier layer (decode), fused: rebase S by -p0 * theta (as above),
 * normalise the T = 1 projections qp, kp, vp ((B, H, D) fp32), gate k by sigmoid(gate) (plain rule, gate (B, H) fp32)
 * or use the write strength beta ((B, H) fp32, delta rule; at most one of gate and beta is non-NULL), decay by
 * exp(la) (la (B, H) fp32), write, and read o = S_new^T q ((B, H, D) fp32). S_out may alias S (in-place update).
 * Replaces the T = 1 torch path of AssocCarrier.forward (src/assoc.py:391-411, :502) that `_generate_graphed`
 * replays (src/bench.py:241-317). */
int pragnosia_aspin_decode_step(const float* S, float* S_out, const float* qp, const float* kp, const float* vp,
                                const float* gate, const float* la, const float* beta, const float* theta,
                                const float* p0_dev, float p0, float* o, int64_t B, int64_t H, int64_t D,
                                void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * The carrier LM's single-token decode step, fused (all fp32, as the reference decodes).
 *
 * The carrier's recurrent step reading its inputs from ONE projection GEMV's output P (B, np): per sequence b,
 * P[b] = [qp (H D) | kp (H D) | vp (H D) | ... ] with the decay logits (before bias) at columns la_col + h and either
 * the write-gate logits (gate_col >= 0, plain rule) or the write-strength logits (beta_col >= 0, delta rule) at
 * their columns (the other -1). Forms la = -softplus(logit + la_bias[h]) exp(A[h]) (floored at la_floor[h] when
 * non-NULL), the gate logit + gate_bias[h], beta = max(sigmoid(logit + beta_bias[h]), beta_min), then runs the step of
 * pragnosia_aspin_decode_step (S_out may equal S: in place) and writes the output per-head RMS-normalised and
 * token-major: o[b][h D + j] = (o_j r) on_weight[j], r = 1 / sqrt(mean_j o_j^2 + on_eps); with on_weight NULL the
 * output is written raw, o[b][h D + j] = o_j (D / 16 workgroups per head below 256 heads, one past it; the consumer
 * applies the RMSNorm, e.g. pragnosia_decode_gemv_rms). D = 64, or 128 with on_weight NULL (PRAGNOSIA_ERR_UNSUPPORTED otherwise). Replaces,
 * inside the reference's graphed decode (src/bench.py:241-317), the T = 1 path of `AssocCarrier.forward` from its
 * projections to `self.on(o).transpose(1, 2).reshape(B, T, D)` (src/assoc.py:384-505). */
int pragnosia_aspin_decode_proj(const float* S, float* S_out, const float* P, int64_t np, int64_t la_col,
                                int64_t gate_col, int64_t beta_col, const float* la_bias, const float* A,
                                const float* la_floor, const float* gate_bias, const float* beta_bias, float beta_min,
                                const float* theta, const float* p0_dev, float p0, const float* on_weight,
                                float on_eps, float* o, int64_t B, int64_t H, int64_t D, void* stream);

/* pragnosia_aspin_decode_proj with on_weight, followed by the gated o-projection and residual, in one launch: for
 * D = 64 (PRAGNOSIA_ERR_UNSUPPORTED otherwise) and the small batches of the GEMV decode, y (B, N) += scale *
 * (Wo o_n) with o_n the per-head RMS-normalised step output (as pragnosia_aspin_decode_proj writes it), Wo (N, H D)
 * row-major, scale a device scalar or NULL (1). One workgroup per (sequence, head, 64 rows of Wo) runs the head's step and adds its
 * 64 columns' products to its rows of y with atomics: y holds the residual on entry and equals the residual plus the
 * projection to fp32 rounding, with the heads summed in arrival order (not bit-identical from run to run). Every
 * workgroup reads the old state, so S_out must not overlap S (the new state goes there), and y must not overlap P or
 * S (PRAGNOSIA_ERR_INVALID_ARGUMENT otherwise). Replaces,
 * inside the reference's graphed decode (src/bench.py:241-317), the T = 1 path of `AssocCarrier.forward` from its
 * projections to `x + F.linear(o, self.o.weight) * sigmoid(self.gate)` (src/assoc.py:384-512), as
 * pragnosia_aspin_decode_proj + pragnosia_decode_gemv_rms do in two launches. */
int pragnosia_aspin_decode_oproj(const float* S, float* S_out, const float* P, int64_t np, int64_t la_col,
                                 int64_t gate_col, int64_t beta_col, const float* la_bias, const float* A,
                                 const float* la_floor, const float* gate_bias, const float* beta_bias,
                                 float beta_min, const float* theta, const float* p0_dev, float p0,
                                 const float* on_weight, float on_eps, const float* Wo, int64_t N,
                                 const float* scale, float* y, int64_t B, int64_t H, int64_t D, void* stream);

/* One dense layer of the decode step over B sequences: y (B, N) = act(scale * (W z) + bias) + resid, with W (N, K)
 * row-major, z = LayerNorm(x) with ln_weight / ln_bias (may be NULL) / ln_eps when ln_weight is non-NULL (K <= 1024),
 * else z = x (B, K); scale a device scalar or NULL (1); bias (N) or NULL; act 0 = identity, 1 = GELU (erf form);
 * resid (B, N) or NULL. y must not alias x or resid. Replaces the LayerNorm + nn.Linear (+ GELU, + residual) calls of
 * the carrier's projections and gated output projection, the MLP (src/model.py:552-560) and the tied head during
 * decoding. */
int pragnosia_decode_gemv(const float* x, int64_t B, int64_t K, const float* ln_weight, const float* ln_bias,
                          float ln_eps, const float* W, int64_t N, const float* bias, const float* scale, int act,
                          const float* resid, float* y, void* stream);

/* pragnosia_decode_gemv with the carrier's per-head RMSNorm on its input instead of a LayerNorm, over heads of
 * group = 64 or 128 channels: z[b][h G + j] = x[b][h G + j] r_{b,h} rms_weight[j], r = 1 / sqrt(mean_j x[b][h G + j]^2
 * + rms_eps), then y = act(scale (W z) + bias) + resid. For B <= 4 and K a multiple of 256 up to 1024
 * (PRAGNOSIA_ERR_UNSUPPORTED otherwise). Replaces `self.on(o)` and the gated o-projection with the residual of the
 * carrier's T = 1 step (src/assoc.py:505-511), reading the raw output of pragnosia_aspin_decode_proj (on_weight
 * NULL). */
int pragnosia_decode_gemv_rms(const float* x, int64_t B, int64_t K, const float* rms_weight, int64_t group,
                              float rms_eps, const float* W, int64_t N, const float* bias, const float* scale, int act,
                              const float* resid, float* y, void* stream);

/* The end of one greedy decode step for B sequences, in one launch: tok = argmax over logits (B, V) fp32 per row
 * (the first index among equal maxima, NaN above every number, as torch.argmax), out[c][b] = tok and tok_out[b] = tok
 * with c = *ctr_in (out (n_rows, B) int64, the row skipped when c >= n_rows), h (B, d) = emb[tok] + pemb[p] fp32 with
 * p = (*pos_in + 1) mod ctx (emb (V, d), pemb (ctx, d): the tied token embedding and the position table), then
 * *pos_out = p, *ctr_out = c + 1, p0s[0 .. L-1] = 1 (the carried states' position offsets after a one-token call), and
 * with logits_rec non-NULL (n_rows, B, V) fp32 the logits copied to row c. The counter and position are read from one
 * int64 and written to another (ctr_in != ctr_out, pos_in != pos_out; the caller alternates them step to step).
 * Replaces the per-token tail of the reference's graphed generate (`src/bench.py:241-317`: argmax, append, position
 * advance modulo ctx, the next input's embedding sum of `src/model.py:822-826`). */
int pragnosia_decode_tail(const float* logits, int64_t B, int64_t V, const float* emb, const float* pemb, int64_t d,
                          int64_t ctx, const int64_t* ctr_in, int64_t* ctr_out, const int64_t* pos_in,
                          int64_t* pos_out, int64_t* out, int64_t n_rows, int64_t* tok, float* h, float* p0s,
                          int64_t L, float* logits_rec, void* stream);

/* The dense layers of the decode step on the fp32 matrix cores, for batches past the GEMV's (any B; 16 rows a
 * workgroup): y (B, N) = act(scale * (W z) + bias) + resid, with z = x (mode 0); z = (x - mean) / sqrt(var + eps) over
 * each row (mode 1: a LayerNorm whose weight is folded into W's columns, W[n][k] ln_weight[k], and whose bias into
 * `bias` as W ln_bias; csum (N) = the row sums of the folded W, required); or z = x / sqrt(mean of squares + eps) over
 * each 64-channel group (mode 2, K a multiple of 64 up to 1024) or each 128-channel group (mode 3, K a multiple of
 * 128 up to 2048): the carrier's per-head RMSNorm, its weight folded into W's columns, W[n][k] rms_weight[k mod G]). scale a device scalar or NULL, bias (N) or NULL, act 0 identity / 1 GELU
 * (erf form), resid (B, N) or NULL. W (N, K) is given tiled: Wt[((t (K / 16) + s) 64 + l) 4 + e] = W[16 t + l % 16][16
 * s + 4 (l / 16) + e], zero for columns past N, so Wt holds ceil(N / 16) 16 K floats. K a multiple of 16; y must not
 * alias x or resid. Deterministic; no workspace. pragnosia_decode_gemm_waves gives the waves a workgroup runs for (K,
 * mode), -1 where the kernel does not cover it (the call then returns PRAGNOSIA_ERR_UNSUPPORTED). Replaces the
 * LayerNorm + nn.Linear (+ GELU, + residual) calls of the carrier's projections, its RMSNorm and gated output
 * projection, the MLP (src/model.py:552-560) and the tied head in the reference's batched graphed decode
 * (src/bench.py:241-317), as pragnosia_decode_gemv does for B <= 4. */
int pragnosia_decode_gemm_waves(int64_t K, int mode);
int pragnosia_decode_gemm(const float* x, int64_t B, int64_t K, int mode, const float* csum, float eps,
                          const float* Wt, int64_t N, const float* bias, const float* scale, int act,
                          const float* resid, float* y, void* stream);

/* y (B, N) += scale * (W z) + bias, with z = x (mode 0) or each 64-channel (mode 2) or 128-channel (mode 3) group
 * RMS-scaled as in pragnosia_decode_gemm, K split over groups of workgroups, each adding its partial products (the
 * first split also the bias) into y with fp32 atomics: y holds the residual on entry, so the layer's residual add
 * needs no read of a separate tensor and the layer spreads over more compute units than its column tiles give.
 * Splits: mode 0 four or two (each at least 512 of K, whole 16-wide steps), the RMS modes up to four of whole channel
 * groups (at least four groups a split); 1 where none fits. x and y must not overlap; calls that write one y on one
 * stream are ordered, the adds within a call are not (the sum's rounding order varies run to run: not
 * bit-deterministic). W tiled (and the RMSNorm's weight folded) as for pragnosia_decode_gemm. Replaces the MLP's
 * second nn.Linear + residual and the carrier's RMSNorm + gated output projection + residual (src/model.py:552-560,
 * src/assoc.py:384-512) in the reference's batched graphed decode (src/bench.py:241-317). */
/* y (B, N) += scale * (W x) + bias for B <= 4, W (N, K) row-major fp32 as for pragnosia_decode_gemv, K a multiple of
 * 256 up to 4096: one-wave workgroups per (row, K split), two splits when each keeps at least 768 of K (else one),
 * each adding its partial sum (the first split also the bias) into y with an fp32 atomic: y holds the residual on
 * entry. x and y must not overlap; not bit-deterministic (the adds' order varies). Replaces the MLP's
 * second nn.Linear + residual (src/model.py:552-560) in the reference's graphed decode (src/bench.py:241-317) at the
 * one-wave GEMV's batch sizes. */
int pragnosia_decode_gemv_acc(const float* x, int64_t B, int64_t K, const float* W, int64_t N, const float* bias,
                              const float* scale, float* y, void* stream);

int pragnosia_decode_gemm_acc(const float* x, int64_t B, int64_t K, int mode, float eps, const float* Wt, int64_t N,
                              const float* bias, const float* scale, float* y, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PRAGNOSIA_HIP_H */
