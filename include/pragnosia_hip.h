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

/* ABI version of this header; bumped on any signature change. */
int pragnosia_abi_version(void);

/* Human-readable name of a return code (static storage). */
const char* pragnosia_error_string(int code);

/* ---------------------------------------------------------------------------------------------------------
 * Complex diagonal recurrence with per-token lambda (fspin):
 *     h_t = exp(logmag_t + i ang_t) h_{t-1} + u_t,   h_{-1} = h0r + i h0i (zero when h0r/h0i are NULL).
 * Forward: writes hr = Re h and hi = Im h for every t (both (B, T, D) fp32; hr is the output y, hi is saved for
 * the backward). Replaces `_Scan.forward` / `_fwd` of src/scan_kernel.py:24-50, :105-119.
 * u, logmag, ang: (B, T, D) fp32. h0r, h0i: (B, D) fp32 or NULL (both or neither). */
int pragnosia_diag_scan_fwd(const float* u, const float* logmag, const float* ang,
                            const float* h0r, const float* h0i,
                            float* hr, float* hi,
                            int64_t B, int64_t T, int64_t D, void* stream);

/* Backward of pragnosia_diag_scan_fwd (the adjoint recurrence run in reverse). Replaces `_Scan.backward` /
 * `_bwd` of src/scan_kernel.py:53-99, :121-140, including the folding of the final-state gradients:
 * g_last_r adds to g at t = T-1 and g_last_i seeds the imaginary adjoint (either may be NULL = zero).
 * g, hr, hi, logmag, ang: (B, T, D) fp32; du, dlogmag, dang: (B, T, D) fp32 outputs.
 * h0r/h0i: the forward's initial state or NULL; dh0r/dh0i: (B, D) outputs or NULL (written only if non-NULL). */
int pragnosia_diag_scan_bwd(const float* g, const float* g_last_r, const float* g_last_i,
                            const float* logmag, const float* ang, const float* hr, const float* hi,
                            const float* h0r, const float* h0i,
                            float* du, float* dlogmag, float* dang, float* dh0r, float* dh0i,
                            int64_t B, int64_t T, int64_t D, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PRAGNOSIA_HIP_H */
