/*
 * kadllm_hip.h -- C ABI of libkadllm_hip.so, the MI355X (gfx950) kernels of
 * the GRBeam shared-prefix beam decode.
 *
 * Conventions
 *   - Every entry point returns int: KAD_OK (0) on success, a negative
 *     KAD_ERR_* code otherwise; kad_last_error() then describes the failure.
 *   - Pointers are device pointers; sizes and strides are in elements.
 *   - Nothing is allocated or retained: outputs and workspaces are caller
 *     owned, inputs marked const (the shared prefix, weights) are never written.
 *   - Work is enqueued on `stream` (the caller's current HIP stream); no entry
 *     point synchronises the host.
 *   - dtype codes: KAD_DTYPE_BF16, KAD_DTYPE_F16, KAD_DTYPE_F32.
 *
 * Each declaration names the reference interface it replaces (file:line in
 * Greek-Guardian/Kadllm); the Python package kadllm_amd binds them through
 * ctypes.
 */
#ifndef KADLLM_HIP_H
#define KADLLM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* kad_stream_t; /* == hipStream_t */

#define KAD_OK 0
#define KAD_ERR_INVALID_ARGUMENT (-1)
#define KAD_ERR_UNSUPPORTED (-2)
#define KAD_ERR_HIP (-3)

#define KAD_DTYPE_BF16 0
#define KAD_DTYPE_F16 1
#define KAD_DTYPE_F32 2

/* Message of the last failed call on this host thread. */
const char* kad_last_error(void);
/* ABI version of this library (bumped on any signature change). */
int kad_abi_version(void);

/* --------------------------------------------------------------------------
 * Gated DeltaNet suffix replay.
 * Replaces src/kadllm/ops.py:70-163 (gated_delta) and its accelerated
 * kernels src/kadllm/kernels/gated_delta.py:14-238 (beam_fused_recurrent_gdn).
 *
 * For request b = n / W, value head hv (qk head h = hv / (HV/H)), each beam n
 * applies its T suffix tokens to the request-shared state S0 = state[b, hv]
 * ([K, V]) without copying it:
 *   S <- S*exp(g_t);  u_t = beta_t (v_t - S^T k_t);  S <- S + k_t u_t^T;
 *   o_t = S^T q_t
 * with q, k L2-normalised (eps 1e-6) and q scaled by `scale`.
 * Layout (element strides): q/k (n,t,h,i) at [(n*T+t)*ld_qk + h*K + i];
 * v/out (n,t,hv,j) at [(n*T+t)*ld_v + hv*V + j] (ld_out for out);
 * log_decay/beta (n,t,hv) at [(n*T+t)*ld_gate + hv];
 * state contiguous [B, HV, K, V].  Supported: K, V in {64, 128}; T <= 4.
 */
int kad_gdn_suffix_replay(const void* q, const void* k, const void* v, int64_t ld_qk,
                          int64_t ld_v, int qkv_dtype, const void* log_decay,
                          int gate_dtype, const void* beta, int beta_dtype,
                          int64_t ld_gate, const void* state, int state_dtype, void* out,
                          int64_t ld_out, int B, int W, int T, int H, int HV, int K,
                          int V, float scale, kad_stream_t stream);

/* --------------------------------------------------------------------------
 * Depthwise causal short convolution over [prefix taps || suffix].
 * Replaces src/kadllm/ops.py:166-226 (causal_conv1d) and
 * src/kadllm/kernels/causal_conv1d.py:10-78 (beam_causal_conv1d_update).
 *
 * y[n,c,t] = act( sum_{i<width} w[c,i] * window[n,c,t+i] ),
 * window = [state[n/W, c, history-(width-1) .. history-1] || x[n, c, 0..T-1]].
 * x, state, out are strided [n, c, t] views (strides in elements); weight is
 * contiguous [C, width].  All tensors share `dtype`.  act = SiLU if
 * activation_silu else identity; bias (nullable, [C]) is added before act.
 * Supported: width <= 4 (width-1 <= history).
 */
int kad_causal_conv_suffix(const void* x, int64_t sx_n, int64_t sx_c, int64_t sx_t,
                           const void* state, int64_t ss_b, int64_t ss_c, int64_t ss_t,
                           int history, const void* weight, int width, const void* bias,
                           void* out, int64_t so_n, int64_t so_c, int64_t so_t, int B,
                           int W, int C, int T, int dtype, int activation_silu,
                           kad_stream_t stream);

/* --------------------------------------------------------------------------
 * MFMA lane-layout self-test (no reference counterpart): C[16x16] = A[16x32]
 * B[32x16] (bf16 in, fp32 out, all row-major) computed by one wave with the
 * operand layout the kernels above assume for v_mfma_f32_16x16x32_bf16, and
 * the same for v_mfma_f32_32x32x16_bf16 (A 32x16, B 16x32, C 32x32).
 */
int kad_selftest_mfma16(const void* a, const void* b, float* c, kad_stream_t stream);
int kad_selftest_mfma32(const void* a, const void* b, float* c, kad_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KADLLM_HIP_H */
