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
 * state contiguous [B, HV, K, V].  Supported: K, V in {64, 128}; T <= 8.
 */
int kad_gdn_suffix_replay(const void* q, const void* k, const void* v, int64_t ld_qk,
                          int64_t ld_v, int qkv_dtype, const void* log_decay,
                          int gate_dtype, const void* beta, int beta_dtype,
                          int64_t ld_gate, const void* state, int state_dtype, void* out,
                          int64_t ld_out, int B, int W, int T, int H, int HV, int K,
                          int V, float scale, kad_stream_t stream);
/* kad_causal_conv_suffix (width 4, SiLU, no bias) followed by
 * kad_gdn_suffix_replay, as one call whose conv output never reaches HBM:
 * proj holds each (beam, token) row's pre-conv channels [q (H*K) | k (H*K) |
 * v (HV*V)] at [(n*T+t)*ld_proj + c] (bf16, ld_proj a multiple of 8, 16-byte
 * aligned); conv_state / history / conv_weight ([C, 4] bf16, 8-byte aligned)
 * as in kad_causal_conv_suffix; the rest as in kad_gdn_suffix_replay.  The
 * outputs are the two calls' bits.  Supported: K = V = 128, T in {1, 2},
 * W % 16 == 0, fp32 log decays and bf16 betas (even ld_gate); anything else
 * is KAD_ERR_UNSUPPORTED (the caller then makes the two calls).  No
 * counterpart in the reference as one call: it fuses the decode's
 * causal_conv1d and gated_delta calls (src/kadllm/adapters/qwen3_5.py:146-174),
 * so the suffix rows make one pass through memory instead of three. */
int kad_gdn_suffix_replay_conv(const void* proj, int64_t ld_proj, const void* conv_state,
                               int64_t ss_b, int64_t ss_c, int64_t ss_t, int history,
                               const void* conv_weight, const void* log_decay, int gate_dtype,
                               const void* beta, int beta_dtype, int64_t ld_gate,
                               const void* state, int state_dtype, void* out, int64_t ld_out,
                               int B, int W, int T, int H, int HV, int K, int V, float scale,
                               kad_stream_t stream);
/* kad_gdn_suffix_replay_conv with the layer's gated RMSNorm applied to each
 * output row of a value head on its way out, as kad_rmsnorm_gated computes
 * it (the same bits as the three calls in a row): out = bf16(bf16(w *
 * bf16(o r)) * silu(z)), r = 1 / sqrt(mean(o^2) + eps).  z: gate rows, (n, t)
 * at [(n*T+t)*ldz + hv*V + j] (bf16, ldz a multiple of 4, 8-byte aligned);
 * norm_w: [V] bf16.  last_token_only: only token T-1 of each beam is normed
 * and written, at out row n (the incremental decode reads no other);
 * otherwise every token, at row n*T + t.  No counterpart in the reference as
 * one call: it fuses the decode's causal_conv1d, gated_delta and
 * Qwen3_5RMSNormGated (src/kadllm/adapters/qwen3_5.py:146-176). */
int kad_gdn_suffix_replay_conv_gated(const void* proj, int64_t ld_proj, const void* conv_state,
                                     int64_t ss_b, int64_t ss_c, int64_t ss_t, int history,
                                     const void* conv_weight, const void* log_decay,
                                     int gate_dtype, const void* beta, int beta_dtype,
                                     int64_t ld_gate, const void* state, int state_dtype,
                                     const void* z, int64_t ldz, const void* norm_w, float eps,
                                     int last_token_only, void* out, int64_t ld_out, int B,
                                     int W, int T, int H, int HV, int K, int V, float scale,
                                     kad_stream_t stream);
/* kad_gdn_suffix_replay_conv_gated (last token only, T = 2) reading each
 * beam's earlier token from its parent's cached projection row in place:
 * prev holds the parent level's rows, (b*Wp + p)*(T-1) + t at stride ld_prev
 * (bf16, 16-byte aligned, ld_prev a multiple of 8); parents [B, W] (int64,
 * clamped to [0, Wp)); cur one row per beam of the new token (b*W + w, stride
 * ld_cur); z the new token's gate rows (one per beam); the gates log_decay /
 * beta still in (n*T + t) rows.  The same bits as gathering the parents'
 * rows (kad_gather_beam_rows) into one [B*W*T] buffer and calling
 * kad_gdn_suffix_replay_conv_gated on it.  No counterpart in the reference:
 * it saves the search's last level the copy of the cached rows that the
 * reference's full replay recomputes (src/kadllm/adapters/qwen3_5.py:216). */
int kad_gdn_suffix_replay_conv_gated_parents(
    const void* prev, int64_t ld_prev, const int64_t* parents, int Wp, const void* cur,
    int64_t ld_cur, const void* conv_state, int64_t ss_b, int64_t ss_c, int64_t ss_t,
    int history, const void* conv_weight, const void* log_decay, int gate_dtype,
    const void* beta, int beta_dtype, int64_t ld_gate, const void* state, int state_dtype,
    const void* z, int64_t ldz, const void* norm_w, float eps, void* out, int64_t ld_out, int B,
    int W, int T, int H, int HV, int K, int V, float scale, kad_stream_t stream);

/* --------------------------------------------------------------------------
 * Depthwise causal short convolution over [prefix taps || suffix].
 * Replaces src/kadllm/ops.py:166-226 (causal_conv1d) and
 * src/kadllm/kernels/causal_conv1d.py:10-78 (beam_causal_conv1d_update).
 *
 * y[n,c,t] = act( sum_{i<width} w[c,i] * window[n,c,t+i] ),
 * window = [state[n/W, c, history-(width-1) .. history-1] || x[n, c, 0..T-1]].
 * x, state, out are strided [n, c, t] views (strides in elements); weight is
 * contiguous [C, width].  All tensors share `dtype` (bf16, fp16, fp32).
 * act = SiLU if activation_silu else identity; bias (nullable, [C]) is added
 * before act.  Supported: width <= 64 (width-1 <= history).
 */
int kad_causal_conv_suffix(const void* x, int64_t sx_n, int64_t sx_c, int64_t sx_t,
                           const void* state, int64_t ss_b, int64_t ss_c, int64_t ss_t,
                           int history, const void* weight, int width, const void* bias,
                           void* out, int64_t so_n, int64_t so_c, int64_t so_t, int B,
                           int W, int C, int T, int dtype, int activation_silu,
                           kad_stream_t stream);

/* --------------------------------------------------------------------------
 * bf16 GEMM with fused epilogues: C[M,N] = A[M,K] W[N,K]^T, fp32 accumulate.
 * Replaces the nn.Linear projections of the decode path
 * (src/kadllm/adapters/qwen3_5.py:146,161-162,169,175,177,181-188,202,234-235)
 * and of the transformers prefill they mirror.  Row strides lda, ldw, ldc,
 * ldr in elements; K % 64 == 0; A, W 16-byte aligned.
 *   KAD_EPI_STORE     C = bf16(acc)
 *   KAD_EPI_RESIDUAL  C = bf16(R + bf16(acc)); R may alias C
 *   KAD_EPI_SWIGLU    W rows interleaved in [gate 32 | up 32] blocks (N % 64
 *                     == 0); C[:, j] = bf16(bf16(silu(bf16 g_j)) * bf16 u_j),
 *                     N/2 output columns
 */
#define KAD_EPI_STORE 0
#define KAD_EPI_RESIDUAL 1
#define KAD_EPI_SWIGLU 2
int kad_gemm_bf16(const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
                  const void* R, int64_t ldr, int M, int N, int K, int epilogue,
                  kad_stream_t stream);

/* kad_gemm_bf16 (KAD_EPI_STORE) of the prefill's GDN input projection with
 * the depthwise causal conv (width 4, SiLU, no bias, zero history) of its
 * first conv_cols columns fused into the epilogue: C[:, :conv_cols] receives
 * the conv outputs kad_causal_conv_prefill would compute from the projection,
 * C[:, conv_cols:N] the plain product, conv_state ([M / seq_len, conv_cols, 4]
 * bf16, nullable) the last 4 inputs of each sequence, all the same bits as
 * the two calls.  Rows are seq_len-token sequences; workspace: at least
 * kad_gemm_bf16_conv_workspace_bytes (16-byte aligned).  Supported: M, N,
 * conv_cols multiples of 256 (conv_cols <= N), K % 64 == 0, seq_len % 128 ==
 * 0; anything else is KAD_ERR_UNSUPPORTED.  No counterpart in the reference
 * as one call: it fuses in_proj_qkv and the causal conv1d of the prefill the
 * reference runs through transformers (src/kadllm/adapters/qwen3_5.py:111),
 * so the conv's input never reaches HBM. */
int kad_gemm_bf16_conv_workspace_bytes(int M, int conv_cols, int64_t* bytes);
int kad_gemm_bf16_conv(const void* A, int64_t lda, const void* W, int64_t ldw, void* C,
                       int64_t ldc, int M, int N, int K, int conv_cols, const void* conv_weight,
                       int seq_len, void* conv_state, void* workspace, int64_t workspace_bytes,
                       kad_stream_t stream);

/* Same with an explicit tile configuration, the forms the automatic choice
 * picks from (0 = automatic choice as kad_gemm_bf16; 1 = 32x256 with 4 waves;
 * 2 = 128x128 with 4 waves; 5 = 256x256 with 8 waves; 11 = 64x32 with 2
 * waves, no SwiGLU epilogue; 12 = 32x64 with 2 waves, no SwiGLU epilogue;
 * 13 = outputs of at most 32 columns, one wave per 32 rows over the whole
 * of K with the weight in LDS, K a multiple of 256 up to 2,048, 16-byte
 * aligned A and W rows, no SwiGLU epilogue; 16 = 256x256 with 8 waves on 16x16x32 MFMAs,
 * direct-to-LDS loads and a 16-byte store epilogue, which needs 16-byte
 * aligned C (and R) with ldc, ldr and the output width multiples of 8;
 * 18 = 16 persistent, one workgroup per CU walking the tiles; 19 = 16's
 * design on 128x128 tiles with 4 waves, two workgroups per CU; 20 = 16 with
 * a third LDS slot for the operand that streams from beyond the L2; 22 =
 * 256x256 persistent with its 8 waves in two groups that alternate between
 * MFMA phases and load phases across workgroup barriers, M and N multiples
 * of 256, 16-byte store epilogue as 16; 24 = 256x256 persistent with 4
 * waves of 128x128, M and N multiples of 256, epilogues from the
 * accumulators, aligned outputs as 16).  Every
 * configuration accumulates K in the same order, so all give bit-identical
 * results (the automatic choice may also split the columns of one call
 * between two of them); other numbers are rejected (KAD_ERR_UNSUPPORTED). */
int kad_gemm_bf16_tiled(const void* A, int64_t lda, const void* W, int64_t ldw, void* C,
                        int64_t ldc, const void* R, int64_t ldr, int M, int N, int K,
                        int epilogue, int tile_config, kad_stream_t stream);

/* --------------------------------------------------------------------------
 * Row-wise layer kernels (bf16).  They replace the transformers modules the
 * reference decode calls between its projections (src/kadllm/adapters/
 * qwen3_5.py:161-176,184-189,216-226,234-235) and reproduce their bf16
 * rounding points.
 *
 * kad_rmsnorm        Qwen3_5RMSNorm: y = bf16(x rsqrt(mean x^2 + eps) (w_offset + w)),
 *                    rows of D (D % 8 == 0), row strides ldx/ldy.
 * kad_rmsnorm_gated  Qwen3_5RMSNormGated over `heads` groups of D per token:
 *                    y = bf16(bf16(w bf16(x r)) silu(z)).
 * kad_gdn_gates      g = -exp(A_log) softplus(a + dt_bias) (fp32, [rows, HV]),
 *                    beta = bf16(sigmoid(b)) ([rows, HV]); a/b strided bf16.
 * kad_qk_norm_rope   per (token, head): optional RMSNorm(1+w) over D, then
 *                    rotate-half RoPE on the first `rot` dims with
 *                    position pos0 + token % pos_period, bf16 cos/sin of
 *                    fp32 angles pos * inv_freq[i]; writes to
 *                    dst + (token / period) s_b + (token % period) s_t + head s_h.
 * kad_scatter_heads  copies [rows, heads, D] head rows into that strided layout.
 * kad_embedding      out[r] = table[ids[r]] (ids clamped into [0, vocab)).
 */
int kad_rmsnorm(const void* x, int64_t ldx, const void* w, float w_offset, void* y, int64_t ldy,
                int64_t rows, int D, float eps, kad_stream_t stream);
int kad_rmsnorm_gated(const void* x, int64_t ldx, const void* z, int64_t ldz, const void* w,
                      void* y, int64_t ldy, int64_t rows, int heads, int D, float eps,
                      kad_stream_t stream);
int kad_gdn_gates(const void* a, int64_t lda, const void* b, int64_t ldb, const void* A_log,
                  const void* dt_bias, float* g, void* beta, int64_t rows, int HV,
                  kad_stream_t stream);
int kad_qk_norm_rope(const void* src, int64_t ld_src, int64_t src_head_stride, int heads,
                     const void* w, void* dst, int64_t period, int64_t s_b, int64_t s_t,
                     int64_t s_h, int64_t rows, int D, int rot, const float* inv_freq,
                     int64_t pos0, int64_t pos_period, float eps, int do_norm,
                     kad_stream_t stream);
int kad_scatter_heads(const void* src, int64_t ld_src, int heads, int D, void* dst,
                      int64_t period, int64_t s_b, int64_t s_t, int64_t s_h, int64_t rows,
                      kad_stream_t stream);
int kad_embedding(const int64_t* ids, const void* table, void* out, int64_t rows, int D,
                  int64_t vocab, kad_stream_t stream);

/* --------------------------------------------------------------------------
 * Prefix-shared gated GQA decode attention (bf16 in/out, fp32 softmax).
 * Replaces src/kadllm/ops.py:229-341 (prefix_attention, merge_attention) and
 * src/kadllm/kernels/flash_attention.py:11-66, with the sigmoid output gate of
 * src/kadllm/adapters/qwen3_5.py:199-201 fused (gate may be null).
 *
 * Row (n, t, h) of q [B*W, T, H, D] attends to the prefix keys of request
 * b = n / W (prefix_k/v [B, L, HK, D] strided views, kv head h / (H/HK),
 * keys with prefix_mask[b, key] == 0 excluded when the mask is given) and to
 * suffix keys j <= t of its own beam (suffix_k/v [B*W, T, HK, D]).  One
 * softmax over both (equal to the reference's LSE merge); out = bf16(o),
 * times bf16(sigmoid(gate)) when gated.  Strides in elements.  T <= 8;
 * D in {64, 128, 256}; prefix_mask is uint8/bool [B, L].
 */
int kad_prefix_attention_decode(
    const void* q, int64_t sq_n, int64_t sq_t, int64_t sq_h, const void* prefix_k,
    const void* prefix_v, int64_t sp_b, int64_t sp_l, int64_t sp_h, const void* suffix_k,
    int64_t ssk_n, int64_t ssk_t, int64_t ssk_h, const void* suffix_v, int64_t ssv_n,
    int64_t ssv_t, int64_t ssv_h, const void* prefix_mask, const void* gate, int64_t sg_n,
    int64_t sg_t, int64_t sg_h, void* out, int64_t so_n, int64_t so_t, int64_t so_h, int B,
    int W, int T, int H, int HK, int L, int D, float scale, kad_stream_t stream);
/* The same for queries that are only the last Tq of a beam's Tk suffix tokens
 * (q/gate/out [B*W, Tq, H, D], suffix_k/v [B*W, Tk, HK, D]): query t sees
 * suffix keys j <= t + Tk - Tq.  Each query row's arithmetic is exactly that
 * of kad_prefix_attention_decode with T = Tk, which lets a level that extends
 * cached suffixes by one token (src/kadllm/grbeam.py:76-77, where the
 * reference replays the whole suffix, src/kadllm/adapters/qwen3_5.py:216) skip
 * the queries of the cached tokens.  Tq <= Tk <= 8. */
int kad_prefix_attention_decode_ex(
    const void* q, int64_t sq_n, int64_t sq_t, int64_t sq_h, const void* prefix_k,
    const void* prefix_v, int64_t sp_b, int64_t sp_l, int64_t sp_h, const void* suffix_k,
    int64_t ssk_n, int64_t ssk_t, int64_t ssk_h, const void* suffix_v, int64_t ssv_n,
    int64_t ssv_t, int64_t ssv_h, const void* prefix_mask, const void* gate, int64_t sg_n,
    int64_t sg_t, int64_t sg_h, void* out, int64_t so_n, int64_t so_t, int64_t so_h, int B,
    int W, int Tq, int Tk, int H, int HK, int L, int D, float scale, kad_stream_t stream);

/* Causal gated GQA attention over full prompts (prefill).  Replaces the
 * causal SDPA of the transformers forward that the reference prefill runs
 * (src/kadllm/adapters/qwen3_5.py:111).  q/out/gate [B, L, H, D]-strided,
 * k/v [B, L, HK, D]-strided (e.g. views of [B, HK, L, D] caches). */
int kad_attention_prefill(const void* q, int64_t sq_b, int64_t sq_l, int64_t sq_h,
                          const void* k, const void* v, int64_t skv_b, int64_t skv_l,
                          int64_t skv_h, const void* gate, int64_t sg_b, int64_t sg_l,
                          int64_t sg_h, void* out, int64_t so_b, int64_t so_l, int64_t so_h,
                          int B, int L, int H, int HK, int D, float scale, kad_stream_t stream);

/* --------------------------------------------------------------------------
 * Beam selection: full-vocabulary log-softmax, optional bool constraint,
 * parent-score add and top-W, without fp32 [W, V] temporaries.  Replaces
 * src/kadllm/grbeam.py:89-104.  Ties are broken by the lower flat index
 * (parent * V + token); torch.topk leaves that order unspecified.
 *
 * kad_beam_row_select    per beam row r (rows = B * Wp, row stride ld of the
 *                        logits, dtype logits_dtype: bf16, fp16 or fp32; mask
 *                        uint8 [rows, V] (ld_mask) or null): writes the row's
 *                        K = min(W, V) best candidates,
 *                        key = ((x - max_r) - log sum exp(x - max_r)) + parent[r]
 *                        (-inf where masked) and flat index (r % Wp) * V + c,
 *                        to cand_key / cand_idx [rows, K].
 * kad_beam_merge_select  per request b: the W best of its ncand = Wp * K
 *                        candidates, sorted by (key desc, index asc): scores
 *                        [B, W] fp32, parents = index / V, tokens = index % V
 *                        (int64), valid = isfinite(score) (uint8).  W <= 16384.
 * kad_beam_merge_select_wide  the same selection for any W (the reference's
 *                        topk has no width cap, src/kadllm/grbeam.py:95):
 *                        the radix rounds histogrammed by many workgroups
 *                        per request, the winners sorted in caller workspace
 *                        of kad_beam_merge_select_wide_workspace_bytes(B, W)
 *                        bytes (16-byte aligned).  Keys are ordered by their
 *                        order-preserving bit pattern, so -0 ranks below +0,
 *                        where kad_beam_merge_select's sort treats them as a
 *                        tie; otherwise the results are identical.
 * kad_beam_history       out[b, w, :] = [history[b, parents[b, w], :step], tokens[b, w]]
 *                        (history [B, Wp, step] int64, out [B, W, step + 1]).
 */
int kad_beam_row_select(const void* logits, int logits_dtype, int64_t ld, const void* mask,
                        int64_t ld_mask, const float* parent_scores, int rows, int Wp, int V,
                        int K, float* cand_key, int* cand_idx, kad_stream_t stream);
int kad_beam_merge_select(const float* cand_key, const int* cand_idx, int B, int ncand, int W,
                          int V, float* scores, int64_t* parents, int64_t* tokens, void* valid,
                          kad_stream_t stream);
int kad_beam_merge_select_wide_workspace_bytes(int B, int W, int64_t* bytes);
int kad_beam_merge_select_wide(const float* cand_key, const int* cand_idx, int B, int ncand,
                               int W, int V, float* scores, int64_t* parents, int64_t* tokens,
                               void* valid, void* workspace, int64_t workspace_bytes,
                               kad_stream_t stream);
/* Allocation-free selection: kad_beam_row_select then kad_beam_merge_select
 * (same arguments, same results bit for bit) with the candidates kept in a
 * 32 MiB device array inside the library instead of caller workspace, so the
 * call makes no hipMalloc and no other allocation.  No counterpart in the
 * reference: it serves callers that cannot allocate (code under stream
 * capture, tight serving loops).  Limit: B * Wp * min(W, V) <= 4,194,304
 * candidates (e.g. 32 requests x 256 beams x 256), else KAD_ERR_UNSUPPORTED.
 * Each GPU has one such array for the life of the process, shared by every
 * call on it: calls that overlap on one GPU (different streams or host
 * threads) race and must be serialised by the caller. */
int kad_beam_select_noalloc(const void* logits, int logits_dtype, int64_t ld, const void* mask,
                            int64_t ld_mask, const float* parent_scores, int B, int Wp, int V,
                            int W, float* scores, int64_t* parents, int64_t* tokens, void* valid,
                            kad_stream_t stream);
int kad_beam_history(const int64_t* history, int Wp, int step, const int64_t* parents,
                     const int64_t* tokens, int64_t* out, int B, int W, kad_stream_t stream);
/* Per-token rows cached for a level's beams follow the beams' parents into the
 * next level: for beam n = b * W + w and t < rows_copy, dst row
 * n * dst_rows_per_beam + t = src row (b * Wp + parents[n]) * src_rows_per_beam
 * + t (row_bytes each, byte strides ld_*; 16-byte aligned; parents clamped to
 * [0, Wp)).  Serves the suffix dedup across levels: the reference recomputes
 * these rows (src/kadllm/adapters/qwen3_5.py:216, README.md:252). */
int kad_gather_beam_rows(const void* src, int64_t ld_src_bytes, int src_rows_per_beam, void* dst,
                         int64_t ld_dst_bytes, int dst_rows_per_beam, int rows_copy,
                         int64_t row_bytes, const int64_t* parents, int B, int W, int Wp,
                         kad_stream_t stream);

/* --------------------------------------------------------------------------
 * Chunked gated delta rule over sequences (chunks of 64 tokens).
 * Replaces the prefill's transformers torch_chunk_gated_delta_rule reached
 * through src/kadllm/adapters/qwen3_5.py:111, and src/kadllm/ops.py:139-163
 * (gated_delta) for suffixes longer than kad_gdn_suffix_replay handles and
 * for final-state requests (ops.py:119-122).
 *
 * N sequences of T tokens; q/k/v/out/gates laid out as in
 * kad_gdn_suffix_replay with n in [0, N).  initial_state (nullable, [N /
 * beams_per_state, HV, K, V]) is read for sequence n at n / beams_per_state;
 * final_state (nullable, fp32 [N, HV, K, V]) receives each sequence's final
 * state.  transformers_l2norm = 1 normalises q and k with the bf16 roundings
 * of transformers' l2norm (prefill); 0 normalises in fp32 as ops.py:147-148.
 * workspace: caller-owned device memory of at least the size reported by
 * kad_gdn_chunk_workspace_bytes (per-chunk intermediates).  bf16 q/k/v;
 * K, V in {64, 128}; q/k/v and out rows 16-byte aligned.
 */
int kad_gdn_chunk_workspace_bytes(int N, int T, int HV, int K, int64_t* bytes);
int kad_gdn_chunk(const void* q, const void* k, const void* v, int64_t ld_qk, int64_t ld_v,
                  int qkv_dtype, const void* log_decay, int gate_dtype, const void* beta,
                  int beta_dtype, int64_t ld_gate, const void* initial_state, int state_dtype,
                  int beams_per_state, void* out, int64_t ld_out, float* final_state,
                  void* workspace, int64_t workspace_bytes, int N, int T, int H, int HV, int K,
                  int V, float scale, int transformers_l2norm, kad_stream_t stream);
/* kad_gdn_chunk (transformers l2norm) with the layer's gated RMSNorm applied
 * to each output row of a value head on its way out: out = bf16(bf16(w *
 * bf16(o r)) * silu(z)), r = 1 / sqrt(mean(o^2) + eps) per (token, value
 * head), o the chunk rule's bf16 output, as kad_rmsnorm_gated computes it
 * (the same bits as the two calls in a row).  z: [N*T rows, HV*V] bf16 row
 * strided (the gate projection columns), ldz a multiple of 8, 16-byte
 * aligned; norm_w: [V] bf16.  No counterpart in the reference as one call:
 * it fuses the chunk rule and the Qwen3_5RMSNormGated that follows it in the
 * prefill the reference runs through transformers
 * (src/kadllm/adapters/qwen3_5.py:111), so the output rows make one pass
 * through memory instead of three. */
int kad_gdn_chunk_gated(const void* q, const void* k, const void* v, int64_t ld_qk, int64_t ld_v,
                        int qkv_dtype, const void* log_decay, int gate_dtype, const void* beta,
                        int beta_dtype, int64_t ld_gate, const void* initial_state,
                        int state_dtype, int beams_per_state, void* out, int64_t ld_out,
                        float* final_state, void* workspace, int64_t workspace_bytes, int N,
                        int T, int H, int HV, int K, int V, float scale, const void* z,
                        int64_t ldz, const void* norm_w, float eps, kad_stream_t stream);

/* Causal width-4 conv + SiLU over whole prompts with zero history, and the
 * conv state (last 4 pre-conv inputs, [B, C, 4], nullable) that decode reads.
 * Replaces the prefill's transformers causal_conv1d_fn and conv-state cache
 * update reached through src/kadllm/adapters/qwen3_5.py:111.  x/out are
 * [B*L, C] row-strided bf16 (row = b*L + t); weight [C, 4]. */
int kad_causal_conv_prefill(const void* x, int64_t ldx, const void* weight, void* out,
                            int64_t ldo, void* state, int B, int L, int C, int activation_silu,
                            kad_stream_t stream);

/* --------------------------------------------------------------------------
 * General-shape kernels: any head dimension <= 256, any suffix length, bf16,
 * fp16 or fp32 tensors, fp32 arithmetic.  They serve the shapes the kernels
 * above do not: the reference operators take any shape and dtype
 * (src/kadllm/ops.py:70-163,252-341), and its toy model runs 8-wide heads in
 * fp32 over whole prompts (src/kadllm/adapters/reference.py:56-91).
 *
 * kad_gdn_recurrent      the token-by-token gated delta rule of ops.py:139-163
 *                        (src/kadllm/ops.py:70-163, gated_delta): layouts as
 *                        kad_gdn_suffix_replay with n in [0, N); q, k
 *                        L2-normalised in fp32 (q / sqrt(sum q^2 + 1e-6) *
 *                        scale); initial_state [N / beams_per_state, HV, K, V]
 *                        (nullable: zeros); final_state fp32 [N, HV, K, V]
 *                        (nullable); out in the q/k/v dtype.  K <= 256.
 * kad_attention_general  kad_prefix_attention_decode_ex's contract (queries
 *                        are the last Tq of Tk suffix tokens; Tk = Tq is the
 *                        reference operator, src/kadllm/ops.py:252-341) for
 *                        any Tq <= Tk, L >= 0 and D <= 256, all tensors of
 *                        `dtype`; fully masked rows give zeros.
 */
int kad_gdn_recurrent(const void* q, const void* k, const void* v, int64_t ld_qk, int64_t ld_v,
                      int qkv_dtype, const void* log_decay, int gate_dtype, const void* beta,
                      int beta_dtype, int64_t ld_gate, const void* initial_state,
                      int state_dtype, int beams_per_state, void* out, int64_t ld_out,
                      float* final_state, int N, int T, int H, int HV, int K, int V, float scale,
                      kad_stream_t stream);
int kad_attention_general(
    const void* q, int64_t sq_n, int64_t sq_t, int64_t sq_h, const void* prefix_k,
    const void* prefix_v, int64_t sp_b, int64_t sp_l, int64_t sp_h, const void* suffix_k,
    int64_t ssk_n, int64_t ssk_t, int64_t ssk_h, const void* suffix_v, int64_t ssv_n,
    int64_t ssv_t, int64_t ssv_h, const void* prefix_mask, const void* gate, int64_t sg_n,
    int64_t sg_t, int64_t sg_h, void* out, int64_t so_n, int64_t so_t, int64_t so_h, int B,
    int W, int Tq, int Tk, int H, int HK, int L, int D, int dtype, float scale,
    kad_stream_t stream);

/* --------------------------------------------------------------------------
 * fp32 models.  The reference adapter runs any float model (src/kadllm/
 * adapters/qwen3_5.py:40-104 wraps the transformers model in its own dtype)
 * and states its fixed-history accuracy for fp32 runs (README.md:152).  These
 * are the projections and row-wise ops of kad_gemm_bf16 / kad_rmsnorm ...
 * in fp32 with no intermediate rounding (same argument meaning, fp32
 * tensors); attention and gated delta of an fp32 model use the general-shape
 * kernels above, the conv kad_causal_conv_suffix.
 *
 * kad_gemm_f32           C = A W^T (v_mfma_f32_16x16x4_f32), epilogues as
 *                        kad_gemm_bf16 (SwiGLU: silu(g) u of interleaved
 *                        [gate 32 | up 32] W rows, N % 64 == 0)
 * kad_rmsnorm_f32        y = x rsqrt(mean x^2 + eps) (w_offset + w)
 * kad_rmsnorm_gated_f32  y = w (x rsqrt(mean x^2 + eps)) silu(z) per head
 * kad_gdn_gates_f32      g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b)
 * kad_qk_norm_rope_f32   kad_qk_norm_rope with fp32 cos/sin and no rounding
 * kad_embedding_f32      out[r] = table[ids[r]]
 */
int kad_gemm_f32(const float* A, int64_t lda, const float* W, int64_t ldw, float* C, int64_t ldc,
                 const float* R, int64_t ldr, int M, int N, int K, int epilogue,
                 kad_stream_t stream);
int kad_rmsnorm_f32(const float* x, int64_t ldx, const float* w, float w_offset, float* y,
                    int64_t ldy, int64_t rows, int D, float eps, kad_stream_t stream);
int kad_rmsnorm_gated_f32(const float* x, int64_t ldx, const float* z, int64_t ldz,
                          const float* w, float* y, int64_t ldy, int64_t rows, int heads, int D,
                          float eps, kad_stream_t stream);
int kad_gdn_gates_f32(const float* a, int64_t lda, const float* b, int64_t ldb,
                      const float* A_log, const float* dt_bias, float* g, float* beta,
                      int64_t rows, int HV, kad_stream_t stream);
int kad_qk_norm_rope_f32(const float* src, int64_t ld_src, int64_t src_head_stride, int heads,
                         const float* w, float* dst, int64_t period, int64_t s_b, int64_t s_t,
                         int64_t s_h, int64_t rows, int D, int rot, const float* inv_freq,
                         int64_t pos0, int64_t pos_period, float eps, int do_norm,
                         kad_stream_t stream);
int kad_embedding_f32(const int64_t* ids, const float* table, float* out, int64_t rows, int D,
                      int64_t vocab, kad_stream_t stream);

/* --------------------------------------------------------------------------
 * HBM streaming probe (no reference counterpart): the bandwidth a plain
 * streaming kernel reaches on this device, for reporting the HBM-bound
 * kernels against it beside the datasheet peak.  mode 0 copies `bytes` from
 * src to dst (read + write), 1 reads src (dst receives at most a few
 * sentinel words), 2 writes dst.  bytes a multiple of 16, buffers 16-byte
 * aligned; src may be NULL for mode 2.
 */
int kad_hbm_probe(const void* src, void* dst, int64_t bytes, int mode, kad_stream_t stream);

/* --------------------------------------------------------------------------
 * Cache prefetch (no reference counterpart; the reference leaves weight
 * traffic to its GEMM library): reads the whole 16-byte pieces of up to two
 * ranges [p0, p0 + bytes0) and [p1, p1 + bytes1) with cache-allocating loads
 * and discards them, so that the next kernels on the stream find those bytes
 * in the last-level cache.  A range with 0 bytes may have a NULL pointer;
 * ranges 16-byte aligned.  Writes nothing; results of later kernels do not
 * depend on it.  The decode levels call it for the MLP and QKV weights ahead
 * of their GEMMs.
 */
int kad_cache_prefetch(const void* p0, int64_t bytes0, const void* p1, int64_t bytes1,
                       kad_stream_t stream);

/* --------------------------------------------------------------------------
 * MFMA lane-layout self-test (no reference counterpart): C[16x16] = A[16x32]
 * B[32x16] (bf16 in, fp32 out, all row-major) computed by one wave with the
 * operand layout the kernels above assume for v_mfma_f32_16x16x32_bf16, and
 * the same for v_mfma_f32_32x32x16_bf16 (A 32x16, B 16x32, C 32x32).
 */
int kad_selftest_mfma16(const void* a, const void* b, float* c, kad_stream_t stream);
int kad_selftest_mfma32(const void* a, const void* b, float* c, kad_stream_t stream);
/* the same for v_mfma_f32_16x16x4_f32 (fp32 A 16x4, B 4x16, C 16x16) */
int kad_selftest_mfma_f32(const float* a, const float* b, float* c, kad_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KADLLM_HIP_H */
