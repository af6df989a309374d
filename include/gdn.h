/*
 * gdn.h -- C ABI of libgdn.so, the MI355X (gfx950) Gated DeltaNet token-mixing path.
 *
 * Plain C: device pointers, int64 sizes, dtype codes and a stream handle (a hipStream_t passed as
 * void*; NULL is the legacy default stream). No entry point allocates device memory; outputs and
 * any workspace are owned by the caller. Every entry point returns GDN_OK or a non-zero status,
 * and gdn_last_error() returns a message for the calling thread's last failure.
 *
 * Layouts (row-major, contiguous, last axis fastest):
 *   q, k        [B, T, H,  K]      v, o  [B, T, HV, V]       g, beta [B, T, HV]
 *   states      [N, HV, K, V] fp32 (V fastest)
 *   cu_seqlens  [N + 1] int32 or int64 on the device, 0 = cu[0] < ... < cu[N] = T, with B == 1.
 *   Without cu_seqlens, N == B and every batch row is one sequence.
 * HV must be a multiple of H: value head i reads q/k head i / (HV / H).
 */
#ifndef SORERNN_AMD_GDN_H
#define SORERNN_AMD_GDN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDN_ABI_VERSION 7

#if defined(__GNUC__) || defined(__clang__)
#define GDN_API __attribute__((visibility("default")))
#else
#define GDN_API
#endif

/* status codes */
#define GDN_OK 0
#define GDN_ERR_INVALID 1 /* an argument violates the contract (shape, dtype, pointer) */
#define GDN_ERR_UNSUPPORTED 2 /* a legal combination this build does not implement */
#define GDN_ERR_HIP 3 /* the HIP runtime reported an error */

/* dtype codes */
#define GDN_DTYPE_F32 0
#define GDN_DTYPE_BF16 1
#define GDN_DTYPE_F16 2

/* flags for the delta-rule entry points */
#define GDN_FLAG_QK_L2NORM 0x1u /* L2-normalise q and k per (token, head) in the kernel */
#define GDN_FLAG_BETA_SIGMOID 0x2u /* beta holds logits: use sigmoid(beta) */
#define GDN_FLAG_GATE_IN_KERNEL 0x4u /* g holds a: use g = -exp(A_log[h]) * softplus(a + dt_bias[h]) */
#define GDN_FLAG_CU_INT32 0x8u /* cu_seqlens is int32 (default int64) */

/* activation codes for the conv and the gated norm */
#define GDN_ACT_NONE 0
#define GDN_ACT_SILU 1
#define GDN_ACT_SILU_ROUNDED 2 /* gdn_qkv_conv_fwd only: the conv output rounded to x_dtype, then SiLU */

/* ABI version of the loaded library (GDN_ABI_VERSION at build time). */
GDN_API int gdn_abi_version(void);

/* Message for the calling thread's last failed call ("" if none). */
GDN_API const char* gdn_last_error(void);

/*
 * Chunked gated delta rule forward (prefill), C = 64 tokens per chunk.
 * Replaces FLA 0.5.2 chunk_gated_delta_rule(q, k, v, g, beta, scale, initial_state,
 * output_final_state, use_qk_l2norm_in_kernel, use_beta_sigmoid_in_kernel, ..., cu_seqlens,
 * cu_seqlens_cpu) as called at sore/model/gdn.py:166-169 (signature:
 * docs/superpowers/plans/2026-10-23-sorernn-v2-core.md:141; gate kwargs gdn.py:157-162).
 * q/k/v/o are bf16; g and beta have their own dtypes. initial_state may be NULL (zero state);
 * final_state may be NULL (not written). A_log/dt_bias [HV] fp32 are read only with
 * GDN_FLAG_GATE_IN_KERNEL. K and V must each be 64 or 128.
 * workspace: caller-owned device memory of at least gdn_chunk_workspace_size(B, T, HV, N,
 * cu_seqlens != NULL) bytes (the per-chunk (I + A)^-1 rows passed between the two kernels of the
 * call; its contents on entry do not matter). Calls that share a workspace must not overlap.
 */
GDN_API int gdn_chunk_fwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                  const float* initial_state, void* o, float* final_state, const void* cu_seqlens,
                  int64_t B, int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, int64_t N,
                  int qkv_dtype, int g_dtype, int beta_dtype, float scale, unsigned flags,
                  const float* A_log, const float* dt_bias, void* workspace, size_t workspace_bytes,
                  void* stream);

/*
 * gdn_chunk_fwd with the layer's gated RMSNorm applied to o in the same call (inference only):
 * o = rmsnorm(o_rule) * norm_weight * silu(gate) per (token, value head) over the V values, with
 * rmsnorm(x) = x / sqrt(mean(x^2) + norm_eps) of the rule's output rounded to bf16 -- what FLA
 * rms_norm_gated(o, gate, weight, None, activation="swish", eps) computes from chunk_gated_delta_rule's
 * o (sore/model/gdn.py:166-169 then 182-186), in fp32 with one rounding, with the arithmetic of
 * gdn_rms_norm_gated_fwd. norm_split != 0 rounds like the reference's unfused route instead,
 * o_norm(o) * F.silu(gate) (gdn.py:188): the norm result and silu(gate) each rounded to bf16, then
 * their product. gate [B, T, HV, V] bf16, norm_weight [V] fp32. The rule's own o is not returned:
 * the result is written over it in o. When the chunk kernel's V / 32 column slices leave at least two
 * CUs per (sequence, head) free, workgroups of the same launch apply the norm to each 64-token
 * tile once all its slices have stored it (progress words in the workspace, which must hold
 * gdn_chunk_gated_norm_workspace_size bytes). Otherwise the norm kernel runs in place after the
 * chunk kernel. On both routes a slice whose fp16 operands overflowed recomputes its columns in
 * fp32 (on the first route from its first non-finite chunk, before that chunk is normalised), as
 * gdn_chunk_fwd does.
 */
GDN_API int gdn_chunk_fwd_gated_norm(const void* q, const void* k, const void* v, const void* g, const void* beta,
                             const float* initial_state, void* o, float* final_state, const void* cu_seqlens,
                             int64_t B, int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, int64_t N,
                             int qkv_dtype, int g_dtype, int beta_dtype, float scale, unsigned flags,
                             const float* A_log, const float* dt_bias, const void* gate, const float* norm_weight,
                             float norm_eps, int norm_split, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes gdn_chunk_fwd_gated_norm needs; 0 for invalid sizes. No counterpart in the reference. */
GDN_API size_t gdn_chunk_gated_norm_workspace_size(int64_t B, int64_t T, int64_t HV, int64_t N, int64_t V, int varlen);

/*
 * Workspace bytes gdn_chunk_fwd needs for these sizes (varlen != 0 when cu_seqlens is passed);
 * 0 for invalid sizes: 128 bytes per token-head, plus 8 bytes per sequence with cu_seqlens. While
 * the environment variable SORERNN_PREFILL=coop selects the cooperative prefill, the size also
 * covers its package ring (up to 8 x 47,360 bytes per sequence and value head); gdn_chunk_fwd reads
 * the variable again, so size and call must see the same value. No counterpart in the reference:
 * FLA allocates its intermediates itself.
 */
GDN_API size_t gdn_chunk_workspace_size(int64_t B, int64_t T, int64_t HV, int64_t N, int varlen);

/*
 * Training forward of the chunked rule: gdn_chunk_fwd plus the state entering every chunk, rounded
 * to bf16 and stored transposed, chunk_states [chunks][HV][V][K] (gdn_chunk_states_size bytes; the
 * backward uses it only as a bf16 MFMA operand; chunk c of sequence n is
 * n * ceil(T / 64) + c, or the running chunk count before n plus c with cu_seqlens), which
 * gdn_chunk_bwd reads. The workspace must also be kept unchanged until gdn_chunk_bwd has run.
 * Replaces the forward half of FLA's chunk_gated_delta_rule autograd function (the call at
 * sore/model/gdn.py:166-169 when the inputs require grad).
 */
GDN_API int gdn_chunk_fwd_train(const void* q, const void* k, const void* v, const void* g, const void* beta,
                        const float* initial_state, void* o, float* final_state, const void* cu_seqlens,
                        int64_t B, int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, int64_t N,
                        int qkv_dtype, int g_dtype, int beta_dtype, float scale, unsigned flags,
                        const float* A_log, const float* dt_bias, void* chunk_states, void* workspace,
                        size_t workspace_bytes, void* stream);

/*
 * gdn_chunk_fwd without a workspace argument; it allocates nothing. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). The workspace is a fixed array in the library's device
 * memory of gdn_chunk_fwd_noalloc_max_workspace() bytes (64 MiB + 64 KiB: up to 524,288 token-heads,
 * e.g. 4 x 4,096 or 32,768 tokens at 16 value heads, with the default prefill), held on every device
 * the library runs on until the process ends.
 * Sizes needing more return GDN_ERR_INVALID. The stream's device must be the current device. Calls
 * on one device share the array: calls that overlap on one device race.
 */
GDN_API int gdn_chunk_fwd_noalloc(const void* q, const void* k, const void* v, const void* g, const void* beta,
                          const float* initial_state, void* o, float* final_state, const void* cu_seqlens,
                          int64_t B, int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, int64_t N,
                          int qkv_dtype, int g_dtype, int beta_dtype, float scale, unsigned flags,
                          const float* A_log, const float* dt_bias, void* stream);

/* Bytes of the array gdn_chunk_fwd_noalloc uses as its workspace. */
GDN_API size_t gdn_chunk_fwd_noalloc_max_workspace(void);

/*
 * Range flag of the chunked forward on `device`. After this call every gdn_chunk_fwd,
 * gdn_chunk_fwd_train and gdn_chunk_fwd_noalloc launch on that device sets *flag to 1 (never back
 * to 0) when it stores an o or final_state element that is inf or NaN. The forward's MFMA operands
 * for S, X, Delta, T - I and scale * P are fp16 (largest finite value 65504); an operand past that
 * range becomes inf and reaches o (and final_state), so a set flag means such an overflow or
 * non-finite inputs. flag: pinned host memory (written with system scope, so the host can poll it
 * without a device synchronisation) or memory of `device`; NULL turns the check off (the default).
 * The caller clears the word. No counterpart in the reference: FLA's bf16 operands keep fp32's
 * exponent range, so its chunk kernel has no such limit to report.
 */
GDN_API int gdn_set_range_flag(int device, unsigned* flag);

/* Bytes of chunk_states for gdn_chunk_fwd_train / gdn_chunk_bwd (0 for invalid sizes). */
GDN_API size_t gdn_chunk_states_size(int64_t B, int64_t T, int64_t HV, int64_t K, int64_t V, int64_t N, int varlen);

/*
 * Backward of the chunked rule. Replaces the backward of FLA 0.5.2's chunk_gated_delta_rule
 * autograd function (its kernels chunk_gated_delta_rule_bwd_kernel_dhu, chunk_bwd_kernel_dqkwg,
 * prepare_wy_repr_bwd and the l2norm backward, named by the profiler at
 * tests/train/test_profiling.py:25,29,31,32,35; gradients checked against autograd through the
 * reference recurrence at tests/model/test_gdn.py:94-101,158-162).
 * Inputs: the forward's q, k, v, g, beta, A_log, dt_bias, cu_seqlens, flags and scale; d_o
 * [B,T,HV,V] bf16; d_final_state [N,HV,K,V] fp32 or NULL (zero); chunk_states and fwd_workspace
 * as left by gdn_chunk_fwd_train.
 * Outputs: dq, dk [B,T,H,K] and dv [B,T,HV,V] bf16 (value heads sharing a q/k head are summed);
 * dg [B,T,HV] in g_dtype and dbeta in beta_dtype (with the flags set, the gradients of the raw
 * gate input a and of the beta logits); d_initial_state [N,HV,K,V] fp32 or NULL (not written);
 * with GDN_FLAG_GATE_IN_KERNEL, dA_log and ddt_bias [HV] fp32 (overwritten, not accumulated).
 * workspace: gdn_chunk_bwd_workspace_size bytes, contents on entry irrelevant.
 */
GDN_API int gdn_chunk_bwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                  const void* d_o, const float* d_final_state, const void* chunk_states,
                  const void* fwd_workspace, const void* cu_seqlens, int64_t B, int64_t T, int64_t H,
                  int64_t HV, int64_t K, int64_t V, int64_t N, int qkv_dtype, int g_dtype, int beta_dtype,
                  float scale, unsigned flags, const float* A_log, const float* dt_bias, void* dq, void* dk,
                  void* dv, void* dg, void* dbeta, float* d_initial_state, float* dA_log, float* ddt_bias,
                  void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes gdn_chunk_bwd needs (0 for invalid sizes). No counterpart in the reference. */
GDN_API size_t gdn_chunk_bwd_workspace_size(int64_t B, int64_t T, int64_t HV, int64_t K, int64_t V, int64_t N,
                                            int varlen);

/*
 * Recurrent gated delta rule forward: tokens in order, the state held on chip for the whole
 * sequence (one read and one write of each state). With T == 1 this is the decode step.
 * Replaces FLA fused_recurrent_gated_delta_rule (named by the profiler rule at
 * sore/train/profiling.py:35; no call site in the reference). final_state may equal
 * initial_state (in-place update). Same layouts, dtypes and flags as gdn_chunk_fwd.
 */
GDN_API int gdn_recurrent_fwd(const void* q, const void* k, const void* v, const void* g, const void* beta,
                      const float* initial_state, void* o, float* final_state, const void* cu_seqlens,
                      int64_t B, int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, int64_t N,
                      int qkv_dtype, int g_dtype, int beta_dtype, float scale, unsigned flags,
                      const float* A_log, const float* dt_bias, void* stream);

/*
 * Fused decode step for one token per sequence: conv-cache update + conv + SiLU on the packed
 * pre-conv projection x_qkv [B, 2*H*D + HV*D] (q | k | v channels), then the gated delta rule
 * step on the updated state. conv_state [B, C, W] (newest input last, updated in place),
 * conv_weight [C, W] fp32 (weight[:, W-1] multiplies the current token), state [B, HV, D, D]
 * fp32 updated in place, o [B, 1, HV, D]. g/beta [B, HV] as in gdn_chunk_fwd (flags apply).
 * No counterpart call in the reference (it has no decode path); composes the conv of
 * sore/model/conv.py:6-23 + SiLU (gdn.py:209), the L2 norm (gdn.py:177) and one step of
 * sore/model/gdn_ref.py:17-21.
 */
GDN_API int gdn_decode_step(const void* x_qkv, void* conv_state, const float* conv_weight, const void* g,
                    const void* beta, float* state, void* o, int64_t B, int64_t H, int64_t HV,
                    int64_t D, int64_t W, int x_dtype, int conv_state_dtype, int g_dtype, int beta_dtype,
                    float scale, unsigned flags, const float* A_log, const float* dt_bias, void* stream);

/*
 * Depthwise causal conv1d (+ optional SiLU) with per-document reset.
 * Replaces FLA causal_conv1d(x, weight, activation="silu", cu_seqlens, cu_seqlens_cpu)
 * (sore/model/gdn.py:199-207) and the torch path causal_conv1d_varlen + F.silu
 * (sore/model/conv.py:6-23, gdn.py:208-209). x, y [B, T, C] (x_dtype); weight [C, W] fp32;
 * bias [C] fp32 or NULL. initial_state [N, C, W] (x_dtype) or NULL supplies the inputs before
 * each sequence; final_state [N, C, W] (x_dtype) or NULL receives the last W inputs of each
 * sequence (zero-padded). Math in fp32, one rounding to x_dtype.
 */
GDN_API int gdn_causal_conv1d_fwd(const void* x, const float* weight, const float* bias, void* y,
                          const void* initial_state, void* final_state, const void* cu_seqlens,
                          int64_t B, int64_t T, int64_t C, int64_t W, int64_t N, int x_dtype,
                          int activation, unsigned flags, void* stream);

/*
 * Row-wise L2 normalisation y = x / max(||x||_2, eps) over the last axis of length D.
 * Replaces F.normalize(q/k, dim=-1) (sore/model/gdn.py:177) and FLA's l2norm_fwd_kernel
 * (tests/train/test_profiling.py:30). Math in fp32, one rounding.
 */
GDN_API int gdn_l2norm_fwd(const void* x, void* y, int64_t rows, int64_t D, int dtype, float eps, void* stream);

/*
 * Gated RMSNorm: y = x * rsqrt(mean(x^2) + eps) * weight (+ bias) * act(gate), per row of D.
 * Replaces FLA rms_norm_gated(o, gate, weight, None, activation="swish", eps) at
 * sore/model/gdn.py:182-186 and o_norm(o) * F.silu(gate) at gdn.py:188 (RMSNorm:
 * sore/model/layers.py:7-18). gate may be NULL (plain RMSNorm). weight [D] fp32 or NULL (ones).
 * Math in fp32, one rounding to dtype.
 */
GDN_API int gdn_rms_norm_gated_fwd(const void* x, const void* gate, const float* weight, const float* bias, void* y,
                           int64_t rows, int64_t D, int dtype, float eps, int activation, void* stream);

/*
 * Backward of gdn_causal_conv1d_fwd (the reference trains through FLA causal_conv1d's backward, or
 * autograd through sore/model/conv.py:6-23 + F.silu, gdn.py:199-209). Inputs as the forward plus
 * dy [B, T, C] (x_dtype). Outputs: dx [B, T, C] (x_dtype); dweight [C, W] and dbias [C] fp32
 * (dbias may be NULL); d_initial_state [N, C, W] fp32 or NULL (written only with initial_state).
 * workspace: gdn_causal_conv1d_bwd_workspace_size bytes (per-block partial sums of dweight/dbias).
 */
GDN_API int gdn_causal_conv1d_bwd(const void* x, const float* weight, const float* bias, const void* dy,
                          const void* initial_state, const void* cu_seqlens, int64_t B, int64_t T, int64_t C,
                          int64_t W, int64_t N, int x_dtype, int activation, unsigned flags, void* dx,
                          float* dweight, float* dbias, float* d_initial_state, void* workspace,
                          size_t workspace_bytes, void* stream);

/* Workspace bytes gdn_causal_conv1d_bwd needs (0 for invalid sizes). No counterpart in the reference. */
GDN_API size_t gdn_causal_conv1d_bwd_workspace_size(int64_t B, int64_t T, int64_t C, int64_t W);

/*
 * Backward of gdn_l2norm_fwd: dx = (dy - y (y . dy)) / max(|x|, eps) per row (dy / eps where the
 * norm is clamped). Replaces the autograd of F.normalize (sore/model/gdn.py:177) and FLA's
 * l2norm backward (tests/train/test_profiling.py:30).
 */
GDN_API int gdn_l2norm_bwd(const void* x, const void* dy, void* dx, int64_t rows, int64_t D, int dtype, float eps,
                   void* stream);

/*
 * Backward of gdn_rms_norm_gated_fwd (FLA rms_norm_gated's backward, sore/model/gdn.py:182-186, or
 * autograd through RMSNorm * silu(gate), gdn.py:188 and layers.py:7-18). Outputs: dx, dgate
 * (dtype; dgate only with a gate), dweight and dbias [D] fp32 (either may be NULL).
 * workspace: gdn_rms_norm_gated_bwd_workspace_size bytes.
 */
GDN_API int gdn_rms_norm_gated_bwd(const void* x, const void* gate, const float* weight, const float* bias,
                           const void* dy, void* dx, void* dgate, float* dweight, float* dbias, int64_t rows,
                           int64_t D, int dtype, float eps, int activation, void* workspace,
                           size_t workspace_bytes, void* stream);

/* Workspace bytes gdn_rms_norm_gated_bwd needs. No counterpart in the reference. */
GDN_API size_t gdn_rms_norm_gated_bwd_workspace_size(int64_t rows, int64_t D);

/*
 * The GDN layer's q/k/v prologue in one pass (inference): x [B, T, >= 2*Cqk + Cv] with row stride
 * x_row_stride elements holds the q | k | v projection outputs (e.g. column slices of one fused
 * projection GEMM); weight [2*Cqk + Cv, 4] fp32 (the q, k, v conv weights stacked), bias or NULL.
 * Depthwise causal conv of width 4 + activation, rounded to x_dtype (GDN_ACT_SILU_ROUNDED rounds the
 * conv output to x_dtype before the SiLU, as gdn.py:208-209's unfused route does with the weight
 * passed already rounded to x_dtype); with GDN_FLAG_QK_L2NORM every
 * head of head_dim channels of q and k is then L2-normalised (x / max(||x||, 1e-12), fp32, rounded).
 * Writes contiguous q, k [B, T, Cqk] and v [B, T, Cv]. Document resets with cu_seqlens (B == 1).
 * bf16 or fp16; head_dim 64 or 128. Replaces the three causal_conv1d calls of
 * sore/model/gdn.py:199-207 (FLA causal_conv1d; torch path causal_conv1d_varlen + F.silu,
 * gdn.py:208-209) and the q/k normalisation of gdn.py:177 (use_qk_l2norm_in_kernel, gdn.py:168):
 * the same fp32 formulas as the separate conv followed by the normalisation (within two ulps).
 */
GDN_API int gdn_qkv_conv_fwd(const void* x, int64_t x_row_stride, const float* weight, const float* bias, void* q,
                     void* k, void* v, const void* cu_seqlens, int64_t B, int64_t T, int64_t Cqk, int64_t Cv,
                     int64_t head_dim, int64_t N, int x_dtype, int activation, unsigned flags, void* stream);

/*
 * Gated attention prologue: per (token, head) row of q_in [B, T, HQ*D] and k_in [B, T, HKV*D]
 * (row strides q_row_stride / k_row_stride elements, e.g. column slices of one fused projection
 * output), RMSNorm over D with weights q_weight / k_weight [D] (w_dtype fp32 or bf16), then the
 * GPT-NeoX rotary embedding on the first rot_dim dims at the token's position (restarting at 0 in
 * every document with cu_seqlens). Writes q_out [B, T, HQ, D] and k_out [B, T, HKV, D] contiguous.
 * bf16 activations. Replaces q_norm(q_proj(x)), k_norm(k_proj(x)) and self.rotary(q, k, positions)
 * in GatedAttention.forward (sore/model/attention.py:105-116; RMSNorm sore/model/layers.py:7-18;
 * PartialRotary sore/model/rope.py:24-41) with the same rounding points.
 */
GDN_API int gdn_attn_qk_norm_rope_fwd(const void* q_in, int64_t q_row_stride, const void* k_in, int64_t k_row_stride,
                              const void* q_weight, const void* k_weight, int w_dtype, void* q_out, void* k_out,
                              const void* cu_seqlens, int64_t B, int64_t T, int64_t HQ, int64_t HKV, int64_t D,
                              int64_t N, int rot_dim, float theta, float eps, unsigned flags, void* stream);

/*
 * Causal GQA attention with the sigmoid output gate: o = softmax(scale q k^T + causal mask) v *
 * sigmoid(gate), q head i reading kv head i / (HQ / HKV). q [B, T, HQ, D], k [B, T, HKV, D]
 * contiguous; v [B, T, HKV*D] and gate [B, T, HQ*D] with row strides v_row_stride /
 * gate_row_stride elements; o [B, T, HQ*D] contiguous. With cu_seqlens (B == 1) a query attends only
 * to keys of its own document. bf16, fp32 softmax and accumulation; D = 64 or 128.
 * Replaces F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True) and its
 * document-causal mask variant (sore/model/attention.py:124-135; flex_attention with
 * doc_causal_block_mask, :28-50,131-135) followed by o * torch.sigmoid(gate_proj(x)) (:122).
 */
GDN_API int gdn_attn_fwd(const void* q, const void* k, const void* v, int64_t v_row_stride, const void* gate,
                 int64_t gate_row_stride, void* o, const void* cu_seqlens, int64_t B, int64_t T, int64_t HQ,
                 int64_t HKV, int64_t D, int64_t N, float scale, unsigned flags, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SORERNN_AMD_GDN_H */
