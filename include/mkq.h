/*
 * mkq.h -- C ABI of the MI355X (gfx950) decode hot path for Qwen3.6.
 *
 * The shared library libmkq.so exports exactly the functions declared here.
 * Every entry point takes plain device pointers, sizes and a HIP stream
 * (passed as void*, so this header needs no HIP include), enqueues its
 * kernels asynchronously on that stream and returns an MKQ_* status.  No
 * entry point allocates device memory, synchronises the stream or queries
 * the device on its call path (the CU count is read once per device and
 * cached), so calls can be captured in a HIP graph.
 *
 * Tensor layouts are the reference's (row-major, contiguous):
 *   x [batch, hidden]; router [experts, hidden];
 *   expert_gate/up [experts, intermediate, hidden]; expert_down [experts, hidden, intermediate];
 *   shared_gate/up [shared_intermediate, hidden]; shared_down [hidden, shared_intermediate];
 *   q [batch, q_heads, head_dim]; k_cache/v_cache [batch, seq_len, kv_heads, head_dim];
 *   linear q/k [batch, k_heads, key_dim]; v [batch, v_heads, value_dim];
 *   state [batch, v_heads, key_dim, value_dim] float32.
 * All weight/activation pointers of one call share the element type `dtype`.
 *
 * Workspace: entry points that need scratch take (workspace, workspace_bytes),
 * 256-byte aligned; *_workspace_bytes() gives the size.  The caller zero-fills
 * a workspace once, before its first use, and gives it to one entry point
 * only: every call leaves the state it keeps there (arrival counters back at
 * zero, the MoE generation word advanced) ready for the next call of the same
 * entry point on the same stream, with any shape, so it need not be cleared
 * again.  Another entry point's scratch data would overwrite that state.  Two
 * calls that run concurrently (different streams) must not share a workspace.
 */
#ifndef MKQ_H_
#define MKQ_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define MKQ_OK 0
#define MKQ_ERR_INVALID 1     /* bad shape / pointer / size: message in mkq_last_error() */
#define MKQ_ERR_UNSUPPORTED 2 /* valid but not supported by these kernels             */
#define MKQ_ERR_HIP 3         /* a HIP runtime call failed                            */

/* element types */
#define MKQ_DTYPE_F32 0
#define MKQ_DTYPE_F16 1
#define MKQ_DTYPE_BF16 2

/* Message of the last failing call on this host thread ("" if none). */
const char* mkq_last_error(void);

/* ABI version (major*100 + minor). */
int mkq_abi_version(void);

/* ------------------------------------------------------------------------
 * MoE decode.  Replaces the kernel side of
 *   _C.moe_decode_persistent      (reference csrc/bindings.cpp:33,
 *                                  csrc/persistent_moe_decode.cu:701-860)
 * as called by moe_decode(backend="persistent") (mega_kernel_qwen36/ops.py:303-304).
 * One persistent launch: RMSNorm -> router -> top-k/softmax -> routed SwiGLU
 * experts -> shared expert (optionally scaled by sigmoid(x_norm . shared_expert_gate))
 * -> down projection + residual.
 * Outputs: out [batch, hidden] (dtype), indices [batch, top_k] int64 (descending
 * logit, ties to the lower index), weights [batch, top_k] float32.
 * shared_expert_gate may be NULL (reference behaviour: no gate).
 * ---------------------------------------------------------------------- */
size_t mkq_moe_decode_workspace_bytes(int batch, int hidden, int experts, int intermediate,
                                      int shared_intermediate, int top_k);
int mkq_moe_decode(int dtype, const void* x, const void* norm_weight, const void* router_weight,
                   const void* expert_gate, const void* expert_up, const void* expert_down,
                   const void* shared_gate, const void* shared_up, const void* shared_down,
                   const void* shared_expert_gate, void* out, int64_t* indices, float* weights,
                   int batch, int hidden, int experts, int intermediate, int shared_intermediate,
                   int top_k, float eps, int add_residual, void* workspace, size_t workspace_bytes,
                   void* stream);

/* Residency and failure.  The workgroups of mkq_moe_decode hand values to
 * each other while they run, so all of them (one per CU) must be resident at
 * once; the entry point checks once per device that one workgroup fits on a
 * CU (else MKQ_ERR_UNSUPPORTED).  The reference gets the same guarantee from
 * cudaLaunchCooperativeKernel (persistent_moe_decode.cu:749-827).  A kernel
 * running concurrently on another stream can still hold CUs and delay some
 * workgroups; every wait is bounded, and a wait that runs out (about 2^21
 * polls) records error 1 in the workspace instead of hanging.  From then on
 * every call on that workspace writes NaN outputs (indices 0, weights NaN)
 * until the workspace is reset: stale tagged words are never read.
 *
 * mkq_moe_decode_status reads the workspace's error word into *error_code
 * (0: no wait has timed out since the last reset; 1: one has) and, with
 * reset != 0 and a nonzero word, zero-fills the whole workspace.  It
 * synchronises `stream` and copies to the host, so it must not be called
 * while the stream is being captured into a graph.  No counterpart in the
 * reference, whose cooperative launch either runs or fails. */
int mkq_moe_decode_status(void* workspace, size_t workspace_bytes, int reset, int* error_code, void* stream);

/* MoE decode that allocates nothing and takes no workspace.  No counterpart
 * in the reference: it is for callers that cannot allocate device memory or
 * own a workspace (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, kernels and results as
 * mkq_moe_decode, minus (workspace, workspace_bytes): the workspace is a
 * static device array of MKQ_MOE_NOALLOC_SCRATCH_BYTES in libmkq.so, one per
 * GPU, zero when the library is loaded and held until the process ends; its
 * address is looked up once per device.  A shape whose workspace
 * (mkq_moe_decode_workspace_bytes) exceeds it returns MKQ_ERR_UNSUPPORTED
 * (config 2 needs about 2.5 MB).  Every call on one GPU shares that array and
 * leaves its generation word advanced for the next call, so calls that
 * overlap on one GPU (several streams, several host threads) race and must
 * be serialised by the caller.  If a wait ever times out (see above), every
 * later call of this entry point on that GPU writes NaN outputs until the
 * process ends: mkq_moe_decode_status cannot reach the static array. */
#define MKQ_MOE_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)
int mkq_moe_decode_noalloc(int dtype, const void* x, const void* norm_weight, const void* router_weight,
                           const void* expert_gate, const void* expert_up, const void* expert_down,
                           const void* shared_gate, const void* shared_up, const void* shared_down,
                           const void* shared_expert_gate, void* out, int64_t* indices, float* weights,
                           int batch, int hidden, int experts, int intermediate, int shared_intermediate,
                           int top_k, float eps, int add_residual, void* stream);

/* ------------------------------------------------------------------------
 * Dense SwiGLU FFN decode: out = down(silu(gate(rms(x))) * up(rms(x))) (+ x).
 * No native counterpart in the reference: replaces the torch composite
 * _dense_ffn_decode_torch (mega_kernel_qwen36/ops.py:202-218) reached from
 * dense_ffn_decode (ops.py:323-364); semantics of reference.py:65-88.
 * ---------------------------------------------------------------------- */
size_t mkq_dense_ffn_decode_workspace_bytes(int batch, int hidden, int intermediate);
int mkq_dense_ffn_decode(int dtype, const void* x, const void* norm_weight, const void* gate_weight,
                         const void* up_weight, const void* down_weight, void* out, int batch,
                         int hidden, int intermediate, float eps, int add_residual, void* workspace,
                         size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * GQA full-attention decode (one query token).  Replaces
 *   _C.full_attention_decode      (csrc/bindings.cpp:34, csrc/attention_decode.cu:152-218)
 * as called by full_attention_decode (ops.py:372-373).
 * out [batch, q_heads, head_dim] (dtype) = softmax(q k^T * scale) v per q head,
 * q head h reading kv head h / (q_heads / kv_heads).  head_dim <= 256.
 * ---------------------------------------------------------------------- */
size_t mkq_full_attention_decode_workspace_bytes(int batch, int q_heads, int kv_heads, int head_dim,
                                                 int seq_len);
int mkq_full_attention_decode(int dtype, const void* q, const void* k_cache, const void* v_cache,
                              void* out, int batch, int q_heads, int kv_heads, int head_dim,
                              int seq_len, float scale, void* workspace, size_t workspace_bytes,
                              void* stream);

/* The same with q and the keys rotated inside the kernel (rotate-half RoPE
 * on their first rotary_dim dims, reference.py:91-114).  It replaces the
 * rotation of q and of the whole k_cache that full_attention_decode
 * (ops.py:368) runs in Python before _C.full_attention_decode when cos/sin
 * are given; the reference has no such entry point.  cos_sin: 2 * rotary_dim
 * floats on the device, cos then sin, the one vector pair the reference
 * broadcasts over every token and head.  q, k_cache are passed unrotated.
 * Both are rotated with the reference's rounding (products and sum in FP32,
 * then dtype), so the result equals the plain entry point on rotated inputs.
 * rotary_dim: a power of two in [16, head_dim]; bf16/f16, head_dim % 8 == 0
 * and 16-byte aligned tensors, else MKQ_ERR_UNSUPPORTED.  Uses the same
 * workspace. */
int mkq_full_attention_decode_rope(int dtype, const void* q, const void* k_cache, const void* v_cache,
                                   void* out, int batch, int q_heads, int kv_heads, int head_dim,
                                   int seq_len, float scale, const float* cos_sin, int rotary_dim,
                                   void* workspace, size_t workspace_bytes, void* stream);

/* KV append fused into the attention step.  The caches are [batch, capacity,
 * kv_heads, head_dim]; tokens 0 .. seq_len-2 are already in them and the new
 * token's k_new, v_new [batch, kv_heads, head_dim] go to row seq_len - 1 of
 * every batch row (written in place).  The result is that of
 * mkq_full_attention_decode(_rope) over the first seq_len tokens after the
 * cache rows were written, bit for bit; the kernel uses k_new/v_new directly
 * for the new token, so it is never read back.  capacity >= seq_len; the
 * batch stride is capacity tokens, so a preallocated cache needs no copy.
 * cos_sin may be NULL (no rotation) or as in the _rope entry point; the
 * cache keeps the new key unrotated, as the reference's caches hold unrotated
 * keys that every call rotates (ops.py:368).  bf16/f16, head_dim % 8 == 0 and
 * 16-byte aligned tensors, else MKQ_ERR_UNSUPPORTED (nothing written).  The
 * workspace is sized for seq_len.  No counterpart in the reference, whose
 * callers write the cache themselves before full_attention_decode
 * (ops.py:367-374). */
int mkq_full_attention_decode_append(int dtype, const void* q, const void* k_new, const void* v_new,
                                     void* k_cache, void* v_cache, void* out, int batch, int q_heads,
                                     int kv_heads, int head_dim, int seq_len, int capacity, float scale,
                                     const float* cos_sin, int rotary_dim, void* workspace,
                                     size_t workspace_bytes, void* stream);

/* Paged KV layout: k_blocks, v_blocks [num_blocks, block_size, kv_heads,
 * head_dim] hold the caches of all sequences in fixed-size blocks, and
 * block_table [batch, max_blocks] (int32, device) lists each batch row's
 * blocks in token order: token t of row b is row t % block_size of block
 * block_table[b, t / block_size].  The result equals
 * mkq_full_attention_decode over the gathered contiguous cache of seq_len
 * tokens, bit for bit.  A block id outside [0, num_blocks) reads as zeros
 * (no fault).  block_size a multiple of 16; max_blocks * block_size >=
 * seq_len; bf16/f16, head_dim % 8 == 0 and 16-byte aligned tensors, else
 * MKQ_ERR_UNSUPPORTED.  The workspace is sized as for the contiguous entry
 * point.  No counterpart in the reference, whose attention reads one
 * contiguous [B, T, Hkv, D] cache (attention_decode.cu:152-218); its task
 * planner assumes paged attention (mpk_graph.py:383-390). */
int mkq_full_attention_decode_paged(int dtype, const void* q, const void* k_blocks, const void* v_blocks,
                                    const int* block_table, void* out, int batch, int q_heads,
                                    int kv_heads, int head_dim, int seq_len, int block_size,
                                    int max_blocks, int num_blocks, float scale, void* workspace,
                                    size_t workspace_bytes, void* stream);

/* Paged KV with the KV append fused in: k_new, v_new [batch, kv_heads,
 * head_dim] are token seq_len - 1 of every batch row and are written (in
 * place) to row (seq_len - 1) % block_size of block
 * block_table[b, (seq_len - 1) / block_size]; the result equals writing that
 * row first and calling mkq_full_attention_decode_paged, bit for bit.  A
 * block id outside the pool is neither read nor written.  Limits as for the
 * two entry points it combines.  No counterpart in the reference. */
int mkq_full_attention_decode_paged_append(int dtype, const void* q, const void* k_new, const void* v_new,
                                           void* k_blocks, void* v_blocks, const int* block_table,
                                           void* out, int batch, int q_heads, int kv_heads, int head_dim,
                                           int seq_len, int block_size, int max_blocks, int num_blocks,
                                           float scale, void* workspace, size_t workspace_bytes,
                                           void* stream);

/* Paged KV with q and the keys rotated in the kernel (cos_sin and
 * rotary_dim as for mkq_full_attention_decode_rope, which must not be NULL);
 * bit-identical to that entry point over the gathered contiguous cache.
 * No counterpart in the reference. */
int mkq_full_attention_decode_paged_rope(int dtype, const void* q, const void* k_blocks,
                                         const void* v_blocks, const int* block_table, void* out,
                                         int batch, int q_heads, int kv_heads, int head_dim, int seq_len,
                                         int block_size, int max_blocks, int num_blocks, float scale,
                                         const float* cos_sin, int rotary_dim, void* workspace,
                                         size_t workspace_bytes, void* stream);

/* Paged KV with both the KV append and the in-kernel RoPE: the new token is
 * written into its block as by mkq_full_attention_decode_paged_append (the
 * key unrotated, as the caches hold keys) and q and the keys are rotated as
 * by mkq_full_attention_decode_paged_rope; bit-identical to
 * mkq_full_attention_decode_append with cos_sin over the gathered contiguous
 * cache.  Limits as for the entry points it combines.  No counterpart in the
 * reference. */
int mkq_full_attention_decode_paged_append_rope(int dtype, const void* q, const void* k_new, const void* v_new,
                                                void* k_blocks, void* v_blocks, const int* block_table,
                                                void* out, int batch, int q_heads, int kv_heads, int head_dim,
                                                int seq_len, int block_size, int max_blocks, int num_blocks,
                                                float scale, const float* cos_sin, int rotary_dim,
                                                void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Recurrent linear-attention decode, reference rule.  Replaces
 *   _C.linear_attention_decode    (csrc/bindings.cpp:35, csrc/linear_attention_decode.cu:46-93)
 * as called by linear_attention_decode (ops.py:378-385):
 *   new_state = decay * state + k (x) v;   out = q^T new_state.
 * state/new_state float32 [batch, heads, key_dim, value_dim]; new_state may
 * equal state (in-place update).
 * ---------------------------------------------------------------------- */
int mkq_linear_attention_decode(int dtype, const void* q, const void* k, const void* v,
                                const float* state, void* out, float* new_state, int batch,
                                int heads, int key_dim, int value_dim, float decay, void* stream);

/* ------------------------------------------------------------------------
 * Gated delta rule decode (Qwen3.6 linear attention).  No counterpart in the
 * reference (its rule is the one above); selected by linear_attention_decode
 * when g/beta are supplied.  Per batch row b and v head j (q/k head
 * h = j / (v_heads / k_heads)):
 *   S <- exp(g[b,j]) S;  S <- S + beta[b,j] k_h (x) (v_j - S^T k_h);  out_j = S^T q_h.
 * g, beta float32 [batch, v_heads]; new_state may equal state.
 * ---------------------------------------------------------------------- */
int mkq_gated_delta_decode(int dtype, const void* q, const void* k, const void* v,
                           const float* state, const float* g, const float* beta, void* out,
                           float* new_state, int batch, int k_heads, int v_heads, int key_dim,
                           int value_dim, void* stream);

/* The same step with q and k L2-normalised inside the kernel, in FP32,
 * x / sqrt(sum x^2 + 1e-6) over key_dim, and q then multiplied by q_scale
 * (1/sqrt(key_dim) in Qwen3.6): the use_qk_l2norm_in_kernel form of the
 * model's linear-attention step, where otherwise the caller normalises q
 * and k with separate ops first.  No counterpart in the reference. */
int mkq_gated_delta_decode_qknorm(int dtype, const void* q, const void* k, const void* v,
                                  const float* state, const float* g, const float* beta, void* out,
                                  float* new_state, int batch, int k_heads, int v_heads, int key_dim,
                                  int value_dim, float q_scale, void* stream);

/* ------------------------------------------------------------------------
 * The ops around the gated delta recurrence in the Qwen3.6 linear-attention
 * decode step.  No counterpart in the reference; they restate the model's
 * causal_conv1d_update and RMSNormGated (transformers 5.15.0,
 * modeling_qwen3_next.py).
 *
 * mkq_causal_conv1d_update: one new token per channel through a depthwise
 * causal convolution of width state_len + 1.  x [batch, channels];
 * conv_state [batch, channels, state_len] (dtype, updated in place: it keeps
 * the last state_len inputs); weight [channels, state_len + 1]; bias
 * [channels] or NULL; out [batch, channels] = silu(conv) (or conv when
 * silu_activation is 0).  The convolution is rounded to dtype before the SiLU.
 * state_len <= 7.
 *
 * mkq_gated_rms_norm: per row of dim values, n = round(x * rsqrt(mean(x^2) +
 * eps)) (FP32 mean and rsqrt), t = round(weight * n), out = round(t *
 * silu(gate)).  x, gate, out [rows, dim]; weight [dim].
 * ---------------------------------------------------------------------- */
int mkq_causal_conv1d_update(int dtype, const void* x, void* conv_state, const void* weight,
                             const void* bias, void* out, int batch, int channels, int state_len,
                             int silu_activation, void* stream);
int mkq_gated_rms_norm(int dtype, const void* x, const void* gate, const void* weight, void* out,
                       int rows, int dim, float eps, void* stream);

/* One Qwen3.6 linear-attention step around and through the recurrence, in
 * one launch on `stream`:
 *   mixed = silu(conv(x_mixed))   (as mkq_causal_conv1d_update, conv_state in place)
 *   q, k, v = the [k_heads*key_dim | k_heads*key_dim | v_heads*value_dim]
 *             parts of mixed
 *   o = gated delta rule with q/k L2 norm and q_scale (state updated in place)
 *   out = gated RMSNorm of o (as mkq_gated_rms_norm(o, z, norm_weight, eps))
 * bit-identical to those three calls in sequence.
 * x_mixed [batch, C] with C = 2*k_heads*key_dim + v_heads*value_dim;
 * conv_state [batch, C, conv_state_len], conv_state_len <= 7;
 * conv_weight [C, conv_state_len+1]; conv_bias [C] or NULL;
 * state [batch, v_heads, key_dim, value_dim] FP32; g, beta [batch, v_heads]
 * FP32; z, out [batch, v_heads, value_dim]; norm_weight [value_dim].  The
 * workspace (the recurrence output handed to the row norms and arrival
 * counts) is sized by mkq_linear_attention_step_workspace_bytes, 256-byte
 * aligned and zero-filled once before its first use: each call leaves its
 * counts at zero.  No counterpart in the reference. */
size_t mkq_linear_attention_step_workspace_bytes(int dtype, int batch, int k_heads, int v_heads,
                                                 int key_dim, int value_dim);
int mkq_linear_attention_step(int dtype, const void* x_mixed, void* conv_state, const void* conv_weight,
                              const void* conv_bias, int conv_state_len, float* state, const float* g,
                              const float* beta, const void* z, const void* norm_weight, void* out,
                              int batch, int k_heads, int v_heads, int key_dim, int value_dim,
                              float q_scale, float eps, void* workspace, size_t workspace_bytes,
                              void* stream);

/* ------------------------------------------------------------------------
 * Plain GEMV used for the optional attention output projections in
 * decode_layer: y[b, n] = sum_k w[n, k] * x[b, k] (+ residual[b, n]).
 * No counterpart in the reference (decode_layer reshapes, ops.py:722,728).
 * residual may be NULL.
 * ---------------------------------------------------------------------- */
int mkq_gemv(int dtype, const void* x, const void* w, const void* residual, void* y, int batch,
             int in_features, int out_features, void* stream);

/* ------------------------------------------------------------------------
 * The same GEMV with the residual add of decode_layer fused in:
 *   y[b, n]   = round(sum_k w[n, k] * x[b, k])
 *   sum[b, n] = round(residual[b, n] + y[b, n])
 * Both outputs carry the roundings of the reference's separate add
 * `residual = residual + attention_output` (ops.py:722-723, 728-729), so
 * sum is bit-identical to that add applied to y.  No counterpart in the
 * reference.  residual, y and sum must not alias.
 * ---------------------------------------------------------------------- */
int mkq_gemv_add(int dtype, const void* x, const void* w, const void* residual, void* y, void* sum,
                 int batch, int in_features, int out_features, void* stream);

/* ------------------------------------------------------------------------
 * Input RMSNorm and projection in one launch:
 *   xn[b, k] = round(x[b, k] * rsqrt(mean_k(x[b, k]^2) + eps) * norm_weight[k])
 *   y[b, n]  = round(sum_k w[n, k] * xn[b, k])
 * (statistics in FP32; round = to the element type, as reference.py:10-13
 * rounds rms_norm's result).  Replaces the reference planner's task pair
 * `rmsnorm` -> `linear` (projection "qkv") of a full-attention layer, and the
 * norm in front of a linear-attention layer's input projection
 * (mega_kernel_qwen36/mpk_graph.py:349-373, 391-405), which the reference
 * plans but never executes.  Every workgroup normalises x itself, so there is
 * no hand-off between workgroups; in_features is limited by staging x
 * (FP32) in LDS.
 * ---------------------------------------------------------------------- */
int mkq_rms_norm_gemv(int dtype, const void* x, const void* norm_weight, float eps, const void* w, void* y,
                      int batch, int in_features, int out_features, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MKQ_H_ */
