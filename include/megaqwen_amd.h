/* C ABI of the MI355X-native Qwen3-0.6B megakernel (gfx950).
 *
 * Drop-in for the reference's `csrc/megakernel` launchers: the entry points
 * below keep the reference's names, argument order and meaning; the
 * differences are (1) `hipStream_t` instead of `cudaStream_t`, (2) every entry
 * returns an int status (MQ_OK or a negative MQ_ERR_*) instead of void, and
 * (3) no cuBLAS handle (prefill uses hand-written MFMA kernels).
 *
 * All pointers are device pointers unless stated otherwise. Buffers belong to
 * the caller; the library keeps one small per-device workspace of its own
 * (exchange buffers, counters), allocated on the first call on that device.
 * Calls that overlap in time on one device race on that workspace.
 */
#ifndef MEGAQWEN_AMD_H
#define MEGAQWEN_AMD_H

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MQ_OK 0
#define MQ_ERR_ARG (-1)      /* invalid argument (checked on the host before any HIP call) */
#define MQ_ERR_HIP (-2)      /* a HIP runtime call failed */
#define MQ_ERR_DEVICE (-3)   /* device cannot hold the decode grid (256 resident workgroups) */
#define MQ_ERR_ALLOC (-4)    /* workspace allocation failed */

/* Per-layer weight pointers, bf16, HF nn.Linear layout [out, in].
 * Same fields and order as the reference's LDGLayerWeights
 * (csrc/megakernel/fused_decode_ldg.cu:24-36) and PrefillLayerWeights
 * (csrc/megakernel/megakernel_decode.py:281-293). */
typedef struct LDGLayerWeights {
  const void* input_layernorm_weight;     /* [1024] */
  const void* q_proj_weight;              /* [2048, 1024] */
  const void* k_proj_weight;              /* [1024, 1024] */
  const void* v_proj_weight;              /* [1024, 1024] */
  const void* q_norm_weight;              /* [128] */
  const void* k_norm_weight;              /* [128] */
  const void* o_proj_weight;              /* [1024, 2048] */
  const void* post_attn_layernorm_weight; /* [1024] */
  const void* gate_proj_weight;           /* [3072, 1024] */
  const void* up_proj_weight;             /* [3072, 1024] */
  const void* down_proj_weight;           /* [1024, 3072] */
} LDGLayerWeights;

typedef LDGLayerWeights PrefillLayerWeights;

/* Device-resident decode step (16 bytes, device memory): the input of the next launch of
 * mq_decode_step_device. Each launch reads it at its start and its last workgroup writes
 * {argmax token, position + 1, epoch used, count + 1} back (a failed step writes its
 * negative status as the token and keeps the position; launches that find a negative
 * token, an invalid position or count == capacity do nothing). */
typedef struct MqDecodeStep {
  int token;      /* input token of the next step */
  int position;   /* KV slot the next step writes (cache_len = position + 1) */
  unsigned epoch; /* output only: the exchange epoch the last step used (launches take their
                     epoch from the library workspace, one more than the previous launch's) */
  int count;      /* steps done: out_ids[count] receives the next step's token */
} MqDecodeStep;

/* One greedy decode step of the full model.
 * Replaces `launch_ldg_decode` (csrc/megakernel/fused_decode_ldg.cu:893-921).
 *   layer_weights : DEVICE array of num_layers structs (as in the reference).
 *   k_cache/v_cache: bf16 [num_layers, 8, max_seq_len, 128]; slot `position` is written.
 *   cache_len must equal position + 1.
 *   On return (stream-ordered): *output_token_id = argmax of the bf16 logits
 *   (lowest index on ties), or a negative value -(1 + flags) if the kernel's
 *   watchdog fired; hidden_buffer = final hidden bf16[1024]; g_normalized =
 *   final-norm output as fp32[1024]. The other scratch pointers
 *   (g_activations .. g_mlp_intermediate, block_max_vals, block_max_idxs) are
 *   accepted for ABI compatibility and not used. */
int launch_ldg_decode(int input_token_id, int* output_token_id, const void* embed_weight,
                      const LDGLayerWeights* layer_weights, const void* final_norm_weight,
                      const void* lm_head_weight, const void* cos_table, const void* sin_table, void* k_cache,
                      void* v_cache, void* hidden_buffer, void* g_activations, void* g_residual, void* g_q,
                      void* g_k, void* g_v, void* g_attn_out, void* g_mlp_intermediate, void* g_normalized,
                      void* block_max_vals, void* block_max_idxs, int num_layers, int position, int cache_len,
                      int max_seq_len, float attn_scale, hipStream_t stream);

/* As launch_ldg_decode, and also writes the bf16-rounded logits (as fp32) of
 * all 151936 vocabulary rows to logits_output.
 * Replaces `launch_ldg_decode_with_logits` (csrc/megakernel/fused_decode_ldg.cu:972-1001). */
int launch_ldg_decode_with_logits(int input_token_id, int* output_token_id, float* logits_output,
                                  const void* embed_weight, const LDGLayerWeights* layer_weights,
                                  const void* final_norm_weight, const void* lm_head_weight, const void* cos_table,
                                  const void* sin_table, void* k_cache, void* v_cache, void* hidden_buffer,
                                  void* g_activations, void* g_residual, void* g_q, void* g_k, void* g_v,
                                  void* g_attn_out, void* g_mlp_intermediate, void* g_normalized,
                                  void* block_max_vals, void* block_max_idxs, int num_layers, int position,
                                  int cache_len, int max_seq_len, float attn_scale, hipStream_t stream);

/* launch_ldg_decode without any allocation, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. Same arguments and results as
 * launch_ldg_decode minus the reference's unused scratch pointers (output_token_id,
 * hidden_buffer and g_normalized are written as there; g_normalized may be NULL). Its
 * kernels use a file-scope device array of about 1.2 MB (the decode workspace) instead
 * of the library's allocated workspace: each GPU holds one copy from the first call on
 * that device until the process ends. The first call on a device does the set-up (a
 * device query and the array's address); call it once before any graph capture.
 * Limits: num_layers <= 32, position < 16384 (MQ_ERR_ARG past them). Calls on one GPU
 * share its array: calls that overlap in time on one device race. */
int launch_ldg_decode_noalloc(int input_token_id, int* output_token_id, const void* embed_weight,
                              const LDGLayerWeights* layer_weights, const void* final_norm_weight,
                              const void* lm_head_weight, const void* cos_table, const void* sin_table, void* k_cache,
                              void* v_cache, void* hidden_buffer, void* g_normalized, int num_layers, int position,
                              int cache_len, int max_seq_len, float attn_scale, hipStream_t stream);

/* Decode-kernel variants of mq_decode_variant. */
#define MQ_VARIANT_BASELINE 0 /* the kernel instance for each step's position (launch_ldg_decode's choice) */
#define MQ_VARIANT_UNSPLIT 1  /* instance 0: one attention workgroup per XCD; positions < 256 only */
#define MQ_VARIANT_SPLIT 2    /* instances 1/2: attention split into chunks; every position */

/* launch_ldg_decode_with_logits (logits_output may be NULL) with the decode-kernel
 * instance fixed by a variant instead of chosen per step. The MI355X counterpart of the
 * reference's variant policy, which compiles one source variant per kernel module
 * (chat.py:17-29, 36-46, 59-64); the reference's C ABI has no such entry. Returns
 * MQ_ERR_ARG for an unknown variant or for MQ_VARIANT_UNSPLIT at position >= 256. All
 * variants give the same tokens, logits and caches (the instances differ only in how
 * the attention work is split across workgroups). */
int mq_decode_variant(int variant, int input_token_id, int* output_token_id, float* logits_output,
                      const void* embed_weight, const LDGLayerWeights* layer_weights, const void* final_norm_weight,
                      const void* lm_head_weight, const void* cos_table, const void* sin_table, void* k_cache,
                      void* v_cache, void* hidden_buffer, void* g_normalized, int num_layers, int position,
                      int cache_len, int max_seq_len, float attn_scale, hipStream_t stream);

/* One decoder block at `position` on a given bf16 hidden vector (no embedding,
 * no LM head): hidden_out = layer(hidden_in); K/V slot `position` of the
 * single-layer caches k_cache/v_cache ([1, 8, max_seq_len, 128]) is written.
 * Debug/parity entry for a single block; the reference has no separate
 * launcher for it (its layer body is ldg_decode_kernel's loop,
 * csrc/megakernel/fused_decode_ldg.cu:655-686). */
int mq_decode_layer(const void* hidden_in, void* hidden_out, const LDGLayerWeights* layer_weights,
                    const void* cos_table, const void* sin_table, void* k_cache, void* v_cache, int position,
                    int max_seq_len, float attn_scale, hipStream_t stream);

/* Prefill of a whole prompt, then the greedy next token.
 * Replaces `launch_prefill_float` (csrc/megakernel/fused_prefill.cu:601-636) with the
 * same arguments minus the cuBLAS handle (the GEMMs are hand-written MFMA kernels).
 *   input_token_ids: device int32 [seq_len]; 1 <= seq_len <= max_seq_len.
 *   layer_weights  : HOST array of num_layers structs (as in the reference,
 *                    csrc/megakernel/megakernel_decode.py:516).
 *   k_cache/v_cache: bf16 [num_layers, 8, max_seq_len, 128]; slots 0..seq_len-1 are written.
 *   Scratch (bf16, device, caller-owned, as the reference sizes them):
 *     hidden_bf16 [seq_len, 1024], normalized [seq_len, 1024], q_proj [seq_len, 2048],
 *     k_proj / v_proj [seq_len, 1024], attn_out [seq_len, 2048], mlp_norm [seq_len, 1024],
 *     mlp_intermediate [seq_len, 3072], gate_out / up_out [seq_len, 3072] (here they,
 *     q_proj and k_proj | v_proj hold fp32 partial sums of the k-split o_proj and
 *     down_proj products once the attention has consumed q, k and v),
 *     final_hidden [1024] (final-norm output of the last row), block_max_vals f32
 *     [1184], block_max_idxs i32 [1184]. Every buffer needs 16-byte alignment.
 *     residual, o_proj_out and down_out are accepted and unused (the epilogues fuse
 *     those steps); they may be NULL.
 *   hidden_bf16_out [1024]: a copy of final_hidden (the last row after the final norm), as
 *                    the reference copies it (csrc/megakernel/fused_prefill.cu:843-849).
 *   On return (stream-ordered): *output_token_id = argmax of the last row's bf16
 *   logits (lowest index on ties), or -2 if an input id was outside [0, 151936). */
int launch_prefill_float(const int* input_token_ids, int* output_token_id, int seq_len, const void* embed_weight,
                         const PrefillLayerWeights* layer_weights, const void* final_norm_weight,
                         const void* lm_head_weight, const void* cos_table, const void* sin_table, void* k_cache,
                         void* v_cache, void* hidden_bf16, void* residual, void* normalized, void* q_proj,
                         void* k_proj, void* v_proj, void* attn_out, void* o_proj_out, void* mlp_norm,
                         void* gate_out, void* up_out, void* mlp_intermediate, void* down_out, void* final_hidden,
                         void* block_max_vals, void* block_max_idxs, void* hidden_bf16_out, int num_layers,
                         int max_seq_len, float attn_scale, hipStream_t stream);

/* Prefill through the reference's fused-prefill launcher name and arguments.
 * Replaces `launch_prefill_megakernel` (csrc/megakernel/fused_prefill_megakernel.cu:938-1016;
 * its Python caller, csrc/megakernel/megakernel_decode.py:911-937). The same MFMA prefill as
 * launch_prefill_float (the same tokens, caches and logits), with the reference's fp32 scratch:
 *   hidden / residual / normalized [seq_len, 1024], q_proj / attn_out [seq_len, 2048],
 *   k_proj / v_proj [seq_len, 1024], mlp_intermediate [seq_len, 3072], all float32 and
 *   16-byte aligned (the bf16 activations and the fp32 partial sums are carved from them).
 *   final_hidden: float32 [1024], the final-norm output of the last row (HF's bf16 values
 *                 as fp32; the reference writes the unrounded fp32 product).
 *   hidden_bf16_out: bf16 [1024], the last row before the final norm, as the reference
 *                 writes it (csrc/megakernel/fused_prefill_megakernel.cu:728).
 *   block_max_vals f32 [1184], block_max_idxs i32 [1184]; other arguments and the result
 *   as launch_prefill_float. The reference's launcher returns void and needs a cooperative
 *   launch; this one returns a status and runs ordinary launches. */
int launch_prefill_megakernel(const int* token_ids, int* output_token_id, int seq_len, const void* embed_weight,
                              const PrefillLayerWeights* layer_weights, const void* final_norm_weight,
                              const void* lm_head_weight, const void* cos_table, const void* sin_table, void* k_cache,
                              void* v_cache, void* hidden, void* residual, void* normalized, void* q_proj,
                              void* k_proj, void* v_proj, void* attn_out, void* mlp_intermediate, void* final_hidden,
                              void* hidden_bf16_out, void* block_max_vals, void* block_max_idxs, int num_layers,
                              int max_seq_len, float attn_scale, hipStream_t stream);

/* Device-resident generation (reference idea: experimental/qwen_persistent_kernel.cu:1028-1033,
 * which reads token and position from device memory so a captured graph can replay).
 * mq_decode_step_init writes {token, position, 0, 0} to `step` (stream-ordered copy of
 * pageable host memory, then a stream synchronisation). Then up to
 * `capacity` launches of mq_decode_step_device (directly, or as nodes of a captured HIP
 * graph: the launch itself does no memset, copy or allocation) each decode one token of
 * the full model like launch_ldg_decode, taking token and position from `step`,
 * appending the greedy token to out_ids[count] and advancing `step`. No host read is
 * needed between steps. split_instance: 0 runs the kernel instance for contexts of at
 * most 256 positions (a step past that fails with a negative token), 1 and 2 the
 * instances for every length (2 pipelines a chunk's LDS passes: the faster one past 4096
 * positions, see mq_decode_plan). Re-initialise `step` before replaying a graph. */
int mq_decode_step_init(MqDecodeStep* step, int token, int position, int capacity, hipStream_t stream);
int mq_decode_step_device(MqDecodeStep* step, int* out_ids, int out_capacity, int split_instance,
                          const void* embed_weight, const LDGLayerWeights* layer_weights,
                          const void* final_norm_weight, const void* lm_head_weight, const void* cos_table,
                          const void* sin_table, void* k_cache, void* v_cache, void* hidden_buffer,
                          void* g_normalized, int num_layers, int max_seq_len, float attn_scale, hipStream_t stream);

/* The decode kernel's work split for the query at `position` (host-side, no GPU needed):
 * *instance = 0 (one attention workgroup per XCD, contexts of at most 256 positions), 1,
 * or 2 (a chunk's LDS passes pipelined, where a chunk takes more than one pass);
 * the attention is split into *nsplit chunks of at most *chunk positions, each attended
 * in at most *npass LDS passes. The MI355X counterpart of the reference's decode-kernel
 * variant choice (chat.py:17-29). MQ_ERR_ARG past the 16384-position limit. */
int mq_decode_plan(int position, int* instance, int* nsplit, int* chunk, int* npass);

/* Launch mode of the decode entry points (process-wide): 0 = ordinary launch (default;
 * all 256 workgroups are resident by construction and every inter-workgroup wait is
 * bounded), 1 = hipLaunchCooperativeKernel (the reference's launch,
 * csrc/megakernel/fused_decode_ldg.cu:947). Returns the previous mode. */
int mq_set_launch_mode(int cooperative);

/* Test hook: sets this device's decode error word, as a failed wait would. The next
 * decode launch then gives up every wait that does not succeed at once, completes, and
 * reports the flags as a negative token; mq_reset_workspace clears them. Synchronous. */
int mq_debug_set_error(int device, unsigned flags);

/* Zero this device's workspaces (exchange buffers and counters): the library's allocated
 * workspace and, once launch_ldg_decode_noalloc has been called on this device, that entry
 * point's file-scope workspace too (a synchronous memset: it allocates nothing). Needed
 * only after a launch reported a watchdog error. Synchronous. */
int mq_reset_workspace(int device);

/* Human-readable name of a status code. */
const char* mq_strerror(int status);

#ifdef __cplusplus
}
#endif

#endif /* MEGAQWEN_AMD_H */
