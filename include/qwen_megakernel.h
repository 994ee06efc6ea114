/* C-ABI of the MI355X Qwen3-0.6B batch-1 decode engine (libqwen_megakernel.so).
 *
 * Drop-in for the launchers of the reference's Tools/megakernel/megakernel.cu,
 * which its pybind11 layer (Tools/megakernel/qwen_ops.cpp:9-27) binds with
 * CUDA streams. Same names, argument order and argument meaning; the stream is
 * a hipStream_t. Plain pointers and sizes only.
 *
 * Buffers: every pointer is device memory owned by the caller, exactly as in
 * the reference (Model/Qwen06B_architecture.py:205-255):
 *   embed_weight      fp16 [151936, 1024]
 *   layer_weights     device array of num_layers LDGLayerWeight (16-B aligned)
 *   final_norm_weight fp16 [1024]
 *   lm_head_weight    fp16 [151936, 1024] (tied: may equal embed_weight)
 *   cos_table/sin_table fp16 [max_seq_len, 128]
 *   k_cache/v_cache   fp16 [num_layers, 8, max_seq_len, 128]
 *   hidden_buffer     fp16 [1024]   out: final-layer residual (before the final norm)
 *   g_normalized      fp32 [1024]   out: final-normed vector fed to the lm_head
 *   g_activations, g_residual, g_q, g_k, g_v, g_attn_out, g_mlp_intermediate,
 *   block_max_vals, block_max_idxs: accepted for signature compatibility and
 *   not touched; the engine keeps its inter-workgroup exchange buffers in its
 *   own per-device workspace (allocated once, like the reference's static
 *   barrier state, megakernel.cu:714-737).
 *
 * Return value: 0 on success, a QWEN_ERR_* code otherwise (the reference's
 * launchers return void; a caller declaring them void still links and runs).
 * Launches are asynchronous on `stream`; kernel-side failures (a wait that
 * exceeded its deadline) are reported by qwen_last_error().
 *
 * One call at a time per device: all calls on a device share its workspace.
 */
#ifndef QWEN_MEGAKERNEL_H
#define QWEN_MEGAKERNEL_H

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Per-layer weight pointers, field order of Tools/megakernel/megakernel.cu:87-100
 * and Model/Qwen06B_architecture.py:148-160; 12 pointers (96 B), ABI version 2. */
typedef struct __attribute__((aligned(16))) LDGLayerWeight {
  const void* input_layernorm_weight;     /* [1024]        */
  const void* q_proj_weight;              /* [2048, 1024]  */
  const void* k_proj_weight;              /* [1024, 1024]  */
  const void* v_proj_weight;              /* [1024, 1024]  */
  const void* q_norm_weight;              /* [128]         */
  const void* k_norm_weight;              /* [128]         */
  const void* o_proj_weight;              /* [1024, 2048]  */
  const void* post_attn_layernorm_weight; /* [1024]        */
  const void* gate_proj_weight;           /* [3072, 1024]  */
  const void* up_proj_weight;             /* [3072, 1024]  */
  const void* down_proj_weight;           /* [1024, 3072]  */
  const void* padding;                    /* 0             */
} LDGLayerWeight;

#define QWEN_ABI_VERSION 2

#define QWEN_OK 0
#define QWEN_ERR_ARG 1        /* bad argument (null pointer, range, alignment) */
#define QWEN_ERR_DEVICE 2     /* not a 256-CU gfx950 device, or no cooperative launch */
#define QWEN_ERR_LAUNCH 3     /* HIP launch/allocation failure */
#define QWEN_ERR_TIMEOUT 4    /* a device-side wait exceeded its deadline (reported by qwen_last_error) */
#define QWEN_ERR_BAD_TOKEN 5  /* a teacher-forced id outside [0, 151936) reached the device (qwen_last_error) */

/* One decode step at `position` (Tools/megakernel/megakernel.cu:1150-1196):
 * embedding of input_token_id, 28 layers writing K/V at `position`, final
 * norm, tied lm_head, argmax -> *output_token_id (device int32). */
int launch_ldg_decode_direct(
    int input_token_id, int* output_token_id, const void* embed_weight,
    const LDGLayerWeight* layer_weights, const void* final_norm_weight,
    const void* lm_head_weight, const void* cos_table, const void* sin_table,
    void* k_cache, void* v_cache, void* hidden_buffer, void* g_activations,
    void* g_residual, void* g_q, void* g_k, void* g_v, void* g_attn_out,
    void* g_mlp_intermediate, void* g_normalized, void* block_max_vals,
    void* block_max_idxs, int num_layers, int position, int max_seq_len,
    float attn_scale, hipStream_t stream);

/* Exported-but-unbound variant of the reference (megakernel.cu:1198-1244):
 * identical to launch_ldg_decode_direct. cache_len is accepted and not used, as
 * in the reference, whose kernel attends over positions 0..position. */
int launch_ldg_decode_persistent(
    int input_token_id, int* output_token_id, const void* embed_weight,
    const LDGLayerWeight* layer_weights, const void* final_norm_weight,
    const void* lm_head_weight, const void* cos_table, const void* sin_table,
    void* k_cache, void* v_cache, void* hidden_buffer, void* g_activations,
    void* g_residual, void* g_q, void* g_k, void* g_v, void* g_attn_out,
    void* g_mlp_intermediate, void* g_normalized, void* block_max_vals,
    void* block_max_idxs, int num_layers, int position, int cache_len,
    int max_seq_len, float attn_scale, hipStream_t stream);

/* num_steps greedy decode steps in ONE kernel launch with no host round trip
 * (megakernel.cu:1247-1314): step s consumes the token at position
 * start_position + s (step 0: first_token_id, later: the previous argmax) and
 * writes its argmax to output_log[s] (device int32[num_steps]). */
int launch_ldg_generate_nosync(
    int first_token_id, int num_steps, const void* embed_weight,
    const LDGLayerWeight* layer_weights, const void* final_norm_weight,
    const void* lm_head_weight, const void* cos_table, const void* sin_table,
    void* k_cache, void* v_cache, void* hidden_buffer, void* g_activations,
    void* g_residual, void* g_q, void* g_k, void* g_v, void* g_attn_out,
    void* g_mlp_intermediate, void* g_normalized, void* block_max_vals,
    void* block_max_idxs, int* output_log, int num_layers, int start_position,
    int max_seq_len, float attn_scale, hipStream_t stream);

/* ---- additions (no counterpart in the reference) ---------------------------------- */

/* generate_nosync with two extras, for prefill and parity checks:
 * forced_tokens (device int32[num_steps], nullable): step s >= 1 consumes
 *   forced_tokens[s] instead of the previous argmax (teacher forcing; a prompt
 *   is prefilled in one launch);
 * logits_out (device fp32[num_steps][151936], nullable): every step's logits;
 * hidden_steps (device fp32[num_steps][1024], nullable): every step's
 *   final-layer residual (the value written to hidden_buffer). */
int qwen_generate_ex(
    int first_token_id, int num_steps, const int* forced_tokens,
    const void* embed_weight, const LDGLayerWeight* layer_weights,
    const void* final_norm_weight, const void* lm_head_weight,
    const void* cos_table, const void* sin_table, void* k_cache, void* v_cache,
    void* hidden_buffer, void* g_normalized, int* output_log, float* logits_out,
    float* hidden_steps, int num_layers, int start_position, int max_seq_len,
    float attn_scale, hipStream_t stream);

/* generate_nosync that ends after the first step whose argmax is eos_token_id
 * (no counterpart in the reference, which truncates on the host after all
 * num_steps: Model/Qwen06B_architecture.py:379-381). output_log[0 .. n) receives
 * the generated ids, the last one eos_token_id when it was reached, where
 * n = *out_count (device int32) <= num_steps; later entries are not written. The
 * K/V cache holds positions start_position .. start_position + n - 1. */
int qwen_generate_until(
    int first_token_id, int num_steps, int eos_token_id, const void* embed_weight,
    const LDGLayerWeight* layer_weights, const void* final_norm_weight,
    const void* lm_head_weight, const void* cos_table, const void* sin_table,
    void* k_cache, void* v_cache, void* hidden_buffer, void* g_normalized,
    int* output_log, int* out_count, int num_layers, int start_position,
    int max_seq_len, float attn_scale, hipStream_t stream);

/* launch_ldg_generate_nosync without any allocation, for callers that cannot
 * allocate device memory (tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. Same arguments, limits and
 * results as launch_ldg_generate_nosync; its exchange workspace is a fixed
 * 2,813,184-byte array in the library's device memory (one per GPU, held until
 * the process ends) instead of the allocated one, and memory is cleared with a
 * kernel, never hipMemset. Not for stream capture: on a stream that is being
 * captured it returns QWEN_ERR_ARG (the exchange tags' token epochs are launch
 * arguments, so a replayed graph would reuse them). Every call on a GPU shares
 * that GPU's array: calls that overlap on one GPU (two streams, two threads)
 * race and must be serialized by the caller. Errors are reported by
 * qwen_last_error(). */
int qwen_generate_nosync_noalloc(
    int first_token_id, int num_steps, const void* embed_weight,
    const LDGLayerWeight* layer_weights, const void* final_norm_weight,
    const void* lm_head_weight, const void* cos_table, const void* sin_table,
    void* k_cache, void* v_cache, void* hidden_buffer, void* g_activations,
    void* g_residual, void* g_q, void* g_k, void* g_v, void* g_attn_out,
    void* g_mlp_intermediate, void* g_normalized, void* block_max_vals,
    void* block_max_idxs, int* output_log, int num_layers, int start_position,
    int max_seq_len, float attn_scale, hipStream_t stream);

/* Batched prefill (no counterpart in the reference, which prefills with one
 * decode step per id, Model/Qwen06B_architecture.py:346-347): the n ids
 * (device int32[n]) at positions start_position .. start_position + n - 1 run
 * through all num_layers layers in one launch, as matrix products on MFMA;
 * writes the K/V cache of every one of those positions and, to hidden_buffer,
 * the last position's final-layer residual. No lm_head: the greedy token after
 * a prompt comes from a decode step of its last id. Ids outside [0, 151936)
 * are reported by qwen_last_error() (QWEN_ERR_BAD_TOKEN). A prompt prefilled
 * in pieces (each at its own start position) leaves the same K/V cache, bit for
 * bit, as one call with all of it. Allocates a 78 MB workspace per device on
 * first use (activations of up to 2048 positions, partial attention results). */
int qwen_prefill(
    const int* ids, int n, const void* embed_weight,
    const LDGLayerWeight* layer_weights, const void* cos_table,
    const void* sin_table, void* k_cache, void* v_cache, void* hidden_buffer,
    int num_layers, int start_position, int max_seq_len, float attn_scale,
    hipStream_t stream);

/* Profiling aid for qwen_prefill: the wall-clock times (s_memrealtime ticks,
 * 100 MHz) at which the last prefill on the current device started and passed
 * each of its grid barriers: [0] start, [1] after the embedding, then for each
 * layer the ends of its QKV, attention, o_proj, gate/up and down phases. Copies
 * min(max_entries, 2 + 5 * 28) entries to host memory `out`. */
int qwen_prefill_timestamps(unsigned long long* out, int max_entries);

/* Token sampling (no counterpart in the reference, which decodes greedily:
 * Model/Qwen06B_architecture.py:343-382). One token from fp32 logits[n] into
 * *out_token (device int32): temperature <= 0 or top_k == 1 gives the argmax
 * (lowest index on ties); otherwise the logits are scaled by 1/temperature,
 * top_k > 0 keeps the tokens whose logit is >= the k-th largest (ties kept),
 * top_p < 1 then keeps the most probable of those until the mass strictly
 * above a token reaches top_p of the kept mass (the boundary token and its
 * ties kept), and the token is drawn from the renormalised softmax over the
 * kept set by a Gumbel-max pick whose noise for token j is Philox4x32-10 of
 * counter (j, step, 0, 0) under key (seed low, seed high) words: the same
 * (logits, parameters, seed, step) always give the same token. NaN logits are
 * never drawn. */
int qwen_sample(const float* logits, int n, float temperature, int top_k, float top_p,
                unsigned long long seed, unsigned int step, int* out_token, hipStream_t stream);

/* Sampled generation (no counterpart in the reference): generate_nosync whose
 * every next token is drawn as qwen_sample draws it from that step's logits
 * (seed, step = the position of the step's input token) instead of the argmax.
 * Every parameter set runs as one launch of num_steps steps in which the decode
 * kernel draws each token itself (the same kept set and draw as qwen_sample):
 * temperature <= 0 or top_k == 1 is the argmax; temperature alone, top-k with
 * 1 <= top_k <= 128 (any top_p), and top-p alone or a larger top_k each have a
 * build of the kernel of their own. The last form decides from the 8 largest
 * logits of each of 256 vocabulary slices when those suffice and otherwise
 * splits its radix selections over every workgroup's slice. No host
 * synchronisation. With eos_token_id >= 0 the generation ends on the device
 * after the first sampled eos: output_log[0 .. n) holds the sampled ids, eos
 * last when it was reached, later entries are -1, and n = *out_count (device
 * int32, nullable) <= num_steps; the K/V cache holds positions start_position ..
 * start_position + n - 1. */
int qwen_generate_sampled(
    int first_token_id, int num_steps, int eos_token_id, const void* embed_weight,
    const LDGLayerWeight* layer_weights, const void* final_norm_weight,
    const void* lm_head_weight, const void* cos_table, const void* sin_table,
    void* k_cache, void* v_cache, void* hidden_buffer, void* g_normalized,
    int* output_log, int* out_count, int num_layers, int start_position,
    int max_seq_len, float attn_scale, float temperature, int top_k, float top_p,
    unsigned long long seed, hipStream_t stream);

/* Isolated lm_head + argmax: *out_token = argmax_r (W[r,:] . h), h fp16 [1024]
 * used as is (no norm), W fp16 [151936, 1024]; logits_out (fp32 [151936]) nullable.
 * Exact ties resolve to the lowest row. */
int qwen_lm_head_argmax(const void* hidden_f16, const void* weight, int* out_token,
                        float* logits_out, hipStream_t stream);

/* Isolated lm_head + draw (no counterpart in the reference): the same logits
 * as qwen_lm_head_argmax, then the token the decode kernel's sampling builds
 * draw inside a sampled generation (temperature > 0, top_k >= 0 and top_p as in
 * qwen_sample; Philox step = position). It equals qwen_sample on logits_out
 * with the same arguments; it exists to test those in-kernel draws. */
int qwen_lm_head_sample(const void* hidden_f16, const void* weight, float temperature, int top_k,
                        float top_p, unsigned long long seed, int position, int* out_token,
                        float* logits_out, hipStream_t stream);

/* Isolated MLP half-layer: y = x + down(silu(gate(n)) * up(n)), n = RMSNorm(x) * post_norm_w,
 * with x fp16 [1024], gate/up fp16 [3072,1024], down fp16 [1024,3072], y fp32 [1024]. */
int qwen_mlp_block(const void* x_f16, const void* post_norm_weight, const void* gate_weight,
                   const void* up_weight, const void* down_weight, float* y_out, hipStream_t stream);

/* Synchronizes the current device and returns the device-side error state of
 * the last launches: QWEN_OK, QWEN_ERR_TIMEOUT (a wait exceeded its deadline)
 * or QWEN_ERR_BAD_TOKEN (a forced id out of range); clears it and resets the
 * workspace when set. (Workgroup placement, workgroup w on XCD w % 8, is checked
 * once per device when the library first uses it: QWEN_ERR_DEVICE from every
 * entry point if it does not hold.) */
int qwen_last_error(void);

/* Test hook (no counterpart in the reference): the wall-clock budget, in
 * microseconds, of every single device-side wait of later launches on the
 * current device; 0 restores the default (500000 us). A tiny budget makes the
 * kernel's bounded waits give up, so the error path (status word, every wave
 * leaving, qwen_last_error resetting the workspace) can be exercised. */
int qwen_set_wait_deadline_us(long long us);

/* 2 (QWEN_ABI_VERSION), as qwen_ops.cpp:30-32. */
int qwen_abi_version(void);

/* Profiling aid: while buf is non-null, every launch on the current device
 * records wall-clock timestamps (s_memrealtime ticks, 100 MHz) for token index
 * `token` of the launch into buf[workgroup][stage][qwen_trace_events()]
 * (device u64, 256 x (8*num_layers+1) x events, `elems` entries in all: a launch
 * whose layers need more is refused with QWEN_ERR_ARG; stage 8*l + s is stage s of
 * layer l in the order QKV, attention, combine, o_proj, o_proj sum, gate/up,
 * down, down sum; stage 8*num_layers is the lm_head input and argmax).
 * Events, all from compute wave 0 of the workgroup: 0 = starts waiting for the
 * stage input, 1 = has its quarter of the input, 2 = passed the compute-wave
 * barrier, 3 = stored its results. Pass buf = NULL to stop. While tracing, the
 * launches run a second build of the kernel that carries the trace points (a few
 * microseconds per token slower); without it, the kernel has none. That build
 * decodes greedily: while tracing, the entry points that draw tokens inside
 * the decode kernel (qwen_generate_sampled's single-launch forms,
 * qwen_lm_head_sample) return QWEN_ERR_ARG. */
int qwen_set_trace(unsigned long long* buf, long long elems, int token);
int qwen_trace_events(void);

#ifdef __cplusplus
}
#endif

#endif /* QWEN_MEGAKERNEL_H */
