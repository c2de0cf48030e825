/*
 * fortai_hip_backend.h -- C ABI of the MI355X (gfx950) FortAI backend.
 *
 * Drop-in counterpart of the reference's CUDA ABI
 * (backend/cuda/fortai_cuda_backend.h:22-152): every fortai_cuda_* entry point
 * exists here as fortai_hip_* with the same arguments, ownership and return
 * codes, so the reference's iso_c_binding wrapper
 * (src/backend/cuda/fortai_backend_cuda.f90:67-413) binds it by renaming the
 * bind(C) names.  Entry points marked [extension] have no reference
 * counterpart: the fp16 LM head / embedding the CUDA path lacks, parity probes
 * for the tests, and a fused whole-token decoder.
 *
 * Conventions (as the reference, fortai_cuda_backend.cu:42-52,805-893):
 *  - return 0 OK, 1 INVALID (argument or shape precondition), 2 RUNTIME_ERROR
 *    (HIP failure; message via fortai_hip_q8_last_error);
 *  - the backend allocates handles and the caller destroys them; layers and
 *    weights borrow their context; destroy(NULL) returns OK;
 *  - one non-blocking stream per context; device ops are asynchronous, ops that
 *    return host data synchronise;
 *  - kernels read the token position from device memory written by
 *    set_position, so a captured graph replays with new positions.
 */
#ifndef FORTAI_HIP_BACKEND_H
#define FORTAI_HIP_BACKEND_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct fortai_hip_q8_context fortai_hip_q8_context;
typedef struct fortai_hip_q8_weights fortai_hip_q8_weights;
typedef struct fortai_hip_qwen35_recurrent fortai_hip_qwen35_recurrent;
typedef struct fortai_hip_qwen35_attention fortai_hip_qwen35_attention;
typedef struct fortai_hip_f16_weights fortai_hip_f16_weights;          /* [extension] */
typedef struct fortai_hip_qwen35_decoder fortai_hip_qwen35_decoder;    /* [extension] */
typedef struct fortai_hip_qwen35_batch fortai_hip_qwen35_batch;        /* [extension] */

enum {
    FORTAI_HIP_OK = 0,
    FORTAI_HIP_INVALID = 1,
    FORTAI_HIP_RUNTIME_ERROR = 2
};

/* ---- context (fortai_cuda_backend.h:22-27) ---- */
int fortai_hip_q8_context_create(int device, fortai_hip_q8_context **context);
int fortai_hip_q8_context_destroy(fortai_hip_q8_context *context);
int fortai_hip_q8_context_set_position(fortai_hip_q8_context *context, int position);
int fortai_hip_q8_context_capture_begin(fortai_hip_q8_context *context);
int fortai_hip_q8_context_capture_end(fortai_hip_q8_context *context);
int fortai_hip_q8_context_graph_launch(fortai_hip_q8_context *context);
/* [extension] bytes of the scratch buffers the context has allocated on
 * demand (quantized activations, FFN hidden, outputs of the host paths) */
int fortai_hip_q8_context_scratch_bytes(const fortai_hip_q8_context *context, size_t *bytes);
/* [extension] wait for all work queued on the context's stream */
int fortai_hip_q8_context_synchronize(fortai_hip_q8_context *context);
/* [extension] HIP events on the context's stream: timer_start records the
 * start event; timer_stop records the stop event, waits for it and returns
 * the elapsed milliseconds of the work enqueued in between. */
int fortai_hip_q8_context_timer_start(fortai_hip_q8_context *context);
int fortai_hip_q8_context_timer_stop(fortai_hip_q8_context *context, float *elapsed_ms);

/* ---- resident Q8_0 weights (fortai_cuda_backend.h:29-32).  Accepts the raw
 * GGUF Q8_0 bytes [rows][width/32][34]; they are repacked on the device into a
 * lane-interleaved int8 plane plus an fp16 scale plane (same 34 B / 32 values). */
int fortai_hip_q8_weights_upload(fortai_hip_q8_context *context,
    const void *host_weights, size_t weight_bytes, int rows, int width,
    fortai_hip_q8_weights **weights);
int fortai_hip_q8_weights_destroy(fortai_hip_q8_weights *weights);

/* ---- device buffers (fortai_cuda_backend.h:34-45) ---- */
int fortai_hip_q8_device_buffer_create(fortai_hip_q8_context *context,
    size_t bytes, void **device_buffer);
int fortai_hip_q8_device_buffer_destroy(fortai_hip_q8_context *context,
    void *device_buffer);
int fortai_hip_q8_device_buffer_upload(fortai_hip_q8_context *context,
    void *device_buffer, const void *host_data, size_t bytes);
int fortai_hip_q8_device_buffer_upload_ptr(fortai_hip_q8_context *context,
    void *device_buffer, const void *host_data, size_t bytes);
int fortai_hip_q8_device_buffer_download(fortai_hip_q8_context *context,
    void *host_data, const void *device_buffer, size_t bytes);

/* ---- resident ops (fortai_cuda_backend.h:47-66).  device_activation of
 * matvec_resident is a device Q8_0 activation in GGUF block layout; kernel_ms
 * times the kernel only. */
int fortai_hip_q8_matvec_resident(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *weights, const void *device_activation,
    void *device_output, float *kernel_ms);
int fortai_hip_q8_matvec_device_f32(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *weights, const void *device_activation,
    size_t activation_elements, void *device_output, size_t output_elements);
int fortai_hip_qwen35_embedding_device(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *weights, int64_t token_id, void *device_output,
    size_t output_elements);
int fortai_hip_qwen35_copy_device(fortai_hip_q8_context *context,
    const void *device_input, void *device_output, size_t bytes);
int fortai_hip_qwen35_add_device(fortai_hip_q8_context *context,
    const void *device_left, const void *device_right, void *device_output,
    size_t elements);
int fortai_hip_qwen35_rms_norm_device(fortai_hip_q8_context *context,
    const void *device_input, const void *device_weights, void *device_output,
    size_t elements, float epsilon);

/* ---- host-controlled ops (fortai_cuda_backend.h:68-110): host Q8_0
 * activation in, host fp32 out; elapsed_ms includes the transfers. */
int fortai_hip_q8_matvec_host(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *weights, const void *host_activation,
    size_t activation_bytes, float *host_output, size_t output_bytes,
    float *elapsed_ms);
int fortai_hip_q8_matvec_host_pair(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *first_weights,
    const fortai_hip_q8_weights *second_weights, const void *host_activation,
    size_t activation_bytes, float *first_output, size_t first_output_bytes,
    float *second_output, size_t second_output_bytes, float *elapsed_ms);
int fortai_hip_q8_matvec_host_triplet(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *first_weights,
    const fortai_hip_q8_weights *second_weights,
    const fortai_hip_q8_weights *third_weights, const void *host_activation,
    size_t activation_bytes, float *first_output, size_t first_output_bytes,
    float *second_output, size_t second_output_bytes, float *third_output,
    size_t third_output_bytes, float *elapsed_ms);
int fortai_hip_q8_matvec_host_triplet_contiguous(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *first_weights,
    const fortai_hip_q8_weights *second_weights,
    const fortai_hip_q8_weights *third_weights, const void *host_activation,
    size_t activation_bytes, float *host_output, size_t host_output_bytes,
    float *elapsed_ms);
int fortai_hip_q8_ffn_host(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *gate_weights,
    const fortai_hip_q8_weights *up_weights,
    const fortai_hip_q8_weights *down_weights, const void *host_activation,
    size_t activation_bytes, float *host_output, size_t output_bytes,
    float *elapsed_ms);
int fortai_hip_q8_ffn_device(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *gate_weights,
    const fortai_hip_q8_weights *up_weights,
    const fortai_hip_q8_weights *down_weights, const void *device_activation,
    size_t activation_elements, void *device_output, size_t output_elements);

/* ---- Qwen3.5 recurrent (Gated DeltaNet) layer (fortai_cuda_backend.h:112-134).
 * Requires state_size == head_size, head_size in {64,128,256},
 * value_heads % key_heads == 0, value_heads * head_size == inner_size. */
int fortai_hip_qwen35_recurrent_create(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *qkv_weights,
    const fortai_hip_q8_weights *gate_weights,
    const fortai_hip_q8_weights *alpha_weights,
    const fortai_hip_q8_weights *beta_weights,
    const fortai_hip_q8_weights *output_weights,
    const void *conv_weights, size_t conv_weight_bytes, int conv_size, int conv_kernel,
    const void *ssm_a, size_t ssm_a_bytes, const void *ssm_dt, size_t ssm_dt_bytes,
    const void *ssm_norm, size_t ssm_norm_bytes, int state_size, int key_heads,
    int value_heads, int head_size, int inner_size, float norm_epsilon,
    fortai_hip_qwen35_recurrent **layer);
int fortai_hip_qwen35_recurrent_destroy(fortai_hip_qwen35_recurrent *layer);
int fortai_hip_qwen35_recurrent_reset(fortai_hip_qwen35_recurrent *layer);
int fortai_hip_qwen35_recurrent_run(fortai_hip_qwen35_recurrent *layer,
    const void *host_activation, size_t activation_bytes, float *host_output,
    size_t output_bytes, float *elapsed_ms);
int fortai_hip_qwen35_recurrent_run_device(fortai_hip_qwen35_recurrent *layer,
    const void *device_activation, size_t activation_elements,
    void *device_output, size_t output_elements);

/* ---- Qwen3.5 gated full-attention layer (fortai_cuda_backend.h:136-150).
 * The KV cache is fp16, [max_context][kv_heads][head_size], written with the
 * reference CPU path's float_to_half (ties away from zero). */
int fortai_hip_qwen35_attention_create(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *query_weights,
    const fortai_hip_q8_weights *key_weights,
    const fortai_hip_q8_weights *value_weights,
    const fortai_hip_q8_weights *output_weights,
    const void *query_norm, size_t query_norm_bytes,
    const void *key_norm, size_t key_norm_bytes,
    int heads, int key_value_heads, int head_size, int value_size,
    int max_context, int rope_dimension, float rope_base, float norm_epsilon,
    fortai_hip_qwen35_attention **layer);
int fortai_hip_qwen35_attention_destroy(fortai_hip_qwen35_attention *layer);
int fortai_hip_qwen35_attention_reset(fortai_hip_qwen35_attention *layer);
int fortai_hip_qwen35_attention_run_device(fortai_hip_qwen35_attention *layer,
    const void *device_activation, size_t activation_elements, int position,
    void *device_output, size_t output_elements);

const char *fortai_hip_q8_last_error(const fortai_hip_q8_context *context);

/* =================== [extension] entry points ======================== */

/* fp16 matrices (tied token embedding / LM head), GGUF F16 row-major
 * [rows][width].  The matvec runs the reference's sequential fp32 dot per row
 * (fortai_gguf_runtime.f90:382-386) and can fuse the first-index argmax
 * (app/fortai_cpu_run.f90:58): device_token (int64, may be NULL). */
int fortai_hip_f16_weights_upload(fortai_hip_q8_context *context,
    const void *host_weights, size_t weight_bytes, int rows, int width,
    fortai_hip_f16_weights **weights);
int fortai_hip_f16_weights_destroy(fortai_hip_f16_weights *weights);
int fortai_hip_f16_matvec_device(fortai_hip_q8_context *context,
    const fortai_hip_f16_weights *weights, const void *device_activation,
    size_t activation_elements, void *device_output, size_t output_elements,
    void *device_token);
int fortai_hip_qwen35_embedding_f16_device(fortai_hip_q8_context *context,
    const fortai_hip_f16_weights *weights, int64_t token_id, void *device_output,
    size_t output_elements);
/* first-index argmax of a device fp32 vector into a device int64 */
int fortai_hip_argmax_device(fortai_hip_q8_context *context,
    const void *device_values, size_t elements, void *device_token);

/* Repacked-weight cache.  A Q8_0 matrix is repacked at upload into this
 * backend's resident layout; these let a host cache those planes and skip
 * the repack next time (the reference keys its pack files by model /
 * backend / variant / ABI version, src/fortai_cache.f90:6-31).
 * pack_bytes: size of the planes of a rows x width matrix (0 if invalid);
 * weights_pack: copy a resident matrix's planes to host memory (synchronous);
 * weights_upload_packed: create a resident matrix from such planes. */
size_t fortai_hip_q8_pack_bytes(int rows, int width);
int fortai_hip_q8_weights_pack(const fortai_hip_q8_weights *weights, void *host, size_t bytes);
int fortai_hip_q8_weights_upload_packed(fortai_hip_q8_context *context, const void *host, size_t bytes, int rows,
    int width, fortai_hip_q8_weights **weights);

/* Parity probes: fortai_q8_quantize on device (GGUF block bytes + fp32
 * scales), and the exact int32 dot of every (row, block) [rows][width/32]. */
int fortai_hip_q8_quantize_device(fortai_hip_q8_context *context,
    const void *device_input, size_t elements, void *device_blocks,
    void *device_scales);
int fortai_hip_q8_block_dots_device(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *weights, const void *device_activation,
    void *device_dots);

/* Batched matvec: device fp32 x [batch][width] (batch 1..8) -> out
 * [batch][rows], every weight read once for all rows of x; each output row
 * is bit-identical to fortai_hip_q8_matvec_device_f32 of that x.  kernel_ms
 * (may be NULL): event-timed duration, synchronising. */
int fortai_hip_q8_batch_matvec_device(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *weights, const void *device_x, int batch,
    void *device_output, float *kernel_ms);
/* [extension, no reference counterpart] fortai_hip_q8_batch_matvec_device
 * without any allocation, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops): the quantized
 * activations go to a fixed per-GPU array inside the library instead of a
 * buffer it allocates on demand.  Limit: batch * ceil(width / 128) * 144 <=
 * 147456 bytes (batch 8 at width 16384); larger requests return INVALID.  The
 * array is shared by every call on a GPU and keeps the last call's contents.
 * Calls from different contexts on one GPU are serialised: a call makes its
 * context's stream wait for the previous other context's call to finish.
 * Outputs are bit-identical to fortai_hip_q8_batch_matvec_device. */
int fortai_hip_q8_batch_matvec_noalloc(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *weights, const void *device_x, int batch, void *device_output);

/* Token blocks (prefill, batches) on the i8 matrix cores.  The reference runs
 * every token through the matvec of fortai_gguf_runtime.f90:424-465; these
 * compute the same product for `tokens` activations at once.
 * quantize_tokens: device fp32 x [tokens][width] (row pitch `width`) ->
 * fortai_q8_quantize (fortai_q8_dot.c:153-198) of every token into a device
 * buffer of fortai_hip_q8_tokens_bytes(tokens, width) bytes.
 * mmq: out[t][rows] (fp32) = W . x_t for every token, plus device_residual
 * [tokens][rows] when it is not NULL (may alias the output).  The int32 block
 * dots are exact; the fp32 accumulation is the scalar reference's
 * result += scale * dot per block (fortai_q8_dot.c:262-284), so results
 * agree with the AVX2 path to fp32 rounding.  kernel_ms (may be NULL):
 * event-timed kernel duration, synchronising.
 * mmq_exact: the same product with the reference's AVX2 accumulation kept
 * (eight fp32 lane chains per output and its horizontal sum,
 * fortai_q8_dot.c:287-331): every output is bit-identical to the decode
 * matvec of its token.  The prompt prefill's default projections.
 * mmq_block_dots: the exact int32 dot of every (token, row, block), device
 * int32 [tokens][rows][width/32] (parity probe). */
size_t fortai_hip_q8_tokens_bytes(int tokens, int width);
int fortai_hip_q8_quantize_tokens_device(fortai_hip_q8_context *context,
    const void *device_x, int tokens, int width, void *device_tokens);
int fortai_hip_q8_mmq_device(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *weights, const void *device_tokens, int tokens,
    void *device_output, const void *device_residual, float *kernel_ms);
int fortai_hip_q8_mmq_exact_device(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *weights, const void *device_tokens, int tokens,
    void *device_output, const void *device_residual, float *kernel_ms);
int fortai_hip_q8_mmq_block_dots(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *weights, const void *device_tokens, int tokens,
    void *device_dots);

/* Recurrent-layer core step (conv1d + SiLU + L2 norm + decay/beta + delta
 * rule; no projections, no gated norm): device fp32 qkv [conv_size], alpha and
 * beta [value_heads] in, raw output [inner_size].  State access uses the
 * reference layouts: gdn [value_heads][head][head] row-major, conv
 * [conv_kernel-1][conv_size] oldest first. */
int fortai_hip_qwen35_recurrent_core_device(fortai_hip_qwen35_recurrent *layer,
    const void *device_qkv, const void *device_alpha, const void *device_beta,
    void *device_output);
/* [extension] `steps` autoregressive core steps in one launch with the state
 * held in registers (state-resident): device qkv
 * [steps][conv_size], alpha and beta [steps][value_heads], out
 * [steps][inner_size]; state, conv windows and outputs bit-identical to
 * `steps` calls of fortai_hip_qwen35_recurrent_core_device.  Head 128. */
int fortai_hip_qwen35_recurrent_core_steps_device(fortai_hip_qwen35_recurrent *layer,
    const void *device_qkv, const void *device_alpha, const void *device_beta, int steps, void *device_output);
int fortai_hip_qwen35_recurrent_state_download(fortai_hip_qwen35_recurrent *layer,
    float *host_gdn_state, size_t gdn_bytes, float *host_conv_state, size_t conv_bytes);
int fortai_hip_qwen35_recurrent_state_upload(fortai_hip_qwen35_recurrent *layer,
    const float *host_gdn_state, size_t gdn_bytes, const float *host_conv_state,
    size_t conv_bytes);

/* Attention-layer core step at the context's device position: q projection
 * output [heads][q | gate], k [kv_heads][head], v [kv_heads][value] (device
 * fp32) -> gated attention output [heads][value].  Cache access in fp16 bits
 * for positions [0, positions). */
int fortai_hip_qwen35_attention_core_device(fortai_hip_qwen35_attention *layer,
    const void *device_query, const void *device_key, const void *device_value,
    void *device_output);
/* The prompt prefill's attention for one sequence of T tokens from position
 * 0 [extension; the reference has no prefill, it runs
 * fortai_qwen35_cpu.f90:990-1031 once per token]: q [T][heads][q | gate],
 * k [T][kv_heads][head], v [T][kv_heads][value] (device fp32) -> gated
 * outputs [T][heads][value]; q is normalised and rotated in place and K/V are
 * appended at positions 0..T-1.  matrix_cores = 0: the exact kernel (the
 * reference's summation orders, the default prefill), 1: the fp16
 * matrix-core kernel of the FORTAI_HIP_PREFILL_FAST prefill mode.  Heads of 64, 128 or 256. */
int fortai_hip_qwen35_attention_prefill_core_device(fortai_hip_qwen35_attention *layer,
    void *device_query, const void *device_key, const void *device_value, int T,
    int matrix_cores, void *device_output);
int fortai_hip_qwen35_attention_cache_download(fortai_hip_qwen35_attention *layer,
    uint16_t *host_keys, uint16_t *host_values, int positions);
int fortai_hip_qwen35_attention_cache_upload(fortai_hip_qwen35_attention *layer,
    const uint16_t *host_keys, const uint16_t *host_values, int positions);

/* Fused whole-token decoder over already created layers and weights.
 * Layer i is recurrent[i] (GDN) or attention[i] (full attention); every layer
 * has ffn_gate/up/down and host fp32 attn_norm/post_norm [hidden].  The token
 * embedding and LM head are fp16 (tied allowed) or Q8_0.  One decode step is a
 * single captured HIP graph: embedding, 5 launches per layer, LM head with
 * the fused argmax; the graph advances the device token and position itself,
 * so generate() replays it back to back with no host round trip per token. */
int fortai_hip_qwen35_decoder_create(fortai_hip_q8_context *context, int layer_count,
    fortai_hip_qwen35_recurrent *const *recurrent,
    fortai_hip_qwen35_attention *const *attention,
    const fortai_hip_q8_weights *const *ffn_gate,
    const fortai_hip_q8_weights *const *ffn_up,
    const fortai_hip_q8_weights *const *ffn_down,
    const float *const *attn_norm, const float *const *post_norm,
    const float *output_norm, int hidden_size,
    const fortai_hip_f16_weights *embedding_f16, const fortai_hip_q8_weights *embedding_q8,
    const fortai_hip_f16_weights *output_f16, const fortai_hip_q8_weights *output_q8,
    int max_context, float norm_epsilon, fortai_hip_qwen35_decoder **decoder);
int fortai_hip_qwen35_decoder_destroy(fortai_hip_qwen35_decoder *decoder);
/* zero every layer state and the token trace */
int fortai_hip_qwen35_decoder_reset(fortai_hip_qwen35_decoder *decoder);
/* one step at (token, position): host_logits (vocab floats) and next_token
 * may be NULL; synchronises only when either is requested */
int fortai_hip_qwen35_decoder_forward(fortai_hip_qwen35_decoder *decoder, int64_t token,
    int position, float *host_logits, int64_t *next_token);
/* greedy decode of `steps` tokens starting from (token, position); the trace
 * (steps ids) is written to host_trace.  Steps are enqueued back to back. */
int fortai_hip_qwen35_decoder_generate(fortai_hip_qwen35_decoder *decoder, int64_t token,
    int position, int steps, int64_t *host_trace);
/* enqueue `steps` further graph replays continuing from the device token and
 * position (no host synchronisation; for timing loops) */
int fortai_hip_qwen35_decoder_replay(fortai_hip_qwen35_decoder *decoder, int steps);
/* wait for the queued steps (RUNTIME_ERROR with the reason in last_error
 * when a step failed) */
int fortai_hip_qwen35_decoder_status(fortai_hip_qwen35_decoder *decoder);
/* The kernels one decode step launches, as the reference's PlanIR steps
 * (src/fortai_plan_ir.f90:7-21: operation, kernel, batch size), recorded when
 * the step was captured (or by the first step): text lines
 * "operation<TAB>kernel<TAB>batch<LF>", NUL-terminated.  *needed (may be NULL)
 * receives the size including the NUL; buffer may be NULL to query it;
 * INVALID when bytes is too small. */
int fortai_hip_qwen35_decoder_plan(const fortai_hip_qwen35_decoder *decoder, char *buffer, size_t bytes,
    size_t *needed);
/* device pointer of the decoder's logits [vocab] */
int fortai_hip_qwen35_decoder_logits(fortai_hip_qwen35_decoder *decoder, void **device_logits);
/* the greedy ids the decoder wrote at positions first .. first+count-1
 * (the token each step chose; synchronises) */
int fortai_hip_qwen35_decoder_trace(fortai_hip_qwen35_decoder *decoder, int first, int count, int64_t *host_trace);

/* [extension] Batched decoder: `batch` (1..8) independent sequences over the
 * same layers and weights as fortai_hip_qwen35_decoder_create (same
 * arguments).  The layer objects supply weights and constants only: the batch
 * object holds every sequence's conv/GDN state and KV cache (max_context
 * positions each).  One step is one captured graph that reads every weight
 * once for all sequences; each sequence's logits and tokens are bit-identical
 * to the single-sequence decoder's.  The reference decodes one sequence at a
 * time (app/fortai_cpu_run.f90:50-64); sequence s here is that loop on its own
 * token and position. */
int fortai_hip_qwen35_batch_create(fortai_hip_q8_context *context, int batch, int layer_count,
    fortai_hip_qwen35_recurrent *const *recurrent,
    fortai_hip_qwen35_attention *const *attention,
    const fortai_hip_q8_weights *const *ffn_gate,
    const fortai_hip_q8_weights *const *ffn_up,
    const fortai_hip_q8_weights *const *ffn_down,
    const float *const *attn_norm, const float *const *post_norm,
    const float *output_norm, int hidden_size,
    const fortai_hip_f16_weights *embedding_f16, const fortai_hip_q8_weights *embedding_q8,
    const fortai_hip_f16_weights *output_f16, const fortai_hip_q8_weights *output_q8,
    int max_context, float norm_epsilon, fortai_hip_qwen35_batch **batch_decoder);
int fortai_hip_qwen35_batch_destroy(fortai_hip_qwen35_batch *batch_decoder);
/* zero every sequence's state, cache and trace */
int fortai_hip_qwen35_batch_reset(fortai_hip_qwen35_batch *batch_decoder);
/* one step of every sequence at (tokens[s], positions[s]); host_logits
 * [batch][vocab] and next_tokens [batch] may be NULL */
int fortai_hip_qwen35_batch_forward(fortai_hip_qwen35_batch *batch_decoder, const int64_t *tokens,
    const int *positions, float *host_logits, int64_t *next_tokens);
/* greedy decode of `steps` tokens per sequence from (tokens[s], positions[s]);
 * host_trace [batch][steps] */
int fortai_hip_qwen35_batch_generate(fortai_hip_qwen35_batch *batch_decoder, const int64_t *tokens,
    const int *positions, int steps, int64_t *host_trace);
/* enqueue `steps` further steps from the device tokens and positions (no
 * synchronisation; for timing loops) */
int fortai_hip_qwen35_batch_replay(fortai_hip_qwen35_batch *batch_decoder, int steps);
/* Prompt prefill of every sequence from position 0 (after create or reset):
 * tokens [batch][T]; all batch x T tokens go through each layer at once (the
 * projections as token-block products on the i8 matrix cores, conv1d / delta
 * rule / causal attention looping over time), leaving every state, cache,
 * token and position as T decode steps of those tokens would (within fp32
 * rounding: the reference has no prefill and runs each prompt token through
 * the decode step, fortai_qwen35_cpu.f90:591-711).  next_tokens [batch]
 * (greedy token after the prompt), host_logits [batch][vocab] and kernel_ms
 * (event-timed prefill) may be NULL. */
int fortai_hip_qwen35_batch_prefill(fortai_hip_qwen35_batch *batch_decoder, const int64_t *tokens, int T,
    int64_t *next_tokens, float *host_logits, float *kernel_ms);
/* As fortai_hip_qwen35_decoder_plan: the launches of one batched step
 * (prefill == 0) or of the last prefill (prefill != 0). */
int fortai_hip_qwen35_batch_plan(const fortai_hip_qwen35_batch *batch_decoder, int prefill, char *buffer,
    size_t bytes, size_t *needed);
/* device pointer of the logits [batch][vocab] */
int fortai_hip_qwen35_batch_logits(fortai_hip_qwen35_batch *batch_decoder, void **device_logits);

/* [extension] Options, set by explicit calls (the library reads nothing from
 * the environment).
 * attention_set_exact_max: the positions up to which the attention output
 * keeps the reference's two-pass summation orders, bit-exact
 * (fortai_qwen35_cpu.f90:1006-1031; default 8192); beyond them split-K with an
 * online-softmax merge, within 1e-3 relative.  Set it before a decoder or
 * batch is created over the layer.
 * attention_set_test_options [test only; results stay bit-identical]:
 * z_skew moves every Z candidate window by that many floats, so that the
 * running sums fall outside them and the walk's own chain runs; force_wide
 * runs the batches' wide output kernel for a single sequence too.
 * decoder_set_mode / batch_set_mode: FORTAI_HIP_DECODER_DIRECT enqueues the
 * kernels every step instead of replaying a captured graph (same kernels,
 * same results; for kernel tracing).  The *_ONLY flags [timing probes,
 * decoder only; any combination] enqueue only those kernel families of the
 * step -- the Q8_0 projections, the GDN delta rule, the attention kernels,
 * the embedding and LM head -- so the values are meaningless.  The step is
 * re-captured.
 * batch_set_prefill_mode: FORTAI_HIP_PREFILL_EXACT (default; bit-identical to
 * token-by-token decoding), _MATVEC (the batched decode matvec, 8 tokens at a
 * time; the same bits), _FAST (whole-block int32 dots on the i8 matrix cores
 * and the fp16 matrix-core attention; within 5e-2, not bit-exact). */
#define FORTAI_HIP_DECODER_DIRECT 1
#define FORTAI_HIP_DECODER_MATVEC_ONLY 2
#define FORTAI_HIP_DECODER_GDN_ONLY 4
#define FORTAI_HIP_DECODER_ATTENTION_ONLY 8
#define FORTAI_HIP_DECODER_HEAD_ONLY 16
#define FORTAI_HIP_PREFILL_EXACT 0
#define FORTAI_HIP_PREFILL_MATVEC 1
#define FORTAI_HIP_PREFILL_FAST 2
int fortai_hip_qwen35_attention_set_exact_max(fortai_hip_qwen35_attention *layer, int exact_max);
int fortai_hip_qwen35_attention_set_test_options(fortai_hip_qwen35_attention *layer, int z_skew, int force_wide);
int fortai_hip_qwen35_decoder_set_mode(fortai_hip_qwen35_decoder *decoder, int flags);
int fortai_hip_qwen35_batch_set_mode(fortai_hip_qwen35_batch *batch_decoder, int flags);
int fortai_hip_qwen35_batch_set_prefill_mode(fortai_hip_qwen35_batch *batch_decoder, int mode);

#ifdef __cplusplus
}
#endif

#endif
