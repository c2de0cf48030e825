/* fortai_hip_stub.c -- weak stand-ins for every entry point of
 * include/fortai_hip_backend.h, for FortAI builds that link the HIP binding
 * module without libfortai_hip.so (as src/backend/cpu/fortai_cuda_stub.c does
 * for the CUDA binding).  As the reference's stub
 * (src/backend/cpu/fortai_cuda_stub.c:13-23) does: a create or upload sets
 * its out-handle to NULL and fails with FORTAI_HIP_RUNTIME_ERROR, every
 * destroy (NULL included) succeeds, every other call fails with
 * FORTAI_HIP_RUNTIME_ERROR and last_error says why.  Linking the real library
 * overrides all of them. */
#include "fortai_hip_backend.h"

#define FORTAI_HIP_WEAK __attribute__((weak))

static const char *const fortai_hip_stub_message = "FortAI was built without the HIP backend (libfortai_hip.so)";

FORTAI_HIP_WEAK int fortai_hip_q8_context_create(int device, fortai_hip_q8_context **context)
{
    (void)device;
    if (context) *context = NULL;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_context_destroy(fortai_hip_q8_context *context)
{
    (void)context;
    return FORTAI_HIP_OK;
}

FORTAI_HIP_WEAK int fortai_hip_q8_context_set_position(fortai_hip_q8_context *context, int position)
{
    (void)context;
    (void)position;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_context_capture_begin(fortai_hip_q8_context *context)
{
    (void)context;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_context_capture_end(fortai_hip_q8_context *context)
{
    (void)context;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_context_graph_launch(fortai_hip_q8_context *context)
{
    (void)context;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_context_synchronize(fortai_hip_q8_context *context)
{
    (void)context;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_context_timer_start(fortai_hip_q8_context *context)
{
    (void)context;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_context_timer_stop(fortai_hip_q8_context *context, float *elapsed_ms)
{
    (void)context;
    (void)elapsed_ms;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_weights_upload(fortai_hip_q8_context *context, const void *host_weights, size_t weight_bytes, int rows, int width, fortai_hip_q8_weights **weights)
{
    (void)context;
    (void)host_weights;
    (void)weight_bytes;
    (void)rows;
    (void)width;
    if (weights) *weights = NULL;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_weights_destroy(fortai_hip_q8_weights *weights)
{
    (void)weights;
    return FORTAI_HIP_OK;
}

FORTAI_HIP_WEAK int fortai_hip_q8_device_buffer_create(fortai_hip_q8_context *context, size_t bytes, void **device_buffer)
{
    (void)context;
    (void)bytes;
    if (device_buffer) *device_buffer = NULL;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_device_buffer_destroy(fortai_hip_q8_context *context, void *device_buffer)
{
    (void)context;
    (void)device_buffer;
    return FORTAI_HIP_OK;
}

FORTAI_HIP_WEAK int fortai_hip_q8_device_buffer_upload(fortai_hip_q8_context *context, void *device_buffer, const void *host_data, size_t bytes)
{
    (void)context;
    (void)device_buffer;
    (void)host_data;
    (void)bytes;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_device_buffer_upload_ptr(fortai_hip_q8_context *context, void *device_buffer, const void *host_data, size_t bytes)
{
    (void)context;
    (void)device_buffer;
    (void)host_data;
    (void)bytes;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_device_buffer_download(fortai_hip_q8_context *context, void *host_data, const void *device_buffer, size_t bytes)
{
    (void)context;
    (void)host_data;
    (void)device_buffer;
    (void)bytes;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_matvec_resident(fortai_hip_q8_context *context, const fortai_hip_q8_weights *weights, const void *device_activation, void *device_output, float *kernel_ms)
{
    (void)context;
    (void)weights;
    (void)device_activation;
    (void)device_output;
    (void)kernel_ms;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_matvec_device_f32(fortai_hip_q8_context *context, const fortai_hip_q8_weights *weights, const void *device_activation, size_t activation_elements, void *device_output, size_t output_elements)
{
    (void)context;
    (void)weights;
    (void)device_activation;
    (void)activation_elements;
    (void)device_output;
    (void)output_elements;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_embedding_device(fortai_hip_q8_context *context, const fortai_hip_q8_weights *weights, int64_t token_id, void *device_output, size_t output_elements)
{
    (void)context;
    (void)weights;
    (void)token_id;
    (void)device_output;
    (void)output_elements;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_copy_device(fortai_hip_q8_context *context, const void *device_input, void *device_output, size_t bytes)
{
    (void)context;
    (void)device_input;
    (void)device_output;
    (void)bytes;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_add_device(fortai_hip_q8_context *context, const void *device_left, const void *device_right, void *device_output, size_t elements)
{
    (void)context;
    (void)device_left;
    (void)device_right;
    (void)device_output;
    (void)elements;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_rms_norm_device(fortai_hip_q8_context *context, const void *device_input, const void *device_weights, void *device_output, size_t elements, float epsilon)
{
    (void)context;
    (void)device_input;
    (void)device_weights;
    (void)device_output;
    (void)elements;
    (void)epsilon;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_matvec_host(fortai_hip_q8_context *context, const fortai_hip_q8_weights *weights, const void *host_activation, size_t activation_bytes, float *host_output, size_t output_bytes, float *elapsed_ms)
{
    (void)context;
    (void)weights;
    (void)host_activation;
    (void)activation_bytes;
    (void)host_output;
    (void)output_bytes;
    (void)elapsed_ms;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_matvec_host_pair(fortai_hip_q8_context *context, const fortai_hip_q8_weights *first_weights, const fortai_hip_q8_weights *second_weights, const void *host_activation, size_t activation_bytes, float *first_output, size_t first_output_bytes, float *second_output, size_t second_output_bytes, float *elapsed_ms)
{
    (void)context;
    (void)first_weights;
    (void)second_weights;
    (void)host_activation;
    (void)activation_bytes;
    (void)first_output;
    (void)first_output_bytes;
    (void)second_output;
    (void)second_output_bytes;
    (void)elapsed_ms;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_matvec_host_triplet(fortai_hip_q8_context *context, const fortai_hip_q8_weights *first_weights, const fortai_hip_q8_weights *second_weights, const fortai_hip_q8_weights *third_weights, const void *host_activation, size_t activation_bytes, float *first_output, size_t first_output_bytes, float *second_output, size_t second_output_bytes, float *third_output, size_t third_output_bytes, float *elapsed_ms)
{
    (void)context;
    (void)first_weights;
    (void)second_weights;
    (void)third_weights;
    (void)host_activation;
    (void)activation_bytes;
    (void)first_output;
    (void)first_output_bytes;
    (void)second_output;
    (void)second_output_bytes;
    (void)third_output;
    (void)third_output_bytes;
    (void)elapsed_ms;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_matvec_host_triplet_contiguous(fortai_hip_q8_context *context, const fortai_hip_q8_weights *first_weights, const fortai_hip_q8_weights *second_weights, const fortai_hip_q8_weights *third_weights, const void *host_activation, size_t activation_bytes, float *host_output, size_t host_output_bytes, float *elapsed_ms)
{
    (void)context;
    (void)first_weights;
    (void)second_weights;
    (void)third_weights;
    (void)host_activation;
    (void)activation_bytes;
    (void)host_output;
    (void)host_output_bytes;
    (void)elapsed_ms;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_ffn_host(fortai_hip_q8_context *context, const fortai_hip_q8_weights *gate_weights, const fortai_hip_q8_weights *up_weights, const fortai_hip_q8_weights *down_weights, const void *host_activation, size_t activation_bytes, float *host_output, size_t output_bytes, float *elapsed_ms)
{
    (void)context;
    (void)gate_weights;
    (void)up_weights;
    (void)down_weights;
    (void)host_activation;
    (void)activation_bytes;
    (void)host_output;
    (void)output_bytes;
    (void)elapsed_ms;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_ffn_device(fortai_hip_q8_context *context, const fortai_hip_q8_weights *gate_weights, const fortai_hip_q8_weights *up_weights, const fortai_hip_q8_weights *down_weights, const void *device_activation, size_t activation_elements, void *device_output, size_t output_elements)
{
    (void)context;
    (void)gate_weights;
    (void)up_weights;
    (void)down_weights;
    (void)device_activation;
    (void)activation_elements;
    (void)device_output;
    (void)output_elements;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_recurrent_create(fortai_hip_q8_context *context, const fortai_hip_q8_weights *qkv_weights, const fortai_hip_q8_weights *gate_weights, const fortai_hip_q8_weights *alpha_weights, const fortai_hip_q8_weights *beta_weights, const fortai_hip_q8_weights *output_weights, const void *conv_weights, size_t conv_weight_bytes, int conv_size, int conv_kernel, const void *ssm_a, size_t ssm_a_bytes, const void *ssm_dt, size_t ssm_dt_bytes, const void *ssm_norm, size_t ssm_norm_bytes, int state_size, int key_heads, int value_heads, int head_size, int inner_size, float norm_epsilon, fortai_hip_qwen35_recurrent **layer)
{
    (void)context;
    (void)qkv_weights;
    (void)gate_weights;
    (void)alpha_weights;
    (void)beta_weights;
    (void)output_weights;
    (void)conv_weights;
    (void)conv_weight_bytes;
    (void)conv_size;
    (void)conv_kernel;
    (void)ssm_a;
    (void)ssm_a_bytes;
    (void)ssm_dt;
    (void)ssm_dt_bytes;
    (void)ssm_norm;
    (void)ssm_norm_bytes;
    (void)state_size;
    (void)key_heads;
    (void)value_heads;
    (void)head_size;
    (void)inner_size;
    (void)norm_epsilon;
    if (layer) *layer = NULL;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_recurrent_destroy(fortai_hip_qwen35_recurrent *layer)
{
    (void)layer;
    return FORTAI_HIP_OK;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_recurrent_reset(fortai_hip_qwen35_recurrent *layer)
{
    (void)layer;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_recurrent_run(fortai_hip_qwen35_recurrent *layer, const void *host_activation, size_t activation_bytes, float *host_output, size_t output_bytes, float *elapsed_ms)
{
    (void)layer;
    (void)host_activation;
    (void)activation_bytes;
    (void)host_output;
    (void)output_bytes;
    (void)elapsed_ms;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_recurrent_run_device(fortai_hip_qwen35_recurrent *layer, const void *device_activation, size_t activation_elements, void *device_output, size_t output_elements)
{
    (void)layer;
    (void)device_activation;
    (void)activation_elements;
    (void)device_output;
    (void)output_elements;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_attention_create(fortai_hip_q8_context *context, const fortai_hip_q8_weights *query_weights, const fortai_hip_q8_weights *key_weights, const fortai_hip_q8_weights *value_weights, const fortai_hip_q8_weights *output_weights, const void *query_norm, size_t query_norm_bytes, const void *key_norm, size_t key_norm_bytes, int heads, int key_value_heads, int head_size, int value_size, int max_context, int rope_dimension, float rope_base, float norm_epsilon, fortai_hip_qwen35_attention **layer)
{
    (void)context;
    (void)query_weights;
    (void)key_weights;
    (void)value_weights;
    (void)output_weights;
    (void)query_norm;
    (void)query_norm_bytes;
    (void)key_norm;
    (void)key_norm_bytes;
    (void)heads;
    (void)key_value_heads;
    (void)head_size;
    (void)value_size;
    (void)max_context;
    (void)rope_dimension;
    (void)rope_base;
    (void)norm_epsilon;
    if (layer) *layer = NULL;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_attention_destroy(fortai_hip_qwen35_attention *layer)
{
    (void)layer;
    return FORTAI_HIP_OK;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_attention_reset(fortai_hip_qwen35_attention *layer)
{
    (void)layer;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_attention_run_device(fortai_hip_qwen35_attention *layer, const void *device_activation, size_t activation_elements, int position, void *device_output, size_t output_elements)
{
    (void)layer;
    (void)device_activation;
    (void)activation_elements;
    (void)position;
    (void)device_output;
    (void)output_elements;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK const char * fortai_hip_q8_last_error(const fortai_hip_q8_context *context)
{
    (void)context;
    return fortai_hip_stub_message;
}

FORTAI_HIP_WEAK int fortai_hip_f16_weights_upload(fortai_hip_q8_context *context, const void *host_weights, size_t weight_bytes, int rows, int width, fortai_hip_f16_weights **weights)
{
    (void)context;
    (void)host_weights;
    (void)weight_bytes;
    (void)rows;
    (void)width;
    if (weights) *weights = NULL;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_f16_weights_destroy(fortai_hip_f16_weights *weights)
{
    (void)weights;
    return FORTAI_HIP_OK;
}

FORTAI_HIP_WEAK int fortai_hip_f16_matvec_device(fortai_hip_q8_context *context, const fortai_hip_f16_weights *weights, const void *device_activation, size_t activation_elements, void *device_output, size_t output_elements, void *device_token)
{
    (void)context;
    (void)weights;
    (void)device_activation;
    (void)activation_elements;
    (void)device_output;
    (void)output_elements;
    (void)device_token;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_embedding_f16_device(fortai_hip_q8_context *context, const fortai_hip_f16_weights *weights, int64_t token_id, void *device_output, size_t output_elements)
{
    (void)context;
    (void)weights;
    (void)token_id;
    (void)device_output;
    (void)output_elements;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_argmax_device(fortai_hip_q8_context *context, const void *device_values, size_t elements, void *device_token)
{
    (void)context;
    (void)device_values;
    (void)elements;
    (void)device_token;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_quantize_device(fortai_hip_q8_context *context, const void *device_input, size_t elements, void *device_blocks, void *device_scales)
{
    (void)context;
    (void)device_input;
    (void)elements;
    (void)device_blocks;
    (void)device_scales;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_block_dots_device(fortai_hip_q8_context *context, const fortai_hip_q8_weights *weights, const void *device_activation, void *device_dots)
{
    (void)context;
    (void)weights;
    (void)device_activation;
    (void)device_dots;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_recurrent_core_steps_device(fortai_hip_qwen35_recurrent *layer,
    const void *device_qkv, const void *device_alpha, const void *device_beta, int steps, void *device_output)
{
    (void)layer; (void)device_qkv; (void)device_alpha; (void)device_beta; (void)steps; (void)device_output;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_recurrent_core_device(fortai_hip_qwen35_recurrent *layer, const void *device_qkv, const void *device_alpha, const void *device_beta, void *device_output)
{
    (void)layer;
    (void)device_qkv;
    (void)device_alpha;
    (void)device_beta;
    (void)device_output;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_recurrent_state_download(fortai_hip_qwen35_recurrent *layer, float *host_gdn_state, size_t gdn_bytes, float *host_conv_state, size_t conv_bytes)
{
    (void)layer;
    (void)host_gdn_state;
    (void)gdn_bytes;
    (void)host_conv_state;
    (void)conv_bytes;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_recurrent_state_upload(fortai_hip_qwen35_recurrent *layer, const float *host_gdn_state, size_t gdn_bytes, const float *host_conv_state, size_t conv_bytes)
{
    (void)layer;
    (void)host_gdn_state;
    (void)gdn_bytes;
    (void)host_conv_state;
    (void)conv_bytes;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_attention_prefill_core_device(fortai_hip_qwen35_attention *layer, void *device_query, const void *device_key, const void *device_value, int T, int matrix_cores, void *device_output)
{
    (void)layer;
    (void)device_query;
    (void)device_key;
    (void)device_value;
    (void)T;
    (void)matrix_cores;
    (void)device_output;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_attention_core_device(fortai_hip_qwen35_attention *layer, const void *device_query, const void *device_key, const void *device_value, void *device_output)
{
    (void)layer;
    (void)device_query;
    (void)device_key;
    (void)device_value;
    (void)device_output;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_attention_cache_download(fortai_hip_qwen35_attention *layer, uint16_t *host_keys, uint16_t *host_values, int positions)
{
    (void)layer;
    (void)host_keys;
    (void)host_values;
    (void)positions;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_attention_cache_upload(fortai_hip_qwen35_attention *layer, const uint16_t *host_keys, const uint16_t *host_values, int positions)
{
    (void)layer;
    (void)host_keys;
    (void)host_values;
    (void)positions;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_decoder_create(fortai_hip_q8_context *context, int layer_count, fortai_hip_qwen35_recurrent *const *recurrent, fortai_hip_qwen35_attention *const *attention, const fortai_hip_q8_weights *const *ffn_gate, const fortai_hip_q8_weights *const *ffn_up, const fortai_hip_q8_weights *const *ffn_down, const float *const *attn_norm, const float *const *post_norm, const float *output_norm, int hidden_size, const fortai_hip_f16_weights *embedding_f16, const fortai_hip_q8_weights *embedding_q8, const fortai_hip_f16_weights *output_f16, const fortai_hip_q8_weights *output_q8, int max_context, float norm_epsilon, fortai_hip_qwen35_decoder **decoder)
{
    (void)context;
    (void)layer_count;
    (void)recurrent;
    (void)attention;
    (void)ffn_gate;
    (void)ffn_up;
    (void)ffn_down;
    (void)attn_norm;
    (void)post_norm;
    (void)output_norm;
    (void)hidden_size;
    (void)embedding_f16;
    (void)embedding_q8;
    (void)output_f16;
    (void)output_q8;
    (void)max_context;
    (void)norm_epsilon;
    if (decoder) *decoder = NULL;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_decoder_destroy(fortai_hip_qwen35_decoder *decoder)
{
    (void)decoder;
    return FORTAI_HIP_OK;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_decoder_reset(fortai_hip_qwen35_decoder *decoder)
{
    (void)decoder;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_decoder_forward(fortai_hip_qwen35_decoder *decoder, int64_t token, int position, float *host_logits, int64_t *next_token)
{
    (void)decoder;
    (void)token;
    (void)position;
    (void)host_logits;
    (void)next_token;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_decoder_generate(fortai_hip_qwen35_decoder *decoder, int64_t token, int position, int steps, int64_t *host_trace)
{
    (void)decoder;
    (void)token;
    (void)position;
    (void)steps;
    (void)host_trace;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_decoder_replay(fortai_hip_qwen35_decoder *decoder, int steps)
{
    (void)decoder;
    (void)steps;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_decoder_status(fortai_hip_qwen35_decoder *decoder)
{
    (void)decoder;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_decoder_trace(fortai_hip_qwen35_decoder *decoder, int first, int count,
    int64_t *host_trace)
{
    (void)decoder; (void)first; (void)count; (void)host_trace;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_decoder_logits(fortai_hip_qwen35_decoder *decoder, void **device_logits)
{
    (void)decoder;
    if (device_logits) *device_logits = NULL;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_batch_matvec_noalloc(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *weights, const void *device_x, int batch, void *device_output)
{
    (void)context; (void)weights; (void)device_x; (void)batch; (void)device_output;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_batch_matvec_device(fortai_hip_q8_context *context,
    const fortai_hip_q8_weights *weights, const void *device_x, int batch, void *device_output, float *kernel_ms)
{
    (void)context; (void)weights; (void)device_x; (void)batch; (void)device_output; (void)kernel_ms;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK size_t fortai_hip_q8_tokens_bytes(int tokens, int width)
{
    (void)tokens; (void)width;
    return 0;
}

FORTAI_HIP_WEAK int fortai_hip_q8_quantize_tokens_device(fortai_hip_q8_context *context, const void *device_x,
    int tokens, int width, void *device_tokens)
{
    (void)context; (void)device_x; (void)tokens; (void)width; (void)device_tokens;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_mmq_device(fortai_hip_q8_context *context, const fortai_hip_q8_weights *weights,
    const void *device_tokens, int tokens, void *device_output, const void *device_residual, float *kernel_ms)
{
    (void)context; (void)weights; (void)device_tokens; (void)tokens; (void)device_output; (void)device_residual;
    (void)kernel_ms;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_mmq_exact_device(fortai_hip_q8_context *context, const fortai_hip_q8_weights *weights,
    const void *device_tokens, int tokens, void *device_output, const void *device_residual, float *kernel_ms)
{
    (void)context; (void)weights; (void)device_tokens; (void)tokens; (void)device_output; (void)device_residual;
    (void)kernel_ms;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_mmq_block_dots(fortai_hip_q8_context *context, const fortai_hip_q8_weights *weights,
    const void *device_tokens, int tokens, void *device_dots)
{
    (void)context; (void)weights; (void)device_tokens; (void)tokens; (void)device_dots;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_batch_create(fortai_hip_q8_context *context, int batch, int layer_count,
    fortai_hip_qwen35_recurrent *const *recurrent, fortai_hip_qwen35_attention *const *attention,
    const fortai_hip_q8_weights *const *ffn_gate, const fortai_hip_q8_weights *const *ffn_up,
    const fortai_hip_q8_weights *const *ffn_down, const float *const *attn_norm, const float *const *post_norm,
    const float *output_norm, int hidden_size, const fortai_hip_f16_weights *embedding_f16,
    const fortai_hip_q8_weights *embedding_q8, const fortai_hip_f16_weights *output_f16,
    const fortai_hip_q8_weights *output_q8, int max_context, float norm_epsilon, fortai_hip_qwen35_batch **batch_decoder)
{
    (void)context; (void)batch; (void)layer_count; (void)recurrent; (void)attention; (void)ffn_gate; (void)ffn_up;
    (void)ffn_down; (void)attn_norm; (void)post_norm; (void)output_norm; (void)hidden_size; (void)embedding_f16;
    (void)embedding_q8; (void)output_f16; (void)output_q8; (void)max_context; (void)norm_epsilon;
    if (batch_decoder) *batch_decoder = NULL;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_batch_destroy(fortai_hip_qwen35_batch *batch_decoder)
{
    (void)batch_decoder;
    return FORTAI_HIP_OK;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_batch_reset(fortai_hip_qwen35_batch *batch_decoder)
{
    (void)batch_decoder;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_batch_forward(fortai_hip_qwen35_batch *batch_decoder, const int64_t *tokens,
    const int *positions, float *host_logits, int64_t *next_tokens)
{
    (void)batch_decoder; (void)tokens; (void)positions; (void)host_logits; (void)next_tokens;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_batch_generate(fortai_hip_qwen35_batch *batch_decoder, const int64_t *tokens,
    const int *positions, int steps, int64_t *host_trace)
{
    (void)batch_decoder; (void)tokens; (void)positions; (void)steps; (void)host_trace;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_batch_replay(fortai_hip_qwen35_batch *batch_decoder, int steps)
{
    (void)batch_decoder; (void)steps;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_batch_prefill(fortai_hip_qwen35_batch *batch_decoder, const int64_t *tokens,
    int T, int64_t *next_tokens, float *host_logits, float *kernel_ms)
{
    (void)batch_decoder; (void)tokens; (void)T; (void)next_tokens; (void)host_logits; (void)kernel_ms;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_batch_logits(fortai_hip_qwen35_batch *batch_decoder, void **device_logits)
{
    (void)batch_decoder; (void)device_logits;
    if (device_logits) *device_logits = NULL;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_decoder_plan(const fortai_hip_qwen35_decoder *decoder, char *buffer, size_t bytes,
    size_t *needed)
{
    (void)decoder; (void)buffer; (void)bytes;
    if (needed) *needed = 0;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_batch_plan(const fortai_hip_qwen35_batch *batch_decoder, int prefill,
    char *buffer, size_t bytes, size_t *needed)
{
    (void)batch_decoder; (void)prefill; (void)buffer; (void)bytes;
    if (needed) *needed = 0;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK size_t fortai_hip_q8_pack_bytes(int rows, int width)
{
    (void)rows; (void)width;
    return 0;
}

FORTAI_HIP_WEAK int fortai_hip_q8_weights_pack(const fortai_hip_q8_weights *weights, void *host, size_t bytes)
{
    (void)weights; (void)host; (void)bytes;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_weights_upload_packed(fortai_hip_q8_context *context, const void *host, size_t bytes,
    int rows, int width, fortai_hip_q8_weights **weights)
{
    (void)context; (void)host; (void)bytes; (void)rows; (void)width;
    if (weights) *weights = NULL;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_attention_set_exact_max(fortai_hip_qwen35_attention *layer, int exact_max)
{
    (void)layer; (void)exact_max;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_attention_set_test_options(fortai_hip_qwen35_attention *layer, int z_skew,
    int force_wide)
{
    (void)layer; (void)z_skew; (void)force_wide;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_decoder_set_mode(fortai_hip_qwen35_decoder *decoder, int flags)
{
    (void)decoder; (void)flags;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_batch_set_mode(fortai_hip_qwen35_batch *batch_decoder, int flags)
{
    (void)batch_decoder; (void)flags;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_qwen35_batch_set_prefill_mode(fortai_hip_qwen35_batch *batch_decoder, int mode)
{
    (void)batch_decoder; (void)mode;
    return FORTAI_HIP_RUNTIME_ERROR;
}

FORTAI_HIP_WEAK int fortai_hip_q8_context_scratch_bytes(const fortai_hip_q8_context *context, size_t *bytes)
{
    (void)context;
    if (bytes) *bytes = 0;
    return FORTAI_HIP_RUNTIME_ERROR;
}
