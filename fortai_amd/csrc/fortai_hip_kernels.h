// Host-side launchers of the gfx950 kernels (defined in the *.hip files next
// to this header).  Every launcher enqueues on the given stream and returns
// hipGetLastError() of the launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace fortai_hip {

// Q8_0 matrix repacked at upload (layout documented in q8_kernels.hip).
struct Q8Matrix {
    const uint4 *quants = nullptr;  // [row_groups][chunks][64 lanes] x 16 B
    const uint2 *scales = nullptr;  // [row_groups][chunks][8 rows] x 4 fp16
    int rows = 0;                   // logical rows
    int blocks = 0;                 // 32-value blocks per row (width / 32)
    int chunks = 0;                 // ceil(blocks / 4)
    int row_groups = 0;             // ceil(rows / 8)
};

// How the activation reaches the workgroup before the row dots.
enum class Prologue : int {
    Q8 = 0,       // already quantized: GGUF Q8_0 blocks in device memory
    F32 = 1,      // f32 vector, quantized in-workgroup (fortai_q8_quantize)
    RMSNORM = 2,  // f32 x -> rms_norm(x, w) -> quantize
    GATED = 3,    // GDN output: o/rms(o)*ssm_norm*silu(z) per head -> quantize
};

// What happens to each row result.
enum class Epilogue : int {
    STORE = 0,      // out[row] = dot
    ADD = 1,        // out[row] = dot + resid[row]   (in place allowed)
    SILU_PAIR = 2,  // out[row] = silu(dot(w)) * dot(w2)  (fortai_silu_product)
};

struct MatvecSegment {
    Q8Matrix w;
    Q8Matrix w2;          // second matrix of a SILU_PAIR, same shape as w
    float *out = nullptr;
    const float *resid = nullptr;
};

struct MatvecInput {
    const float *x = nullptr;     // F32 / RMSNORM: [width]; GATED: o [width]
    const int8_t *xq = nullptr;   // Q8: GGUF blocks [blocks][34]
    const float *norm = nullptr;  // RMSNORM: weights [width]; GATED: ssm_norm [head]
    const float *gate = nullptr;  // GATED: z [width] (before SiLU)
    float eps = 0.0f;
    int width = 0;                // activation elements (multiple of 32)
    int head = 0;                 // GATED: values per head
};

// Evaluate up to four matrices that share one activation in one launch.
hipError_t launch_q8_matvec(const MatvecSegment *segments, int count, const MatvecInput &in,
    Prologue prologue, Epilogue epilogue, hipStream_t stream);

// Repack GGUF Q8_0 bytes [rows][blocks][34] (device) into the Q8Matrix planes.
hipError_t launch_q8_repack(const uint8_t *gguf, int rows, int blocks, uint4 *quants,
    uint2 *scales, hipStream_t stream);

// Test entry points: fortai_q8_quantize on device (GGUF block bytes + float
// scales) and the exact int32 per-block dots [rows][blocks].
hipError_t launch_q8_quantize(const float *x, int width, int8_t *out34, float *scales,
    hipStream_t stream);
hipError_t launch_q8_block_dots(const Q8Matrix &w, const int8_t *xq34, int32_t *out,
    hipStream_t stream);

// Small elementwise / norm kernels of the reference ABI.
hipError_t launch_q8_embedding(const Q8Matrix &w, const uint8_t *unused, const int64_t *token,
    int64_t token_value, float *out, hipStream_t stream);
hipError_t launch_f16_embedding(const uint16_t *table, int width, const int64_t *token,
    int64_t token_value, float *out, hipStream_t stream);
hipError_t launch_add(const float *a, const float *b, float *out, int n, hipStream_t stream);
hipError_t launch_rms_norm(const float *x, const float *w, float *out, int n, float eps,
    hipStream_t stream);

// fp16 matrix x f32 vector with the reference's sequential fp32 dot per row
// (fortai_gguf_runtime.f90:382-386), optional RMSNorm prologue and a fused
// first-index argmax whose final reduction is done by the last workgroup.
struct ArgmaxState {
    float *partial_value = nullptr;   // [max workgroups]
    int32_t *partial_index = nullptr; // [max workgroups]
    unsigned int *done = nullptr;     // zero between launches (the last WG resets it)
    int64_t *token = nullptr;         // argmax result (0-based row)
    int64_t *trace = nullptr;         // optional: trace[*position] = token
    int *position = nullptr;          // optional: advanced by one after the trace write
    int trace_capacity = 0;           // entries of trace
};
hipError_t launch_f16_matvec(const uint16_t *w, int rows, int width, const float *x,
    const float *norm, float eps, float *out, const ArgmaxState *argmax, hipStream_t stream);
int f16_matvec_workgroups(int rows);
hipError_t launch_argmax(const float *values, int n, const ArgmaxState &state, hipStream_t stream);

// ---- Gated DeltaNet ------------------------------------------------------
struct GdnParams {
    const float *qkv = nullptr;       // [conv_size] projection output (pre-conv)
    const float *alpha = nullptr;     // [value_heads]
    const float *beta = nullptr;      // [value_heads]
    const float *ssm_a = nullptr;     // [value_heads]
    const float *ssm_dt = nullptr;    // [value_heads]
    const float *conv_w = nullptr;    // [conv_size][kernel]
    float *conv_ring = nullptr;       // [kernel][conv_size]: x_t lives in slot t % kernel
    float *state = nullptr;           // [value_heads][head][8 lanes][head/8] (lane-major rows)
    float *out = nullptr;             // [value_heads * head] raw o (before the gated norm)
    int *step = nullptr;              // device step counter t of this layer
    unsigned int *done = nullptr;     // workgroup completion counter (self-resetting)
    int conv_size = 0, kernel = 0, state_size = 0, key_heads = 0, value_heads = 0, head = 0;
    float eps = 0.0f;
};
hipError_t launch_gdn_step(const GdnParams &p, hipStream_t stream);

// ---- attention -------------------------------------------------------------
struct AttentionParams {
    const float *q = nullptr;       // [heads][q(head) | gate(head)] projection output
    const float *k = nullptr;       // [kv_heads][head] projection output
    const float *v = nullptr;       // [kv_heads][value]
    const float *q_norm = nullptr;  // [head]
    const float *k_norm = nullptr;  // [head]
    const float2 *rope = nullptr;   // [max_context][rope_dim/2] (cos, sin)
    uint16_t *kcache = nullptr;     // [max_context][kv_heads][head] fp16 bits
    uint16_t *vcache = nullptr;     // [max_context][kv_heads][value] fp16 bits
    float *partial = nullptr;       // [kv_heads][chunks][group][value + 2]
    unsigned int *done = nullptr;   // [kv_heads] self-resetting counters
    float *out = nullptr;           // [heads][value]
    const int *position = nullptr;  // device position (the new token's index)
    int heads = 0, kv_heads = 0, head = 0, value = 0, max_context = 0, rope_dim = 0;
    int chunk = 0;                  // positions per workgroup
    float eps = 0.0f;
};
hipError_t launch_attention(const AttentionParams &p, hipStream_t stream);
int attention_chunk(int max_context);

}  // namespace fortai_hip
