// Host-side launchers of the gfx950 kernels (defined in the *.hip files next
// to this header).  Every launcher enqueues on the given stream and returns
// hipGetLastError() of the launch.
//
// Cross-workgroup results are handed over only at kernel boundaries: a
// device-scope fence inside a kernel costs an L2 writeback per workgroup on
// this part, so every split reduction (attention chunks, argmax partials) is
// finished by a small follow-up kernel instead.
#pragma once

#include "fastdiv.h"
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

// "Q8L": a quantized activation in the lane layout the matvec consumes, so a
// consumer copies it to LDS with plain 16-byte loads:
//   u32[(c * 8 + l) * 4 + j] = int8 x4 of lane l (values 4l..4l+3) of block 4c+j
//   f32[chunks * 32 + b]     = fp32 scale of block b (fp16-rounded, as the
//                              reference quantizer stores it)
// Blocks past the width (up to a multiple of 4) hold zeros.
__host__ __device__ inline size_t q8l_bytes(int width) {
    const int chunks = (width / 32 + 3) / 4;
    return static_cast<size_t>(chunks) * 144;
}

// How the activation reaches the workgroup before the row dots.
enum class Prologue : int {
    Q8 = 0,       // GGUF Q8_0 blocks in device memory (host-quantized input)
    F32 = 1,      // f32 vector, quantized in-workgroup (fortai_q8_quantize)
    RMSNORM = 2,  // f32 x -> rms_norm(x, w) -> quantize
    Q8L = 3,      // producer-quantized activation in the Q8L layout
    GATED = 4,    // raw GDN output x with the gate already through SiLU (z):
                  // per-head gated RMSNorm ((x / rms(x)) * norm) * z
                  // (fortai_qwen35_cpu.f90:907-915)
};

// What happens to each row result.
enum class Epilogue : int {
    STORE = 0,      // out[row] = dot
    ADD = 1,        // out[row] = dot + resid[row]   (in place allowed)
    SILU_PAIR = 2,  // h[row] = silu(dot(w)) * dot(w2)  (fortai_silu_product);
                    // f32 to out (optional) and Q8L to out_q8l (optional)
};

struct MatvecSegment {
    Q8Matrix w;
    Q8Matrix w2;             // second matrix of a SILU_PAIR, same shape as w
    float *out = nullptr;
    const float *resid = nullptr;
    void *out_q8l = nullptr; // SILU_PAIR: quantized h for the next matvec
    // STORE with conv_w: the causal conv1d + SiLU of each row's channel over
    // its window conv_state[kernel-1][conv_size] (oldest first), which the
    // row's thread then shifts (fortai_qwen35_cpu.f90:856-879)
    const float *conv_w = nullptr;  // [rows][kernel]
    float *conv_state = nullptr;
    int conv_size = 0, kernel = 0;
    int conv_rows = 0;              // > 0: only rows below it have the conv (rows past it: STORE)
    bool silu = false;              // STORE without conv: out[row] = silu(dot)
    int silu_begin = 0, silu_end = 0;  // STORE: rows in [silu_begin, silu_end) also through SiLU
};

struct MatvecInput {
    const float *x = nullptr;     // F32 / RMSNORM: [width]
    const int8_t *xq = nullptr;   // Q8: GGUF blocks [blocks][34]
    const void *xq8l = nullptr;   // Q8L
    const float *norm = nullptr;  // RMSNORM: weights [width]; GATED: [head]
    const float *z = nullptr;     // GATED: silu(gate) [width]
    int head = 0;                 // GATED: head size (the norm's span)
    float eps = 0.0f;
    int width = 0;                // activation elements (multiple of 32)
};

// Plan recording: every launcher notes the kernel variant it launched
// (printf-style); last_launch() returns the note of this thread's last launch.
void note_launch(const char *fmt, ...);
const char *last_launch();
const char *prologue_name(Prologue p);
const char *epilogue_name(Epilogue e);

// Activation widths: the fp32-input prologues quantize up to
// kMatvecF32MaxWidth values in-kernel; the Q8L layout (producer-quantized, or
// launch_q8l_prep) serves up to kQ8lPrepMaxWidth.
constexpr int kMatvecF32MaxWidth = 8192;
constexpr int kQ8lPrepMaxWidth = 12288;

// Evaluate up to four matrices that share one activation in one launch.
hipError_t launch_q8_matvec(const MatvecSegment *segments, int count, const MatvecInput &in,
    Prologue prologue, Epilogue epilogue, hipStream_t stream);

// Batches of up to 8 sequences.  launch_q8l_prep builds each sequence's
// quantized activation (F32, RMSNORM or GATED prologue; x and z [batch][width])
// into q8l [batch][q8l_bytes(width)]; launch_q8_batch_matvec evaluates the
// segments for every sequence from it, outputs [batch][rows] (SILU_PAIR's
// out_q8l [batch][q8l_bytes(rows)], conv windows [batch][kernel-1][conv_size]).
hipError_t launch_q8l_prep(const MatvecInput &in, Prologue prologue, void *q8l, int batch, hipStream_t stream);
hipError_t launch_q8_batch_matvec(const MatvecSegment *segments, int count, const void *q8l, int width, int batch,
    Epilogue epilogue, hipStream_t stream);

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
// batch > 1 (device tokens only): token[s] -> out + s * width
hipError_t launch_q8_embedding(const Q8Matrix &w, const int64_t *token, int64_t token_value, float *out,
    hipStream_t stream, int batch = 1);
hipError_t launch_f16_embedding(const uint16_t *table, int rows, int width, const int64_t *token,
    int64_t token_value, float *out, hipStream_t stream, int batch = 1);
hipError_t launch_add(const float *a, const float *b, float *out, int n, hipStream_t stream);
hipError_t launch_rms_norm(const float *x, const float *w, float *out, int n, float eps,
    hipStream_t stream);

// fp16 matrix x f32 vector with the reference's sequential fp32 dot per row
// (fortai_gguf_runtime.f90:382-386), optional RMSNorm prologue, and per
// workgroup first-maximum partials finished by launch_argmax_finish.
struct ArgmaxState {
    float *partial_value = nullptr;   // [max workgroups]
    int32_t *partial_index = nullptr; // [max workgroups]
    int64_t *token = nullptr;         // argmax result (0-based row)
    int64_t *trace = nullptr;         // optional: trace[*position] = token
    int *position = nullptr;          // optional: advanced by one after the trace write
    int trace_capacity = 0;           // entries of trace
    // optional, single sequence: the token the next decode step embeds when
    // >= 0; -1 when it is still the argmax of the partials.  The producer of
    // the partials writes -1 and leaves the finish to launch_step_embedding
    // (or to launch_argmax_finish, which writes the resolved token here)
    int64_t *embed = nullptr;
};
hipError_t launch_f16_matvec(const uint16_t *w, int rows, int width, bool finite_halves, const float *x,
    const float *norm, float eps, float *out, const ArgmaxState *argmax, hipStream_t stream);
int f16_matvec_workgroups(int rows);
// The fp16 LM head for `batch` (<= 8) sequences at once: final RMSNorm
// (norm required) of x [batch][width] into xnorm [width][8] (interleaved), then
// out [batch][rows], argmax partials [batch][f16_batch_lm_head_workgroups(rows)]
// and the per-sequence finish.
hipError_t launch_f16_batch_lm_head(const uint16_t *w, int rows, int width, bool finite, int batch, const float *x,
    const float *norm, float eps, float *xnorm, float *out, const ArgmaxState &argmax, hipStream_t stream);
int f16_batch_lm_head_workgroups(int rows);
hipError_t launch_argmax(const float *values, int n, const ArgmaxState &state, hipStream_t stream);
// reduce `partials` argmax partials and publish token / trace / position
// batch > 1: sequence s reduces partials [s * partials, (s + 1) * partials)
// into token[s], trace[s * trace_capacity + position[s]], position[s]
// With state.embed: nothing when *embed >= 0 already, else the finish above and
// *embed = token.
hipError_t launch_argmax_finish(int partials, const ArgmaxState &state, hipStream_t stream, int batch = 1);
// A decode step's first kernel, the token embedding (fp16 table16 or Q8_0
// table8) with the previous step's argmax finish folded in: *state.embed >= 0
// is embedded as is; otherwise every workgroup reduces the `partials` partials
// (the first maximum, as launch_argmax_finish) and workgroup 0 publishes token,
// trace and position.  One launch fewer per token than finish + embedding.
hipError_t launch_step_embedding(const uint16_t *table16, const Q8Matrix *table8, int rows, int width,
    const ArgmaxState &state, int partials, float *out, hipStream_t stream);
// scan an fp16 table for exponent-31 patterns (inf/NaN), counted into *count
hipError_t launch_count_nonfinite_halves(const uint16_t *w, size_t n, unsigned int *count, hipStream_t stream);

// ---- token blocks on the i8 matrix cores (mmq.hip) --------------------------
// X8 token activations: [blocks_pad][ld][32] int8 then [blocks_pad][ld] f32
// scales, ld = q8_tokens_ld(tokens), blocks_pad = 4 * ceil(width / 128).
int q8_tokens_ld(int tokens);
size_t q8_tokens_bytes(int tokens, int width);
hipError_t launch_q8_quantize_tokens(const float *x, int tokens, int width, int ld_x, void *x8, hipStream_t stream);
// out[t * ld_out + row] = W . x_t (+ resid at the same index); optional
// int32 block dots [tokens][rows][blocks]
hipError_t launch_q8_mmq(const Q8Matrix &w, const void *x8, int tokens, float *out, int ld_out, const float *resid,
    int32_t *dots, hipStream_t stream);
// The same product with the reference's eight-lane fp32 order kept: every
// output is bit-identical to the decode matvec of its token.
hipError_t launch_q8_mmq_exact(const Q8Matrix &w, const void *x8, int tokens, float *out, int ld_out,
    const float *resid, hipStream_t stream);

// ---- Gated DeltaNet ------------------------------------------------------
struct GdnParams {
    const float *qkv = nullptr;       // [conv_size] conv + SiLU outputs (q | k | v channels)
    const float *alpha = nullptr;     // [value_heads]
    const float *beta = nullptr;      // [value_heads]
    const float *ssm_a = nullptr;     // [value_heads]
    const float *ssm_dt = nullptr;    // [value_heads]
    float *state = nullptr;           // [value_heads][head][8 lanes][head/8] (lane-major rows)
    float *out = nullptr;             // [value_heads * head] raw o (before the gated norm)
    int state_size = 0, key_heads = 0, value_heads = 0, head = 0;
    float eps = 0.0f;
};
// The delta rule, 16 state rows per workgroup: writes the raw output o.
// batch > 1: sequences along blockIdx.y, every buffer [batch][single size]
// `steps` autoregressive core steps (conv1d + SiLU + delta rule) in one launch
// with the state held in registers: qkv [steps][conv_size] projection outputs,
// alpha / beta [steps][value_heads], out [steps][value_heads * head]; p.qkv,
// p.alpha, p.beta, p.out point at those arrays; conv_in: a copy of
// conv_state taken before the launch.  head 128 only.
hipError_t launch_gdn_recurrence(const GdnParams &p, const float *conv_w, const float *conv_in, float *conv_state,
    int conv_size, int K, int steps, hipStream_t stream);
hipError_t launch_gdn_delta(const GdnParams &p, hipStream_t stream, int batch = 1);
// The delta rule of one whole value head per workgroup followed by the
// head's gated RMSNorm and Q8_0 quantization into q8l [batch][q8l_bytes(width)]
// (width = value_heads * head): the bits of launch_gdn_delta then
// launch_q8l_prep(GATED), in one launch.  head 64 or 128, width % 128 == 0;
// z: SiLU'd gate [batch][width]; norm: [head]; eps: the gated norm's.
hipError_t launch_gdn_delta_gated(const GdnParams &p, const float *z, const float *norm, float eps, void *q8l,
    hipStream_t stream, int batch);
// Causal conv1d + SiLU of every channel of x, shifting the windows
// conv_state[K-1][channels] (oldest first).
hipError_t launch_conv_silu(const float *x, const float *conv_w, float *conv_state, float *out, int channels, int K,
    hipStream_t stream);

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
    float *partial = nullptr;       // workspace (attention_scores_floats): scores, e values, Z tables
    int *cache_flags = nullptr;     // [kv_heads]: 1 once the cache holds an exponent-31 half
    float *out = nullptr;           // [heads][value] gated output
    // optional (batches): the same output also as the Q8L activation of the o
    // projection, [batch][q8l_bytes(heads * value)], written by the wide and
    // merge kernels (value % 64 == 0 and heads * value % 128 == 0)
    void *out_q8l = nullptr;
    const int *position = nullptr;  // device position (the new token's index)
    int heads = 0, kv_heads = 0, head = 0, value = 0, max_context = 0, rope_dim = 0;
    float eps = 0.0f;
    // Up to exact_max positions the output is the reference's two-pass softmax
    // with its summation orders (bit-exact); beyond, split-K over chunks of
    // the context with an online-softmax merge (within 1e-3 relative).  The
    // split-K kernels are launched only when max_context > exact_max.
    int exact_max = 1 << 30;
    float *split = nullptr;         // [heads][attention_split_chunks][value + 2]
    int z_skew = 0;                 // test hook: offset of the Z candidate windows (0 in use)
    int force_wide = 0;             // test hook: the batches' wide output kernel for one sequence too
    // the kernels' divisors, set by launch_attention from the fields above:
    // heads, kv_heads, heads / kv_heads, head, head / 8, value / 8, value / 64
    FastDiv div_heads, div_kv_heads, div_group, div_head, div_segs, div_slices, div_vd64;
};
int attention_split_chunks(int max_context);
// batch > 1: sequences along blockIdx.y, every buffer [batch][single size],
// position[batch]
hipError_t launch_attention(const AttentionParams &p, hipStream_t stream, int batch = 1);
// whether launch_attention honours p.out_q8l for this shape and batch (the
// wide output kernel and the split-K merge write it)
bool attention_quantizes_output(const AttentionParams &p, int batch);
size_t attention_scores_floats(int heads, int max_context);

// ---- prompt prefill (prefill.hip): rows are tokens, row s * T + t ---------------
// rows [r0, r0 + count) of an X8 buffer -> Q8L [count][q8l_bytes(width)]
hipError_t launch_x8_to_q8l(const void *x8, int tokens, int width, int r0, int count, void *q8l, hipStream_t stream);
// x [rows][width] -> optional RMSNorm -> X8 (q8_tokens_bytes(rows, width))
hipError_t launch_rms_quantize_tokens(const float *x, int rows, int width, const float *norm, float eps, void *x8,
    hipStream_t stream);
// GDN o and raw gate z [rows][width] -> per-head gated RMSNorm -> X8
hipError_t launch_gated_quantize_tokens(const float *o, const float *z, const float *norm, float eps, int rows,
    int width, int head, void *x8, hipStream_t stream);
// silu(gate) * up [rows][width] -> X8
hipError_t launch_silu_product_quantize(const float *gate, const float *up, int rows, int width, void *x8,
    hipStream_t stream);
// causal conv1d + SiLU over T tokens of every sequence, continuing conv_state
hipError_t launch_conv_silu_tokens(const float *x, const float *conv_w, float *conv_state, float *out, int batch, int T,
    int C, int K, hipStream_t stream);
// the delta rule over T tokens (p.qkv: conv outputs [rows][C], p.alpha/beta
// raw projections [rows][value_heads], p.out [rows][inner], p.state
// [batch][...] as the decode kernel keeps it); scratch [rows][key_heads] x 2
// and [rows][value_heads] x 2
hipError_t launch_gdn_prefill(const GdnParams &p, int batch, int T, float *qinv, float *kinv, float *beta_t,
    float *decay_t, hipStream_t stream);
// q/k norm + RoPE, fp16 K/V append at positions 0..T-1 and causal attention:
// p.q [rows][heads][2 head] (normalized in place), p.k/p.v [rows][kv_heads][head],
// caches and flags [batch][...]; out [rows][heads][head]
// matrix_cores: fp16 MFMA scores and P.V (the default prefill mode); false:
// the fp32 kernel throughout (the exact mode)
hipError_t launch_attention_prefill(const AttentionParams &p, int batch, int T, float *out, hipStream_t stream,
    bool matrix_cores);

}  // namespace fortai_hip
