// C ABI of the gfx950 FortAI backend (include/fortai_hip_backend.h).
//
// Host orchestration only: handles, validation, device allocation, and the
// enqueue order of the kernels in q8_kernels.hip, gdn.hip, attention.hip and
// lm_head.hip.  Entry points follow the reference CUDA ABI
// (backend/cuda/fortai_cuda_backend.cu:805-1736) in arguments, ownership and
// return codes; each carries the citation of the function it replaces.
#include "../../include/fortai_hip_backend.h"
#include "fortai_hip_internal.h"
#include "fortai_hip_kernels.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <new>
#include <initializer_list>
#include <mutex>
#include <string>
#include <vector>
#include <initializer_list>

using namespace fortai_hip;

// per-workgroup (value, index) partials of a fused argmax held by a context
// (the fp16 LM head uses one per 128 rows: vocabularies up to 524,288)
constexpr int kArgmaxParts = 4096;

// one recorded launch: the reference's PlanIR step (src/fortai_plan_ir.f90:7-11)
struct plan_step {
    std::string operation, kernel;
    int batch = 1;
};

struct fortai_hip_q8_context {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t start = nullptr, stop = nullptr;
    int *position = nullptr;    // device: current token position
    int64_t *token = nullptr;   // device: current token id
    int8_t *scratch_act = nullptr;
    size_t scratch_act_bytes = 0;
    float *scratch_out = nullptr;
    size_t scratch_out_bytes = 0;
    float *scratch_aux = nullptr;
    size_t scratch_aux_bytes = 0;
    float *argmax_value = nullptr;
    int32_t *argmax_index = nullptr;
    void *scratch_q8l = nullptr;  // quantized FFN hidden of the ABI FFN paths
    size_t scratch_q8l_bytes = 0;
    void *noalloc_scratch = nullptr;  // device address of this GPU's `scratch` array (set at create)
    hipEvent_t noalloc_done = nullptr;  // recorded after this context's last use of that array
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    char error[256] = {};
};

struct fortai_hip_q8_weights {
    fortai_hip_q8_context *context = nullptr;
    int width = 0;
    Q8Matrix m;
    uint4 *quants = nullptr;
    uint2 *scales = nullptr;
};

struct fortai_hip_f16_weights {
    fortai_hip_q8_context *context = nullptr;
    int rows = 0, width = 0;
    bool finite = false;  // no exponent-31 halves: the plain conversion is exact
    uint16_t *data = nullptr;
};

struct fortai_hip_qwen35_recurrent {
    fortai_hip_q8_context *context = nullptr;
    const fortai_hip_q8_weights *qkv = nullptr, *gate = nullptr, *alpha = nullptr, *beta = nullptr, *out = nullptr;
    int conv_size = 0, kernel = 0, state_size = 0, key_heads = 0, value_heads = 0, head = 0, inner = 0;
    float eps = 0.0f;
    float *conv_w = nullptr, *ssm_a = nullptr, *ssm_dt = nullptr, *ssm_norm = nullptr;
    float *conv_state = nullptr, *state = nullptr;
    float *proj = nullptr;  // projection outputs, one buffer: qkv | z | alpha | beta
    float *qkv_out = nullptr, *z_out = nullptr, *alpha_out = nullptr, *beta_out = nullptr;  // views of proj
    float *o_raw = nullptr;  // GDN output before the gated norm (ssm_out input)
    float *conv_snap = nullptr;  // recurrent_core_steps: the conv windows before a launch
    // qkv | gate | alpha | beta as one matrix (when each is whole 8-row
    // groups): the four projections then run as one single-segment launch
    Q8Matrix in_m;
    uint4 *in_quants = nullptr;
    uint2 *in_scales = nullptr;
};

struct fortai_hip_qwen35_attention {
    fortai_hip_q8_context *context = nullptr;
    const fortai_hip_q8_weights *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
    int heads = 0, kv_heads = 0, head = 0, value = 0, max_context = 0, rope_dim = 0;
    float rope_base = 0.0f, eps = 0.0f;
    float *q_norm = nullptr, *k_norm = nullptr;
    float2 *rope = nullptr;
    uint16_t *kcache = nullptr, *vcache = nullptr;
    float *proj = nullptr;  // projection outputs, one buffer: q | k | v
    float *q_out = nullptr, *k_out = nullptr, *v_out = nullptr;  // views of proj
    float *partial = nullptr;
    Q8Matrix in_m;  // q | k | v as one matrix (whole 8-row groups each)
    uint4 *in_quants = nullptr;
    uint2 *in_scales = nullptr;
    int *cache_flags = nullptr;  // per kv head: the cache holds an exponent-31 half
    float *attn_out = nullptr;   // gated attention output (o_proj input)
    int exact_max = 0;           // positions with the bit-exact two-pass softmax; split-K beyond
    int z_skew = 0;              // test option: offset of the Z candidate windows
    int force_wide = 0;          // test option: the wide output kernel for one sequence
    float *split = nullptr;      // split-K partials (allocated when max_context > exact_max)
};

constexpr int kDefaultExactMax = 8192;
// Kernel families of a decode step.  A decoder in a timing-probe mode
// enqueues only some of them (their values are then meaningless).
constexpr unsigned kFamMatvec = 1, kFamGdn = 2, kFamAttention = 4, kFamHead = 8, kFamAll = 15;
// prompt prefill projections: the exact token-block product (default), the
// batched decode matvec (same bits), or whole-block int32 dots (not exact)
enum class PrefillMode { EXACT = 0, MATVEC = 1, FAST = 2 };

struct decoder_layer {
    fortai_hip_qwen35_recurrent *recurrent = nullptr;
    fortai_hip_qwen35_attention *attention = nullptr;
    const fortai_hip_q8_weights *gate = nullptr, *up = nullptr, *down = nullptr;
    float *attn_norm = nullptr, *post_norm = nullptr;
};

struct fortai_hip_qwen35_decoder {
    fortai_hip_q8_context *context = nullptr;
    std::vector<decoder_layer> layers;
    int hidden = 0, vocab = 0, ffn = 0, max_context = 0;
    float eps = 0.0f;
    const fortai_hip_f16_weights *emb16 = nullptr, *out16 = nullptr;
    const fortai_hip_q8_weights *emb8 = nullptr, *out8 = nullptr;
    float *output_norm = nullptr, *x = nullptr, *logits = nullptr;
    void *h_q8l = nullptr;  // quantized FFN hidden
    float *argmax_value = nullptr;
    int32_t *argmax_index = nullptr;
    int64_t *trace = nullptr;
    int64_t *embed = nullptr;  // the next step's token, or -1: the argmax of the LM head's partials
    int next_position = 0;  // host mirror of the device position after the queued steps
    bool use_graph = true;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    // the *_ONLY timing-probe modes: a step enqueues only the selected kernel
    // families (same kernels, weights and arguments; the others are left out,
    // so the values are meaningless) -- for timing each family of a decode
    // step as the graph replays it
    unsigned families = kFamAll;  // kernel families a step enqueues (a timing probe: a subset)
    std::vector<plan_step> plan;  // the launches of one step (PlanIR steps)
};

// Batched decoder: `batch` independent sequences over one set of layers and
// weights.  The layer objects supply weights and constants; every sequence
// has its own conv/GDN state and KV cache, all [batch][single size].
struct batch_layer {
    fortai_hip_qwen35_recurrent *rec = nullptr;
    fortai_hip_qwen35_attention *att = nullptr;
    const fortai_hip_q8_weights *gate = nullptr, *up = nullptr, *down = nullptr;
    float *attn_norm = nullptr, *post_norm = nullptr;
    // recurrent
    float *conv_state = nullptr, *state = nullptr, *qkv = nullptr, *z = nullptr, *alpha = nullptr, *beta = nullptr,
          *o_raw = nullptr;
    // attention
    uint16_t *kcache = nullptr, *vcache = nullptr;
    float *q = nullptr, *k = nullptr, *v = nullptr, *partial = nullptr, *attn_out = nullptr, *split = nullptr;
    int *flags = nullptr;
};

struct fortai_hip_qwen35_batch {
    fortai_hip_q8_context *context = nullptr;
    int batch = 0, hidden = 0, vocab = 0, ffn = 0, max_context = 0, parts = 0, act_width = 0;
    float eps = 0.0f;
    std::vector<batch_layer> layers;
    const fortai_hip_f16_weights *emb16 = nullptr, *out16 = nullptr;
    const fortai_hip_q8_weights *emb8 = nullptr, *out8 = nullptr;
    float *output_norm = nullptr, *x = nullptr, *logits = nullptr;
    float *xnorm = nullptr;  // output-RMSNormed x [hidden][8 slots], the fp16 LM head input
    void *act = nullptr;     // quantized activations [batch][q8l_bytes(act_width)]
    void *h_q8l = nullptr;   // quantized FFN hidden [batch][q8l_bytes(ffn)]
    float *argmax_value = nullptr;
    int32_t *argmax_index = nullptr;
    int64_t *tokens = nullptr, *trace = nullptr;  // trace [batch][max_context]
    int *positions = nullptr;
    std::vector<int> next_positions;  // host mirror after the queued steps
    // prompt prefill buffers, rows = batch * T (grown on demand)
    int prefill_rows = 0;
    float *px = nullptr;                                   // residual stream [rows][hidden]
    void *px8 = nullptr;                                   // quantized tokens of the widest input
    float *pa = nullptr, *pb = nullptr, *pc = nullptr, *pd = nullptr;  // projections / stage outputs
    float *palpha = nullptr, *pbeta = nullptr, *pqinv = nullptr, *pkinv = nullptr, *pbt = nullptr, *pdt = nullptr;
    int64_t *ptokens = nullptr;
    void *pq8l = nullptr;                                  // exact mode: 8 tokens in the matvec layout
    bool use_graph = true;            // FORTAI_HIP_DECODER_DIRECT mode: enqueue the kernels every step
    PrefillMode prefill_mode = PrefillMode::EXACT;
    std::vector<plan_step> plan, prefill_plan;  // launches of one step / of the last prefill
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace {

int fail(fortai_hip_q8_context *ctx, int code, const char *op, hipError_t err = hipSuccess) {
    if (ctx) {
        if (err == hipSuccess) std::snprintf(ctx->error, sizeof(ctx->error), "%s", op);
        else std::snprintf(ctx->error, sizeof(ctx->error), "%s: %s", op, hipGetErrorString(err));
    }
    return code;
}

thread_local unsigned g_families = kFamAll;
inline bool fam(unsigned f) { return (g_families & f) != 0; }
// PlanIR recording (src/fortai_plan_ir.f90:7-21): while a plan is being
// recorded, every successful launch appends (operation, kernel, batch).
thread_local std::vector<plan_step> *g_plan = nullptr;
thread_local int g_plan_batch = 1;

hipError_t rec(hipError_t e, const char *operation) {
    if (e == hipSuccess && g_plan) g_plan->push_back({operation, last_launch(), g_plan_batch});
    return e;
}

// "operation\tkernel\tbatch\n" lines
std::string plan_text(const std::vector<plan_step> &plan) {
    std::string t;
    for (const auto &s : plan) t += s.operation + "\t" + s.kernel + "\t" + std::to_string(s.batch) + "\n";
    return t;
}

int copy_plan(const std::vector<plan_step> &plan, char *buffer, size_t bytes, size_t *needed) {
    const std::string t = plan_text(plan);
    if (needed) *needed = t.size() + 1;
    if (!buffer) return FORTAI_HIP_OK;
    if (bytes < t.size() + 1) return FORTAI_HIP_INVALID;
    std::memcpy(buffer, t.c_str(), t.size() + 1);
    return FORTAI_HIP_OK;
}

int done(fortai_hip_q8_context *ctx, hipError_t err, const char *op) {
    return err == hipSuccess ? FORTAI_HIP_OK : fail(ctx, FORTAI_HIP_RUNTIME_ERROR, op, err);
}

template <typename T>
hipError_t alloc(T **ptr, size_t count) {
    *ptr = nullptr;
    if (count == 0) return hipSuccess;
    return hipMalloc(reinterpret_cast<void **>(ptr), count * sizeof(T));
}

template <typename T>
void release(T *&ptr) {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
}

// The planes of several Q8_0 matrices of one width, one after the other, as
// one matrix (the planes are row-group major, so this is a concatenation).
// Only when every matrix is whole 8-row groups; returns hipSuccess with
// *quants left null otherwise.
hipError_t fuse_q8(std::initializer_list<const fortai_hip_q8_weights *> parts, Q8Matrix *m, uint4 **quants,
    uint2 **scales, hipStream_t stream) {
    *quants = nullptr;
    *scales = nullptr;
    int rows = 0;
    const fortai_hip_q8_weights *first = *parts.begin();
    for (const auto *w : parts) {
        if (w->m.rows % kRowsPerWave || w->m.chunks != first->m.chunks) return hipSuccess;
        rows += w->m.rows;
    }
    Q8Matrix f = first->m;
    f.rows = rows;
    f.row_groups = rows / kRowsPerWave;
    const size_t per_group = static_cast<size_t>(f.chunks);
    hipError_t e = alloc(quants, static_cast<size_t>(f.row_groups) * per_group * 64);
    if (e == hipSuccess) e = alloc(scales, static_cast<size_t>(f.row_groups) * per_group * 8);
    size_t at = 0;
    for (const auto *w : parts) {
        const size_t groups = static_cast<size_t>(w->m.row_groups) * per_group;
        if (e == hipSuccess)
            e = hipMemcpyAsync(*quants + at * 64, w->m.quants, groups * 64 * sizeof(uint4), hipMemcpyDeviceToDevice, stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(*scales + at * 8, w->m.scales, groups * 8 * sizeof(uint2), hipMemcpyDeviceToDevice, stream);
        at += groups;
    }
    f.quants = *quants;
    f.scales = *scales;
    *m = f;
    return e;
}

hipError_t upload_f32(float **dst, const void *src, size_t count, hipStream_t stream) {
    hipError_t e = alloc(dst, count);
    if (e == hipSuccess) e = hipMemcpyAsync(*dst, src, count * sizeof(float), hipMemcpyHostToDevice, stream);
    return e;
}

hipError_t ensure(void **buf, size_t *have, size_t need) {
    if (*have >= need) return hipSuccess;
    if (*buf) (void)hipFree(*buf);
    *buf = nullptr;
    *have = 0;
    const hipError_t e = hipMalloc(buf, need);
    if (e == hipSuccess) *have = need;
    return e;
}

hipError_t ensure_scratch(fortai_hip_q8_context *c, size_t act, size_t out, size_t q8l) {
    hipError_t e = ensure(reinterpret_cast<void **>(&c->scratch_act), &c->scratch_act_bytes, act);
    if (e == hipSuccess) e = ensure(reinterpret_cast<void **>(&c->scratch_out), &c->scratch_out_bytes, out);
    if (e == hipSuccess && q8l > c->scratch_q8l_bytes) {
        e = ensure(&c->scratch_q8l, &c->scratch_q8l_bytes, q8l);
        if (e == hipSuccess) e = hipMemsetAsync(c->scratch_q8l, 0, q8l, c->stream);  // padding blocks stay zero
    }
    return e;
}

hipError_t alloc_q8l(void **buf, int width, hipStream_t stream) {
    const size_t bytes = q8l_bytes(width);
    hipError_t e = hipMalloc(buf, bytes);
    if (e == hipSuccess) e = hipMemsetAsync(*buf, 0, bytes, stream);
    return e;
}

__global__ void set_position_kernel(int *dst, int value) { *dst = value; }
__global__ void set_token_kernel(int64_t *dst, int64_t value) { *dst = value; }

MatvecSegment segment(const fortai_hip_q8_weights *w, float *out, const float *resid = nullptr,
    const fortai_hip_q8_weights *w2 = nullptr, void *out_q8l = nullptr) {
    MatvecSegment s;
    s.w = w->m;
    if (w2) s.w2 = w2->m;
    s.out = out;
    s.resid = resid;
    s.out_q8l = out_q8l;
    return s;
}

MatvecInput q8l_input(const void *xq8l, int width) {
    MatvecInput in;
    in.xq8l = xq8l;
    in.width = width;
    return in;
}

MatvecInput f32_input(const float *x, int width) {
    MatvecInput in;
    in.x = x;
    in.width = width;
    return in;
}

MatvecInput q8_input(const int8_t *xq, int width) {
    MatvecInput in;
    in.xq = xq;
    in.width = width;
    return in;
}

bool owned(const fortai_hip_q8_context *c, const fortai_hip_q8_weights *w) { return w && w->context == c; }

GdnParams gdn_params(fortai_hip_qwen35_recurrent *L, const float *qkv, const float *alpha, const float *beta,
    float *out) {
    GdnParams p;
    p.qkv = qkv; p.alpha = alpha; p.beta = beta; p.ssm_a = L->ssm_a; p.ssm_dt = L->ssm_dt;
    p.state = L->state; p.out = out;
    p.state_size = L->state_size; p.key_heads = L->key_heads; p.value_heads = L->value_heads; p.head = L->head;
    p.eps = L->eps;
    return p;
}

// enqueue the GDN projections (the qkv rows through conv1d + SiLU in the
// epilogue) -> delta rule -> ssm_out with the gated RMSNorm as its prologue
hipError_t enqueue_recurrent(fortai_hip_qwen35_recurrent *L, const MatvecInput &in, Prologue pro, float *out,
    const float *resid, hipStream_t stream) {
    MatvecSegment segs[4] = {segment(L->qkv, L->qkv_out), segment(L->gate, L->z_out),
        segment(L->alpha, L->alpha_out), segment(L->beta, L->beta_out)};
    segs[0].conv_w = L->conv_w;
    segs[0].conv_state = L->conv_state;
    segs[0].conv_size = L->conv_size;
    segs[0].kernel = L->kernel;
    segs[1].silu = true;  // the gate is only used through SiLU
    int count = 4;
    if (L->in_quants) {
        // the fused matrix: rows [0, conv_size) qkv through the conv, the gate
        // rows through SiLU, then alpha and beta, into proj (laid out alike)
        segs[0].w = L->in_m;
        segs[0].out = L->proj;
        segs[0].conv_rows = L->conv_size;
        segs[0].silu_begin = L->conv_size;
        segs[0].silu_end = L->conv_size + L->inner;
        count = 1;
    }
    hipError_t e = !fam(kFamMatvec) ? hipSuccess : rec(launch_q8_matvec(segs, count, in, pro, Epilogue::STORE, stream),
        "GDN qkv/gate/alpha/beta projections, conv1d + SiLU");
    if (e == hipSuccess && fam(kFamGdn))
        e = rec(launch_gdn_delta(gdn_params(L, L->qkv_out, L->alpha_out, L->beta_out, L->o_raw), stream),
            "GDN L2 norms, decay/beta, delta rule");
    if (e != hipSuccess) return e;
    MatvecInput gated;
    gated.x = L->o_raw;
    gated.z = L->z_out;
    gated.norm = L->ssm_norm;
    gated.eps = L->eps;
    gated.head = L->head;
    gated.width = L->inner;
    const MatvecSegment oseg = segment(L->out, out, resid);
    if (!fam(kFamMatvec)) return hipSuccess;
    return rec(launch_q8_matvec(&oseg, 1, gated, Prologue::GATED, resid ? Epilogue::ADD : Epilogue::STORE, stream),
        "GDN gated RMSNorm, ssm_out projection + residual");
}

AttentionParams attention_params(fortai_hip_qwen35_attention *A, const float *q, const float *k, const float *v,
    float *out) {
    AttentionParams p;
    p.q = q; p.k = k; p.v = v; p.q_norm = A->q_norm; p.k_norm = A->k_norm; p.rope = A->rope;
    p.kcache = A->kcache; p.vcache = A->vcache; p.partial = A->partial; p.cache_flags = A->cache_flags; p.out = out;
    p.position = A->context->position; p.heads = A->heads; p.kv_heads = A->kv_heads; p.head = A->head;
    p.value = A->value; p.max_context = A->max_context; p.rope_dim = A->rope_dim;
    p.eps = A->eps; p.exact_max = A->exact_max; p.split = A->split; p.z_skew = A->z_skew;
    p.force_wide = A->force_wide;
    return p;
}

hipError_t enqueue_attention(fortai_hip_qwen35_attention *A, const MatvecInput &in, Prologue pro, float *out,
    const float *resid, hipStream_t stream) {
    MatvecSegment segs[3] = {segment(A->q, A->q_out), segment(A->k, A->k_out), segment(A->v, A->v_out)};
    int count = 3;
    if (A->in_quants) {
        segs[0].w = A->in_m;  // q | k | v into proj (laid out alike)
        segs[0].out = A->proj;
        count = 1;
    }
    hipError_t e = !fam(kFamMatvec) ? hipSuccess
        : rec(launch_q8_matvec(segs, count, in, pro, Epilogue::STORE, stream), "attention q/k/v projections");
    if (e != hipSuccess) return e;
    if (fam(kFamAttention))
        e = rec(launch_attention(attention_params(A, A->q_out, A->k_out, A->v_out, A->attn_out), stream),
            "q/k norm, RoPE, KV append, softmax.V, gate");
    if (e != hipSuccess) return e;
    const MatvecSegment oseg = segment(A->o, out, resid);
    MatvecInput oin;
    oin.x = A->attn_out;
    oin.width = A->heads * A->value;
    if (!fam(kFamMatvec)) return hipSuccess;
    return rec(launch_q8_matvec(&oseg, 1, oin, Prologue::F32, resid ? Epilogue::ADD : Epilogue::STORE, stream),
        "attention o projection + residual");
}

hipError_t enqueue_ffn(const fortai_hip_q8_weights *gate, const fortai_hip_q8_weights *up,
    const fortai_hip_q8_weights *down, const MatvecInput &in, Prologue pro, void *h_q8l, float *out,
    const float *resid, hipStream_t stream) {
    if (!fam(kFamMatvec)) return hipSuccess;
    const MatvecSegment pair = segment(gate, nullptr, nullptr, up, h_q8l);
    hipError_t e = rec(launch_q8_matvec(&pair, 1, in, pro, Epilogue::SILU_PAIR, stream),
        "FFN post-norm, gate/up projections, SiLU product");
    if (e != hipSuccess) return e;
    const MatvecSegment dseg = segment(down, out, resid);
    return rec(launch_q8_matvec(&dseg, 1, q8l_input(h_q8l, gate->m.rows), Prologue::Q8L,
        resid ? Epilogue::ADD : Epilogue::STORE, stream), "FFN down projection + residual");
}

bool ffn_shapes_ok(const fortai_hip_q8_weights *g, const fortai_hip_q8_weights *u, const fortai_hip_q8_weights *d) {
    return g->m.blocks == u->m.blocks && g->m.rows == u->m.rows && g->m.rows == d->m.blocks * kQ8Block &&
        g->m.rows % kQ8Block == 0;
}

}  // namespace

extern "C" {

// ------------------------------------------------------ allocation-free path
// `scratch`: the quantized activations (Q8L, batch x q8l_bytes(width)) of
// fortai_hip_q8_batch_matvec_noalloc.  Every GPU the library runs on holds one
// copy until the process ends; its device address is looked up once per
// context (with the context's device current) and kept in the context.
constexpr size_t kNoAllocScratchBytes = 8 * 18432;  // batch 8 x q8l_bytes(16384)
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

// The last user of each GPU's array: its context (stream) and the event
// recorded after its launches.  A call from another context makes its own
// stream wait for that event first, so calls from different contexts on one
// GPU run one after the other instead of overwriting each other's
// activations; calls on one stream are in order anyway.
constexpr int kNoAllocDevices = 64;
struct NoAllocUser {
    fortai_hip_q8_context *context = nullptr;
    hipEvent_t done = nullptr;
};
std::mutex g_noalloc_mutex;
NoAllocUser g_noalloc_user[kNoAllocDevices];

// ------------------------------------------------------------------ context
// fortai_cuda_backend.cu:805-833
int fortai_hip_q8_context_create(int device, fortai_hip_q8_context **context) {
    if (!context || device < 0) return FORTAI_HIP_INVALID;
    *context = nullptr;
    auto *c = new (std::nothrow) fortai_hip_q8_context;
    if (!c) return FORTAI_HIP_RUNTIME_ERROR;
    c->device = device;
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&c->start);
    if (e == hipSuccess) e = hipEventCreate(&c->stop);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&c->noalloc_done, hipEventDisableTiming);
    if (e == hipSuccess) e = alloc(&c->position, 1);
    if (e == hipSuccess) e = alloc(&c->token, 1);
    if (e == hipSuccess) e = alloc(&c->argmax_value, kArgmaxParts);
    if (e == hipSuccess) e = alloc(&c->argmax_index, kArgmaxParts);
    if (e == hipSuccess) e = hipMemsetAsync(c->position, 0, sizeof(int), c->stream);
    if (e == hipSuccess) e = hipMemsetAsync(c->token, 0, sizeof(int64_t), c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e == hipSuccess) {
        // the allocation-free entry point's array on this device (on failure
        // that entry point reports it; nothing else depends on it)
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) == hipSuccess) c->noalloc_scratch = ptr;
        else (void)hipGetLastError();
    }
    if (e != hipSuccess) {
        fortai_hip_q8_context_destroy(c);
        return FORTAI_HIP_RUNTIME_ERROR;
    }
    *context = c;
    return FORTAI_HIP_OK;
}

// fortai_cuda_backend.cu:835-850
int fortai_hip_q8_context_destroy(fortai_hip_q8_context *c) {
    if (!c) return FORTAI_HIP_OK;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    if (c->device < kNoAllocDevices) {
        std::lock_guard<std::mutex> lock(g_noalloc_mutex);
        if (g_noalloc_user[c->device].context == c) g_noalloc_user[c->device] = NoAllocUser{};
    }
    if (c->noalloc_done) (void)hipEventDestroy(c->noalloc_done);
    if (c->graph_exec) (void)hipGraphExecDestroy(c->graph_exec);
    if (c->graph) (void)hipGraphDestroy(c->graph);
    release(c->position); release(c->token); release(c->scratch_act); release(c->scratch_out);
    release(c->scratch_aux); release(c->argmax_value); release(c->argmax_index);
    if (c->scratch_q8l) (void)hipFree(c->scratch_q8l);
    if (c->start) (void)hipEventDestroy(c->start);
    if (c->stop) (void)hipEventDestroy(c->stop);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
    return FORTAI_HIP_OK;
}

// fortai_cuda_backend.cu:852-859.  Written by a one-thread kernel (the value
// travels as a kernel argument): stream ordered and capturable.
int fortai_hip_q8_context_set_position(fortai_hip_q8_context *c, int position) {
    if (!c || !c->position || position < 0) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    hipLaunchKernelGGL(set_position_kernel, dim3(1), dim3(1), 0, c->stream, c->position, position);
    return done(c, hipGetLastError(), "set device position");
}

// fortai_cuda_backend.cu:861-868
int fortai_hip_q8_context_capture_begin(fortai_hip_q8_context *c) {
    if (!c || c->graph || c->graph_exec) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    return done(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeGlobal), "begin HIP graph capture");
}

// fortai_cuda_backend.cu:870-885
int fortai_hip_q8_context_capture_end(fortai_hip_q8_context *c) {
    if (!c) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    hipError_t e = hipStreamEndCapture(c->stream, &c->graph);
    if (e == hipSuccess) e = hipGraphInstantiate(&c->graph_exec, c->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        if (c->graph_exec) (void)hipGraphExecDestroy(c->graph_exec);
        if (c->graph) (void)hipGraphDestroy(c->graph);
        c->graph_exec = nullptr;
        c->graph = nullptr;
        return fail(c, FORTAI_HIP_RUNTIME_ERROR, "end HIP graph capture", e);
    }
    return FORTAI_HIP_OK;
}

// fortai_cuda_backend.cu:887-893
int fortai_hip_q8_context_graph_launch(fortai_hip_q8_context *c) {
    if (!c || !c->graph_exec) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    return done(c, hipGraphLaunch(c->graph_exec, c->stream), "launch HIP graph");
}

int fortai_hip_q8_context_synchronize(fortai_hip_q8_context *c) {
    if (!c) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    return done(c, hipStreamSynchronize(c->stream), "stream synchronize");
}

int fortai_hip_q8_context_timer_start(fortai_hip_q8_context *c) {
    if (!c) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    return done(c, hipEventRecord(c->start, c->stream), "timer start");
}

int fortai_hip_q8_context_timer_stop(fortai_hip_q8_context *c, float *ms) {
    if (!c || !ms) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    hipError_t e = hipEventRecord(c->stop, c->stream);
    if (e == hipSuccess) e = hipEventSynchronize(c->stop);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, c->start, c->stop);
    return done(c, e, "timer stop");
}

// ------------------------------------------------------------------ weights
// fortai_cuda_backend.cu:895-931 (+ the repack to the lane-interleaved layout)
int fortai_hip_q8_weights_upload(fortai_hip_q8_context *c, const void *host_weights, size_t weight_bytes,
    int rows, int width, fortai_hip_q8_weights **weights) {
    if (!c || !host_weights || !weights || rows <= 0 || width <= 0 || width % kQ8Block) return FORTAI_HIP_INVALID;
    *weights = nullptr;
    const int blocks = width / kQ8Block;
    const size_t expected = static_cast<size_t>(rows) * blocks * kQ8Bytes;
    if (weight_bytes < expected) return FORTAI_HIP_INVALID;
    auto *w = new (std::nothrow) fortai_hip_q8_weights;
    if (!w) return FORTAI_HIP_RUNTIME_ERROR;
    w->context = c;
    w->width = width;
    w->m.rows = rows;
    w->m.blocks = blocks;
    w->m.chunks = (blocks + 3) / 4;
    w->m.row_groups = (rows + kRowsPerWave - 1) / kRowsPerWave;
    (void)hipSetDevice(c->device);
    uint8_t *staging = nullptr;
    const size_t groups = static_cast<size_t>(w->m.row_groups) * w->m.chunks;
    hipError_t e = alloc(&w->quants, groups * 64);
    if (e == hipSuccess) e = alloc(&w->scales, groups * 8);
    if (e == hipSuccess) e = alloc(&staging, expected);
    if (e == hipSuccess) e = hipMemcpyAsync(staging, host_weights, expected, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = launch_q8_repack(staging, rows, blocks, w->quants, w->scales, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    release(staging);
    if (e != hipSuccess) {
        release(w->quants);
        release(w->scales);
        delete w;
        return fail(c, FORTAI_HIP_RUNTIME_ERROR, "weight upload", e);
    }
    w->m.quants = w->quants;
    w->m.scales = w->scales;
    *weights = w;
    return FORTAI_HIP_OK;
}

// ------------------------------------------------- repacked-weight cache
// The resident planes (quants, then scales) of a rows x width Q8_0 matrix,
// as a weight-pack cache stores them (the reference keys its pack files by
// model / backend / variant / ABI version, src/fortai_cache.f90:6-31).
size_t fortai_hip_q8_pack_bytes(int rows, int width) {
    if (rows <= 0 || width <= 0 || width % kQ8Block) return 0;
    const size_t groups = static_cast<size_t>((rows + kRowsPerWave - 1) / kRowsPerWave) * ((width / kQ8Block + 3) / 4);
    return groups * (64 * sizeof(uint4) + 8 * sizeof(uint2));
}

int fortai_hip_q8_weights_pack(const fortai_hip_q8_weights *w, void *host, size_t bytes) {
    if (!w || !host || bytes < fortai_hip_q8_pack_bytes(w->m.rows, w->width)) return FORTAI_HIP_INVALID;
    auto *c = w->context;
    (void)hipSetDevice(c->device);
    const size_t groups = static_cast<size_t>(w->m.row_groups) * w->m.chunks;
    uint8_t *h = static_cast<uint8_t *>(host);
    hipError_t e = hipMemcpyAsync(h, w->quants, groups * 64 * sizeof(uint4), hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(h + groups * 64 * sizeof(uint4), w->scales, groups * 8 * sizeof(uint2), hipMemcpyDeviceToHost,
            c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    return done(c, e, "weight pack");
}

int fortai_hip_q8_weights_upload_packed(fortai_hip_q8_context *c, const void *host, size_t bytes, int rows, int width,
    fortai_hip_q8_weights **weights) {
    if (!c || !host || !weights || rows <= 0 || width <= 0 || width % kQ8Block ||
        bytes < fortai_hip_q8_pack_bytes(rows, width))
        return FORTAI_HIP_INVALID;
    *weights = nullptr;
    auto *w = new (std::nothrow) fortai_hip_q8_weights;
    if (!w) return FORTAI_HIP_RUNTIME_ERROR;
    w->context = c;
    w->width = width;
    w->m.rows = rows;
    w->m.blocks = width / kQ8Block;
    w->m.chunks = (w->m.blocks + 3) / 4;
    w->m.row_groups = (rows + kRowsPerWave - 1) / kRowsPerWave;
    (void)hipSetDevice(c->device);
    const size_t groups = static_cast<size_t>(w->m.row_groups) * w->m.chunks;
    const uint8_t *h = static_cast<const uint8_t *>(host);
    hipError_t e = alloc(&w->quants, groups * 64);
    if (e == hipSuccess) e = alloc(&w->scales, groups * 8);
    if (e == hipSuccess) e = hipMemcpyAsync(w->quants, h, groups * 64 * sizeof(uint4), hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(w->scales, h + groups * 64 * sizeof(uint4), groups * 8 * sizeof(uint2), hipMemcpyHostToDevice,
            c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        release(w->quants);
        release(w->scales);
        delete w;
        return fail(c, FORTAI_HIP_RUNTIME_ERROR, "packed weight upload", e);
    }
    w->m.quants = w->quants;
    w->m.scales = w->scales;
    *weights = w;
    return FORTAI_HIP_OK;
}

// fortai_cuda_backend.cu:925-931
int fortai_hip_q8_weights_destroy(fortai_hip_q8_weights *w) {
    if (!w) return FORTAI_HIP_OK;
    if (w->context) (void)hipSetDevice(w->context->device);
    release(w->quants);
    release(w->scales);
    delete w;
    return FORTAI_HIP_OK;
}

int fortai_hip_f16_weights_upload(fortai_hip_q8_context *c, const void *host_weights, size_t weight_bytes, int rows,
    int width, fortai_hip_f16_weights **weights) {
    if (!c || !host_weights || !weights || rows <= 0 || width <= 0 || width % 64) return FORTAI_HIP_INVALID;
    *weights = nullptr;
    const size_t expected = static_cast<size_t>(rows) * width * 2;
    if (weight_bytes < expected) return FORTAI_HIP_INVALID;
    auto *w = new (std::nothrow) fortai_hip_f16_weights;
    if (!w) return FORTAI_HIP_RUNTIME_ERROR;
    w->context = c;
    w->rows = rows;
    w->width = width;
    (void)hipSetDevice(c->device);
    hipError_t e = alloc(&w->data, static_cast<size_t>(rows) * width);
    unsigned int *count = nullptr;
    unsigned int nonfinite = 1;
    if (e == hipSuccess) e = alloc(&count, 1);
    if (e == hipSuccess) e = hipMemcpyAsync(w->data, host_weights, expected, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemsetAsync(count, 0, sizeof(unsigned), c->stream);
    if (e == hipSuccess) e = launch_count_nonfinite_halves(w->data, static_cast<size_t>(rows) * width, count, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(&nonfinite, count, sizeof(unsigned), hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    release(count);
    w->finite = nonfinite == 0;
    if (e != hipSuccess) {
        release(w->data);
        delete w;
        return fail(c, FORTAI_HIP_RUNTIME_ERROR, "f16 weight upload", e);
    }
    *weights = w;
    return FORTAI_HIP_OK;
}

int fortai_hip_f16_weights_destroy(fortai_hip_f16_weights *w) {
    if (!w) return FORTAI_HIP_OK;
    if (w->context) (void)hipSetDevice(w->context->device);
    release(w->data);
    delete w;
    return FORTAI_HIP_OK;
}

// ------------------------------------------------------------------ buffers
// fortai_cuda_backend.cu:933-990
int fortai_hip_q8_device_buffer_create(fortai_hip_q8_context *c, size_t bytes, void **buffer) {
    if (!c || !buffer || bytes == 0) return FORTAI_HIP_INVALID;
    *buffer = nullptr;
    (void)hipSetDevice(c->device);
    return done(c, hipMalloc(buffer, bytes), "device buffer allocation");
}

int fortai_hip_q8_device_buffer_destroy(fortai_hip_q8_context *c, void *buffer) {
    if (!c || !buffer) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    return done(c, hipFree(buffer), "device buffer free");
}

int fortai_hip_q8_device_buffer_upload(fortai_hip_q8_context *c, void *buffer, const void *host, size_t bytes) {
    if (!c || !buffer || !host || bytes == 0) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    hipError_t e = hipMemcpyAsync(buffer, host, bytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    return done(c, e, "device upload");
}

int fortai_hip_q8_device_buffer_upload_ptr(fortai_hip_q8_context *c, void *buffer, const void *host, size_t bytes) {
    if (!c || !buffer || !host || bytes == 0) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    return done(c, hipMemcpyAsync(buffer, host, bytes, hipMemcpyHostToDevice, c->stream), "async device upload");
}

int fortai_hip_q8_device_buffer_download(fortai_hip_q8_context *c, void *host, const void *buffer, size_t bytes) {
    if (!c || !buffer || !host || bytes == 0) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    hipError_t e = hipMemcpyAsync(host, buffer, bytes, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    return done(c, e, "device download");
}

// --------------------------------------------------------------- device ops
// fortai_cuda_backend.cu:992-1012
int fortai_hip_q8_matvec_resident(fortai_hip_q8_context *c, const fortai_hip_q8_weights *w,
    const void *device_activation, void *device_output, float *kernel_ms) {
    if (!c || !owned(c, w) || !device_activation || !device_output || !kernel_ms) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    const MatvecSegment s = segment(w, static_cast<float *>(device_output));
    hipError_t e = hipEventRecord(c->start, c->stream);
    if (e == hipSuccess)
        e = launch_q8_matvec(&s, 1, q8_input(static_cast<const int8_t *>(device_activation), w->width), Prologue::Q8,
            Epilogue::STORE, c->stream);
    if (e == hipSuccess) e = hipEventRecord(c->stop, c->stream);
    if (e == hipSuccess) e = hipEventSynchronize(c->stop);
    if (e == hipSuccess) e = hipEventElapsedTime(kernel_ms, c->start, c->stop);
    return done(c, e, "resident matvec");
}

// fortai_cuda_backend.cu:1014-1039 (quantize fused into the matvec)
int fortai_hip_q8_matvec_device_f32(fortai_hip_q8_context *c, const fortai_hip_q8_weights *w,
    const void *device_activation, size_t activation_elements, void *device_output, size_t output_elements) {
    if (!c || !owned(c, w) || !device_activation || !device_output ||
        activation_elements != static_cast<size_t>(w->width) || output_elements < static_cast<size_t>(w->m.rows))
        return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    const MatvecSegment s = segment(w, static_cast<float *>(device_output));
    const MatvecInput in = f32_input(static_cast<const float *>(device_activation), w->width);
    if (w->width <= kMatvecF32MaxWidth)
        return done(c, launch_q8_matvec(&s, 1, in, Prologue::F32, Epilogue::STORE, c->stream), "device F32 matvec");
    // wider than the in-kernel quantizer holds (e.g. the 4B FFN down, 9216):
    // quantize once into the Q8L layout (the same quantizer, so the same
    // bits), then the matvec reads it as a producer-quantized activation
    if (w->width > kQ8lPrepMaxWidth) return FORTAI_HIP_INVALID;
    hipError_t e = ensure_scratch(c, 0, 0, q8l_bytes(w->width));
    if (e == hipSuccess) e = launch_q8l_prep(in, Prologue::F32, c->scratch_q8l, 1, c->stream);
    if (e == hipSuccess)
        e = launch_q8_matvec(&s, 1, q8l_input(c->scratch_q8l, w->width), Prologue::Q8L, Epilogue::STORE, c->stream);
    return done(c, e, "device F32 matvec (wide)");
}

// fortai_cuda_backend.cu:1041-1055
int fortai_hip_qwen35_embedding_device(fortai_hip_q8_context *c, const fortai_hip_q8_weights *w, int64_t token_id,
    void *device_output, size_t output_elements) {
    if (!c || !owned(c, w) || !device_output || token_id < 0 || token_id >= w->m.rows ||
        output_elements < static_cast<size_t>(w->width))
        return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    return done(c, launch_q8_embedding(w->m, nullptr, token_id, static_cast<float *>(device_output), c->stream),
        "device Q8 embedding");
}

int fortai_hip_qwen35_embedding_f16_device(fortai_hip_q8_context *c, const fortai_hip_f16_weights *w,
    int64_t token_id, void *device_output, size_t output_elements) {
    if (!c || !w || w->context != c || !device_output || token_id < 0 || token_id >= w->rows ||
        output_elements < static_cast<size_t>(w->width))
        return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    return done(c, launch_f16_embedding(w->data, w->rows, w->width, nullptr, token_id, static_cast<float *>(device_output),
        c->stream), "device F16 embedding");
}

// fortai_cuda_backend.cu:1057-1065
int fortai_hip_qwen35_copy_device(fortai_hip_q8_context *c, const void *in, void *out, size_t bytes) {
    if (!c || !in || !out || bytes == 0) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    return done(c, hipMemcpyAsync(out, in, bytes, hipMemcpyDeviceToDevice, c->stream), "device copy");
}

// fortai_cuda_backend.cu:1067-1080
int fortai_hip_qwen35_add_device(fortai_hip_q8_context *c, const void *left, const void *right, void *out,
    size_t elements) {
    if (!c || !left || !right || !out || elements == 0 || elements > static_cast<size_t>(INT32_MAX))
        return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    return done(c, launch_add(static_cast<const float *>(left), static_cast<const float *>(right),
        static_cast<float *>(out), static_cast<int>(elements), c->stream), "device add");
}

// fortai_cuda_backend.cu:1082-1095
int fortai_hip_qwen35_rms_norm_device(fortai_hip_q8_context *c, const void *in, const void *weights, void *out,
    size_t elements, float epsilon) {
    if (!c || !in || !weights || !out || elements == 0 || elements > static_cast<size_t>(INT32_MAX) ||
        epsilon <= 0.0f)
        return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    return done(c, launch_rms_norm(static_cast<const float *>(in), static_cast<const float *>(weights),
        static_cast<float *>(out), static_cast<int>(elements), epsilon, c->stream), "device RMS norm");
}

int fortai_hip_f16_matvec_device(fortai_hip_q8_context *c, const fortai_hip_f16_weights *w,
    const void *device_activation, size_t activation_elements, void *device_output, size_t output_elements,
    void *device_token) {
    if (!c || !w || w->context != c || !device_activation || !device_output ||
        activation_elements != static_cast<size_t>(w->width) || output_elements < static_cast<size_t>(w->rows))
        return FORTAI_HIP_INVALID;
    if (device_token && f16_matvec_workgroups(w->rows) > kArgmaxParts) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    ArgmaxState st;
    st.partial_value = c->argmax_value;
    st.partial_index = c->argmax_index;
    st.token = static_cast<int64_t *>(device_token);
    return done(c, launch_f16_matvec(w->data, w->rows, w->width, w->finite, static_cast<const float *>(device_activation),
        nullptr, 0.0f, static_cast<float *>(device_output), device_token ? &st : nullptr, c->stream),
        "device F16 matvec");
}

int fortai_hip_argmax_device(fortai_hip_q8_context *c, const void *values, size_t elements, void *device_token) {
    if (!c || !values || !device_token || elements == 0 || elements > static_cast<size_t>(INT32_MAX))
        return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    ArgmaxState st;
    st.partial_value = c->argmax_value;
    st.partial_index = c->argmax_index;
    st.token = static_cast<int64_t *>(device_token);
    return done(c, launch_argmax(static_cast<const float *>(values), static_cast<int>(elements), st, c->stream),
        "device argmax");
}

int fortai_hip_q8_quantize_device(fortai_hip_q8_context *c, const void *in, size_t elements, void *blocks,
    void *scales) {
    if (!c || !in || !blocks || !scales || elements == 0 || elements % kQ8Block ||
        elements > static_cast<size_t>(INT32_MAX))
        return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    return done(c, launch_q8_quantize(static_cast<const float *>(in), static_cast<int>(elements),
        static_cast<int8_t *>(blocks), static_cast<float *>(scales), c->stream), "device quantize");
}

int fortai_hip_q8_block_dots_device(fortai_hip_q8_context *c, const fortai_hip_q8_weights *w,
    const void *device_activation, void *device_dots) {
    if (!c || !owned(c, w) || !device_activation || !device_dots) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    return done(c, launch_q8_block_dots(w->m, static_cast<const int8_t *>(device_activation),
        static_cast<int32_t *>(device_dots), c->stream), "device block dots");
}

// ------------------------------------------------------ batched matvec
int fortai_hip_q8_context_scratch_bytes(const fortai_hip_q8_context *c, size_t *bytes) {
    if (!c || !bytes) return FORTAI_HIP_INVALID;
    *bytes = c->scratch_act_bytes + c->scratch_out_bytes + c->scratch_aux_bytes + c->scratch_q8l_bytes;
    return FORTAI_HIP_OK;
}

int fortai_hip_q8_batch_matvec_noalloc(fortai_hip_q8_context *c, const fortai_hip_q8_weights *w, const void *x,
    int batch, void *out) {
    if (!c || !owned(c, w) || !x || !out || batch < 1 || batch > 8) return FORTAI_HIP_INVALID;
    const size_t q8l = static_cast<size_t>(batch) * q8l_bytes(w->width);
    if (q8l > kNoAllocScratchBytes || w->width > 16384) {
        char msg[160];
        std::snprintf(msg, sizeof(msg), "batch_matvec_noalloc: batch %d x width %d needs %zu scratch bytes (limit %zu)",
            batch, w->width, q8l, kNoAllocScratchBytes);
        return fail(c, FORTAI_HIP_INVALID, msg);
    }
    if (!c->noalloc_scratch) return fail(c, FORTAI_HIP_RUNTIME_ERROR, "batch_matvec_noalloc: scratch address unavailable");
    if (c->device >= kNoAllocDevices) return fail(c, FORTAI_HIP_INVALID, "batch_matvec_noalloc: device index");
    (void)hipSetDevice(c->device);
    std::lock_guard<std::mutex> lock(g_noalloc_mutex);
    NoAllocUser &user = g_noalloc_user[c->device];
    hipError_t e = hipSuccess;
    // another context's calls on this GPU: wait for them (no overlap on the array)
    if (user.context && user.context != c) e = hipStreamWaitEvent(c->stream, user.done, 0);
    // the prologue writes every byte the matvec reads (padding blocks as zeros)
    MatvecInput in = f32_input(static_cast<const float *>(x), w->width);
    if (e == hipSuccess) e = launch_q8l_prep(in, Prologue::F32, c->noalloc_scratch, batch, c->stream);
    const MatvecSegment seg = segment(w, static_cast<float *>(out));
    if (e == hipSuccess) e = launch_q8_batch_matvec(&seg, 1, c->noalloc_scratch, w->width, batch, Epilogue::STORE, c->stream);
    if (e == hipSuccess) e = hipEventRecord(c->noalloc_done, c->stream);
    if (e == hipSuccess) user = NoAllocUser{c, c->noalloc_done};
    return done(c, e, "batched matvec (no allocation)");
}

int fortai_hip_q8_batch_matvec_device(fortai_hip_q8_context *c, const fortai_hip_q8_weights *w, const void *x,
    int batch, void *out, float *kernel_ms) {
    if (!c || !owned(c, w) || !x || !out || batch < 1 || batch > 8) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    const size_t q8l = static_cast<size_t>(batch) * q8l_bytes(w->width);
    hipError_t e = ensure(&c->scratch_q8l, &c->scratch_q8l_bytes, q8l);
    if (e == hipSuccess && kernel_ms) e = hipEventRecord(c->start, c->stream);
    MatvecInput in = f32_input(static_cast<const float *>(x), w->width);
    if (e == hipSuccess) e = launch_q8l_prep(in, Prologue::F32, c->scratch_q8l, batch, c->stream);
    const MatvecSegment seg = segment(w, static_cast<float *>(out));
    if (e == hipSuccess) e = launch_q8_batch_matvec(&seg, 1, c->scratch_q8l, w->width, batch, Epilogue::STORE, c->stream);
    if (kernel_ms) {
        if (e == hipSuccess) e = hipEventRecord(c->stop, c->stream);
        if (e == hipSuccess) e = hipEventSynchronize(c->stop);
        if (e == hipSuccess) e = hipEventElapsedTime(kernel_ms, c->start, c->stop);
    }
    return done(c, e, "batched matvec");
}

// ------------------------------------------------------ token blocks (MFMA)
size_t fortai_hip_q8_tokens_bytes(int tokens, int width) {
    if (tokens <= 0 || width <= 0 || width % kQ8Block) return 0;
    return q8_tokens_bytes(tokens, width);
}

int fortai_hip_q8_quantize_tokens_device(fortai_hip_q8_context *c, const void *x, int tokens, int width, void *x8) {
    if (!c || !x || !x8 || tokens <= 0 || width <= 0 || width % kQ8Block) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    return done(c, launch_q8_quantize_tokens(static_cast<const float *>(x), tokens, width, width, x8, c->stream),
        "quantize tokens");
}

int fortai_hip_q8_mmq_device(fortai_hip_q8_context *c, const fortai_hip_q8_weights *w, const void *x8, int tokens,
    void *out, const void *resid, float *kernel_ms) {
    if (!c || !owned(c, w) || !x8 || !out || tokens <= 0) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    hipError_t e = hipSuccess;
    if (kernel_ms) e = hipEventRecord(c->start, c->stream);
    if (e == hipSuccess)
        e = launch_q8_mmq(w->m, x8, tokens, static_cast<float *>(out), w->m.rows, static_cast<const float *>(resid),
            nullptr, c->stream);
    if (kernel_ms) {
        if (e == hipSuccess) e = hipEventRecord(c->stop, c->stream);
        if (e == hipSuccess) e = hipEventSynchronize(c->stop);
        if (e == hipSuccess) e = hipEventElapsedTime(kernel_ms, c->start, c->stop);
    }
    return done(c, e, "token-block matmul");
}

int fortai_hip_q8_mmq_exact_device(fortai_hip_q8_context *c, const fortai_hip_q8_weights *w, const void *x8, int tokens,
    void *out, const void *resid, float *kernel_ms) {
    if (!c || !owned(c, w) || !x8 || !out || tokens <= 0) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    hipError_t e = hipSuccess;
    if (kernel_ms) e = hipEventRecord(c->start, c->stream);
    if (e == hipSuccess)
        e = launch_q8_mmq_exact(w->m, x8, tokens, static_cast<float *>(out), w->m.rows,
            static_cast<const float *>(resid), c->stream);
    if (kernel_ms) {
        if (e == hipSuccess) e = hipEventRecord(c->stop, c->stream);
        if (e == hipSuccess) e = hipEventSynchronize(c->stop);
        if (e == hipSuccess) e = hipEventElapsedTime(kernel_ms, c->start, c->stop);
    }
    return done(c, e, "token-block matmul (lane order)");
}

int fortai_hip_q8_mmq_block_dots(fortai_hip_q8_context *c, const fortai_hip_q8_weights *w, const void *x8,
    int tokens, void *dots) {
    if (!c || !owned(c, w) || !x8 || !dots || tokens <= 0) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    float *scratch = nullptr;
    hipError_t e = hipMalloc(&scratch, static_cast<size_t>(tokens) * w->m.rows * sizeof(float));
    if (e == hipSuccess)
        e = launch_q8_mmq(w->m, x8, tokens, scratch, w->m.rows, nullptr, static_cast<int32_t *>(dots), c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (scratch) (void)hipFree(scratch);
    return done(c, e, "token-block dots");
}

// ----------------------------------------------------------------- host ops
namespace {
struct host_request {
    const fortai_hip_q8_weights *w;
    float *host;
    size_t bytes;
};

// fortai_cuda_backend.cu host matvec paths (:1097-1187): upload the Q8
// activation once, evaluate each resident matrix, copy the outputs back.
int matvec_host_many(fortai_hip_q8_context *c, const host_request *req, int count, const void *host_activation,
    size_t activation_bytes, float *elapsed_ms, float *contiguous) {
    if (!c || !host_activation || !elapsed_ms) return FORTAI_HIP_INVALID;
    size_t total = 0;
    for (int i = 0; i < count; ++i) {
        const fortai_hip_q8_weights *w = req[i].w;
        if (!owned(c, w) || !req[i].host || w->width != req[0].w->width ||
            req[i].bytes < static_cast<size_t>(w->m.rows) * sizeof(float))
            return FORTAI_HIP_INVALID;
        total += static_cast<size_t>(w->m.rows) * sizeof(float);
    }
    const size_t act = static_cast<size_t>(req[0].w->m.blocks) * kQ8Bytes;
    if (activation_bytes < act) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    hipError_t e = ensure_scratch(c, act, total, 0);
    if (e == hipSuccess) e = hipEventRecord(c->start, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(c->scratch_act, host_activation, act, hipMemcpyHostToDevice, c->stream);
    MatvecSegment segs[4];
    size_t offset = 0;
    for (int i = 0; i < count; ++i) {
        segs[i] = segment(req[i].w, c->scratch_out + offset);
        offset += static_cast<size_t>(req[i].w->m.rows);
    }
    if (e == hipSuccess)
        e = launch_q8_matvec(segs, count, q8_input(c->scratch_act, req[0].w->width), Prologue::Q8, Epilogue::STORE,
            c->stream);
    if (contiguous) {
        if (e == hipSuccess) e = hipMemcpyAsync(contiguous, c->scratch_out, total, hipMemcpyDeviceToHost, c->stream);
    } else {
        offset = 0;
        for (int i = 0; i < count && e == hipSuccess; ++i) {
            const size_t bytes = static_cast<size_t>(req[i].w->m.rows) * sizeof(float);
            e = hipMemcpyAsync(req[i].host, c->scratch_out + offset, bytes, hipMemcpyDeviceToHost, c->stream);
            offset += static_cast<size_t>(req[i].w->m.rows);
        }
    }
    if (e == hipSuccess) e = hipEventRecord(c->stop, c->stream);
    if (e == hipSuccess) e = hipEventSynchronize(c->stop);
    if (e == hipSuccess) e = hipEventElapsedTime(elapsed_ms, c->start, c->stop);
    return done(c, e, "host matvec");
}
}  // namespace

int fortai_hip_q8_matvec_host(fortai_hip_q8_context *c, const fortai_hip_q8_weights *w, const void *act,
    size_t act_bytes, float *out, size_t out_bytes, float *ms) {
    if (!w || !out) return FORTAI_HIP_INVALID;
    const host_request r[] = {{w, out, out_bytes}};
    return matvec_host_many(c, r, 1, act, act_bytes, ms, nullptr);
}

int fortai_hip_q8_matvec_host_pair(fortai_hip_q8_context *c, const fortai_hip_q8_weights *w1,
    const fortai_hip_q8_weights *w2, const void *act, size_t act_bytes, float *o1, size_t b1, float *o2, size_t b2,
    float *ms) {
    if (!w1 || !w2) return FORTAI_HIP_INVALID;
    const host_request r[] = {{w1, o1, b1}, {w2, o2, b2}};
    return matvec_host_many(c, r, 2, act, act_bytes, ms, nullptr);
}

int fortai_hip_q8_matvec_host_triplet(fortai_hip_q8_context *c, const fortai_hip_q8_weights *w1,
    const fortai_hip_q8_weights *w2, const fortai_hip_q8_weights *w3, const void *act, size_t act_bytes, float *o1,
    size_t b1, float *o2, size_t b2, float *o3, size_t b3, float *ms) {
    if (!w1 || !w2 || !w3) return FORTAI_HIP_INVALID;
    const host_request r[] = {{w1, o1, b1}, {w2, o2, b2}, {w3, o3, b3}};
    return matvec_host_many(c, r, 3, act, act_bytes, ms, nullptr);
}

int fortai_hip_q8_matvec_host_triplet_contiguous(fortai_hip_q8_context *c, const fortai_hip_q8_weights *w1,
    const fortai_hip_q8_weights *w2, const fortai_hip_q8_weights *w3, const void *act, size_t act_bytes, float *out,
    size_t out_bytes, float *ms) {
    if (!w1 || !w2 || !w3 || !out) return FORTAI_HIP_INVALID;
    const size_t n1 = static_cast<size_t>(w1->m.rows), n2 = static_cast<size_t>(w2->m.rows),
                 n3 = static_cast<size_t>(w3->m.rows);
    if (out_bytes < (n1 + n2 + n3) * sizeof(float)) return FORTAI_HIP_INVALID;
    const host_request r[] = {{w1, out, n1 * 4}, {w2, out + n1, n2 * 4}, {w3, out + n1 + n2, n3 * 4}};
    return matvec_host_many(c, r, 3, act, act_bytes, ms, out);
}

// fortai_cuda_backend.cu:1189-1245
int fortai_hip_q8_ffn_host(fortai_hip_q8_context *c, const fortai_hip_q8_weights *gate,
    const fortai_hip_q8_weights *up, const fortai_hip_q8_weights *down, const void *act, size_t act_bytes, float *out,
    size_t out_bytes, float *ms) {
    if (!c || !owned(c, gate) || !owned(c, up) || !owned(c, down) || !act || !out || !ms) return FORTAI_HIP_INVALID;
    if (!ffn_shapes_ok(gate, up, down)) return FORTAI_HIP_INVALID;
    const size_t in_bytes = static_cast<size_t>(gate->m.blocks) * kQ8Bytes;
    const size_t o_bytes = static_cast<size_t>(down->m.rows) * sizeof(float);
    if (act_bytes < in_bytes || out_bytes < o_bytes) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    hipError_t e = ensure_scratch(c, in_bytes, o_bytes, q8l_bytes(gate->m.rows));
    if (e == hipSuccess) e = hipEventRecord(c->start, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(c->scratch_act, act, in_bytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess)
        e = enqueue_ffn(gate, up, down, q8_input(c->scratch_act, gate->width), Prologue::Q8, c->scratch_q8l,
            c->scratch_out, nullptr, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(out, c->scratch_out, o_bytes, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipEventRecord(c->stop, c->stream);
    if (e == hipSuccess) e = hipEventSynchronize(c->stop);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, c->start, c->stop);
    return done(c, e, "Qwen FFN host");
}

// fortai_cuda_backend.cu:1247-1296
int fortai_hip_q8_ffn_device(fortai_hip_q8_context *c, const fortai_hip_q8_weights *gate,
    const fortai_hip_q8_weights *up, const fortai_hip_q8_weights *down, const void *act, size_t act_elements,
    void *out, size_t out_elements) {
    if (!c || !owned(c, gate) || !owned(c, up) || !owned(c, down) || !act || !out) return FORTAI_HIP_INVALID;
    if (!ffn_shapes_ok(gate, up, down) || act_elements != static_cast<size_t>(gate->width) ||
        out_elements < static_cast<size_t>(down->m.rows))
        return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    hipError_t e = ensure_scratch(c, 0, 0, q8l_bytes(gate->m.rows));
    if (e == hipSuccess)
        e = enqueue_ffn(gate, up, down, f32_input(static_cast<const float *>(act), gate->width), Prologue::F32,
            c->scratch_q8l, static_cast<float *>(out), nullptr, c->stream);
    return done(c, e, "Qwen FFN device");
}

// --------------------------------------------------------- recurrent layer
// fortai_cuda_backend.cu:1298-1346
int fortai_hip_qwen35_recurrent_create(fortai_hip_q8_context *c, const fortai_hip_q8_weights *qkv,
    const fortai_hip_q8_weights *gate, const fortai_hip_q8_weights *alpha, const fortai_hip_q8_weights *beta,
    const fortai_hip_q8_weights *outw, const void *conv_weights, size_t conv_weight_bytes, int conv_size,
    int conv_kernel, const void *ssm_a, size_t ssm_a_bytes, const void *ssm_dt, size_t ssm_dt_bytes,
    const void *ssm_norm, size_t ssm_norm_bytes, int state_size, int key_heads, int value_heads, int head_size,
    int inner_size, float norm_epsilon, fortai_hip_qwen35_recurrent **layer) {
    if (!c || !layer || !qkv || !gate || !alpha || !beta || !outw || !conv_weights || !ssm_a || !ssm_dt ||
        !ssm_norm || conv_size <= 0 || conv_kernel < 2 || state_size <= 0 || key_heads <= 0 || value_heads <= 0 ||
        head_size <= 0 || inner_size <= 0 || value_heads % key_heads != 0 || value_heads * head_size != inner_size)
        return FORTAI_HIP_INVALID;
    *layer = nullptr;
    if (!owned(c, qkv) || !owned(c, gate) || !owned(c, alpha) || !owned(c, beta) || !owned(c, outw))
        return FORTAI_HIP_INVALID;
    // this backend's step kernel covers the Qwen3.5 geometry: q/k slices of
    // head_size, power-of-two heads of 64..256
    if (state_size != head_size || (head_size != 64 && head_size != 128 && head_size != 256) ||
        conv_size != 2 * state_size * key_heads + inner_size || qkv->m.rows != conv_size ||
        gate->m.rows != inner_size || alpha->m.rows != value_heads || beta->m.rows != value_heads ||
        outw->width != inner_size || gate->width != qkv->width || alpha->width != qkv->width ||
        beta->width != qkv->width)
        return FORTAI_HIP_INVALID;
    if (conv_weight_bytes < static_cast<size_t>(conv_size) * conv_kernel * sizeof(float) ||
        ssm_a_bytes < static_cast<size_t>(value_heads) * sizeof(float) ||
        ssm_dt_bytes < static_cast<size_t>(value_heads) * sizeof(float) ||
        ssm_norm_bytes < static_cast<size_t>(head_size) * sizeof(float))
        return FORTAI_HIP_INVALID;
    auto *L = new (std::nothrow) fortai_hip_qwen35_recurrent;
    if (!L) return FORTAI_HIP_RUNTIME_ERROR;
    L->context = c; L->qkv = qkv; L->gate = gate; L->alpha = alpha; L->beta = beta; L->out = outw;
    L->conv_size = conv_size; L->kernel = conv_kernel; L->state_size = state_size; L->key_heads = key_heads;
    L->value_heads = value_heads; L->head = head_size; L->inner = inner_size; L->eps = norm_epsilon;
    (void)hipSetDevice(c->device);
    const size_t state_n = static_cast<size_t>(value_heads) * head_size * head_size;
    hipError_t e = upload_f32(&L->conv_w, conv_weights, static_cast<size_t>(conv_size) * conv_kernel, c->stream);
    if (e == hipSuccess) e = upload_f32(&L->ssm_a, ssm_a, value_heads, c->stream);
    if (e == hipSuccess) e = upload_f32(&L->ssm_dt, ssm_dt, value_heads, c->stream);
    if (e == hipSuccess) e = upload_f32(&L->ssm_norm, ssm_norm, head_size, c->stream);
    if (e == hipSuccess) e = alloc(&L->conv_state, static_cast<size_t>(conv_kernel - 1) * conv_size);
    if (e == hipSuccess) e = alloc(&L->state, state_n);
    if (e == hipSuccess) e = alloc(&L->proj, static_cast<size_t>(conv_size) + inner_size + 2 * value_heads);
    if (e == hipSuccess) {
        L->qkv_out = L->proj;
        L->z_out = L->qkv_out + conv_size;
        L->alpha_out = L->z_out + inner_size;
        L->beta_out = L->alpha_out + value_heads;
    }
    if (e == hipSuccess) e = fuse_q8({qkv, gate, alpha, beta}, &L->in_m, &L->in_quants, &L->in_scales, c->stream);
    if (e == hipSuccess) e = alloc(&L->o_raw, inner_size);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        fortai_hip_qwen35_recurrent_destroy(L);
        return fail(c, FORTAI_HIP_RUNTIME_ERROR, "Qwen recurrent create", e);
    }
    const int rc = fortai_hip_qwen35_recurrent_reset(L);
    if (rc != FORTAI_HIP_OK) {
        fortai_hip_qwen35_recurrent_destroy(L);
        return rc;
    }
    *layer = L;
    return FORTAI_HIP_OK;
}

int fortai_hip_qwen35_recurrent_destroy(fortai_hip_qwen35_recurrent *L) {
    if (!L) return FORTAI_HIP_OK;
    if (L->context) {
        (void)hipSetDevice(L->context->device);
        (void)hipStreamSynchronize(L->context->stream);
    }
    release(L->conv_w); release(L->ssm_a); release(L->ssm_dt); release(L->ssm_norm); release(L->conv_state);
    release(L->state); release(L->proj); release(L->in_quants); release(L->in_scales); release(L->conv_snap);
    release(L->o_raw);
    delete L;
    return FORTAI_HIP_OK;
}

// fortai_cuda_backend.cu:1395-1408
int fortai_hip_qwen35_recurrent_reset(fortai_hip_qwen35_recurrent *L) {
    if (!L || !L->context) return FORTAI_HIP_INVALID;
    auto *c = L->context;
    (void)hipSetDevice(c->device);
    hipError_t e = hipMemsetAsync(L->conv_state, 0,
        static_cast<size_t>(L->kernel - 1) * L->conv_size * sizeof(float), c->stream);
    if (e == hipSuccess)
        e = hipMemsetAsync(L->state, 0, static_cast<size_t>(L->value_heads) * L->head * L->head * sizeof(float),
            c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    return done(c, e, "Qwen recurrent reset");
}

// fortai_cuda_backend.cu:1410-1489
int fortai_hip_qwen35_recurrent_run(fortai_hip_qwen35_recurrent *L, const void *act, size_t act_bytes,
    float *out, size_t out_bytes, float *ms) {
    if (!L || !L->context || !act || !out || !ms) return FORTAI_HIP_INVALID;
    auto *c = L->context;
    const size_t in_bytes = static_cast<size_t>(L->qkv->m.blocks) * kQ8Bytes;
    const size_t o_bytes = static_cast<size_t>(L->out->m.rows) * sizeof(float);
    if (act_bytes < in_bytes || out_bytes < o_bytes) return FORTAI_HIP_INVALID;
    (void)hipSetDevice(c->device);
    hipError_t e = ensure_scratch(c, in_bytes, o_bytes, 0);
    if (e == hipSuccess) e = hipEventRecord(c->start, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(c->scratch_act, act, in_bytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess)
        e = enqueue_recurrent(L, q8_input(c->scratch_act, L->qkv->width), Prologue::Q8, c->scratch_out, nullptr,
            c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(out, c->scratch_out, o_bytes, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipEventRecord(c->stop, c->stream);
    if (e == hipSuccess) e = hipEventSynchronize(c->stop);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, c->start, c->stop);
    return done(c, e, "Qwen recurrent run");
}

// fortai_cuda_backend.cu:1491-1562
int fortai_hip_qwen35_recurrent_run_device(fortai_hip_qwen35_recurrent *L, const void *act, size_t act_elements,
    void *out, size_t out_elements) {
    if (!L || !L->context || !act || !out) return FORTAI_HIP_INVALID;
    if (act_elements != static_cast<size_t>(L->qkv->width) || out_elements < static_cast<size_t>(L->out->m.rows))
        return FORTAI_HIP_INVALID;
    auto *c = L->context;
    (void)hipSetDevice(c->device);
    return done(c, enqueue_recurrent(L, f32_input(static_cast<const float *>(act), L->qkv->width), Prologue::F32,
        static_cast<float *>(out), nullptr, c->stream), "Qwen recurrent device run");
}

int fortai_hip_qwen35_recurrent_core_device(fortai_hip_qwen35_recurrent *L, const void *qkv, const void *alpha,
    const void *beta, void *out) {
    if (!L || !L->context || !qkv || !alpha || !beta || !out) return FORTAI_HIP_INVALID;
    auto *c = L->context;
    (void)hipSetDevice(c->device);
    // conv1d + SiLU into the layer's qkv buffer (the caller's qkv is only read), then the delta rule
    hipError_t e = launch_conv_silu(static_cast<const float *>(qkv), L->conv_w, L->conv_state, L->qkv_out, L->conv_size,
        L->kernel, c->stream);
    if (e == hipSuccess)
        e = launch_gdn_delta(gdn_params(L, L->qkv_out, static_cast<const float *>(alpha),
            static_cast<const float *>(beta), static_cast<float *>(out)), c->stream);
    return done(c, e, "Qwen recurrent core");
}

int fortai_hip_qwen35_recurrent_core_steps_device(fortai_hip_qwen35_recurrent *L, const void *qkv, const void *alpha,
    const void *beta, int steps, void *out) {
    if (!L || !L->context || !qkv || !alpha || !beta || !out || steps < 1) return FORTAI_HIP_INVALID;
    auto *c = L->context;
    (void)hipSetDevice(c->device);
    const size_t window = static_cast<size_t>(L->kernel - 1) * L->conv_size;
    hipError_t e = L->conv_snap ? hipSuccess : alloc(&L->conv_snap, window);
    if (e == hipSuccess)
        e = hipMemcpyAsync(L->conv_snap, L->conv_state, window * sizeof(float), hipMemcpyDeviceToDevice, c->stream);
    GdnParams p = gdn_params(L, static_cast<const float *>(qkv), static_cast<const float *>(alpha),
        static_cast<const float *>(beta), static_cast<float *>(out));
    if (e == hipSuccess)
        e = launch_gdn_recurrence(p, L->conv_w, L->conv_snap, L->conv_state, L->conv_size, L->kernel, steps, c->stream);
    if (e == hipErrorInvalidValue) return fail(c, FORTAI_HIP_INVALID, "recurrent core steps: head 128 layers only");
    return done(c, e, "Qwen recurrent core steps");
}

int fortai_hip_qwen35_recurrent_state_download(fortai_hip_qwen35_recurrent *L, float *gdn, size_t gdn_bytes,
    float *conv, size_t conv_bytes) {
    if (!L || !L->context) return FORTAI_HIP_INVALID;
    const int H = L->head, cols = H / 8;
    const size_t sn = static_cast<size_t>(L->value_heads) * H * H;
    const size_t cn = static_cast<size_t>(L->kernel - 1) * L->conv_size;
    if ((gdn && gdn_bytes < sn * 4) || (conv && conv_bytes < cn * 4)) return FORTAI_HIP_INVALID;
    auto *c = L->context;
    (void)hipSetDevice(c->device);
    std::vector<float> st(sn);
    hipError_t e = hipMemcpyAsync(st.data(), L->state, sn * 4, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess && conv) e = hipMemcpyAsync(conv, L->conv_state, cn * 4, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return fail(c, FORTAI_HIP_RUNTIME_ERROR, "recurrent state download", e);
    if (gdn)
        for (size_t hr = 0; hr < static_cast<size_t>(L->value_heads) * H; ++hr)
            for (int l = 0; l < 8; ++l)
                for (int i = 0; i < cols; ++i) gdn[hr * H + 8 * i + l] = st[(hr * 8 + l) * cols + i];
    return FORTAI_HIP_OK;
}

int fortai_hip_qwen35_recurrent_state_upload(fortai_hip_qwen35_recurrent *L, const float *gdn, size_t gdn_bytes,
    const float *conv, size_t conv_bytes) {
    if (!L || !L->context || !gdn || !conv) return FORTAI_HIP_INVALID;
    const int H = L->head, cols = H / 8;
    const size_t sn = static_cast<size_t>(L->value_heads) * H * H;
    const size_t cn = static_cast<size_t>(L->kernel - 1) * L->conv_size;
    if (gdn_bytes < sn * 4 || conv_bytes < cn * 4) return FORTAI_HIP_INVALID;
    std::vector<float> st(sn);
    for (size_t hr = 0; hr < static_cast<size_t>(L->value_heads) * H; ++hr)
        for (int l = 0; l < 8; ++l)
            for (int i = 0; i < cols; ++i) st[(hr * 8 + l) * cols + i] = gdn[hr * H + 8 * i + l];
    auto *c = L->context;
    (void)hipSetDevice(c->device);
    hipError_t e = hipMemcpyAsync(L->state, st.data(), sn * 4, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(L->conv_state, conv, cn * 4, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    return done(c, e, "recurrent state upload");
}

// --------------------------------------------------------- attention layer
// fortai_cuda_backend.cu:1564-1621 (+ the RoPE table, computed on the host
// with the reference's expression, fortai_qwen35_cpu.f90:1487-1490)
int fortai_hip_qwen35_attention_create(fortai_hip_q8_context *c, const fortai_hip_q8_weights *q,
    const fortai_hip_q8_weights *k, const fortai_hip_q8_weights *v, const fortai_hip_q8_weights *o,
    const void *query_norm, size_t query_norm_bytes, const void *key_norm, size_t key_norm_bytes, int heads,
    int kv_heads, int head_size, int value_size, int max_context, int rope_dimension, float rope_base,
    float norm_epsilon, fortai_hip_qwen35_attention **layer) {
    if (!c || !layer || !q || !k || !v || !o || !query_norm || !key_norm || heads <= 0 || kv_heads <= 0 ||
        head_size <= 0 || value_size <= 0 || max_context <= 0 || heads % kv_heads != 0 || rope_dimension < 0 ||
        (rope_dimension > 0 && (rope_dimension > head_size || rope_dimension % 2 != 0)) || rope_base <= 0.0f ||
        norm_epsilon <= 0.0f)
        return FORTAI_HIP_INVALID;
    if (!owned(c, q) || !owned(c, k) || !owned(c, v) || !owned(c, o) || q->m.rows != heads * 2 * head_size ||
        k->m.rows != kv_heads * head_size || v->m.rows != kv_heads * value_size ||
        o->width != heads * value_size || query_norm_bytes < static_cast<size_t>(head_size) * sizeof(float) ||
        key_norm_bytes < static_cast<size_t>(head_size) * sizeof(float) || q->width != k->width ||
        q->width != v->width)
        return FORTAI_HIP_INVALID;
    // this backend's attention kernels: GQA groups of <= 4, head <= 256, value <= head (multiple of 8);
    // the scores live in global memory, so the context only bounds the buffers' sizes
    if (heads / kv_heads > 4 || head_size > 256 || value_size > head_size || head_size % 8 || value_size % 8 ||
        max_context > (1 << 20))
        return FORTAI_HIP_INVALID;
    *layer = nullptr;
    auto *A = new (std::nothrow) fortai_hip_qwen35_attention;
    if (!A) return FORTAI_HIP_RUNTIME_ERROR;
    A->context = c; A->q = q; A->k = k; A->v = v; A->o = o; A->heads = heads; A->kv_heads = kv_heads;
    A->head = head_size; A->value = value_size; A->max_context = max_context; A->rope_dim = rope_dimension;
    A->rope_base = rope_base; A->eps = norm_epsilon;
    const int half = rope_dimension / 2;
    std::vector<float2> table(static_cast<size_t>(max_context) * (half > 0 ? half : 1));
    for (int p = 0; p < max_context; ++p)
        for (int i = 0; i < half; ++i) {
            const float angle = static_cast<float>(p) /
                powf(rope_base, static_cast<float>(2 * i) / static_cast<float>(rope_dimension));
            table[static_cast<size_t>(p) * half + i] = make_float2(cosf(angle), sinf(angle));
        }
    (void)hipSetDevice(c->device);
    const size_t kv_n = static_cast<size_t>(max_context) * kv_heads;
    hipError_t e = upload_f32(&A->q_norm, query_norm, head_size, c->stream);
    if (e == hipSuccess) e = upload_f32(&A->k_norm, key_norm, head_size, c->stream);
    if (e == hipSuccess) e = alloc(&A->rope, table.size());
    if (e == hipSuccess)
        e = hipMemcpyAsync(A->rope, table.data(), table.size() * sizeof(float2), hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = alloc(&A->kcache, kv_n * head_size);
    if (e == hipSuccess) e = alloc(&A->vcache, kv_n * value_size);
    if (e == hipSuccess)
        e = alloc(&A->proj, static_cast<size_t>(heads) * 2 * head_size + static_cast<size_t>(kv_heads) * (head_size + value_size));
    if (e == hipSuccess) {
        A->q_out = A->proj;
        A->k_out = A->q_out + static_cast<size_t>(heads) * 2 * head_size;
        A->v_out = A->k_out + static_cast<size_t>(kv_heads) * head_size;
    }
    if (e == hipSuccess) e = fuse_q8({q, k, v}, &A->in_m, &A->in_quants, &A->in_scales, c->stream);
    if (e == hipSuccess) e = alloc(&A->attn_out, static_cast<size_t>(heads) * value_size);
    if (e == hipSuccess) e = alloc(&A->partial, attention_scores_floats(heads, max_context));
    // the positions up to which the attention output keeps the reference's
    // summation orders (default 8192); beyond them the split-K path (within
    // 1e-3 relative) takes over.  fortai_hip_qwen35_attention_set_exact_max
    // changes it.
    A->exact_max = kDefaultExactMax;
    if (e == hipSuccess && max_context > A->exact_max)
        e = alloc(&A->split, static_cast<size_t>(heads) * attention_split_chunks(max_context) * (value_size + 2));
    if (e == hipSuccess) e = alloc(&A->cache_flags, kv_heads);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        fortai_hip_qwen35_attention_destroy(A);
        return fail(c, FORTAI_HIP_RUNTIME_ERROR, "Qwen attention create", e);
    }
    const int rc = fortai_hip_qwen35_attention_reset(A);
    if (rc != FORTAI_HIP_OK) {
        fortai_hip_qwen35_attention_destroy(A);
        return rc;
    }
    *layer = A;
    return FORTAI_HIP_OK;
}

int fortai_hip_qwen35_attention_destroy(fortai_hip_qwen35_attention *A) {
    if (!A) return FORTAI_HIP_OK;
    if (A->context) {
        (void)hipSetDevice(A->context->device);
        (void)hipStreamSynchronize(A->context->stream);
    }
    release(A->q_norm); release(A->k_norm); release(A->rope); release(A->kcache); release(A->vcache);
    release(A->proj); release(A->in_quants); release(A->in_scales); release(A->partial); release(A->cache_flags);
    release(A->attn_out); release(A->split);
    delete A;
    return FORTAI_HIP_OK;
}

// fortai_cuda_backend.cu:1650-1663
int fortai_hip_qwen35_attention_reset(fortai_hip_qwen35_attention *A) {
    if (!A || !A->context) return FORTAI_HIP_INVALID;
    auto *c = A->context;
    (void)hipSetDevice(c->device);
    const size_t kv_n = static_cast<size_t>(A->max_context) * A->kv_heads;
    hipError_t e = hipMemsetAsync(A->kcache, 0, kv_n * A->head * 2, c->stream);
    if (e == hipSuccess) e = hipMemsetAsync(A->vcache, 0, kv_n * A->value * 2, c->stream);
    if (e == hipSuccess) e = hipMemsetAsync(A->cache_flags, 0, static_cast<size_t>(A->kv_heads) * sizeof(int), c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    return done(c, e, "Qwen attention reset");
}

// fortai_cuda_backend.cu:1665-1731.  As in the reference, the kernels read the
// context's device position; `position` is validated against max_context.
int fortai_hip_qwen35_attention_run_device(fortai_hip_qwen35_attention *A, const void *act, size_t act_elements,
    int position, void *out, size_t out_elements) {
    if (!A || !A->context || !act || !out || position < 0 || position >= A->max_context) return FORTAI_HIP_INVALID;
    if (act_elements != static_cast<size_t>(A->q->width) || out_elements < static_cast<size_t>(A->o->m.rows))
        return FORTAI_HIP_INVALID;
    auto *c = A->context;
    (void)hipSetDevice(c->device);
    return done(c, enqueue_attention(A, f32_input(static_cast<const float *>(act), A->q->width), Prologue::F32,
        static_cast<float *>(out), nullptr, c->stream), "Qwen attention device run");
}

int fortai_hip_qwen35_attention_core_device(fortai_hip_qwen35_attention *A, const void *q, const void *k,
    const void *v, void *out) {
    if (!A || !A->context || !q || !k || !v || !out) return FORTAI_HIP_INVALID;
    auto *c = A->context;
    (void)hipSetDevice(c->device);
    return done(c, launch_attention(attention_params(A, static_cast<const float *>(q), static_cast<const float *>(k),
        static_cast<const float *>(v), static_cast<float *>(out)), c->stream), "Qwen attention core");
}

int fortai_hip_qwen35_attention_prefill_core_device(fortai_hip_qwen35_attention *A, void *q, const void *k,
    const void *v, int T, int matrix_cores, void *out) {
    if (!A || !A->context || !q || !k || !v || !out || T < 1 || T > A->max_context) return FORTAI_HIP_INVALID;
    auto *c = A->context;
    (void)hipSetDevice(c->device);
    AttentionParams ap = attention_params(A, static_cast<const float *>(q), static_cast<const float *>(k),
        static_cast<const float *>(v), static_cast<float *>(out));
    const hipError_t e = launch_attention_prefill(ap, 1, T, static_cast<float *>(out), c->stream, matrix_cores != 0);
    if (e == hipErrorInvalidValue) return fail(c, FORTAI_HIP_INVALID, "prefill attention: unsupported layer shape", e);
    return done(c, e, "Qwen prefill attention core");
}

int fortai_hip_qwen35_attention_cache_download(fortai_hip_qwen35_attention *A, uint16_t *keys, uint16_t *values,
    int positions) {
    if (!A || !A->context || positions <= 0 || positions > A->max_context) return FORTAI_HIP_INVALID;
    auto *c = A->context;
    (void)hipSetDevice(c->device);
    const size_t n = static_cast<size_t>(positions) * A->kv_heads;
    hipError_t e = hipSuccess;
    if (keys) e = hipMemcpyAsync(keys, A->kcache, n * A->head * 2, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess && values) e = hipMemcpyAsync(values, A->vcache, n * A->value * 2, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    return done(c, e, "attention cache download");
}

int fortai_hip_qwen35_attention_cache_upload(fortai_hip_qwen35_attention *A, const uint16_t *keys,
    const uint16_t *values, int positions) {
    if (!A || !A->context || !keys || !values || positions <= 0 || positions > A->max_context)
        return FORTAI_HIP_INVALID;
    auto *c = A->context;
    (void)hipSetDevice(c->device);
    const size_t n = static_cast<size_t>(positions) * A->kv_heads;
    // exponent-31 halves force the exact gguf_fp16_to_real decode path
    std::vector<int> flags(static_cast<size_t>(A->kv_heads), 0);
    for (size_t i = 0; i < n * A->head; ++i)
        if ((keys[i] & 0x7c00u) == 0x7c00u) flags[(i / A->head) % A->kv_heads] = 1;
    for (size_t i = 0; i < n * A->value; ++i)
        if ((values[i] & 0x7c00u) == 0x7c00u) flags[(i / A->value) % A->kv_heads] = 1;
    hipError_t e = hipMemcpyAsync(A->kcache, keys, n * A->head * 2, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(A->vcache, values, n * A->value * 2, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(A->cache_flags, flags.data(), flags.size() * sizeof(int), hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    return done(c, e, "attention cache upload");
}

// fortai_cuda_backend.cu:1733-1736
const char *fortai_hip_q8_last_error(const fortai_hip_q8_context *c) {
    return c ? c->error : "invalid HIP context";
}

// ------------------------------------------------------------------ decoder
namespace {
hipError_t enqueue_lm_head(fortai_hip_qwen35_decoder *d, hipStream_t stream);
// the greedy argmax state of the decoder: partials of the LM head (or of the
// argmax over the Q8_0 head's logits), token, trace, position, next token
ArgmaxState decoder_argmax(fortai_hip_qwen35_decoder *d, int *partials) {
    auto *c = d->context;
    ArgmaxState st;
    st.partial_value = d->argmax_value;
    st.partial_index = d->argmax_index;
    st.token = c->token;
    st.trace = d->trace;
    st.trace_capacity = d->max_context;
    st.position = c->position;
    st.embed = d->embed;
    if (partials) *partials = d->out16 ? f16_matvec_workgroups(d->vocab) : std::min((d->vocab + 255) / 256, 1024);
    return st;
}
hipError_t enqueue_decoder_step(fortai_hip_qwen35_decoder *d, hipStream_t stream) {
    g_families = d->families;
    hipError_t e = hipSuccess;
    if (fam(kFamHead)) {
        // the embedding finishes the previous step's argmax (token, trace, position)
        int parts = 0;
        const ArgmaxState st = decoder_argmax(d, &parts);
        e = rec(launch_step_embedding(d->emb16 ? d->emb16->data : nullptr, d->emb8 ? &d->emb8->m : nullptr,
                    d->emb16 ? d->emb16->rows : d->emb8->m.rows, d->hidden, st, parts, d->x, stream),
            "token embedding");
    }
    for (size_t i = 0; i < d->layers.size() && e == hipSuccess; ++i) {
        const decoder_layer &L = d->layers[i];
        MatvecInput in;
        in.x = d->x;
        in.norm = L.attn_norm;
        in.eps = d->eps;
        in.width = d->hidden;
        if (L.recurrent) e = enqueue_recurrent(L.recurrent, in, Prologue::RMSNORM, d->x, d->x, stream);
        else e = enqueue_attention(L.attention, in, Prologue::RMSNORM, d->x, d->x, stream);
        if (e != hipSuccess) break;
        in.norm = L.post_norm;
        e = enqueue_ffn(L.gate, L.up, L.down, in, Prologue::RMSNORM, d->h_q8l, d->x, d->x, stream);
    }
    const bool head = fam(kFamHead);
    g_families = kFamAll;
    if (e != hipSuccess || !head) return e;
    return enqueue_lm_head(d, stream);
}
// final RMSNorm + LM head + greedy argmax partials from d->x; the next step's
// embedding (or finish_decoder_steps) turns them into token, trace and position
hipError_t enqueue_lm_head(fortai_hip_qwen35_decoder *d, hipStream_t stream) {
    hipError_t e = hipSuccess;
    const ArgmaxState st = decoder_argmax(d, nullptr);
    if (d->out16)
        return rec(launch_f16_matvec(d->out16->data, d->vocab, d->hidden, d->out16->finite, d->x, d->output_norm, d->eps,
            d->logits, &st, stream), "output RMSNorm, LM head, greedy argmax");
    MatvecInput in;
    in.x = d->x;
    in.norm = d->output_norm;
    in.eps = d->eps;
    in.width = d->hidden;
    const MatvecSegment s = segment(d->out8, d->logits);
    e = rec(launch_q8_matvec(&s, 1, in, Prologue::RMSNORM, Epilogue::STORE, stream), "output RMSNorm, LM head");
    if (e == hipSuccess) e = rec(launch_argmax(d->logits, d->vocab, st, stream), "greedy argmax");
    return e;
}
// The decode step as one captured graph (unless the decoder is in direct
// mode); the plan is recorded at capture (direct mode: by the first step).
hipError_t capture_decoder(fortai_hip_qwen35_decoder *d) {
    auto *c = d->context;
    if (d->exec) (void)hipGraphExecDestroy(d->exec);
    if (d->graph) (void)hipGraphDestroy(d->graph);
    d->exec = nullptr;
    d->graph = nullptr;
    d->plan.clear();
    if (!d->use_graph) return hipSuccess;
    hipError_t e = hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return e;
    g_plan = &d->plan;
    g_plan_batch = 1;
    const hipError_t ce = enqueue_decoder_step(d, c->stream);
    g_plan = nullptr;
    e = hipStreamEndCapture(c->stream, &d->graph);
    if (ce != hipSuccess) e = ce;
    if (e == hipSuccess) e = hipGraphInstantiate(&d->exec, d->graph, nullptr, nullptr, 0);
    return e;
}
hipError_t run_step(fortai_hip_qwen35_decoder *d) {
    // the plan is recorded by the first step (at capture for the graph)
    std::vector<plan_step> *saved = g_plan;
    if (d->plan.empty() && !d->use_graph) g_plan = &d->plan;
    const hipError_t e = d->use_graph ? hipGraphLaunch(d->exec, d->context->stream)
                                      : enqueue_decoder_step(d, d->context->stream);
    g_plan = saved;
    return e;
}
// after a call's last step: the pending argmax finish, so token, trace and
// position are current for the host (nothing when already finished)
hipError_t finish_decoder_steps(fortai_hip_qwen35_decoder *d) {
    if (!(d->families & kFamHead)) return hipSuccess;
    int parts = 0;
    const ArgmaxState st = decoder_argmax(d, &parts);
    return launch_argmax_finish(parts, st, d->context->stream);
}
// the token the next step embeds, as given by the host
hipError_t set_decoder_token(fortai_hip_qwen35_decoder *d, int64_t token, int position) {
    auto *c = d->context;
    hipLaunchKernelGGL(set_token_kernel, dim3(1), dim3(1), 0, c->stream, c->token, token);
    hipLaunchKernelGGL(set_token_kernel, dim3(1), dim3(1), 0, c->stream, d->embed, token);
    hipLaunchKernelGGL(set_position_kernel, dim3(1), dim3(1), 0, c->stream, c->position, position);
    return hipGetLastError();
}
}  // namespace

int fortai_hip_qwen35_decoder_create(fortai_hip_q8_context *c, int layer_count,
    fortai_hip_qwen35_recurrent *const *recurrent, fortai_hip_qwen35_attention *const *attention,
    const fortai_hip_q8_weights *const *ffn_gate, const fortai_hip_q8_weights *const *ffn_up,
    const fortai_hip_q8_weights *const *ffn_down, const float *const *attn_norm, const float *const *post_norm,
    const float *output_norm, int hidden, const fortai_hip_f16_weights *emb16, const fortai_hip_q8_weights *emb8,
    const fortai_hip_f16_weights *out16, const fortai_hip_q8_weights *out8, int max_context, float eps,
    fortai_hip_qwen35_decoder **decoder) {
    if (!c || !decoder || layer_count <= 0 || !recurrent || !attention || !ffn_gate || !ffn_up || !ffn_down ||
        !attn_norm || !post_norm || !output_norm || hidden <= 0 || hidden % 64 || max_context <= 0 || eps <= 0.0f ||
        (!emb16 == !emb8) || (!out16 == !out8))
        return FORTAI_HIP_INVALID;
    *decoder = nullptr;
    if ((emb16 && (emb16->context != c || emb16->width != hidden)) || (emb8 && (!owned(c, emb8) || emb8->width != hidden)) ||
        (out16 && (out16->context != c || out16->width != hidden)) || (out8 && (!owned(c, out8) || out8->width != hidden)))
        return FORTAI_HIP_INVALID;
    const int vocab = out16 ? out16->rows : out8->m.rows;
    if (out16 && f16_matvec_workgroups(vocab) > 1 << 20) return FORTAI_HIP_INVALID;
    auto *d = new (std::nothrow) fortai_hip_qwen35_decoder;
    if (!d) return FORTAI_HIP_RUNTIME_ERROR;
    d->context = c; d->hidden = hidden; d->vocab = vocab; d->max_context = max_context; d->eps = eps;
    d->emb16 = emb16; d->emb8 = emb8; d->out16 = out16; d->out8 = out8;
    int ffn = 0;
    for (int i = 0; i < layer_count; ++i) {
        decoder_layer L;
        L.recurrent = recurrent[i];
        L.attention = attention[i];
        L.gate = ffn_gate[i]; L.up = ffn_up[i]; L.down = ffn_down[i];
        const bool ok = (!L.recurrent != !L.attention) && owned(c, L.gate) && owned(c, L.up) && owned(c, L.down) &&
            ffn_shapes_ok(L.gate, L.up, L.down) && L.gate->width == hidden && L.down->m.rows == hidden &&
            attn_norm[i] && post_norm[i] &&
            (L.recurrent ? (L.recurrent->context == c && L.recurrent->qkv->width == hidden && L.recurrent->out->m.rows == hidden)
                         : (L.attention->context == c && L.attention->q->width == hidden && L.attention->o->m.rows == hidden &&
                            L.attention->max_context >= max_context));
        if (!ok) {
            delete d;
            return FORTAI_HIP_INVALID;
        }
        if (L.gate->m.rows > ffn) ffn = L.gate->m.rows;
        d->layers.push_back(L);
    }
    d->ffn = ffn;
    (void)hipSetDevice(c->device);
    const int parts = out16 ? f16_matvec_workgroups(vocab) : 1024;
    hipError_t e = hipSuccess;
    for (auto &L : d->layers) {
        if (e == hipSuccess) e = upload_f32(&L.attn_norm, attn_norm[&L - d->layers.data()], hidden, c->stream);
        if (e == hipSuccess) e = upload_f32(&L.post_norm, post_norm[&L - d->layers.data()], hidden, c->stream);
    }
    if (e == hipSuccess) e = upload_f32(&d->output_norm, output_norm, hidden, c->stream);
    if (e == hipSuccess) e = alloc(&d->x, hidden);
    if (e == hipSuccess) e = alloc_q8l(&d->h_q8l, ffn, c->stream);
    if (e == hipSuccess) e = alloc(&d->logits, vocab);
    if (e == hipSuccess) e = alloc(&d->argmax_value, parts);
    if (e == hipSuccess) e = alloc(&d->argmax_index, parts);
    if (e == hipSuccess) e = alloc(&d->trace, max_context + 1);
    if (e == hipSuccess) e = hipMemsetAsync(d->trace, 0, (max_context + 1) * sizeof(int64_t), c->stream);
    if (e == hipSuccess) e = alloc(&d->embed, 1);
    if (e == hipSuccess) e = hipMemsetAsync(d->embed, 0, sizeof(int64_t), c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e == hipSuccess) e = capture_decoder(d);
    if (e != hipSuccess) {
        fortai_hip_qwen35_decoder_destroy(d);
        return fail(c, FORTAI_HIP_RUNTIME_ERROR, "Qwen decoder create", e);
    }
    *decoder = d;
    return FORTAI_HIP_OK;
}

int fortai_hip_qwen35_decoder_destroy(fortai_hip_qwen35_decoder *d) {
    if (!d) return FORTAI_HIP_OK;
    auto *c = d->context;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    if (d->exec) (void)hipGraphExecDestroy(d->exec);
    if (d->graph) (void)hipGraphDestroy(d->graph);
    for (auto &L : d->layers) {
        release(L.attn_norm);
        release(L.post_norm);
    }
    release(d->output_norm); release(d->x); release(d->logits); release(d->argmax_value);
    release(d->argmax_index); release(d->trace); release(d->embed);
    if (d->h_q8l) (void)hipFree(d->h_q8l);
    delete d;
    return FORTAI_HIP_OK;
}

int fortai_hip_qwen35_decoder_reset(fortai_hip_qwen35_decoder *d) {
    if (!d) return FORTAI_HIP_INVALID;
    for (auto &L : d->layers) {
        const int rc = L.recurrent ? fortai_hip_qwen35_recurrent_reset(L.recurrent)
                                   : fortai_hip_qwen35_attention_reset(L.attention);
        if (rc != FORTAI_HIP_OK) return rc;
    }
    auto *c = d->context;
    (void)hipSetDevice(c->device);
    d->next_position = 0;
    hipError_t e = hipMemsetAsync(d->trace, 0, (d->max_context + 1) * sizeof(int64_t), c->stream);
    if (e == hipSuccess) e = hipMemsetAsync(d->x, 0, d->hidden * sizeof(float), c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    return done(c, e, "decoder reset");
}

int fortai_hip_qwen35_decoder_forward(fortai_hip_qwen35_decoder *d, int64_t token, int position, float *logits,
    int64_t *next_token) {
    if (!d || token < 0 || token >= (d->emb16 ? d->emb16->rows : d->emb8->m.rows) || position < 0 ||
        position >= d->max_context)
        return FORTAI_HIP_INVALID;
    auto *c = d->context;
    (void)hipSetDevice(c->device);
    hipError_t e = set_decoder_token(d, token, position);
    if (e == hipSuccess) e = run_step(d);
    if (e == hipSuccess) e = finish_decoder_steps(d);
    d->next_position = position + 1;
    if (e == hipSuccess && logits)
        e = hipMemcpyAsync(logits, d->logits, static_cast<size_t>(d->vocab) * 4, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess && next_token)
        e = hipMemcpyAsync(next_token, c->token, sizeof(int64_t), hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess && (logits || next_token)) e = hipStreamSynchronize(c->stream);
    return done(c, e, "decoder forward");
}

int fortai_hip_qwen35_decoder_generate(fortai_hip_qwen35_decoder *d, int64_t token, int position, int steps,
    int64_t *trace) {
    if (!d || !trace || steps <= 0 || position < 0 || position + steps > d->max_context || token < 0 ||
        token >= (d->emb16 ? d->emb16->rows : d->emb8->m.rows))
        return FORTAI_HIP_INVALID;
    auto *c = d->context;
    (void)hipSetDevice(c->device);
    hipError_t e = set_decoder_token(d, token, position);
    for (int s = 0; s < steps && e == hipSuccess; ++s) e = run_step(d);
    if (e == hipSuccess) e = finish_decoder_steps(d);
    d->next_position = position + steps;
    if (e == hipSuccess)
        e = hipMemcpyAsync(trace, d->trace + position, static_cast<size_t>(steps) * sizeof(int64_t),
            hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    return done(c, e, "decoder generate");
}

int fortai_hip_qwen35_decoder_replay(fortai_hip_qwen35_decoder *d, int steps) {
    if (!d || steps <= 0 || d->next_position + steps > d->max_context) return FORTAI_HIP_INVALID;
    auto *c = d->context;
    (void)hipSetDevice(c->device);
    hipError_t e = hipSuccess;
    for (int s = 0; s < steps && e == hipSuccess; ++s) e = run_step(d);
    if (e == hipSuccess) e = finish_decoder_steps(d);
    d->next_position += steps;
    return done(c, e, "decoder replay");
}

int fortai_hip_qwen35_decoder_status(fortai_hip_qwen35_decoder *d) {
    if (!d) return FORTAI_HIP_INVALID;
    auto *c = d->context;
    (void)hipSetDevice(c->device);
    return done(c, hipStreamSynchronize(c->stream), "decoder status");
}

int fortai_hip_qwen35_decoder_plan(const fortai_hip_qwen35_decoder *d, char *buffer, size_t bytes, size_t *needed) {
    if (!d) return FORTAI_HIP_INVALID;
    return copy_plan(d->plan, buffer, bytes, needed);
}

int fortai_hip_qwen35_decoder_logits(fortai_hip_qwen35_decoder *d, void **logits) {
    if (!d || !logits) return FORTAI_HIP_INVALID;
    *logits = d->logits;
    return FORTAI_HIP_OK;
}

int fortai_hip_qwen35_decoder_trace(fortai_hip_qwen35_decoder *d, int first, int count, int64_t *host_trace) {
    if (!d || !host_trace || first < 0 || count <= 0 || count > d->max_context - first) return FORTAI_HIP_INVALID;
    auto *c = d->context;
    (void)hipSetDevice(c->device);
    hipError_t e = hipMemcpyAsync(host_trace, d->trace + first, static_cast<size_t>(count) * sizeof(int64_t),
        hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    return done(c, e, "decoder trace");
}

// ------------------------------------------------------------ batched decoder
namespace {
hipError_t enqueue_batch_step(fortai_hip_qwen35_batch *b, hipStream_t stream) {
    const int B = b->batch, H = b->hidden;
    hipError_t e = rec(b->emb16 ? launch_f16_embedding(b->emb16->data, b->emb16->rows, H, b->tokens, 0, b->x, stream, B)
                                : launch_q8_embedding(b->emb8->m, b->tokens, 0, b->x, stream, B), "token embeddings");
    for (size_t i = 0; i < b->layers.size() && e == hipSuccess; ++i) {
        batch_layer &L = b->layers[i];
        MatvecInput in;
        in.x = b->x;
        in.norm = L.attn_norm;
        in.eps = b->eps;
        in.width = H;
        e = rec(launch_q8l_prep(in, Prologue::RMSNORM, b->act, B, stream), "attention-norm and quantize");
        if (e != hipSuccess) break;
        if (L.rec) {
            auto *R = L.rec;
            MatvecSegment segs[4] = {segment(R->qkv, L.qkv), segment(R->gate, L.z), segment(R->alpha, L.alpha),
                segment(R->beta, L.beta)};
            segs[0].conv_w = R->conv_w;
            segs[0].conv_state = L.conv_state;
            segs[0].conv_size = R->conv_size;
            segs[0].kernel = R->kernel;
            segs[1].silu = true;
            e = rec(launch_q8_batch_matvec(segs, 4, b->act, H, B, Epilogue::STORE, stream),
                "GDN qkv/gate/alpha/beta projections, conv1d + SiLU");
            GdnParams gp = gdn_params(R, L.qkv, L.alpha, L.beta, L.o_raw);
            gp.state = L.state;
            if (e == hipSuccess && (R->head == 64 || R->head == 128) && R->inner % 128 == 0) {
                // one workgroup per (value head, sequence): the delta rule, then
                // the gated norm and quantization for ssm_out in the same launch
                e = rec(launch_gdn_delta_gated(gp, L.z, R->ssm_norm, R->eps, b->act, stream, B),
                    "GDN L2 norms, decay/beta, delta rule, gated RMSNorm and quantize");
            } else {
                if (e == hipSuccess) e = rec(launch_gdn_delta(gp, stream, B), "GDN L2 norms, decay/beta, delta rule");
                MatvecInput gated;
                gated.x = L.o_raw;
                gated.z = L.z;
                gated.norm = R->ssm_norm;
                gated.eps = R->eps;
                gated.head = R->head;
                gated.width = R->inner;
                if (e == hipSuccess)
                    e = rec(launch_q8l_prep(gated, Prologue::GATED, b->act, B, stream), "GDN gated RMSNorm and quantize");
            }
            const MatvecSegment oseg = segment(R->out, b->x, b->x);
            if (e == hipSuccess)
                e = rec(launch_q8_batch_matvec(&oseg, 1, b->act, R->inner, B, Epilogue::ADD, stream),
                    "GDN ssm_out projection + residual");
        } else {
            auto *A = L.att;
            const MatvecSegment segs[3] = {segment(A->q, L.q), segment(A->k, L.k), segment(A->v, L.v)};
            e = rec(launch_q8_batch_matvec(segs, 3, b->act, H, B, Epilogue::STORE, stream), "attention q/k/v projections");
            AttentionParams ap = attention_params(A, L.q, L.k, L.v, L.attn_out);
            ap.kcache = L.kcache; ap.vcache = L.vcache; ap.partial = L.partial; ap.cache_flags = L.flags;
            ap.split = L.split; ap.position = b->positions; ap.max_context = b->max_context;
            // the output kernels also quantize the o projection's input when they can
            ap.out_q8l = b->act;
            if (!attention_quantizes_output(ap, B)) ap.out_q8l = nullptr;
            if (e == hipSuccess) e = rec(launch_attention(ap, stream, B), "q/k norm, RoPE, KV append, softmax.V, gate");
            MatvecInput oin;
            oin.x = L.attn_out;
            oin.width = A->heads * A->value;
            if (e == hipSuccess && !ap.out_q8l)
                e = rec(launch_q8l_prep(oin, Prologue::F32, b->act, B, stream), "quantize attention output");
            const MatvecSegment oseg = segment(A->o, b->x, b->x);
            if (e == hipSuccess)
                e = rec(launch_q8_batch_matvec(&oseg, 1, b->act, oin.width, B, Epilogue::ADD, stream),
                    "attention o projection + residual");
        }
        if (e != hipSuccess) break;
        in.norm = L.post_norm;
        e = rec(launch_q8l_prep(in, Prologue::RMSNORM, b->act, B, stream), "FFN post-norm and quantize");
        const MatvecSegment pair = segment(L.gate, nullptr, nullptr, L.up, b->h_q8l);
        if (e == hipSuccess)
            e = rec(launch_q8_batch_matvec(&pair, 1, b->act, H, B, Epilogue::SILU_PAIR, stream),
                "FFN gate/up projections, SiLU product");
        const MatvecSegment dseg = segment(L.down, b->x, b->x);
        if (e == hipSuccess)
            e = rec(launch_q8_batch_matvec(&dseg, 1, b->h_q8l, L.gate->m.rows, B, Epilogue::ADD, stream),
                "FFN down projection + residual");
    }
    if (e != hipSuccess) return e;
    ArgmaxState st;
    st.partial_value = b->argmax_value;
    st.partial_index = b->argmax_index;
    st.token = b->tokens;
    st.trace = b->trace;
    st.trace_capacity = b->max_context;
    st.position = b->positions;
    if (b->out16)
        return rec(launch_f16_batch_lm_head(b->out16->data, b->vocab, H, b->out16->finite, B, b->x, b->output_norm,
            b->eps, b->xnorm, b->logits, st, stream), "output RMSNorm, LM head, greedy argmax");
    // Q8_0 LM head: the batched matvec, then the argmax of each sequence
    MatvecInput in;
    in.x = b->x;
    in.norm = b->output_norm;
    in.eps = b->eps;
    in.width = H;
    e = launch_q8l_prep(in, Prologue::RMSNORM, b->act, B, stream);
    const MatvecSegment s8 = segment(b->out8, b->logits);
    if (e == hipSuccess) e = launch_q8_batch_matvec(&s8, 1, b->act, H, B, Epilogue::STORE, stream);
    for (int q = 0; q < B && e == hipSuccess; ++q) {
        ArgmaxState sq = st;
        sq.partial_value += static_cast<size_t>(q) * b->parts;
        sq.partial_index += static_cast<size_t>(q) * b->parts;
        sq.token += q;
        sq.trace += static_cast<size_t>(q) * b->max_context;
        sq.position += q;
        e = launch_argmax(b->logits + static_cast<size_t>(q) * b->vocab, b->vocab, sq, stream);
    }
    return e;
}

hipError_t batch_step(fortai_hip_qwen35_batch *b) {
    if (b->use_graph) return hipGraphLaunch(b->exec, b->context->stream);
    std::vector<plan_step> *saved = g_plan;
    if (b->plan.empty()) {
        g_plan = &b->plan;
        g_plan_batch = b->batch;
    }
    const hipError_t e = enqueue_batch_step(b, b->context->stream);
    g_plan = saved;
    g_plan_batch = 1;
    return e;
}

hipError_t batch_zero_state(fortai_hip_qwen35_batch *b, hipStream_t stream) {
    const size_t B = static_cast<size_t>(b->batch);
    hipError_t e = hipSuccess;
    for (auto &L : b->layers) {
        if (L.rec) {
            const auto *R = L.rec;
            if (e == hipSuccess)
                e = hipMemsetAsync(L.conv_state, 0, B * (R->kernel - 1) * R->conv_size * sizeof(float), stream);
            if (e == hipSuccess)
                e = hipMemsetAsync(L.state, 0, B * R->value_heads * R->head * R->head * sizeof(float), stream);
        } else {
            const auto *A = L.att;
            const size_t cache = B * b->max_context * A->kv_heads;
            if (e == hipSuccess) e = hipMemsetAsync(L.kcache, 0, cache * A->head * sizeof(uint16_t), stream);
            if (e == hipSuccess) e = hipMemsetAsync(L.vcache, 0, cache * A->value * sizeof(uint16_t), stream);
            if (e == hipSuccess) e = hipMemsetAsync(L.flags, 0, B * A->kv_heads * sizeof(int), stream);
        }
    }
    if (e == hipSuccess) e = hipMemsetAsync(b->trace, 0, B * b->max_context * sizeof(int64_t), stream);
    if (e == hipSuccess) e = hipMemsetAsync(b->x, 0, B * b->hidden * sizeof(float), stream);
    return e;
}

int batch_set_inputs(fortai_hip_qwen35_batch *b, const int64_t *tokens, const int *positions, int steps) {
    const int rows = b->emb16 ? b->emb16->rows : b->emb8->m.rows;
    auto *c = b->context;
    for (int q = 0; q < b->batch; ++q)
        if (tokens[q] < 0 || tokens[q] >= rows || positions[q] < 0 || positions[q] + steps > b->max_context) {
            std::snprintf(c->error, sizeof(c->error), "batch inputs: sequence %d token %lld position %d steps %d "
                "outside vocabulary %d / context %d", q, static_cast<long long>(tokens[q]), positions[q], steps,
                rows, b->max_context);
            return FORTAI_HIP_INVALID;
        }
    hipError_t e = hipMemcpyAsync(b->tokens, tokens, b->batch * sizeof(int64_t), hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(b->positions, positions, b->batch * sizeof(int), hipMemcpyHostToDevice, c->stream);
    // the host arrays are borrowed for the call only
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    for (int q = 0; q < b->batch; ++q) b->next_positions[q] = positions[q];
    return done(c, e, "batch inputs");
}
}  // namespace

// One batched step as a captured graph (unless in direct mode).
hipError_t capture_batch(fortai_hip_qwen35_batch *b) {
    auto *c = b->context;
    if (b->exec) (void)hipGraphExecDestroy(b->exec);
    if (b->graph) (void)hipGraphDestroy(b->graph);
    b->exec = nullptr;
    b->graph = nullptr;
    b->plan.clear();
    if (!b->use_graph) return hipSuccess;
    hipError_t e = hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return e;
    g_plan = &b->plan;
    g_plan_batch = b->batch;
    const hipError_t ce = enqueue_batch_step(b, c->stream);
    g_plan = nullptr;
    g_plan_batch = 1;
    e = hipStreamEndCapture(c->stream, &b->graph);
    if (ce != hipSuccess) e = ce;
    if (e == hipSuccess) e = hipGraphInstantiate(&b->exec, b->graph, nullptr, nullptr, 0);
    return e;
}

int fortai_hip_qwen35_batch_create(fortai_hip_q8_context *c, int batch, int layer_count,
    fortai_hip_qwen35_recurrent *const *recurrent, fortai_hip_qwen35_attention *const *attention,
    const fortai_hip_q8_weights *const *ffn_gate, const fortai_hip_q8_weights *const *ffn_up,
    const fortai_hip_q8_weights *const *ffn_down, const float *const *attn_norm, const float *const *post_norm,
    const float *output_norm, int hidden, const fortai_hip_f16_weights *emb16, const fortai_hip_q8_weights *emb8,
    const fortai_hip_f16_weights *out16, const fortai_hip_q8_weights *out8, int max_context, float eps,
    fortai_hip_qwen35_batch **out) {
    if (!c || !out || batch < 1 || batch > 8 || layer_count <= 0 || !recurrent || !attention || !ffn_gate ||
        !ffn_up || !ffn_down || !attn_norm || !post_norm || !output_norm || hidden <= 0 || hidden % 64 ||
        max_context <= 0 || eps <= 0.0f || (!emb16 == !emb8) || (!out16 == !out8))
        return FORTAI_HIP_INVALID;
    *out = nullptr;
    if ((emb16 && (emb16->context != c || emb16->width != hidden)) || (emb8 && (!owned(c, emb8) || emb8->width != hidden)) ||
        (out16 && (out16->context != c || out16->width != hidden)) || (out8 && (!owned(c, out8) || out8->width != hidden)))
        return FORTAI_HIP_INVALID;
    auto *b = new (std::nothrow) fortai_hip_qwen35_batch;
    if (!b) return FORTAI_HIP_RUNTIME_ERROR;
    b->context = c; b->batch = batch; b->hidden = hidden; b->max_context = max_context; b->eps = eps;
    b->emb16 = emb16; b->emb8 = emb8; b->out16 = out16; b->out8 = out8;
    b->vocab = out16 ? out16->rows : out8->m.rows;
    b->parts = out16 ? f16_batch_lm_head_workgroups(b->vocab) : (b->vocab + 255) / 256;
    b->next_positions.assign(batch, 0);
    int ffn = 0, width = hidden;
    for (int i = 0; i < layer_count; ++i) {
        batch_layer L;
        L.rec = recurrent[i];
        L.att = attention[i];
        L.gate = ffn_gate[i]; L.up = ffn_up[i]; L.down = ffn_down[i];
        const bool ok = (!L.rec != !L.att) && owned(c, L.gate) && owned(c, L.up) && owned(c, L.down) &&
            ffn_shapes_ok(L.gate, L.up, L.down) && L.gate->width == hidden && L.down->m.rows == hidden &&
            attn_norm[i] && post_norm[i] &&
            (L.rec ? (L.rec->context == c && L.rec->qkv->width == hidden && L.rec->out->m.rows == hidden)
                   : (L.att->context == c && L.att->q->width == hidden && L.att->o->m.rows == hidden &&
                      L.att->max_context >= max_context));
        if (!ok) {
            delete b;
            return FORTAI_HIP_INVALID;
        }
        ffn = std::max(ffn, L.gate->m.rows);
        width = std::max(width, L.rec ? L.rec->inner : L.att->heads * L.att->value);
        b->layers.push_back(L);
    }
    b->ffn = ffn;
    b->act_width = width;
    (void)hipSetDevice(c->device);
    const size_t B = static_cast<size_t>(batch);
    hipError_t e = hipSuccess;
    for (size_t i = 0; i < b->layers.size(); ++i) {
        batch_layer &L = b->layers[i];
        if (e == hipSuccess) e = upload_f32(&L.attn_norm, attn_norm[i], hidden, c->stream);
        if (e == hipSuccess) e = upload_f32(&L.post_norm, post_norm[i], hidden, c->stream);
        if (L.rec) {
            const auto *R = L.rec;
            if (e == hipSuccess) e = alloc(&L.conv_state, B * (R->kernel - 1) * R->conv_size);
            if (e == hipSuccess) e = alloc(&L.state, B * R->value_heads * R->head * R->head);
            if (e == hipSuccess) e = alloc(&L.qkv, B * R->conv_size);
            if (e == hipSuccess) e = alloc(&L.z, B * R->inner);
            if (e == hipSuccess) e = alloc(&L.alpha, B * R->value_heads);
            if (e == hipSuccess) e = alloc(&L.beta, B * R->value_heads);
            if (e == hipSuccess) e = alloc(&L.o_raw, B * R->inner);
        } else {
            const auto *A = L.att;
            const size_t cache = B * max_context * A->kv_heads;
            if (e == hipSuccess) e = alloc(&L.kcache, cache * A->head);
            if (e == hipSuccess) e = alloc(&L.vcache, cache * A->value);
            if (e == hipSuccess) e = alloc(&L.q, B * A->heads * 2 * A->head);
            if (e == hipSuccess) e = alloc(&L.k, B * A->kv_heads * A->head);
            if (e == hipSuccess) e = alloc(&L.v, B * A->kv_heads * A->value);
            if (e == hipSuccess) e = alloc(&L.partial, B * attention_scores_floats(A->heads, max_context));
            if (e == hipSuccess) e = alloc(&L.attn_out, B * A->heads * A->value);
            if (e == hipSuccess) e = alloc(&L.flags, B * A->kv_heads);
            if (e == hipSuccess && max_context > A->exact_max)
                e = alloc(&L.split, B * A->heads * attention_split_chunks(max_context) * (A->value + 2));
        }
    }
    if (e == hipSuccess) e = upload_f32(&b->output_norm, output_norm, hidden, c->stream);
    if (e == hipSuccess) e = alloc(&b->x, B * hidden);
    if (e == hipSuccess) e = alloc(&b->xnorm, static_cast<size_t>(8) * hidden);
    if (e == hipSuccess) e = hipMalloc(&b->act, B * q8l_bytes(width));
    if (e == hipSuccess) e = hipMemsetAsync(b->act, 0, B * q8l_bytes(width), c->stream);
    if (e == hipSuccess) e = hipMalloc(&b->h_q8l, B * q8l_bytes(ffn));
    if (e == hipSuccess) e = hipMemsetAsync(b->h_q8l, 0, B * q8l_bytes(ffn), c->stream);
    if (e == hipSuccess) e = alloc(&b->logits, B * b->vocab);
    if (e == hipSuccess) e = alloc(&b->argmax_value, B * b->parts);
    if (e == hipSuccess) e = alloc(&b->argmax_index, B * b->parts);
    if (e == hipSuccess) e = alloc(&b->tokens, B);
    if (e == hipSuccess) e = alloc(&b->positions, B);
    if (e == hipSuccess) e = alloc(&b->trace, B * max_context);
    if (e == hipSuccess) e = hipMemsetAsync(b->tokens, 0, B * sizeof(int64_t), c->stream);
    if (e == hipSuccess) e = hipMemsetAsync(b->positions, 0, B * sizeof(int), c->stream);
    if (e == hipSuccess) e = batch_zero_state(b, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    // one step captured as a graph (state, tokens and positions are device-side)
    if (e == hipSuccess) e = capture_batch(b);
    if (e != hipSuccess) {
        fortai_hip_qwen35_batch_destroy(b);
        return fail(c, FORTAI_HIP_RUNTIME_ERROR, "Qwen batch create", e);
    }
    *out = b;
    return FORTAI_HIP_OK;
}

int fortai_hip_qwen35_batch_destroy(fortai_hip_qwen35_batch *b) {
    if (!b) return FORTAI_HIP_OK;
    auto *c = b->context;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    release(b->px); release(b->pa); release(b->pb); release(b->pc); release(b->pd); release(b->palpha);
    release(b->pbeta); release(b->pqinv); release(b->pkinv); release(b->pbt); release(b->pdt); release(b->ptokens);
    if (b->px8) (void)hipFree(b->px8);
    if (b->pq8l) (void)hipFree(b->pq8l);
    b->pq8l = nullptr;
    if (b->exec) (void)hipGraphExecDestroy(b->exec);
    if (b->graph) (void)hipGraphDestroy(b->graph);
    for (auto &L : b->layers) {
        release(L.attn_norm); release(L.post_norm);
        release(L.conv_state); release(L.state); release(L.qkv); release(L.z); release(L.alpha); release(L.beta);
        release(L.o_raw);
        release(L.kcache); release(L.vcache); release(L.q); release(L.k); release(L.v); release(L.partial);
        release(L.attn_out); release(L.split); release(L.flags);
    }
    release(b->output_norm); release(b->x); release(b->xnorm); release(b->logits); release(b->argmax_value); release(b->argmax_index);
    release(b->tokens); release(b->positions); release(b->trace);
    if (b->act) (void)hipFree(b->act);
    if (b->h_q8l) (void)hipFree(b->h_q8l);
    delete b;
    return FORTAI_HIP_OK;
}

int fortai_hip_qwen35_batch_reset(fortai_hip_qwen35_batch *b) {
    if (!b) return FORTAI_HIP_INVALID;
    auto *c = b->context;
    (void)hipSetDevice(c->device);
    hipError_t e = batch_zero_state(b, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    b->next_positions.assign(b->batch, 0);
    return done(c, e, "batch reset");
}

int fortai_hip_qwen35_batch_forward(fortai_hip_qwen35_batch *b, const int64_t *tokens, const int *positions,
    float *logits, int64_t *next_tokens) {
    if (!b || !tokens || !positions) return FORTAI_HIP_INVALID;
    auto *c = b->context;
    (void)hipSetDevice(c->device);
    const int rc = batch_set_inputs(b, tokens, positions, 1);
    if (rc != FORTAI_HIP_OK) return rc;
    hipError_t e = batch_step(b);
    for (auto &p : b->next_positions) ++p;
    if (e == hipSuccess && logits)
        e = hipMemcpyAsync(logits, b->logits, static_cast<size_t>(b->batch) * b->vocab * sizeof(float),
            hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess && next_tokens)
        e = hipMemcpyAsync(next_tokens, b->tokens, b->batch * sizeof(int64_t), hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess && (logits || next_tokens)) e = hipStreamSynchronize(c->stream);
    return done(c, e, "batch forward");
}

int fortai_hip_qwen35_batch_generate(fortai_hip_qwen35_batch *b, const int64_t *tokens, const int *positions,
    int steps, int64_t *trace) {
    if (!b || !tokens || !positions || !trace || steps <= 0) return FORTAI_HIP_INVALID;
    auto *c = b->context;
    (void)hipSetDevice(c->device);
    const int rc = batch_set_inputs(b, tokens, positions, steps);
    if (rc != FORTAI_HIP_OK) return rc;
    hipError_t e = hipSuccess;
    for (int s = 0; s < steps && e == hipSuccess; ++s) e = batch_step(b);
    for (int q = 0; q < b->batch && e == hipSuccess; ++q) {
        e = hipMemcpyAsync(trace + static_cast<size_t>(q) * steps,
            b->trace + static_cast<size_t>(q) * b->max_context + positions[q], steps * sizeof(int64_t),
            hipMemcpyDeviceToHost, c->stream);
        b->next_positions[q] = positions[q] + steps;
    }
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    return done(c, e, "batch generate");
}

int fortai_hip_qwen35_batch_replay(fortai_hip_qwen35_batch *b, int steps) {
    if (!b || steps <= 0) return FORTAI_HIP_INVALID;
    for (int q = 0; q < b->batch; ++q)
        if (b->next_positions[q] + steps > b->max_context) return FORTAI_HIP_INVALID;
    auto *c = b->context;
    (void)hipSetDevice(c->device);
    hipError_t e = hipSuccess;
    for (int s = 0; s < steps && e == hipSuccess; ++s) e = batch_step(b);
    for (auto &p : b->next_positions) p += steps;
    return done(c, e, "batch replay");
}

namespace {
// widths of the prefill buffers
struct prefill_widths {
    int x8 = 0, a = 0, b = 0, c = 0, d = 0, vh = 0, kh = 0;
};
prefill_widths batch_prefill_widths(const fortai_hip_qwen35_batch *b) {
    prefill_widths w;
    w.x8 = std::max(b->hidden, b->ffn);
    w.a = w.b = b->ffn;
    for (const auto &L : b->layers) {
        if (L.rec) {
            const auto *R = L.rec;
            w.x8 = std::max(w.x8, R->inner);
            w.a = std::max(w.a, R->conv_size);
            w.b = std::max(w.b, R->inner);
            w.c = std::max(w.c, R->conv_size);
            w.d = std::max(w.d, R->inner);
            w.vh = std::max(w.vh, R->value_heads);
            w.kh = std::max(w.kh, R->key_heads);
        } else {
            const auto *A = L.att;
            w.x8 = std::max(w.x8, A->heads * A->value);
            w.a = std::max(w.a, A->heads * 2 * A->head);
            w.b = std::max(w.b, A->kv_heads * A->head);
            w.c = std::max(w.c, A->kv_heads * A->value);
            w.d = std::max(w.d, A->heads * A->value);
        }
    }
    return w;
}

hipError_t batch_prefill_buffers(fortai_hip_qwen35_batch *b, int rows) {
    if (rows <= b->prefill_rows) return hipSuccess;
    release(b->px); release(b->pa); release(b->pb); release(b->pc); release(b->pd); release(b->palpha);
    release(b->pbeta); release(b->pqinv); release(b->pkinv); release(b->pbt); release(b->pdt); release(b->ptokens);
    if (b->px8) (void)hipFree(b->px8);
    if (b->pq8l) (void)hipFree(b->pq8l);
    b->pq8l = nullptr;
    b->px8 = nullptr;
    b->prefill_rows = 0;
    const prefill_widths w = batch_prefill_widths(b);
    const size_t n = static_cast<size_t>(rows);
    hipError_t e = alloc(&b->px, n * b->hidden);
    if (e == hipSuccess) e = hipMalloc(&b->px8, q8_tokens_bytes(rows, w.x8));
    if (e == hipSuccess) e = alloc(&b->pa, n * w.a);
    if (e == hipSuccess) e = alloc(&b->pb, n * w.b);
    if (e == hipSuccess) e = alloc(&b->pc, n * std::max(w.c, 1));
    if (e == hipSuccess) e = alloc(&b->pd, n * w.d);
    if (e == hipSuccess) e = alloc(&b->palpha, n * std::max(w.vh, 1));
    if (e == hipSuccess) e = alloc(&b->pbeta, n * std::max(w.vh, 1));
    if (e == hipSuccess) e = alloc(&b->pbt, n * std::max(w.vh, 1));
    if (e == hipSuccess) e = alloc(&b->pdt, n * std::max(w.vh, 1));
    if (e == hipSuccess) e = alloc(&b->pqinv, n * std::max(w.kh, 1));
    if (e == hipSuccess) e = alloc(&b->pkinv, n * std::max(w.kh, 1));
    if (e == hipSuccess) e = alloc(&b->ptokens, n);
    if (e == hipSuccess) e = hipMalloc(&b->pq8l, 8 * q8l_bytes(w.x8));
    if (e == hipSuccess) b->prefill_rows = rows;
    return e;
}

// Every layer over batch * T prompt tokens (positions 0..T-1), then the LM
// head on each sequence's last token, which leaves tokens / positions / trace
// as after T decode steps.
// The modes (FORTAI_HIP_PREFILL):
//  exact (default): the projections in the reference's lane order on the
//    matrix cores (q8_mmq_exact_kernel) and the fp32 causal attention: every
//    logit and state bit-identical to token-by-token decoding;
//  fast: the projections as whole-block int32 dots (q8_mmq_kernel) and the
//    fp16 matrix-core attention (outputs within fp32 rounding of the
//    reference, not bit for bit);
//  matvec: the projections through the batched decode matvec, 8 tokens at a
//    time (a cross-check of the exact mode).
hipError_t enqueue_batch_prefill(fortai_hip_qwen35_batch *b, int T, PrefillMode mode, hipStream_t stream) {
    const int B = b->batch, H = b->hidden, N = B * T;
    hipError_t e = rec(b->emb16 ? launch_f16_embedding(b->emb16->data, b->emb16->rows, H, b->ptokens, 0, b->px, stream, N)
                                : launch_q8_embedding(b->emb8->m, b->ptokens, 0, b->px, stream, N), "token embeddings");
    auto mmq = [&](const fortai_hip_q8_weights *w, float *out, const float *resid, const char *op) {
        if (mode == PrefillMode::EXACT)
            return rec(launch_q8_mmq_exact(w->m, b->px8, N, out, w->m.rows, resid, stream), op);
        if (mode == PrefillMode::FAST) return rec(launch_q8_mmq(w->m, b->px8, N, out, w->m.rows, resid, nullptr, stream), op);
        hipError_t r = hipSuccess;
        for (int r0 = 0; r0 < N && r == hipSuccess; r0 += 8) {
            const int cnt = std::min(8, N - r0);
            r = launch_x8_to_q8l(b->px8, N, w->width, r0, cnt, b->pq8l, stream);
            MatvecSegment sg = segment(w, out + static_cast<size_t>(r0) * w->m.rows,
                resid ? resid + static_cast<size_t>(r0) * w->m.rows : nullptr);
            if (r == hipSuccess)
                r = launch_q8_batch_matvec(&sg, 1, b->pq8l, w->width, cnt, resid ? Epilogue::ADD : Epilogue::STORE,
                    stream);
        }
        return r;
    };
    for (size_t i = 0; i < b->layers.size() && e == hipSuccess; ++i) {
        batch_layer &L = b->layers[i];
        e = rec(launch_rms_quantize_tokens(b->px, N, H, L.attn_norm, b->eps, b->px8, stream), "attention-norm and quantize");
        if (L.rec) {
            const auto *R = L.rec;
            if (e == hipSuccess) e = mmq(R->qkv, b->pa, nullptr, "GDN qkv projection");
            if (e == hipSuccess) e = mmq(R->gate, b->pb, nullptr, "GDN gate projection");
            if (e == hipSuccess) e = mmq(R->alpha, b->palpha, nullptr, "GDN alpha projection");
            if (e == hipSuccess) e = mmq(R->beta, b->pbeta, nullptr, "GDN beta projection");
            if (e == hipSuccess)
                e = rec(launch_conv_silu_tokens(b->pa, R->conv_w, L.conv_state, b->pc, B, T, R->conv_size, R->kernel, stream),
                    "GDN conv1d + SiLU over time");
            GdnParams gp = gdn_params(const_cast<fortai_hip_qwen35_recurrent *>(R), b->pc, b->palpha, b->pbeta, b->pd);
            gp.state = L.state;
            if (e == hipSuccess)
                e = rec(launch_gdn_prefill(gp, B, T, b->pqinv, b->pkinv, b->pbt, b->pdt, stream),
                    "GDN L2 norms, decay/beta, delta rule over time");
            if (e == hipSuccess)
                e = rec(launch_gated_quantize_tokens(b->pd, b->pb, R->ssm_norm, R->eps, N, R->inner, R->head, b->px8, stream),
                    "GDN gated RMSNorm and quantize");
            if (e == hipSuccess) e = mmq(R->out, b->px, b->px, "GDN ssm_out projection + residual");
        } else {
            const auto *A = L.att;
            if (e == hipSuccess) e = mmq(A->q, b->pa, nullptr, "attention q projection");
            if (e == hipSuccess) e = mmq(A->k, b->pb, nullptr, "attention k projection");
            if (e == hipSuccess) e = mmq(A->v, b->pc, nullptr, "attention v projection");
            AttentionParams ap = attention_params(const_cast<fortai_hip_qwen35_attention *>(A), b->pa, b->pb, b->pc, b->pd);
            ap.kcache = L.kcache; ap.vcache = L.vcache; ap.cache_flags = L.flags; ap.max_context = b->max_context;
            if (e == hipSuccess)
                e = rec(launch_attention_prefill(ap, B, T, b->pd, stream, mode == PrefillMode::FAST), "q/k norm, RoPE, KV append, causal attention");
            if (e == hipSuccess)
                e = rec(launch_rms_quantize_tokens(b->pd, N, A->heads * A->value, nullptr, 0.0f, b->px8, stream),
                    "quantize attention output");
            if (e == hipSuccess) e = mmq(A->o, b->px, b->px, "attention o projection + residual");
        }
        if (e == hipSuccess)
            e = rec(launch_rms_quantize_tokens(b->px, N, H, L.post_norm, b->eps, b->px8, stream), "FFN post-norm and quantize");
        if (e == hipSuccess) e = mmq(L.gate, b->pa, nullptr, "FFN gate projection");
        if (e == hipSuccess) e = mmq(L.up, b->pb, nullptr, "FFN up projection");
        if (e == hipSuccess)
            e = rec(launch_silu_product_quantize(b->pa, b->pb, N, L.gate->m.rows, b->px8, stream),
                "FFN SiLU product and quantize");
        if (e == hipSuccess) e = mmq(L.down, b->px, b->px, "FFN down projection + residual");
    }
    if (e != hipSuccess) return e;
    // each sequence's last token -> x [batch][hidden]; the LM head then
    // writes trace[T - 1] and advances the positions to T
    e = hipMemcpy2DAsync(b->x, H * sizeof(float), b->px + static_cast<size_t>(T - 1) * H, static_cast<size_t>(T) * H * sizeof(float),
        H * sizeof(float), B, hipMemcpyDeviceToDevice, stream);
    if (e != hipSuccess) return e;
    ArgmaxState st;
    st.partial_value = b->argmax_value;
    st.partial_index = b->argmax_index;
    st.token = b->tokens;
    st.trace = b->trace;
    st.trace_capacity = b->max_context;
    st.position = b->positions;
    if (b->out16)
        return rec(launch_f16_batch_lm_head(b->out16->data, b->vocab, H, b->out16->finite, B, b->x, b->output_norm,
            b->eps, b->xnorm, b->logits, st, stream), "output RMSNorm, LM head, greedy argmax (last prompt tokens)");
    MatvecInput in;
    in.x = b->x;
    in.norm = b->output_norm;
    in.eps = b->eps;
    in.width = H;
    e = launch_q8l_prep(in, Prologue::RMSNORM, b->act, B, stream);
    const MatvecSegment s8 = segment(b->out8, b->logits);
    if (e == hipSuccess) e = launch_q8_batch_matvec(&s8, 1, b->act, H, B, Epilogue::STORE, stream);
    for (int q = 0; q < B && e == hipSuccess; ++q) {
        ArgmaxState sq = st;
        sq.partial_value += static_cast<size_t>(q) * b->parts;
        sq.partial_index += static_cast<size_t>(q) * b->parts;
        sq.token += q;
        sq.trace += static_cast<size_t>(q) * b->max_context;
        sq.position += q;
        e = launch_argmax(b->logits + static_cast<size_t>(q) * b->vocab, b->vocab, sq, stream);
    }
    return e;
}
}  // namespace

int fortai_hip_qwen35_batch_prefill(fortai_hip_qwen35_batch *b, const int64_t *tokens, int T, int64_t *next_tokens,
    float *logits, float *kernel_ms) {
    if (!b || !tokens || T < 1 || T > b->max_context) return FORTAI_HIP_INVALID;
    const int rows = b->emb16 ? b->emb16->rows : b->emb8->m.rows;
    const size_t N = static_cast<size_t>(b->batch) * T;
    for (size_t i = 0; i < N; ++i)
        if (tokens[i] < 0 || tokens[i] >= rows) return FORTAI_HIP_INVALID;
    auto *c = b->context;
    (void)hipSetDevice(c->device);
    hipError_t e = batch_prefill_buffers(b, static_cast<int>(N));
    if (e == hipSuccess) e = hipMemcpyAsync(b->ptokens, tokens, N * sizeof(int64_t), hipMemcpyHostToDevice, c->stream);
    // the LM head of the last prompt token writes trace[T - 1] and moves to T
    std::vector<int> last(b->batch, T - 1);
    if (e == hipSuccess) e = hipMemcpyAsync(b->positions, last.data(), b->batch * sizeof(int), hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);  // the host arrays are borrowed for the call
    if (e == hipSuccess && kernel_ms) e = hipEventRecord(c->start, c->stream);
    const PrefillMode mode = b->prefill_mode;
    b->prefill_plan.clear();
    g_plan = &b->prefill_plan;
    g_plan_batch = static_cast<int>(N);
    if (e == hipSuccess) e = enqueue_batch_prefill(b, T, mode, c->stream);
    g_plan = nullptr;
    g_plan_batch = 1;
    if (e == hipSuccess && kernel_ms) e = hipEventRecord(c->stop, c->stream);
    if (e == hipSuccess && logits)
        e = hipMemcpyAsync(logits, b->logits, static_cast<size_t>(b->batch) * b->vocab * sizeof(float),
            hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess && next_tokens)
        e = hipMemcpyAsync(next_tokens, b->tokens, b->batch * sizeof(int64_t), hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e == hipSuccess && kernel_ms) e = hipEventElapsedTime(kernel_ms, c->start, c->stop);
    b->next_positions.assign(b->batch, T);
    return done(c, e, "batch prefill");
}

int fortai_hip_qwen35_batch_plan(const fortai_hip_qwen35_batch *b, int prefill, char *buffer, size_t bytes,
    size_t *needed) {
    if (!b) return FORTAI_HIP_INVALID;
    return copy_plan(prefill ? b->prefill_plan : b->plan, buffer, bytes, needed);
}

int fortai_hip_qwen35_batch_logits(fortai_hip_qwen35_batch *b, void **logits) {
    if (!b || !logits) return FORTAI_HIP_INVALID;
    *logits = b->logits;
    return FORTAI_HIP_OK;
}

// ---- options (explicit calls; nothing is read from the environment) ----

int fortai_hip_qwen35_attention_set_exact_max(fortai_hip_qwen35_attention *A, int exact_max) {
    if (!A || !A->context || exact_max < 0) return FORTAI_HIP_INVALID;
    auto *c = A->context;
    (void)hipSetDevice(c->device);
    hipError_t e = hipSuccess;
    if (A->max_context > exact_max && !A->split)
        e = alloc(&A->split, static_cast<size_t>(A->heads) * attention_split_chunks(A->max_context) * (A->value + 2));
    if (e == hipSuccess) A->exact_max = exact_max;
    return done(c, e, "Qwen attention exact_max");
}

int fortai_hip_qwen35_attention_set_test_options(fortai_hip_qwen35_attention *A, int z_skew, int force_wide) {
    if (!A || !A->context) return FORTAI_HIP_INVALID;
    A->z_skew = z_skew;
    A->force_wide = force_wide != 0;
    return FORTAI_HIP_OK;
}

int fortai_hip_qwen35_decoder_set_mode(fortai_hip_qwen35_decoder *d, int flags) {
    constexpr int kOnly = FORTAI_HIP_DECODER_MATVEC_ONLY | FORTAI_HIP_DECODER_GDN_ONLY |
        FORTAI_HIP_DECODER_ATTENTION_ONLY | FORTAI_HIP_DECODER_HEAD_ONLY;
    if (!d || (flags & ~(FORTAI_HIP_DECODER_DIRECT | kOnly))) return FORTAI_HIP_INVALID;
    auto *c = d->context;
    (void)hipSetDevice(c->device);
    hipError_t e = hipStreamSynchronize(c->stream);
    d->use_graph = !(flags & FORTAI_HIP_DECODER_DIRECT);
    unsigned f = 0;
    if (flags & FORTAI_HIP_DECODER_MATVEC_ONLY) f |= kFamMatvec;
    if (flags & FORTAI_HIP_DECODER_GDN_ONLY) f |= kFamGdn;
    if (flags & FORTAI_HIP_DECODER_ATTENTION_ONLY) f |= kFamAttention;
    if (flags & FORTAI_HIP_DECODER_HEAD_ONLY) f |= kFamHead;
    d->families = f ? f : kFamAll;
    if (e == hipSuccess) e = capture_decoder(d);
    return done(c, e, "Qwen decoder mode");
}

int fortai_hip_qwen35_batch_set_mode(fortai_hip_qwen35_batch *b, int flags) {
    if (!b || (flags & ~FORTAI_HIP_DECODER_DIRECT)) return FORTAI_HIP_INVALID;
    auto *c = b->context;
    (void)hipSetDevice(c->device);
    hipError_t e = hipStreamSynchronize(c->stream);
    b->use_graph = !(flags & FORTAI_HIP_DECODER_DIRECT);
    if (e == hipSuccess) e = capture_batch(b);
    return done(c, e, "Qwen batch mode");
}

int fortai_hip_qwen35_batch_set_prefill_mode(fortai_hip_qwen35_batch *b, int mode) {
    if (!b || mode < FORTAI_HIP_PREFILL_EXACT || mode > FORTAI_HIP_PREFILL_FAST) return FORTAI_HIP_INVALID;
    b->prefill_mode = static_cast<PrefillMode>(mode);
    return FORTAI_HIP_OK;
}

}  // extern "C"


