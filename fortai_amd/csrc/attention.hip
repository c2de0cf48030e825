// Gated GQA decode attention for gfx950 (per-op path): per-head RMSNorm of q
// and k, RoPE, the fp16 KV append, and the reference's two-pass softmax with
// its summation orders kept (attention_exact.h), so the output is
// bit-identical to the CPU path (fortai_qwen35_cpu.f90:990-1033).
//
// Two kernels: scores (one workgroup per kv head x 64 positions; the one
// that holds the new position also appends it) and output (one workgroup per
// head x 8 value dims: softmax weights, the P.V chains and the sigmoid gate).
#include "attention_exact.h"
#include "fortai_hip_internal.h"
#include "fortai_hip_kernels.h"

namespace fortai_hip {

namespace {

namespace ea = exact_attention;

constexpr int kMaxGroup = 4;
constexpr int kMaxHead = 256;
constexpr int kLoads = ea::kPosBlock * (kMaxHead / 8) / ea::kThreads;
constexpr int kQLoads = kMaxGroup * kMaxHead / ea::kThreads;

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kChunk = 256;  // positions per split-K chunk (long contexts)

// The per-sequence workspace behind AttentionParams::partial, in floats:
//   scores [heads][max_context] | e values [heads][max_context] |
//   Z tables [heads][z_segments(max_context)][kZStride] |
//   block statistics [heads][score blocks][2] (the scores kernel's per
//   64-position block max m_b and sum of exp(s - m_b), for the softmax's
//   estimates of the running sums)
__host__ __device__ inline int score_blocks(int max_context) { return (max_context + ea::kPosBlock - 1) / ea::kPosBlock; }
__host__ __device__ inline size_t workspace_floats(int heads, int max_context) {
    return static_cast<size_t>(heads) * max_context * 2 +
        static_cast<size_t>(heads) * ea::z_segments(max_context) * ea::kZStride +
        static_cast<size_t>(heads) * score_blocks(max_context) * 2;
}
__device__ __forceinline__ float2 *block_stats_of(const AttentionParams &p) {
    return reinterpret_cast<float2 *>(p.partial + static_cast<size_t>(p.heads) * p.max_context * 2 +
        static_cast<size_t>(p.heads) * ea::z_segments(p.max_context) * ea::kZStride);
}
__device__ __forceinline__ float *evals_of(const AttentionParams &p) {
    return p.partial + static_cast<size_t>(p.heads) * p.max_context;
}
__device__ __forceinline__ float *ztab_of(const AttentionParams &p) {
    return p.partial + static_cast<size_t>(p.heads) * p.max_context * 2;
}

// Sequence s of a batch (blockIdx.y): every per-sequence buffer is laid out
// [batch][...] with the single-sequence size, and position[s] is its own.
__device__ __forceinline__ AttentionParams attention_seq(AttentionParams p, int s) {
    const size_t nmax = (static_cast<size_t>(p.max_context) + kChunk - 1) / kChunk;
    p.q += static_cast<size_t>(s) * p.heads * 2 * p.head;
    p.k += static_cast<size_t>(s) * p.kv_heads * p.head;
    p.v += static_cast<size_t>(s) * p.kv_heads * p.value;
    p.kcache += static_cast<size_t>(s) * p.max_context * p.kv_heads * p.head;
    p.vcache += static_cast<size_t>(s) * p.max_context * p.kv_heads * p.value;
    p.partial += static_cast<size_t>(s) * workspace_floats(p.heads, p.max_context);
    p.cache_flags += static_cast<size_t>(s) * p.kv_heads;
    p.out += static_cast<size_t>(s) * p.heads * p.value;
    if (p.out_q8l) p.out_q8l = static_cast<unsigned char *>(p.out_q8l) + static_cast<size_t>(s) * q8l_bytes(p.heads * p.value);
    p.position += s;
    if (p.split) p.split += static_cast<size_t>(s) * p.heads * nmax * (p.value + 2);
    return p;
}

// Wave 0 of a workgroup holding 64 consecutive outputs (lane d: output
// h * value + d0 + d, 64-aligned): their Q8_0 quantization into p.out_q8l,
// the two blocks as the matvec's f32 prologue forms them (lane j of 16: the
// 4-value group j, fortai_q8_quantize's amax, scale and rounding).  lds: 64
// floats of the caller's LDS, free for this wave.
__device__ __forceinline__ void out_quantize64(const AttentionParams &p, int h, int d0, float val, float *lds) {
    const int lane = static_cast<int>(threadIdx.x) & 63;
    lds[lane] = val;
    wave_lds_fence();
    const float4 y = reinterpret_cast<const float4 *>(lds)[lane & 15];
    float scale;
    uint16_t bits;
    const uint32_t packed = quantize_group(y, scale, bits);
    if (lane < 16) {
        const int g = (h * p.value + d0) / 4 + lane, b = g >> 3, l = g & 7;
        unsigned char *base = static_cast<unsigned char *>(p.out_q8l);
        reinterpret_cast<uint32_t *>(base)[((b >> 2) * 8 + l) * 4 + (b & 3)] = packed;
        const int chunks = p.heads * p.value / 128;
        if (l == 0) reinterpret_cast<float *>(base + static_cast<size_t>(chunks) * 128)[b] = scale;
    }
}

__global__ __launch_bounds__(ea::kThreads) void attention_scores_kernel(const AttentionParams p_batch) {
    FORTAI_TRACE_SCOPE(3);
    const AttentionParams p = attention_seq(p_batch, static_cast<int>(blockIdx.y));
    __shared__ __align__(16) float qh[kMaxGroup * kMaxHead];
    __shared__ __align__(16) float kn[kMaxHead];
    __shared__ __align__(16) float2 rs[kMaxHead / 2];
    __shared__ __align__(16) uint16_t ktile[ea::kPosBlock][kMaxHead + 8];
    __shared__ int overflow;
    const int tid = static_cast<int>(threadIdx.x), wave = tid >> 6, lane = tid & 63;
    FORTAI_ATT_MARK(16);
    const int pos = *p.position;
    if (pos < 0 || pos >= p.max_context) return;  // never index past the cache
    const int positions = pos + 1, nblk_max = (p.max_context + ea::kPosBlock - 1) / ea::kPosBlock;
    // block-major: the blocks that hold positions are dispatched first, the
    // ones past the current position (which only read it and exit) last
    const int b = div(static_cast<int>(blockIdx.x), p.div_kv_heads);
    const int kvh = static_cast<int>(blockIdx.x) - b * p.kv_heads;
    const int p0 = b * ea::kPosBlock;
    if (p0 >= positions) return;
    const int n = min(ea::kPosBlock, positions - p0);
    const bool owns_new = pos >= p0 && pos < p0 + n;
    const int group = static_cast<int>(p.div_group.d), HD = p.head, VD = p.value, NKV = p.kv_heads;
    const int half = p.rope_dim / 2;

    // q, k, the norm weights, v and the rope entry first (indices clamped in
    // bounds), then the key rows: the loads complete in order, so the q/k
    // norms and RoPE run while the key rows (the only HBM stream of this
    // kernel) are still arriving
    float qv[kQLoads];
#pragma unroll
    for (int i = 0; i < kQLoads; ++i) {
        const int e = min(tid + i * ea::kThreads, group * HD - 1);
        const int eh = div(e, p.div_head);
        qv[i] = p.q[static_cast<size_t>(kvh * group + eh) * 2 * HD + (e - eh * HD)];
    }
    const int th = min(tid, HD - 1), tv = min(tid, VD - 1);
    const float knv = p.k[static_cast<size_t>(kvh) * HD + th];
    // the q and k norm weights a lane applies (elements lane + 64 j of a head)
    constexpr int kNW = kMaxHead / 64;
    float qwr[kNW], kwr[kNW];
#pragma unroll
    for (int j = 0; j < kNW; ++j) {
        qwr[j] = p.q_norm[min(lane + 64 * j, HD - 1)];
        kwr[j] = p.k_norm[min(lane + 64 * j, HD - 1)];
    }
    const float vnv = p.v[static_cast<size_t>(kvh) * VD + tv];
    const float2 rsv = half > 0 ? p.rope[static_cast<size_t>(pos) * half + min(tid, half - 1)] : make_float2(0.0f, 0.0f);
    const int flag = p.cache_flags[kvh];
    v4u kr[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int li = tid + i * ea::kThreads;
        const int jj = div(li, p.div_segs), sg = li - jj * static_cast<int>(p.div_segs.d);
        const int j = min(jj, n - 1);  // rows past n re-read row n-1 (in bounds)
        kr[i] = reinterpret_cast<const v4u *>(p.kcache + (static_cast<size_t>(p0 + j) * NKV + kvh) * HD)[sg];
    }
#pragma unroll
    for (int i = 0; i < kQLoads; ++i)
        if (tid + i * ea::kThreads < group * HD) qh[tid + i * ea::kThreads] = qv[i];
    if (tid < HD) kn[tid] = knv;
    if (tid < half) rs[tid] = rsv;
    if (tid == 0) overflow = 0;
    FORTAI_ATT_MARK(17);
    __syncthreads();
    for (int sl = wave; sl < group + (owns_new ? 1 : 0); sl += ea::kThreads / 64) {
        if (sl < group) ea::norm_rope_regs(qh + sl * HD, HD, qwr, p.eps, rs, p.rope_dim, lane);
        else ea::norm_rope_regs(kn, HD, kwr, p.eps, rs, p.rope_dim, lane);
    }
    FORTAI_ATT_MARK(18);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int li = tid + i * ea::kThreads;
        const int j = div(li, p.div_segs), sg = li - j * static_cast<int>(p.div_segs.d);
        if (j < n) *reinterpret_cast<v4u *>(&ktile[j][sg * 8]) = kr[i];
    }
    __syncthreads();
    FORTAI_ATT_MARK(19);
    if (owns_new) {
        // append at pos (fortai_qwen35_cpu.f90:1594-1601)
        if (tid < HD) {
            const uint16_t kb = float_to_half_kv(kn[tid]);
            p.kcache[(static_cast<size_t>(pos) * NKV + kvh) * HD + tid] = kb;
            ktile[pos - p0][tid] = kb;
            if ((kb & 0x7c00u) == 0x7c00u) overflow = 1;
        }
        if (tid < VD) {
            const uint16_t vb = float_to_half_kv(vnv);
            p.vcache[(static_cast<size_t>(pos) * NKV + kvh) * VD + tid] = vb;
            if ((vb & 0x7c00u) == 0x7c00u) overflow = 1;
        }
        __syncthreads();
        if (tid == 0 && overflow) p.cache_flags[kvh] = 1;
    }
    const bool finite = flag == 0 && overflow == 0;
    const float sqrt_head = sqrtf(static_cast<float>(HD));
    const int gi = tid >> 6, j = tid & 63;
    if (gi < group) {  // wave gi: head kvh * group + gi, positions p0 + lane
        constexpr float kLowest = -3.402823466e38f;  // -huge(1.0_real32)
        float sc = kLowest;
        if (j < n) {
            const float *qg = qh + gi * HD;
            const uint16_t *kr = &ktile[j][0];
            if (finite) sc = HD == 256 ? ea::score_n<true, 256>(qg, kr, sqrt_head) : ea::score<true>(qg, kr, HD, sqrt_head);
            else sc = ea::score<false>(qg, kr, HD, sqrt_head);
            p.partial[static_cast<size_t>(kvh * group + gi) * p.max_context + p0 + j] = sc;
        }
        // the block's max and sum of exp(s - max) (a fast exp, in double): the
        // softmax kernel's estimates start from these, not from every score
        const float mb = wave_max(sc);
        double t = j < n ? static_cast<double>(__expf(sc - mb)) : 0.0;
        t = wave_sum(t);
        if (j == 0)
            block_stats_of(p)[static_cast<size_t>(kvh * group + gi) * score_blocks(p.max_context) + b] =
                make_float2(mb, static_cast<float>(t));
    }
    FORTAI_ATT_MARK(20);
}

// e_p = expf(s_p - m) of kSeg-position segments of one head, stored for the
// output kernels, and each segment's Z candidate table (attention_exact.h,
// resolve_z): thread c runs the segment's left-to-right chain from candidate
// starting sum c.  grid (heads x G, batch): workgroup (k0, h) takes segments
// k0, k0 + G, ... of head h (G = z_segments(max_context) for one sequence, so
// one segment each; at most 8 for a batch, so that at a short position in a
// long cache few workgroups load the scores and exit idle), segments holding
// positions dispatched first.
__global__ __launch_bounds__(ea::kThreads) void attention_softmax_kernel(const AttentionParams p_batch) {
    FORTAI_TRACE_SCOPE(4);
    const AttentionParams p = attention_seq(p_batch, static_cast<int>(blockIdx.y));
    __shared__ __align__(16) float e_seg[ea::kSeg];
    __shared__ double dred[2 * ea::kWaves];
    __shared__ float fred[ea::kWaves];
    __shared__ MathTables mt;  // loaded after the scores are issued (the wait for it is theirs)
    static_assert(ea::kZCand == ea::kThreads && ea::kSeg == ea::kThreads, "one candidate and one position per thread");
    const int pos = *p.position;
    const int k0 = div(static_cast<int>(blockIdx.x), p.div_heads), h = static_cast<int>(blockIdx.x) - k0 * p.heads;
    const int G = div(static_cast<int>(gridDim.x), p.div_heads);
    const int tid = static_cast<int>(threadIdx.x), wave = tid >> 6, lane = tid & 63;
    const float *sc = p.partial + static_cast<size_t>(h) * p.max_context;
    FORTAI_ATT_MARK(21);
    // the statistics of every 64-position score block (max m_b, sum of
    // exp(s - m_b)) written by the scores kernel: one block per thread and
    // register up to kStatRegs * 256 blocks (clamped in bounds; those past the
    // position are masked), and the first segment's own scores
    constexpr int kStatRegs = 2;
    const int cap = p.max_context < p.exact_max ? p.max_context : p.exact_max;
    const int nb_cap = score_blocks(cap);
    const float2 *bst = block_stats_of(p) + static_cast<size_t>(h) * score_blocks(p.max_context);
    float2 st[kStatRegs];
#pragma unroll
    for (int i = 0; i < kStatRegs; ++i)
        if (i * ea::kThreads < nb_cap) st[i] = bst[min(tid + i * ea::kThreads, nb_cap - 1)];
    const float sv0 = sc[min(k0 * ea::kSeg + tid, cap - 1)];
    mt.load();  // visible after the barrier of the max below
    if (pos < 0 || pos >= p.max_context) return;
    const int n = pos + 1;
    if (n > p.exact_max) return;  // the split-K kernels cover this position
    if (k0 * ea::kSeg >= n) return;
    const int nb = score_blocks(n);
    // m = max over every score = max over the blocks' maxima (any order and
    // grouping gives the same value)
    constexpr float kLowest = -3.402823466e38f;  // -huge(1.0_real32)
    float m = kLowest;
#pragma unroll
    for (int i = 0; i < kStatRegs; ++i)
        if (tid + i * ea::kThreads < nb) m = fmaxf(m, st[i].x);
    for (int b = tid + kStatRegs * ea::kThreads; b < nb; b += ea::kThreads) m = fmaxf(m, bst[b].x);
    m = wave_max(m);
    if (lane == 0) fred[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(fred[0], fred[1]), fmaxf(fred[2], fred[3]));
    // block b's share of the running sum, rescaled to m (a fast exp, in double)
    double tb[kStatRegs];
#pragma unroll
    for (int i = 0; i < kStatRegs; ++i) {
        const int b = tid + i * ea::kThreads;
        tb[i] = b < nb ? static_cast<double>(st[i].y) * static_cast<double>(__expf(st[i].x - m)) : 0.0;
    }
    FORTAI_ATT_MARK(22);
    for (int k = k0; k * ea::kSeg < n; k += G) {
    if (k != k0) __syncthreads();  // the previous segment's chains have read e_seg and dred
    const int p0 = k * ea::kSeg;
    const int cnt = min(ea::kSeg, n - p0);
    // the segment's own e values, exactly as the reference computes them
    const float sv = k == k0 ? sv0 : sc[min(p0 + tid, n - 1)];
    const float e = tid < cnt ? mt.expf(sv - m) : -0.0f;  // -0 leaves a sum unchanged
    e_seg[tid] = e;
    if (tid < cnt) evals_of(p)[static_cast<size_t>(h) * p.max_context + p0 + tid] = e;
    // the estimates of the running sums entering this segment and the next:
    // the blocks before it, and those before the next one (the next
    // segment's workgroup forms the same sum in the same order)
    const int b_in = p0 / ea::kPosBlock, b_next = (p0 + ea::kSeg) / ea::kPosBlock;
    double est = 0.0, est_next = 0.0;
#pragma unroll
    for (int i = 0; i < kStatRegs; ++i) {
        const int b = tid + i * ea::kThreads;
        if (b < b_in) est += tb[i];
        if (b < b_next) est_next += tb[i];
    }
    for (int b = tid + kStatRegs * ea::kThreads; b < nb && b < b_next; b += ea::kThreads) {
        const float2 sb = bst[b];
        const double t = static_cast<double>(sb.y) * static_cast<double>(__expf(sb.x - m));
        if (b < b_in) est += t;
        est_next += t;
    }
    est = wave_sum(est);
    est_next = wave_sum(est_next);
    if (lane == 0) {
        dred[wave] = est;
        dred[ea::kWaves + wave] = est_next;
    }
    __syncthreads();
    est = (dred[0] + dred[1]) + (dred[2] + dred[3]);
    est_next = (dred[4] + dred[5]) + (dred[6] + dred[7]);
    if (k == k0) FORTAI_ATT_MARK(23);
    const uint32_t skew = static_cast<uint32_t>(p.z_skew);
    const uint32_t centre = k == 0 ? 0u : __float_as_uint(static_cast<float>(est)) + skew;
    const uint32_t centre_next = __float_as_uint(static_cast<float>(est_next)) + skew;
    float acc = k == 0 ? 0.0f : __uint_as_float(centre + static_cast<uint32_t>(tid) - ea::kZCand / 2);
#pragma unroll 16
    for (int j = 0; j < ea::kSeg; j += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(e_seg + j);
        acc = acc + v.x;
        acc = acc + v.y;
        acc = acc + v.z;
        acc = acc + v.w;
    }
    if (k == k0) FORTAI_ATT_MARK(24);
    const bool last = p0 + ea::kSeg >= n;
    float *tab = ztab_of(p) + (static_cast<size_t>(h) * ea::z_segments(p.max_context) + k) * ea::kZStride;
    tab[tid] = acc;
    tab[ea::kZNext + tid] = last ? acc : __int_as_float(ea::z_index(acc, centre_next));
    if (tid == 0) tab[ea::kZCentre] = __uint_as_float(centre);
    }
    FORTAI_ATT_MARK(25);
}

// Z of head h: the walk words of the candidate tables into LDS (up to
// kZLdsSegments segments; longer contexts walk in global memory), then
// resolve_z by one thread.  walk_lds: min(z_segments(n), kZLdsSegments) *
// kZCand words.  Returns Z in every thread.
constexpr int kZLdsSegments = 32;
__host__ __device__ inline int z_lds_segments(int positions) {
    return ea::z_segments(positions) < kZLdsSegments ? ea::z_segments(positions) : kZLdsSegments;
}
__device__ __forceinline__ const float *head_tab(const AttentionParams &p, int h) {
    return ztab_of(p) + static_cast<size_t>(h) * ea::z_segments(p.max_context) * ea::kZStride;
}
__device__ __forceinline__ float head_z(const AttentionParams &p, int h, int n, int32_t *walk_lds, float *slot) {
    const int tid = static_cast<int>(threadIdx.x);
    const int nseg = (n + ea::kSeg - 1) / ea::kSeg;
    const float *tab = head_tab(p, h);
    if (nseg <= kZLdsSegments) {
        for (int i = tid; i < nseg * ea::kZCand; i += ea::kThreads)
            walk_lds[i] = __float_as_int(tab[static_cast<size_t>(i / ea::kZCand) * ea::kZStride + ea::kZNext + i % ea::kZCand]);
    }
    __syncthreads();
    if (tid == 0) {
        const float *ev = evals_of(p) + static_cast<size_t>(h) * p.max_context;
        *slot = nseg <= kZLdsSegments
            ? ea::resolve_z(walk_lds, ea::kZCand, tab, ev, n)
            : ea::resolve_z(reinterpret_cast<const int32_t *>(tab + ea::kZNext), ea::kZStride, tab, ev, n);
    }
    __syncthreads();
    return *slot;
}

// The output of one head x kDims value dims.  Workgroups are numbered so
// that the ones reading the same 128-byte value lines (the 64 dims of a kv
// head that 8 slices x the GQA group share) are consecutive on one XCD
// (workgroup b runs on XCD b % 8).  Every load that does not depend on the
// position (the first value pieces, e values and the Z tables, all clamped to
// the cache) is issued together with the position's, in one round trip.
constexpr int kTabRegs = kZLdsSegments * ea::kZCand / ea::kThreads;  // walk words per thread
__global__ __launch_bounds__(ea::kThreads) void attention_output_kernel(const AttentionParams p_batch) {
    FORTAI_TRACE_SCOPE(5);
    const AttentionParams p = attention_seq(p_batch, static_cast<int>(blockIdx.y));
    extern __shared__ __align__(16) float lds[];
    // sigmoid of the gate: wave 1 forms it while thread 0 resolves Z
    __shared__ float gate_sig[ea::kDims];
    const int tid = static_cast<int>(threadIdx.x);
    FORTAI_ATT_MARK(0);
    const int pos = *p.position;
    const int group = static_cast<int>(p.div_group.d), HD = p.head, VD = p.value, NKV = p.kv_heads;
    const int slices = static_cast<int>(p.div_slices.d), nwg = p.heads * slices;
    const int b = static_cast<int>(blockIdx.x);
    int h, d0;
    if (nwg % 8 == 0 && VD % 64 == 0) {
        const int i = (b % 8) * (nwg / 8) + b / 8;  // logical index, consecutive on one XCD
        const int i8 = i / 8, sl = i % 8;
        const int t = div(i8, p.div_group), g = i8 - t * group;
        const int kvh = div(t, p.div_vd64), lg = t - kvh * static_cast<int>(p.div_vd64.d);
        h = kvh * group + g;
        d0 = (lg * 8 + sl) * ea::kDims;
    } else {
        h = div(b, p.div_slices);
        d0 = (b - h * slices) * ea::kDims;
    }
    const int kvh = div(h, p.div_group);
    const int cap = p.max_context < p.exact_max ? p.max_context : p.exact_max;  // positions this kernel serves
    const uint16_t *vbase = p.vcache + static_cast<size_t>(kvh) * VD + d0;
    const size_t vstride = static_cast<size_t>(NKV) * VD;
    const float *ev = evals_of(p) + static_cast<size_t>(h) * p.max_context;
    const float *tab = head_tab(p, h);
    const int rows = z_lds_segments(cap);
    ea::ValuePieces v;
    float e4[ea::kPieces];
    int32_t tr[kTabRegs];  // walk word tid of segment r
    ea::value_prefetch(vbase, vstride, p.max_context, v);
    ea::e_prefetch(ev, p.max_context, e4);
    static_assert(ea::kZCand == ea::kThreads, "one walk word per thread and segment");
    // unconditional loads (a branch around each would make the compiler wait
    // for it): rows past the cached ones re-read the last (row 0 always exists)
    const int last_row = max(rows, 1) - 1;
#pragma unroll
    for (int r = 0; r < kTabRegs; ++r)
        tr[r] = __float_as_int(tab[static_cast<size_t>(min(r, last_row)) * ea::kZStride + ea::kZNext + tid]);
    const float gate = p.q[static_cast<size_t>(h) * 2 * HD + HD + d0 + (tid & (ea::kDims - 1))];
    const int flag = p.cache_flags[kvh];
    FORTAI_ATT_MARK(3);
    if (pos < 0 || pos >= p.max_context) return;
    const int positions = pos + 1;
    if (positions > p.exact_max) return;  // the split-K kernels cover this position
    float *work = lds;
    int32_t *walk_lds = reinterpret_cast<int32_t *>(lds + ea::work_floats());
    const int nseg = ea::z_segments(positions);
    if (nseg <= kZLdsSegments) {
#pragma unroll
        for (int r = 0; r < kTabRegs; ++r)
            if (r < nseg) walk_lds[r * ea::kZCand + tid] = tr[r];
    }
    __syncthreads();
    FORTAI_ATT_MARK(1);
    if (tid == 0)
        work[0] = nseg <= kZLdsSegments
            ? ea::resolve_z(walk_lds, ea::kZCand, tab, ev, positions)
            : ea::resolve_z(reinterpret_cast<const int32_t *>(tab + ea::kZNext), ea::kZStride, tab, ev, positions);
    // (glibc's algorithm with its table in constant memory: one lookup, off
    // the critical path; seen by wave 0 after the output step's barriers)
    if (tid >= 64 && tid < 64 + ea::kDims) gate_sig[tid - 64] = sigmoid_ref(gate);
    FORTAI_ATT_MARK(2);
    __syncthreads();
    const float z = work[0];
    FORTAI_ATT_MARK(5);
    const float acc = flag == 0 ? ea::attend_given_z<true>(ev, z, positions, vbase, vstride, work, v, e4)
                                : ea::attend_given_z<false>(ev, z, positions, vbase, vstride, work, v, e4);
    if (tid < ea::kDims) p.out[static_cast<size_t>(h) * VD + d0 + tid] = acc * gate_sig[tid];
    FORTAI_ATT_MARK(4);
}

size_t output_lds_bytes(int positions) {
    return (ea::work_floats() + static_cast<size_t>(z_lds_segments(positions)) * ea::kZCand) * sizeof(float);
}

// ------------------------------------------------------- exact, batches
// The same arithmetic as attention_output_kernel (the reference's two-pass
// softmax and P.V with its summation orders, fortai_qwen35_cpu.f90:1016-1031)
// with one workgroup per (head, 64 value dims, sequence) instead of one per
// (head, 8 value dims): Z from the candidate tables (head_z), then lane d of
// wave 0 runs the P.V chain of value dim d0 + d over the positions in order,
// out_d = fl(w_0 v_0,d) + fl(w_1 v_1,d) + ... with w_p = e_p / Z.  A batch has
// many (head, sequence) pairs, so this fills the chip with 1/8 as many
// workgroups, each chain step using all 64 lanes; a single sequence keeps the
// per-slice kernel, whose chains are shorter per workgroup.
//
// Values reach LDS in tiles of kWideTile positions, loaded by all four waves
// two tiles ahead of the chain: each thread loads 8 positions x 8 dims (eight
// 16-byte pieces), transposes them in registers and stores one 16-byte row
// of 8 positions per dim, so the tile is [dim][position] and a chain lane
// reads 8 positions of its dim with one 16-byte LDS read (and w_p of the tile,
// divided when the tile is stored, with two).  Row R (dim R) keeps its group g
// of 8 positions at column g + 2 (R / 16): with a row pitch of 49 16-byte bank
// groups (1 mod 16), the 16 lanes of a store pass (8 rows 8 apart, two column
// groups) and of a read pass (16 consecutive rows, one group) all fall on
// different banks.  The Z walk words use the tile's LDS before the first tile
// is stored; nothing is sized by the context.
constexpr int kWideTile = 256;                   // positions per value tile
constexpr int kWideDims = 64;                    // value dims per workgroup
constexpr int kWidePitchT = 392;                 // halves per LDS row: 32 + 6 column groups, 49 x 16 bytes
constexpr int kWideMaxPositions = 8192;
static_assert(kWideTile / 8 * (kWideDims / 8) == ea::kThreads, "one 8 x 8 block of (position, dim) per thread");
static_assert(kWidePitchT >= (kWideTile / 8 + 2 * (kWideDims / 16 - 1)) * 8 && kWidePitchT % 8 == 0 &&
    (kWidePitchT / 8) % 16 == 1, "every shifted column in the row; 16-byte rows one bank group apart");
static_assert(kWideDims * kWidePitchT * 2 >= kZLdsSegments * ea::kZCand * 4, "the Z walk words fit the tile's LDS");

// dynamic LDS of attention_output_wide_kernel: the transposed tile, then w of the tile
constexpr size_t kWideLdsBytes = static_cast<size_t>(kWideDims) * kWidePitchT * 2 + kWideTile * 4;

// halves k of dwords a (low half of the result) and b (high half)
__device__ __forceinline__ uint32_t pick_halves(uint32_t a, uint32_t b, int hi) {
    return hi ? __builtin_amdgcn_perm(b, a, 0x07060302u) : __builtin_amdgcn_perm(b, a, 0x05040100u);
}

template <bool FINITE>
__device__ __forceinline__ void attend_wide(const AttentionParams &p, int h, int d0, int n, uint16_t *vt, float *wt,
    float *red) {
    const int tid = static_cast<int>(threadIdx.x), wave = tid >> 6, lane = tid & 63;
    const int group = p.heads / p.kv_heads, HD = p.head, VD = p.value, NKV = p.kv_heads;
    const int kvh = h / group;
    const uint16_t *vb = p.vcache + static_cast<size_t>(kvh) * VD + d0;
    const size_t vs = static_cast<size_t>(NKV) * VD;
    const int tiles = (n + kWideTile - 1) / kWideTile;
    const float *ev = evals_of(p) + static_cast<size_t>(h) * p.max_context;
    // this thread's block: positions pg * 8 .. + 7 of a tile, dims pc * 8 .. + 7
    const int pc = tid & 7, pg = tid >> 3;
    const int pcl = min(pc, (min(kWideDims, VD - d0) >> 3) - 1);  // dims past VD re-read the last piece
    FORTAI_ATTW_MARK(0);
    // tile t: eight 16-byte pieces and e of position t * kWideTile + tid (all clamped to the last position)
    auto fetch = [&](int t, uint4 (&regs)[8], float &e) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int pp = min(t * kWideTile + pg * 8 + i, n - 1);
            regs[i] = *reinterpret_cast<const uint4 *>(vb + static_cast<size_t>(pp) * vs + pcl * 8);
        }
        e = ev[min(t * kWideTile + tid, n - 1)];
    };
    // Z first: its table loads would otherwise return after the whole value
    // fetch (loads complete in order)
    const float z = head_z(p, h, n, reinterpret_cast<int32_t *>(vt), red + 4);  // ends with a barrier
    FORTAI_ATTW_MARK(3);
    uint4 ra[8], rb[8];
    float ea_ = 0.0f, eb_ = 0.0f;
    fetch(0, ra, ea_);
    if (tiles > 1) fetch(1, rb, eb_);
    FORTAI_ATTW_MARK(1);
    // the block transposed: row of dim pc * 8 + k holds positions pg * 8 .. + 7
    auto stash = [&](const uint4 (&r)[8], float e) {
        const uint32_t *w32 = reinterpret_cast<const uint32_t *>(r);  // w32[4 i + m]: dims 2m, 2m + 1 of position i
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int m = k >> 1, hi = k & 1;
            uint4 row;
            row.x = pick_halves(w32[0 * 4 + m], w32[1 * 4 + m], hi);
            row.y = pick_halves(w32[2 * 4 + m], w32[3 * 4 + m], hi);
            row.z = pick_halves(w32[4 * 4 + m], w32[5 * 4 + m], hi);
            row.w = pick_halves(w32[6 * 4 + m], w32[7 * 4 + m], hi);
            *reinterpret_cast<uint4 *>(vt + (pc * 8 + k) * kWidePitchT + (pg + 2 * (pc >> 1)) * 8) = row;
        }
        wt[tid] = e / z;
    };
    const int d = d0 + lane;
    // this lane's row from its shifted column 0 (lanes past VD read a row they do not write)
    const uint16_t *myrow = vt + lane * kWidePitchT + 2 * (lane >> 4) * 8;
    // the chain of one tile: groups of 8 positions from a ring of three
    // register sets, each group's LDS reads issued two groups before its adds
    struct Grp {
        uint4 v;
        float4 w0, w1;
    };
    // group g of the tile (a compile-time index: immediate LDS offsets)
    auto ld = [&](int g, Grp &r) {
        r.v = *reinterpret_cast<const uint4 *>(myrow + g * 8);
        r.w0 = *reinterpret_cast<const float4 *>(wt + g * 8);
        r.w1 = *reinterpret_cast<const float4 *>(wt + g * 8 + 4);
    };
    auto add8 = [&](const Grp &r, float acc) {
        if constexpr (FINITE) {
            // fl(w * f32(v)) in one instruction (exact widening, one rounding)
            acc = acc + half_times<false>(r.v.x, r.w0.x);
            acc = acc + half_times<true>(r.v.x, r.w0.y);
            acc = acc + half_times<false>(r.v.y, r.w0.z);
            acc = acc + half_times<true>(r.v.y, r.w0.w);
            acc = acc + half_times<false>(r.v.z, r.w1.x);
            acc = acc + half_times<true>(r.v.z, r.w1.y);
            acc = acc + half_times<false>(r.v.w, r.w1.z);
            acc = acc + half_times<true>(r.v.w, r.w1.w);
        } else {
            const uint32_t q[4] = {r.v.x, r.v.y, r.v.z, r.v.w};
            const float wv[8] = {r.w0.x, r.w0.y, r.w0.z, r.w0.w, r.w1.x, r.w1.y, r.w1.z, r.w1.w};
#pragma unroll
            for (int k = 0; k < 8; ++k)
                acc = acc + wv[k] * ea::kv<false>(static_cast<uint16_t>(q[k >> 1] >> (16 * (k & 1))));
        }
        return acc;
    };
    auto chain = [&](int t, float acc) {
        const int cnt = min(kWideTile, n - t * kWideTile);
        const int full = cnt >> 3;
        constexpr int kGroups = kWideTile / 8;
        Grp ring[3];
        ld(0, ring[0]);
        ld(1, ring[1]);
        // fully unrolled: every LDS offset is an immediate, and the scheduling
        // barriers keep each group's reads two groups ahead of its adds
#pragma unroll
        for (int g = 0; g < kGroups; ++g) {
            if (g < full) {  // uniform
                if (g + 2 < kGroups) ld(g + 2, ring[(g + 2) % 3]);
                __builtin_amdgcn_sched_barrier(0);
                acc = add8(ring[g % 3], acc);
            }
        }
        // the last cnt % 8 positions
        for (int k = 0; k < (cnt & 7); ++k) {
            const int pp = full * 8 + k;
            acc = acc + wt[pp] * ea::kv<FINITE>(myrow[pp]);
        }
        return acc;
    };
    float acc = 0.0f;
    for (int t = 0; t < tiles; t += 2) {
        stash(ra, ea_);
        __syncthreads();
        if (t + 2 < tiles) fetch(t + 2, ra, ea_);
        if (wave == 0) acc = chain(t, acc);
        __syncthreads();
        if (t + 1 >= tiles) break;
        stash(rb, eb_);
        __syncthreads();
        if (t + 3 < tiles) fetch(t + 3, rb, eb_);
        if (wave == 0) acc = chain(t + 1, acc);
        __syncthreads();
    }
    FORTAI_ATTW_MARK(5);
    if (wave == 0 && d < VD) {
        const float gate = p.q[static_cast<size_t>(h) * 2 * HD + HD + d];
        const float o = acc * sigmoid_ref(gate);
        p.out[static_cast<size_t>(h) * VD + d] = o;
        if (p.out_q8l) out_quantize64(p, h, d0, o, wt);  // (the tile is consumed: wt is free)
    }
}

// grid: (heads x ceil(value / 64), batch)
__global__ __launch_bounds__(ea::kThreads) void attention_output_wide_kernel(const AttentionParams p_batch) {
    FORTAI_TRACE_SCOPE(12);
    const AttentionParams p = attention_seq(p_batch, static_cast<int>(blockIdx.y));
    extern __shared__ __align__(16) float wide_lds[];
    __shared__ float red[8];
    const int pos = *p.position;
    if (pos < 0 || pos >= p.max_context) return;
    const int n = pos + 1;
    if (n > p.exact_max) return;  // the split-K kernels cover this position
    const int slices = (p.value + kWideDims - 1) / kWideDims;
    const int h = static_cast<int>(blockIdx.x) / slices, d0 = (static_cast<int>(blockIdx.x) % slices) * kWideDims;
    const int kvh = h / (p.heads / p.kv_heads);
    uint16_t *vt = reinterpret_cast<uint16_t *>(wide_lds);
    float *wt = wide_lds + kWideDims * kWidePitchT / 2;
    if (p.cache_flags[kvh] == 0)
        attend_wide<true>(p, h, d0, n, vt, wt, red);
    else
        attend_wide<false>(p, h, d0, n, vt, wt, red);
}


// ---------------------------------------------------------------- split-K
// Beyond exact_max positions: each workgroup takes one kv head and a chunk of
// kChunk positions for the whole GQA group: the chunk's max m_c, Z_c =
// sum exp(s - m_c) and o_c = sum exp(s - m_c) v, which the merge kernel
// combines per head: M = max m_c, Z = sum Z_c e^(m_c - M),
// out = (sum o_c e^(m_c - M)) / Z * sigmoid(gate) (flash-decoding).  The
// scores are the scores kernel's (the reference's per-position dots).

__device__ __forceinline__ float block_max256(float v, float *red) {
    v = wave_max(v);
    const int tid = static_cast<int>(threadIdx.x);
    __syncthreads();
    if ((tid & 63) == 0) red[tid >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ __forceinline__ float block_sum256(float v, float *red) {
    v = wave_sum(v);
    const int tid = static_cast<int>(threadIdx.x);
    __syncthreads();
    if ((tid & 63) == 0) red[tid >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// Per-workgroup split-K partials of one kv head and chunk for the GQA group.
// Thread t takes the 8-dim value slice t % 32 of positions t / 32 + 8 i (all
// 32 of its 16-byte value loads in flight at once), then the 8 position
// groups are summed through LDS.
constexpr int kSplitSlices = 32;                    // 8-dim slices: value dims <= 256
constexpr int kSplitGroups = 256 / kSplitSlices;    // position groups
constexpr int kSplitPer = kChunk / kSplitGroups;    // positions per thread
static_assert(kChunk <= 256 && kChunk % kSplitGroups == 0, "one score per thread; whole position groups");

struct SplitLds {
    float e[kMaxGroup][kChunk];
    float red4[kMaxGroup][4];
    float part[kMaxGroup][kSplitGroups][kSplitSlices * 8];
};

template <bool FINITE>
__device__ __forceinline__ void split_chunk(const AttentionParams &p, int kvh, int c, int nmax, int p0, int n,
    SplitLds &L) {
    const int tid = static_cast<int>(threadIdx.x);
    const int group = p.heads / p.kv_heads, VD = p.value, NKV = p.kv_heads;
    const int slice = tid % kSplitSlices, pg = tid / kSplitSlices;
    // the scores of every head, then the value loads (the in-order wait for
    // the scores then does not include the values)
    float sc[kMaxGroup], m[kMaxGroup], z[kMaxGroup];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g)
        sc[g] = g < group ? p.partial[static_cast<size_t>(kvh * group + g) * p.max_context + p0 + min(tid, n - 1)]
                          : 0.0f;
    // slices past VD re-read slice 0
    const int d0 = (slice * 8 < VD ? slice : 0) * 8;
    const uint16_t *vb = p.vcache + (static_cast<size_t>(p0) * NKV + kvh) * VD + d0;
    const size_t vs = static_cast<size_t>(NKV) * VD;
    uint4 vv[kSplitPer];
#pragma unroll
    for (int i = 0; i < kSplitPer; ++i)
        vv[i] = *reinterpret_cast<const uint4 *>(vb + static_cast<size_t>(min(pg + kSplitGroups * i, n - 1)) * vs);
    FORTAI_ATT_MARK(12);
    // the four heads' max and sum, reduced together
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
        m[g] = tid < n ? sc[g] : -__builtin_inff();
        m[g] = wave_max(m[g]);
    }
    if ((tid & 63) == 0)
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) L.red4[g][tid >> 6] = m[g];
    __syncthreads();
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
        m[g] = fmaxf(fmaxf(L.red4[g][0], L.red4[g][1]), fmaxf(L.red4[g][2], L.red4[g][3]));
        const float ev = (g < group && tid < n) ? expf_libm(sc[g] - m[g]) : 0.0f;
        if (tid < kChunk) L.e[g][tid] = ev;
        z[g] = ev;
        z[g] = wave_sum(z[g]);
    }
    __syncthreads();  // every wave has read red4
    if ((tid & 63) == 0)
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) L.red4[g][tid >> 6] = z[g];
    __syncthreads();
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) z[g] = (L.red4[g][0] + L.red4[g][1]) + (L.red4[g][2] + L.red4[g][3]);
    FORTAI_ATT_MARK(13);
    float acc[kMaxGroup][8];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g)
#pragma unroll
        for (int d = 0; d < 8; ++d) acc[g][d] = 0.0f;
#pragma unroll
    for (int i = 0; i < kSplitPer; ++i) {
        const int j = pg + kSplitGroups * i;
        if (j >= n) continue;
        const uint32_t hw[4] = {vv[i].x, vv[i].y, vv[i].z, vv[i].w};
        float v8[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            v8[2 * q] = ea::kv<FINITE>(static_cast<uint16_t>(hw[q] & 0xffffu));
            v8[2 * q + 1] = ea::kv<FINITE>(static_cast<uint16_t>(hw[q] >> 16));
        }
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) {
            if (g >= group) break;
            const float ej = L.e[g][j];
#pragma unroll
            for (int d = 0; d < 8; ++d) acc[g][d] = __builtin_fmaf(ej, v8[d], acc[g][d]);
        }
    }
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
        if (g >= group) break;
#pragma unroll
        for (int d = 0; d < 8; ++d) L.part[g][pg][slice * 8 + d] = acc[g][d];
    }
    __syncthreads();
    FORTAI_ATT_MARK(14);
    if (tid >= VD) return;
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
        if (g >= group) break;
        float o = 0.0f;
#pragma unroll
        for (int k = 0; k < kSplitGroups; ++k) o += L.part[g][k][tid];
        float *dst = p.split + (static_cast<size_t>(kvh * group + g) * nmax + c) * (VD + 2);
        dst[tid] = o;
        if (tid == 0) {
            dst[VD] = m[g];
            dst[VD + 1] = z[g];
        }
    }
}

__global__ __launch_bounds__(ea::kThreads) void attention_split_kernel(const AttentionParams p_batch) {
    const AttentionParams p = attention_seq(p_batch, static_cast<int>(blockIdx.y));
    __shared__ SplitLds L;
    const int pos = *p.position;
    if (pos < 0 || pos >= p.max_context) return;
    const int positions = pos + 1;
    if (positions <= p.exact_max) return;  // the exact kernel covers this position
    const int nmax = (p.max_context + kChunk - 1) / kChunk;
    // chunk-major, like the scores kernel: chunks holding positions dispatch first
    const int kvh = static_cast<int>(blockIdx.x) % p.kv_heads, c = static_cast<int>(blockIdx.x) / p.kv_heads;
    const int p0 = c * kChunk;
    if (p0 >= positions) return;
    const int n = min(kChunk, positions - p0);
    if (p.cache_flags[kvh] == 0) split_chunk<true>(p, kvh, c, nmax, p0, n, L);
    else split_chunk<false>(p, kvh, c, nmax, p0, n, L);
}

// Per head and 64 value dims: the chunks' scale factors e^(m_c - M) once into
// LDS, then each dim's chunk partials summed by four threads (a quarter of the
// chunks each, 32 loads in flight) and combined through LDS.
constexpr int kMaxSplitChunks = 4096;  // contexts up to 1M positions
constexpr int kMergeDims = 64;
constexpr int kMergeParts = ea::kThreads / kMergeDims;
constexpr int kMergeBatch = 32;

__global__ __launch_bounds__(ea::kThreads) void attention_merge_kernel(const AttentionParams p_batch) {
    const AttentionParams p = attention_seq(p_batch, static_cast<int>(blockIdx.y));
    __shared__ float f[kMaxSplitChunks];
    __shared__ float red[4];
    __shared__ float part[kMergeParts][kMergeDims];
    const int pos = *p.position;
    if (pos < 0 || pos >= p.max_context) return;
    const int positions = pos + 1;
    if (positions <= p.exact_max) return;
    const int tid = static_cast<int>(threadIdx.x);
    const int VD = p.value, HD = p.head;
    const int slices = (VD + kMergeDims - 1) / kMergeDims;
    const int h = static_cast<int>(blockIdx.x) / slices, d0 = (static_cast<int>(blockIdx.x) % slices) * kMergeDims;
    const int nmax = (p.max_context + kChunk - 1) / kChunk, chunks = (positions + kChunk - 1) / kChunk;
    const float *base = p.split + static_cast<size_t>(h) * nmax * (VD + 2);
    float mx = -__builtin_inff();
    for (int c = tid; c < chunks; c += ea::kThreads) mx = fmaxf(mx, base[static_cast<size_t>(c) * (VD + 2) + VD]);
    mx = block_max256(mx, red);
    float zp = 0.0f;
    for (int c = tid; c < chunks; c += ea::kThreads) {
        const float *row = base + static_cast<size_t>(c) * (VD + 2);
        const float fc = expf_libm(row[VD] - mx);
        f[c] = fc;
        zp = __builtin_fmaf(row[VD + 1], fc, zp);
    }
    const float z = block_sum256(zp, red);  // (its barriers also publish f)
    const int dl = tid % kMergeDims, q = tid / kMergeDims, d = min(d0 + dl, VD - 1);
    const int per = (chunks + kMergeParts - 1) / kMergeParts, c0 = q * per, c1 = min(chunks, c0 + per);
    float o = 0.0f;
    for (int cb = c0; cb < c1; cb += kMergeBatch) {
        float x[kMergeBatch];
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) x[u] = base[static_cast<size_t>(min(cb + u, c1 - 1)) * (VD + 2) + d];
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u)
            if (cb + u < c1) o = __builtin_fmaf(x[u], f[cb + u], o);
    }
    part[q][dl] = o;
    __syncthreads();
    if (q != 0 || d0 + dl >= VD) return;
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < kMergeParts; ++k) sum += part[k][dl];
    const float gate = p.q[static_cast<size_t>(h) * 2 * HD + HD + d0 + dl];
    const float out = (sum / z) * sigmoid_ref(gate);
    p.out[static_cast<size_t>(h) * VD + d0 + dl] = out;
    if (p.out_q8l) out_quantize64(p, h, d0, out, &part[1][0]);  // (wave 0 has read part)
}

}  // namespace

size_t attention_scores_floats(int heads, int max_context) { return workspace_floats(heads, max_context); }

int attention_split_chunks(int max_context) { return (max_context + kChunk - 1) / kChunk; }

// workgroups per head of attention_softmax_kernel: one per segment for a
// single sequence, at most 8 (each looping over segments) for a batch
int softmax_groups(int positions, int batch) {
    const int segs = ea::z_segments(positions);
    return batch > 1 && segs > 8 ? 8 : segs;
}

bool attention_quantizes_output(const AttentionParams &p, int batch) {
    const int exact_positions = p.max_context < p.exact_max ? p.max_context : p.exact_max;
    const bool wide = (batch > 1 || p.force_wide) && exact_positions <= kWideMaxPositions && p.value <= ea::kThreads;
    return wide && p.value % 64 == 0 && (p.heads * p.value) % 128 == 0;
}

hipError_t launch_attention(const AttentionParams &params, hipStream_t stream, int batch) {
    if (batch < 1) return hipErrorInvalidValue;
    if (params.out_q8l && !attention_quantizes_output(params, batch)) return hipErrorInvalidValue;
    const int group = params.kv_heads > 0 ? params.heads / params.kv_heads : 0;
    AttentionParams p = params;
    p.div_heads = fast_div(static_cast<uint32_t>(p.heads));
    p.div_kv_heads = fast_div(static_cast<uint32_t>(p.kv_heads));
    p.div_group = fast_div(static_cast<uint32_t>(group));
    p.div_head = fast_div(static_cast<uint32_t>(p.head));
    p.div_segs = fast_div(static_cast<uint32_t>(p.head / 8));
    p.div_slices = fast_div(static_cast<uint32_t>(p.value / ea::kDims));
    p.div_vd64 = fast_div(static_cast<uint32_t>(p.value / 64));
    if (p.max_context > p.exact_max && (!p.split || attention_split_chunks(p.max_context) > kMaxSplitChunks))
        return hipErrorInvalidValue;
    if (group < 1 || group > kMaxGroup || p.heads % p.kv_heads || p.head > kMaxHead || p.head % 8 ||
        p.value % ea::kDims || p.value > p.head || p.rope_dim > p.head || p.rope_dim % 2 || !p.out || !p.partial)
        return hipErrorInvalidValue;
    const int exact_positions = p.max_context < p.exact_max ? p.max_context : p.exact_max;
    const int nblk_max = (p.max_context + ea::kPosBlock - 1) / ea::kPosBlock;
    hipLaunchKernelGGL(attention_scores_kernel, dim3(p.kv_heads * nblk_max, batch), dim3(ea::kThreads), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (exact_positions > 0) {
        hipLaunchKernelGGL(attention_softmax_kernel, dim3(p.heads * softmax_groups(exact_positions, batch), batch),
            dim3(ea::kThreads), 0, stream, p);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const bool wide = (batch > 1 || p.force_wide) && exact_positions <= kWideMaxPositions && p.value <= ea::kThreads;
    if (wide) {
        const size_t wlds = kWideLdsBytes;
        const int wgrid = p.heads * ((p.value + kWideDims - 1) / kWideDims);
        hipLaunchKernelGGL(attention_output_wide_kernel, dim3(wgrid, batch), dim3(ea::kThreads), wlds, stream, p);
        e = hipGetLastError();
        note_launch("attention_scores_kernel grid %dx%d + attention_softmax_kernel grid %dx%d + "
            "attention_output_wide_kernel grid %dx%d", p.kv_heads * nblk_max, batch,
            p.heads * softmax_groups(exact_positions, batch), batch, wgrid, batch);
    } else {
        hipLaunchKernelGGL(attention_output_kernel, dim3(p.heads * (p.value / ea::kDims), batch), dim3(ea::kThreads),
            output_lds_bytes(exact_positions), stream, p);
        e = hipGetLastError();
        note_launch("attention_scores_kernel grid %dx%d + attention_softmax_kernel grid %dx%d + "
            "attention_output_kernel grid %dx%d", p.kv_heads * nblk_max, batch,
            p.heads * softmax_groups(exact_positions, batch), batch, p.heads * (p.value / ea::kDims), batch);
    }
    if (e != hipSuccess || p.max_context <= p.exact_max) return e;
    // long contexts: the split-K pair (each kernel picks its regime from the device position)
    hipLaunchKernelGGL(attention_split_kernel, dim3(p.kv_heads * attention_split_chunks(p.max_context), batch),
        dim3(ea::kThreads), 0, stream, p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attention_merge_kernel, dim3(p.heads * ((p.value + kMergeDims - 1) / kMergeDims), batch),
        dim3(ea::kThreads), 0, stream, p);
    note_launch("attention_scores_kernel + attention_softmax_kernel + attention_output_kernel (positions <= %d) + "
        "attention_split_kernel grid "
        "%dx%d + attention_merge_kernel (beyond)", p.exact_max, p.kv_heads * attention_split_chunks(p.max_context), batch);
    return hipGetLastError();
}

}  // namespace fortai_hip
