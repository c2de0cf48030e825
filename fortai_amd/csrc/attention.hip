// Gated GQA decode attention for gfx950: per-head RMSNorm of q and k, RoPE,
// fp16 KV append, split-K attention with an online softmax, and the
// cross-chunk merge with the sigmoid output gate.
//
// Reference: forward_attention, fortai_qwen35_cpu.f90:990-1033 (two-pass
// softmax over positions 0..pos, serial per head).  Here the context is split
// into chunks across workgroups (flash-decoding); one workgroup serves the
// whole GQA group of a kv head, so every K/V row is read from HBM once.
//
// Bit-exact parts: q/k normalisation (double sum of squares), RoPE from a
// host-computed table holding the reference's cos/sin values, and the fp16
// append through the reference's float_to_half (fortai_q8_dot.c:85-113, which
// rounds ties away from zero).  The softmax and P.V sums are re-associated
// (fp32, within the 1e-3 relative gate).  The chunk partials are merged by a
// second small kernel (a cross-workgroup handoff inside one kernel would need
// a device-scope fence, i.e. an L2 writeback, per workgroup).
#include "fortai_hip_internal.h"
#include "fortai_hip_kernels.h"

namespace fortai_hip {

namespace {

constexpr int kThreads = 256;
constexpr int kTile = 64;        // positions per LDS tile
constexpr int kMaxGroup = 4;     // q heads per kv head handled per workgroup
constexpr int kMaxHead = 256;
constexpr int kMaxChunks = 128;  // attention_chunk() keeps the chunk count below this

// RMSNorm with weights over a head slice in LDS (fortai_qwen35_cpu.f90:1434-1453),
// then RoPE on the first rope_dim values (:1473-1497).  One wave per slice.
__device__ __forceinline__ void norm_rope(float *v, int head, const float *w, float eps, const float2 *rope,
    int rope_dim, int lane) {
    double ss = 0.0;
    for (int i = lane; i < head; i += 64) ss += static_cast<double>(v[i]) * static_cast<double>(v[i]);
    ss = wave_sum(ss);
    const float mean = static_cast<float>(ss / static_cast<double>(head));
    const float inv = 1.0f / sqrtf(mean + eps);
    for (int i = lane; i < head; i += 64) v[i] = (v[i] * inv) * w[i];
    __builtin_amdgcn_wave_barrier();
    const int half = rope_dim / 2;
    for (int i = lane; i < half; i += 64) {
        const float2 cs = rope[i];
        const float a = v[i], b = v[i + half];
        v[i] = a * cs.x - b * cs.y;
        v[i + half] = a * cs.y + b * cs.x;
    }
    __builtin_amdgcn_wave_barrier();
}

template <bool FINITE>
__device__ __forceinline__ float kv_value(uint16_t h) {
    return FINITE ? half_bits_to_float(h) : gguf_half_to_real(h);
}

// scores of the 64 positions of a tile: wave g = q head g, lane = position
template <bool FINITE>
__device__ __forceinline__ float tile_score(const float *q, const uint16_t *krow, int head) {
    const float4 *q4 = reinterpret_cast<const float4 *>(q);
    const uint4 *k8 = reinterpret_cast<const uint4 *>(krow);
    float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;
#pragma unroll 4
    for (int i = 0; i < head / 8; ++i) {
        const uint4 h8 = k8[i];
        const float4 qa = q4[2 * i], qb = q4[2 * i + 1];
        d0 = __builtin_fmaf(qa.x, kv_value<FINITE>(static_cast<uint16_t>(h8.x)), d0);
        d1 = __builtin_fmaf(qa.y, kv_value<FINITE>(static_cast<uint16_t>(h8.x >> 16)), d1);
        d2 = __builtin_fmaf(qa.z, kv_value<FINITE>(static_cast<uint16_t>(h8.y)), d2);
        d3 = __builtin_fmaf(qa.w, kv_value<FINITE>(static_cast<uint16_t>(h8.y >> 16)), d3);
        d0 = __builtin_fmaf(qb.x, kv_value<FINITE>(static_cast<uint16_t>(h8.z)), d0);
        d1 = __builtin_fmaf(qb.y, kv_value<FINITE>(static_cast<uint16_t>(h8.z >> 16)), d1);
        d2 = __builtin_fmaf(qb.z, kv_value<FINITE>(static_cast<uint16_t>(h8.w)), d2);
        d3 = __builtin_fmaf(qb.w, kv_value<FINITE>(static_cast<uint16_t>(h8.w >> 16)), d3);
    }
    return (d0 + d1) + (d2 + d3);
}

template <bool FINITE>
__device__ __forceinline__ void tile_pv(float (&acc)[kMaxGroup], const float (*prob)[kTile],
    const uint16_t (*vtile)[kMaxHead], int n, int group, int d) {
#pragma unroll 4
    for (int j = 0; j < n; ++j) {
        const float vv = kv_value<FINITE>(vtile[j][d]);
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g)
            if (g < group) acc[g] = __builtin_fmaf(prob[g][j], vv, acc[g]);
    }
}

constexpr int kLoads = kTile * (kMaxHead / 8) / kThreads;  // 16-byte loads per thread per K (or V) tile

// issue the K and V rows [t0, t0+n) of a kv head (rows contiguous, 16 B per load)
__device__ __forceinline__ void fetch_tile(const AttentionParams &p, int kvh, int t0, int n, int tid,
    uint4 (&kr)[kLoads], uint4 (&vr)[kLoads]) {
    const int segs_k = p.head / 8, segs_v = p.value / 8;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int li = tid + i * kThreads;
        // rows past the tile re-read row n-1 (always in bounds); stash_tile skips them
        const int jk = min(li / segs_k, n - 1), sk = li % segs_k;
        const int jv = min(li / segs_v, n - 1), sv = li % segs_v;
        kr[i] = reinterpret_cast<const uint4 *>(p.kcache + (static_cast<size_t>(t0 + jk) * p.kv_heads + kvh) * p.head)[sk];
        vr[i] = reinterpret_cast<const uint4 *>(p.vcache + (static_cast<size_t>(t0 + jv) * p.kv_heads + kvh) * p.value)[sv];
    }
}

__device__ __forceinline__ void stash_tile(const AttentionParams &p, int n, int tid, const uint4 (&kr)[kLoads],
    const uint4 (&vr)[kLoads], uint16_t (*ktile)[kMaxHead + 8], uint16_t (*vtile)[kMaxHead]) {
    const int segs_k = p.head / 8, segs_v = p.value / 8;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int li = tid + i * kThreads;
        const int jk = li / segs_k, sk = li % segs_k;
        const int jv = li / segs_v, sv = li % segs_v;
        if (jk < n) *reinterpret_cast<uint4 *>(&ktile[jk][sk * 8]) = kr[i];
        if (jv < n) *reinterpret_cast<uint4 *>(&vtile[jv][sv * 8]) = vr[i];
    }
}

__global__ __launch_bounds__(kThreads) void attention_kernel(const AttentionParams p) {
    __shared__ __align__(16) float qh[kMaxGroup * kMaxHead];
    __shared__ __align__(16) float kn[kMaxHead];
    __shared__ __align__(16) float vn[kMaxHead];
    __shared__ __align__(16) float qw[kMaxHead];
    __shared__ __align__(16) float kw[kMaxHead];
    __shared__ __align__(16) float2 rs[kMaxHead / 2];
    __shared__ __align__(16) uint16_t ktile[kTile][kMaxHead + 8];
    __shared__ __align__(16) uint16_t vtile[kTile][kMaxHead];
    __shared__ float prob[kMaxGroup][kTile];
    __shared__ float rescale[kMaxGroup];
    __shared__ int overflow;

    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid >> 6, lane = tid & 63;
    const int pos = *p.position;
    if (pos < 0 || pos >= p.max_context) return;  // never index past the cache
    const int L = pos + 1;
    const int nchunk = (p.max_context + p.chunk - 1) / p.chunk;
    const int kvh = static_cast<int>(blockIdx.x) / nchunk;
    const int c = static_cast<int>(blockIdx.x) % nchunk;
    const int active = (L + p.chunk - 1) / p.chunk;
    if (c >= active) return;
    const int group = p.heads / p.kv_heads;
    const int head = p.head, value = p.value;
    const int p0 = c * p.chunk;
    const int p1 = (p0 + p.chunk < L) ? p0 + p.chunk : L;
    const bool owns_new = (pos >= p0 && pos < p1);
    const int h4 = head / 4, v4 = value / 4, half = p.rope_dim / 2;

    // every prologue load is issued before the first use
    const int qn = group * h4;
    float4 qv = make_float4(0.0f, 0.0f, 0.0f, 0.0f), aux = qv, vv4 = qv;
    float2 rv = make_float2(0.0f, 0.0f);
    if (tid < qn) {
        const int g = tid / h4, i = tid % h4;
        qv = reinterpret_cast<const float4 *>(p.q + static_cast<size_t>(kvh * group + g) * 2 * head)[i];
    }
    if (tid < h4) aux = reinterpret_cast<const float4 *>(p.q_norm)[tid];
    else if (tid >= 64 && tid - 64 < h4) aux = reinterpret_cast<const float4 *>(p.k_norm)[tid - 64];
    else if (owns_new && tid >= 192 && tid - 192 < h4)
        aux = reinterpret_cast<const float4 *>(p.k + static_cast<size_t>(kvh) * head)[tid - 192];
    if (tid >= 128 && tid - 128 < half) rv = p.rope[static_cast<size_t>(pos) * half + (tid - 128)];
    if (owns_new && tid < v4) vv4 = reinterpret_cast<const float4 *>(p.v + static_cast<size_t>(kvh) * value)[tid];
    const int flag = p.cache_flags ? p.cache_flags[kvh] : 1;

    if (tid < qn) reinterpret_cast<float4 *>(qh)[tid] = qv;
    if (tid < h4) reinterpret_cast<float4 *>(qw)[tid] = aux;
    else if (tid >= 64 && tid - 64 < h4) reinterpret_cast<float4 *>(kw)[tid - 64] = aux;
    else if (owns_new && tid >= 192 && tid - 192 < h4) reinterpret_cast<float4 *>(kn)[tid - 192] = aux;
    if (tid >= 128 && tid - 128 < half) rs[tid - 128] = rv;
    if (owns_new && tid < v4) reinterpret_cast<float4 *>(vn)[tid] = vv4;
    if (tid == 0) overflow = 0;
    __syncthreads();

    // q heads and the new key: normalise + rotate, one wave per slice
    for (int sl = wave; sl < group + (owns_new ? 1 : 0); sl += kThreads / 64) {
        if (sl < group) norm_rope(qh + sl * head, head, qw, p.eps, rs, p.rope_dim, lane);
        else norm_rope(kn, head, kw, p.eps, rs, p.rope_dim, lane);
    }
    __syncthreads();
    // append at pos with the reference's float_to_half (fortai_qwen35_cpu.f90:1594-1601);
    // the bits also replace the (not yet written) row in the LDS tile below
    uint16_t kbits = 0, vbits = 0;
    if (owns_new) {
        uint16_t *kdst = p.kcache + (static_cast<size_t>(pos) * p.kv_heads + kvh) * head;
        uint16_t *vdst = p.vcache + (static_cast<size_t>(pos) * p.kv_heads + kvh) * value;
        if (tid < head) {
            kbits = float_to_half_kv(kn[tid]);
            kdst[tid] = kbits;
            if ((kbits & 0x7c00u) == 0x7c00u) overflow = 1;
        }
        if (tid < value) {
            vbits = float_to_half_kv(vn[tid]);
            vdst[tid] = vbits;
            if ((vbits & 0x7c00u) == 0x7c00u) overflow = 1;
        }
        __syncthreads();
        if (tid == 0 && overflow && p.cache_flags) p.cache_flags[kvh] = 1;
    }
    const bool finite = flag == 0 && overflow == 0;

    const float scale_div = sqrtf(static_cast<float>(head));
    float m_run = -__builtin_inff();  // per wave = per q head (wave g handles head g)
    float l_run = 0.0f;
    float acc[kMaxGroup];
    for (int g = 0; g < kMaxGroup; ++g) acc[g] = 0.0f;

    for (int t0 = p0; t0 < p1; t0 += kTile) {
        const int n = (p1 - t0 < kTile) ? p1 - t0 : kTile;
        {
            uint4 kr[kLoads], vr[kLoads];
            fetch_tile(p, kvh, t0, n, tid, kr, vr);
            stash_tile(p, n, tid, kr, vr, ktile, vtile);
        }
        if (pos >= t0 && pos < t0 + n) {
            if (tid < head) ktile[pos - t0][tid] = kbits;
            if (tid < value) vtile[pos - t0][tid] = vbits;
        }
        __syncthreads();
        if (wave < group) {
            float sc = -__builtin_inff();
            if (lane < n) {
                const float dot = finite ? tile_score<true>(qh + wave * head, &ktile[lane][0], head)
                                         : tile_score<false>(qh + wave * head, &ktile[lane][0], head);
                sc = dot / scale_div;
            }
            float tmax = sc;
            for (int m = 32; m >= 1; m >>= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, m));
            const float m_new = fmaxf(m_run, tmax);
            const float e = (lane < n) ? expf(sc - m_new) : 0.0f;
            const float r = expf(m_run - m_new);
            l_run = l_run * r + wave_sum(e);
            m_run = m_new;
            prob[wave][lane] = e;
            if (lane == 0) rescale[wave] = r;
        }
        __syncthreads();
        // P.V: thread d owns value dim d for every head of the group
        for (int g = 0; g < kMaxGroup; ++g)
            if (g < group) acc[g] *= rescale[g];
        if (tid < value) {
            if (finite) tile_pv<true>(acc, prob, vtile, n, group, tid);
            else tile_pv<false>(acc, prob, vtile, n, group, tid);
        }
        __syncthreads();
    }

    // chunk partial: [kvh][c][g][m, l, acc[value]]
    const size_t stride = static_cast<size_t>(value) + 2;
    float *part = p.partial + (static_cast<size_t>(kvh) * nchunk + c) * group * stride;
    if (wave < group && lane == 0) {
        part[wave * stride] = m_run;
        part[wave * stride + 1] = l_run;
    }
    if (tid < value)
        for (int g = 0; g < group; ++g) part[g * stride + 2 + tid] = acc[g];
}

// Merge the chunk partials of one head (log-sum-exp rescale), apply the
// sigmoid output gate (fortai_qwen35_cpu.f90:1030-1031) and quantize the
// result for the o_proj matvec.  One 64-thread workgroup per (head, 64 dims).
__global__ __launch_bounds__(64) void attention_merge_kernel(const AttentionParams p) {
    __shared__ float vals[64];
    const int tid = static_cast<int>(threadIdx.x);
    const int pos = *p.position;
    if (pos < 0 || pos >= p.max_context) return;
    const int slices = p.value / 64;
    const int h = static_cast<int>(blockIdx.x) / slices;
    const int d = (static_cast<int>(blockIdx.x) % slices) * 64 + tid;
    const int group = p.heads / p.kv_heads;
    const int kvh = h / group, g = h % group;
    const int nchunk = (p.max_context + p.chunk - 1) / p.chunk;
    const int active = (pos + 1 + p.chunk - 1) / p.chunk;
    const size_t stride = static_cast<size_t>(p.value) + 2;
    const float *base = p.partial + (static_cast<size_t>(kvh) * nchunk * group + g) * stride;
    // chunk maxima and weights once per workgroup, then the weighted sum of
    // this thread's dimension; loads are batched so their latencies overlap
    __shared__ float wts[kMaxChunks];
    __shared__ float lsums[kMaxChunks];
    const size_t cstride = static_cast<size_t>(group) * stride;
    float M = -__builtin_inff();
    for (int c = tid; c < active; c += 64) M = fmaxf(M, base[c * cstride]);
    for (int m = 32; m >= 1; m >>= 1) M = fmaxf(M, __shfl_xor(M, m));
    for (int c = tid; c < active; c += 64) {
        const float w = expf(base[c * cstride] - M);
        wts[c] = w;
        lsums[c] = base[c * cstride + 1] * w;
    }
    __syncthreads();
    float lsum = 0.0f, o = 0.0f;
    for (int c0 = 0; c0 < active; c0 += 16) {
        float a[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) a[i] = (c0 + i < active) ? base[(c0 + i) * cstride + 2 + d] : 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            if (c0 + i < active) {
                lsum = lsum + lsums[c0 + i];
                o = __builtin_fmaf(a[i], wts[c0 + i], o);
            }
        }
    }
    const float gate = p.q[static_cast<size_t>(h) * 2 * p.head + p.head + d];
    const float y = (o / lsum) * sigmoid_ref(gate);
    if (p.out) p.out[static_cast<size_t>(h) * p.value + d] = y;
    if (!p.out_q8l) return;
    vals[tid] = y;
    __syncthreads();
    if (tid < 16) {
        const float4 v4 = make_float4(vals[4 * tid], vals[4 * tid + 1], vals[4 * tid + 2], vals[4 * tid + 3]);
        float scale;
        uint16_t bits;
        const uint32_t packed = quantize_group(v4, scale, bits);
        const int gi = (h * p.value + d - tid) / 4 + tid;  // 4-value group index in [heads*value]
        const int b = gi >> 3, ll = gi & 7;
        const int chunks = (p.heads * p.value / kQ8Block + 3) / 4;
        uint32_t *dq = static_cast<uint32_t *>(p.out_q8l);
        dq[((b >> 2) * 8 + ll) * 4 + (b & 3)] = packed;
        if (ll == 0) reinterpret_cast<float *>(dq + chunks * 32)[b] = scale;
    }
}

}  // namespace

int attention_chunk(int max_context) {
    // at most ~128 chunks per kv head keeps the merge short; at least one tile
    int chunk = kTile;
    while ((max_context + chunk - 1) / chunk > 128) chunk *= 2;
    return chunk;
}

hipError_t launch_attention(const AttentionParams &p, hipStream_t stream) {
    const int group = p.kv_heads > 0 ? p.heads / p.kv_heads : 0;
    if (group < 1 || group > kMaxGroup || p.heads % p.kv_heads || p.head > kMaxHead || p.value > kThreads ||
        p.head % 8 || p.value % 64 || p.rope_dim > p.head || p.rope_dim % 2 || p.chunk < 1)
        return hipErrorInvalidValue;
    const int nchunk = (p.max_context + p.chunk - 1) / p.chunk;
    hipLaunchKernelGGL(attention_kernel, dim3(p.kv_heads * nchunk), dim3(kThreads), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attention_merge_kernel, dim3(p.heads * (p.value / 64)), dim3(64), 0, stream, p);
    return hipGetLastError();
}

}  // namespace fortai_hip
