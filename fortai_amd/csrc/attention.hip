// Gated GQA decode attention for gfx950: per-head RMSNorm of q and k, RoPE,
// fp16 KV append, split-K attention with an online softmax, and the
// cross-chunk merge with the sigmoid output gate.
//
// Reference: forward_attention, fortai_qwen35_cpu.f90:990-1033 (two-pass
// softmax over positions 0..pos, serial per head).  Here the context is split
// into chunks across workgroups (flash-decoding); one workgroup serves the
// whole GQA group of a kv head, so every K/V row is read from HBM once.  The
// last workgroup of a kv head (device-scope counter) merges the chunk
// partials with the usual log-sum-exp rescale.
//
// Bit-exact parts: q/k normalisation (double sum of squares), RoPE from a
// host-computed table holding the reference's cos/sin values, and the fp16
// append through the reference's float_to_half (fortai_q8_dot.c:85-113, which
// rounds ties away from zero).  The softmax and P.V sums are re-associated
// (fp32, within the 1e-3 relative gate).
#include "fortai_hip_internal.h"
#include "fortai_hip_kernels.h"

namespace fortai_hip {

namespace {

constexpr int kThreads = 256;
constexpr int kTile = 64;        // positions per LDS tile
constexpr int kMaxGroup = 4;     // q heads per kv head handled per workgroup
constexpr int kMaxHead = 256;

// RMSNorm with weights over a head slice in LDS (fortai_qwen35_cpu.f90:1434-1453),
// then RoPE on the first rope_dim values (:1473-1497).  One wave per slice.
__device__ void norm_rope(float *v, int head, const float *w, float eps, const float2 *rope, int rope_dim,
    int lane) {
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

__global__ __launch_bounds__(kThreads) void attention_kernel(const AttentionParams p) {
    __shared__ float qh[kMaxGroup][kMaxHead];
    __shared__ float kn[kMaxHead];
    __shared__ float vn[kMaxHead];
    __shared__ uint16_t ktile[kTile][kMaxHead + 8];
    __shared__ uint16_t vtile[kTile][kMaxHead];
    __shared__ float prob[kMaxGroup][kTile];
    __shared__ float rescale[kMaxGroup];
    __shared__ bool last;

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
    const float2 *rope = p.rope + static_cast<size_t>(pos) * (p.rope_dim / 2);
    const bool owns_new = (pos >= p0 && pos < p1);

    // q of the group's heads: normalise + rotate (one wave per head)
    for (int g = wave; g < group; g += kThreads / 64) {
        const float *src = p.q + static_cast<size_t>(kvh * group + g) * 2 * head;
        for (int i = lane; i < head; i += 64) qh[g][i] = src[i];
        __builtin_amdgcn_wave_barrier();
        norm_rope(qh[g], head, p.q_norm, p.eps, rope, p.rope_dim, lane);
    }
    if (owns_new && wave == 0) {
        for (int i = lane; i < head; i += 64) kn[i] = p.k[static_cast<size_t>(kvh) * head + i];
        __builtin_amdgcn_wave_barrier();
        norm_rope(kn, head, p.k_norm, p.eps, rope, p.rope_dim, lane);
        uint16_t *kdst = p.kcache + (static_cast<size_t>(pos) * p.kv_heads + kvh) * head;
        uint16_t *vdst = p.vcache + (static_cast<size_t>(pos) * p.kv_heads + kvh) * value;
        for (int i = lane; i < head; i += 64) {
            const uint16_t bits = float_to_half_kv(kn[i]);
            kdst[i] = bits;
            kn[i] = gguf_half_to_real(bits);
        }
        for (int i = lane; i < value; i += 64) {
            const uint16_t bits = float_to_half_kv(p.v[static_cast<size_t>(kvh) * value + i]);
            vdst[i] = bits;
            vn[i] = gguf_half_to_real(bits);
        }
    }
    __syncthreads();

    const float scale_div = sqrtf(static_cast<float>(head));
    float m_run = -__builtin_inff();  // per wave = per q head (wave g handles head g)
    float l_run = 0.0f;
    float acc[kMaxGroup];
    for (int g = 0; g < kMaxGroup; ++g) acc[g] = 0.0f;

    for (int t0 = p0; t0 < p1; t0 += kTile) {
        const int n = (p1 - t0 < kTile) ? p1 - t0 : kTile;
        // stage K and V rows (16 B per thread per step, rows contiguous)
        const int segs_k = head / 8, segs_v = value / 8;
        for (int li = tid; li < n * segs_k; li += kThreads) {
            const int j = li / segs_k, s = li % segs_k;
            const uint4 *src = reinterpret_cast<const uint4 *>(
                p.kcache + (static_cast<size_t>(t0 + j) * p.kv_heads + kvh) * head) + s;
            *reinterpret_cast<uint4 *>(&ktile[j][s * 8]) = *src;
        }
        for (int li = tid; li < n * segs_v; li += kThreads) {
            const int j = li / segs_v, s = li % segs_v;
            const uint4 *src = reinterpret_cast<const uint4 *>(
                p.vcache + (static_cast<size_t>(t0 + j) * p.kv_heads + kvh) * value) + s;
            *reinterpret_cast<uint4 *>(&vtile[j][s * 8]) = *src;
        }
        __syncthreads();
        // scores: wave g = q head g, lane j = position t0 + j
        if (wave < group) {
            float sc = -__builtin_inff();
            if (lane < n) {
                const int pj = t0 + lane;
                float dot = 0.0f;
                if (pj == pos) {
                    for (int i = 0; i < head; ++i) dot = __builtin_fmaf(qh[wave][i], kn[i], dot);
                } else {
                    const uint16_t *kr = &ktile[lane][0];
                    for (int i = 0; i < head; i += 8) {
                        const uint4 h8 = *reinterpret_cast<const uint4 *>(kr + i);
                        const uint32_t hw[4] = {h8.x, h8.y, h8.z, h8.w};
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            dot = __builtin_fmaf(qh[wave][i + 2 * q], gguf_half_to_real(static_cast<uint16_t>(hw[q] & 0xffffu)), dot);
                            dot = __builtin_fmaf(qh[wave][i + 2 * q + 1], gguf_half_to_real(static_cast<uint16_t>(hw[q] >> 16)), dot);
                        }
                    }
                }
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
        for (int g = 0; g < group; ++g) acc[g] *= rescale[g];
        if (tid < value) {
            for (int j = 0; j < n; ++j) {
                const float vv = (t0 + j == pos) ? vn[tid] : gguf_half_to_real(vtile[j][tid]);
                for (int g = 0; g < group; ++g) acc[g] = __builtin_fmaf(prob[g][j], vv, acc[g]);
            }
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
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = atomicAdd(p.done + kvh, 1u);
        last = (prev == static_cast<unsigned>(active) - 1u);
    }
    __syncthreads();
    if (!last) return;
    __threadfence();

    // merge the active chunks of this kv head, then the output gate
    if (tid < value) {
        const float *base = p.partial + static_cast<size_t>(kvh) * nchunk * group * stride;
        for (int g = 0; g < group; ++g) {
            float M = -__builtin_inff();
            for (int cc = 0; cc < active; ++cc)
                M = fmaxf(M, __hip_atomic_load(base + (static_cast<size_t>(cc) * group + g) * stride,
                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            float lsum = 0.0f, o = 0.0f;
            for (int cc = 0; cc < active; ++cc) {
                const float *pc = base + (static_cast<size_t>(cc) * group + g) * stride;
                const float m = __hip_atomic_load(pc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const float l = __hip_atomic_load(pc + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const float a = __hip_atomic_load(pc + 2 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const float w = expf(m - M);
                lsum = __builtin_fmaf(l, w, lsum);
                o = __builtin_fmaf(a, w, o);
            }
            const int h = kvh * group + g;
            const float gate = p.q[static_cast<size_t>(h) * 2 * head + head + tid];
            p.out[static_cast<size_t>(h) * value + tid] = (o / lsum) * sigmoid_ref(gate);
        }
    }
    if (tid == 0) __hip_atomic_store(p.done + kvh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
        p.head % 8 || p.value % 8 || p.rope_dim > p.head || p.rope_dim % 2 || p.chunk < 1)
        return hipErrorInvalidValue;
    const int nchunk = (p.max_context + p.chunk - 1) / p.chunk;
    hipLaunchKernelGGL(attention_kernel, dim3(p.kv_heads * nchunk), dim3(kThreads), 0, stream, p);
    return hipGetLastError();
}

}  // namespace fortai_hip
