// Exact gated GQA decode attention: the reference's two-pass softmax
// (fortai_qwen35_cpu.f90:1006-1031) with its summation orders kept, so the
// attention output is bit-identical to the CPU path:
//   score_p = (sum_i q_i * k_p,i, left to right, separately rounded) / sqrt(d)
//   m = max_p score_p;  e_p = expf(score_p - m);  Z = sum_p e_p (left to right)
//   out_j = sum_p (e_p / Z) * v_p,j (left to right) * sigmoid(gate_j)
// A greedy trace depends on every rounding: the o_proj input is quantized to
// Q8_0, so a one-ulp change of an output flips an int8 now and then and the
// trace drifts.  The parallel parts (the score of each position, e_p, e_p/Z,
// every product) run on many lanes; only the left-to-right sums are chains.
// The P.V chains are fed by producer waves through an LDS ring, so the chain
// lane issues one add per position.
#pragma once

#include "fortai_hip_internal.h"

namespace fortai_hip {
namespace exact_attention {

constexpr int kThreads = 256;
constexpr int kPosBlock = 64;   // positions per score unit
constexpr int kDims = 16;       // value dims per output unit
constexpr int kRing = 128;      // positions per ring block
constexpr int kRingPitch = kRing + 4;

template <bool FINITE>
__device__ __forceinline__ float kv(uint16_t h) { return FINITE ? half_bits_to_float(h) : gguf_half_to_real(h); }

// RMSNorm with weights over a head slice, then RoPE on the first rope_dim
// values (fortai_qwen35_cpu.f90:1434-1453, 1473-1497).  One wave.
__device__ __forceinline__ void norm_rope(float *v, int head, const float *w, float eps, const float2 *rope,
    int rope_dim, int lane) {
    double ss = 0.0;
    for (int i = lane; i < head; i += 64) ss += static_cast<double>(v[i]) * static_cast<double>(v[i]);
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(static_cast<float>(ss / static_cast<double>(head)) + eps);
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

// One position's score: the sequential dot of fortai_qwen35_cpu.f90:1009-1014.
// q in LDS (broadcast reads), the key row in LDS, 8 halves per read.
template <bool FINITE>
__device__ __forceinline__ float score(const float *q, const uint16_t *krow, int head, float sqrt_head) {
    float acc = 0.0f;
    for (int i = 0; i < head; i += 8) {
        const uint4 h8 = *reinterpret_cast<const uint4 *>(krow + i);
        const float4 qa = *reinterpret_cast<const float4 *>(q + i);
        const float4 qb = *reinterpret_cast<const float4 *>(q + i + 4);
        acc = acc + qa.x * kv<FINITE>(static_cast<uint16_t>(h8.x));
        acc = acc + qa.y * kv<FINITE>(static_cast<uint16_t>(h8.x >> 16));
        acc = acc + qa.z * kv<FINITE>(static_cast<uint16_t>(h8.y));
        acc = acc + qa.w * kv<FINITE>(static_cast<uint16_t>(h8.y >> 16));
        acc = acc + qb.x * kv<FINITE>(static_cast<uint16_t>(h8.z));
        acc = acc + qb.y * kv<FINITE>(static_cast<uint16_t>(h8.z >> 16));
        acc = acc + qb.z * kv<FINITE>(static_cast<uint16_t>(h8.w));
        acc = acc + qb.w * kv<FINITE>(static_cast<uint16_t>(h8.w >> 16));
    }
    return acc / sqrt_head;
}

// s[0..n) (LDS, the scores of one head) -> w[p] = expf(s_p - max) / Z in
// place, with Z summed left to right by one lane (fortai_qwen35_cpu.f90:
// 1016-1020).  red: >= 8 floats of LDS.  All threads of the block call it.
__device__ __forceinline__ void softmax_weights(float *s, int n, float *red) {
    const int tid = static_cast<int>(threadIdx.x);
    float m = -3.402823466e38f;  // -huge(1.0_real32)
    for (int p = tid; p < n; p += kThreads) m = fmaxf(m, s[p]);
    for (int k = 32; k >= 1; k >>= 1) m = fmaxf(m, __shfl_xor(m, k));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int p = tid; p < n; p += kThreads) s[p] = expf_libm(s[p] - m);
    __syncthreads();
    if (tid == 0) {
        // left-to-right sum; LDS reads are issued a batch ahead of the adds
        float z = 0.0f;
        int p = 0;
        float4 cur[8];
        const int full = n / 32;
        if (full > 0) {
#pragma unroll
            for (int k = 0; k < 8; ++k) cur[k] = *reinterpret_cast<const float4 *>(s + 4 * k);
        }
        for (int b = 0; b < full; ++b, p += 32) {
            float4 nxt[8];
            if (b + 1 < full) {
#pragma unroll
                for (int k = 0; k < 8; ++k) nxt[k] = *reinterpret_cast<const float4 *>(s + p + 32 + 4 * k);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                z = z + cur[k].x;
                z = z + cur[k].y;
                z = z + cur[k].z;
                z = z + cur[k].w;
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) cur[k] = nxt[k];
        }
        for (; p < n; ++p) z = z + s[p];
        red[4] = z;
    }
    __syncthreads();
    const float z = red[4];
    for (int p = tid; p < n; p += kThreads) s[p] = s[p] / z;
    __syncthreads();
}

// out_j = sum_p w_p * v_p,j left to right for kDims consecutive value dims:
// lanes 0..kDims-1 of wave 0 run the chains; waves 1..3 write the products
// fl(w_p * v_p,j) into a double-buffered LDS ring [dim][position], with the
// value rows of the next kPrefetch blocks already in their registers (the
// chains need ~0.2 us per block, a row fetch ~1-2 us).  The value row of
// position p starts at vbase + p * vstride (fp16 bits, kDims contiguous).
// The result is valid in threads 0..kDims-1.  ring: 2 * kDims * kRingPitch.
constexpr int kPrefetch = 8;
constexpr int kSegs = kRing * kDims / 8;                 // 16-byte value pieces per block
constexpr int kSegsPerProducer = (kSegs + kThreads - 65) / (kThreads - 64);

template <bool FINITE>
__device__ __forceinline__ void pv_fetch(const uint16_t *vbase, size_t vstride, int n, int b, int ptid,
    uint4 (&dst)[kSegsPerProducer]) {
#pragma unroll
    for (int i = 0; i < kSegsPerProducer; ++i) {
        const int c = ptid + i * (kThreads - 64);
        const int p = b * kRing + c / 2;
        dst[i] = (c < kSegs && p < n)
                     ? *reinterpret_cast<const uint4 *>(vbase + static_cast<size_t>(p) * vstride + (c & 1) * 8)
                     : make_uint4(0u, 0u, 0u, 0u);
    }
}

template <bool FINITE>
__device__ __forceinline__ float pv_chains(const float *w, int n, const uint16_t *vbase, size_t vstride,
    float *ring) {
    static_assert(kDims == 16, "two 16-byte pieces per position");
    const int tid = static_cast<int>(threadIdx.x);
    const int blocks = (n + kRing - 1) / kRing;
    const int ptid = tid - 64;
    uint4 pre[kPrefetch][kSegsPerProducer];
    if (tid >= 64) {
#pragma unroll
        for (int k = 0; k < kPrefetch; ++k)
            if (k < blocks) pv_fetch<FINITE>(vbase, vstride, n, k, ptid, pre[k]);
    }
    auto produce = [&](int b, const uint4 (&vr)[kSegsPerProducer], float *buf) {
#pragma unroll
        for (int i = 0; i < kSegsPerProducer; ++i) {
            const int c = ptid + i * (kThreads - 64);
            const int j = c / 2, d0 = (c & 1) * 8;
            const int p = b * kRing + j;
            if (c < kSegs && p < n) {
                const float wp = w[p];
                const uint32_t hw[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    buf[(d0 + 2 * q) * kRingPitch + j] = wp * kv<FINITE>(static_cast<uint16_t>(hw[q] & 0xffffu));
                    buf[(d0 + 2 * q + 1) * kRingPitch + j] = wp * kv<FINITE>(static_cast<uint16_t>(hw[q] >> 16));
                }
            }
        }
    };
    if (tid >= 64) produce(0, pre[0], ring);
    __syncthreads();
    float acc = 0.0f;
    for (int b0 = 0; b0 < blocks; b0 += kPrefetch) {
#pragma unroll
        for (int s = 0; s < kPrefetch; ++s) {
            const int b = b0 + s;
            if (b >= blocks) break;
            float *cur = ring + (b & 1) * kDims * kRingPitch;
            if (tid >= 64) {
                // slot s now feeds block b + kPrefetch; block b + 1 comes from slot s + 1
                if (b + kPrefetch < blocks) pv_fetch<FINITE>(vbase, vstride, n, b + kPrefetch, ptid, pre[s]);
                if (b + 1 < blocks) produce(b + 1, pre[(s + 1) % kPrefetch], ring + ((b + 1) & 1) * kDims * kRingPitch);
            } else if (tid < kDims) {
                const float *t = cur + tid * kRingPitch;
                const int cnt = min(kRing, n - b * kRing);
                int j = 0;
                for (; j + 16 <= cnt; j += 16) {
                    const float4 a0 = *reinterpret_cast<const float4 *>(t + j);
                    const float4 a1 = *reinterpret_cast<const float4 *>(t + j + 4);
                    const float4 a2 = *reinterpret_cast<const float4 *>(t + j + 8);
                    const float4 a3 = *reinterpret_cast<const float4 *>(t + j + 12);
                    acc = acc + a0.x; acc = acc + a0.y; acc = acc + a0.z; acc = acc + a0.w;
                    acc = acc + a1.x; acc = acc + a1.y; acc = acc + a1.z; acc = acc + a1.w;
                    acc = acc + a2.x; acc = acc + a2.y; acc = acc + a2.z; acc = acc + a2.w;
                    acc = acc + a3.x; acc = acc + a3.y; acc = acc + a3.z; acc = acc + a3.w;
                }
                for (; j < cnt; ++j) acc = acc + t[j];
            }
            __syncthreads();
        }
    }
    return acc;
}

}  // namespace exact_attention
}  // namespace fortai_hip
