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
// The chains run from registers, handed from wave to wave (attend_given_z).
#pragma once

#include "fortai_hip_internal.h"

#ifndef FORTAI_ATT_MARK
#define FORTAI_ATT_MARK(i)
#endif
#ifndef FORTAI_ATTW_MARK
#define FORTAI_ATTW_MARK(i)
#endif

namespace fortai_hip {
namespace exact_attention {

constexpr int kThreads = 256;
constexpr int kPosBlock = 64;   // positions per score unit
constexpr int kDims = 8;        // value dims per output unit

template <bool FINITE>
__device__ __forceinline__ float kv(uint16_t h) { return FINITE ? half_bits_to_float(h) : gguf_half_to_real(h); }

// RMSNorm with weights over a head slice, then RoPE on the first rope_dim
// values (fortai_qwen35_cpu.f90:1434-1453, 1473-1497).  One wave.
__device__ __forceinline__ void norm_rope(float *v, int head, const float *w, float eps, const float2 *rope,
    int rope_dim, int lane) {
    double ss = 0.0;
    for (int i = lane; i < head; i += 64) ss += static_cast<double>(v[i]) * static_cast<double>(v[i]);
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(static_cast<float>(div_count(ss, head)) + eps);
    for (int i = lane; i < head; i += 64) v[i] = (v[i] * inv) * w[i];
    wave_lds_fence();
    const int half = rope_dim / 2;
    for (int i = lane; i < half; i += 64) {
        const float2 cs = rope[i];
        const float a = v[i], b = v[i + half];
        v[i] = a * cs.x - b * cs.y;
        v[i + half] = a * cs.y + b * cs.x;
    }
    wave_lds_fence();
}

// The same with the weights in registers: wr[j] = w[lane + 64 j] (loaded by
// the caller ahead of time), head <= 64 * NW.
template <int NW>
__device__ __forceinline__ void norm_rope_regs(float *v, int head, const float (&wr)[NW], float eps,
    const float2 *rope, int rope_dim, int lane) {
    double ss = 0.0;
    for (int i = lane; i < head; i += 64) ss += static_cast<double>(v[i]) * static_cast<double>(v[i]);
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(static_cast<float>(div_count(ss, head)) + eps);
#pragma unroll
    for (int j = 0; j < NW; ++j)
        if (lane + 64 * j < head) v[lane + 64 * j] = (v[lane + 64 * j] * inv) * wr[j];
    wave_lds_fence();
    const int half = rope_dim / 2;
    for (int i = lane; i < half; i += 64) {
        const float2 cs = rope[i];
        const float a = v[i], b = v[i + half];
        v[i] = a * cs.x - b * cs.y;
        v[i + half] = a * cs.y + b * cs.x;
    }
    wave_lds_fence();
}

// One position's score: the sequential dot of fortai_qwen35_cpu.f90:1009-1014.
// q in LDS (broadcast reads), the key row in LDS, 8 halves per read.  The
// products of a group of 8 are formed one group ahead of their adds, so the
// chain never waits on a product just issued, and the reads run two groups
// ahead of the products.
template <bool FINITE>
__device__ __forceinline__ void score_products(float (&p)[8], uint4 h8, float4 qa, float4 qb) {
    if constexpr (FINITE) {
        // fl(q_i * f32(k_i)) straight from the fp16 half: one v_fma_mix_f32 each
        p[0] = half_times<false>(h8.x, qa.x);
        p[1] = half_times<true>(h8.x, qa.y);
        p[2] = half_times<false>(h8.y, qa.z);
        p[3] = half_times<true>(h8.y, qa.w);
        p[4] = half_times<false>(h8.z, qb.x);
        p[5] = half_times<true>(h8.z, qb.y);
        p[6] = half_times<false>(h8.w, qb.z);
        p[7] = half_times<true>(h8.w, qb.w);
    } else {
        p[0] = qa.x * kv<FINITE>(static_cast<uint16_t>(h8.x));
        p[1] = qa.y * kv<FINITE>(static_cast<uint16_t>(h8.x >> 16));
        p[2] = qa.z * kv<FINITE>(static_cast<uint16_t>(h8.y));
        p[3] = qa.w * kv<FINITE>(static_cast<uint16_t>(h8.y >> 16));
        p[4] = qb.x * kv<FINITE>(static_cast<uint16_t>(h8.z));
        p[5] = qb.y * kv<FINITE>(static_cast<uint16_t>(h8.z >> 16));
        p[6] = qb.z * kv<FINITE>(static_cast<uint16_t>(h8.w));
        p[7] = qb.w * kv<FINITE>(static_cast<uint16_t>(h8.w >> 16));
    }
}

template <bool FINITE>
__device__ __forceinline__ float score(const float *q, const uint16_t *krow, int head, float sqrt_head) {
    const uint4 *k8 = reinterpret_cast<const uint4 *>(krow);
    const float4 *q4 = reinterpret_cast<const float4 *>(q);
    const int groups = head / 8, last = groups - 1;  // head % 8 == 0
    float p[8];
    score_products<FINITE>(p, k8[0], q4[0], q4[1]);
    const int g1 = min(1, last), g2 = min(2, last);
    uint4 h1 = k8[g1], h2 = k8[g2];
    float4 a1 = q4[2 * g1], b1 = q4[2 * g1 + 1], a2 = q4[2 * g2], b2 = q4[2 * g2 + 1];
    float acc = 0.0f;
    for (int g = 0; g < groups; ++g) {
        // group g + 3's reads (clamped; the clamped copies are not used)
        const int g3 = min(g + 3, last);
        const uint4 h3 = k8[g3];
        const float4 a3 = q4[2 * g3], b3 = q4[2 * g3 + 1];
        float pn[8];
        score_products<FINITE>(pn, h1, a1, b1);  // group g + 1 (unused past the end)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = acc + p[i];
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = pn[i];
        h1 = h2; a1 = a2; b1 = b2;
        h2 = h3; a2 = a3; b2 = b3;
    }
    return acc / sqrt_head;
}

// The same for a head width known at compile time, fully unrolled (the
// reads become immediate offsets and the scheduler can run them ahead).
template <bool FINITE, int HEAD>
__device__ __forceinline__ float score_n(const float *q, const uint16_t *krow, float sqrt_head) {
    const uint4 *k8 = reinterpret_cast<const uint4 *>(krow);
    const float4 *q4 = reinterpret_cast<const float4 *>(q);
    float acc = 0.0f;
    float p[8];
    score_products<FINITE>(p, k8[0], q4[0], q4[1]);
#pragma unroll
    for (int g = 0; g < HEAD / 8; ++g) {
        float pn[8];
        if (g + 1 < HEAD / 8) score_products<FINITE>(pn, k8[g + 1], q4[2 * g + 2], q4[2 * g + 3]);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = acc + p[i];
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = pn[i];
    }
    return acc / sqrt_head;
}

// ------------------------------------------------------------ fp32 chains
// A left-to-right fp32 sum is a chain of dependent adds: one add issues every
// ~4.7 cycles on gfx950, and any other instruction of the summing wave takes
// an issue slot from the chain.  So a chain is cut into segments of kSeg
// positions that the four waves take in turn: segment k is summed by wave
// k % 4 from registers only, while the other three waves compute the values
// of their next segments (expf, or e/Z times the value row) and load them into
// their registers.  The running sum passes from wave to wave through a tagged
// 64-bit LDS word per chain (tag = index of the segment it starts).

constexpr int kWaves = kThreads / 64;
constexpr int kSeg = 256;            // positions per chain segment
constexpr int kSegVec = kSeg / 4;    // 16-byte registers per lane per segment
constexpr int kStagePitch = kSeg + 4;
constexpr int kTurnSpin = 1 << 22;   // polls of a handoff word before giving up

typedef float f4 __attribute__((ext_vector_type(4)));


// A segment's values into registers.  The reads are ordinary loads, so the
// compiler tracks them; seg_held() then makes the compiler complete them at
// that point (an empty asm that uses every value), before the wave waits for
// its turn, instead of sinking each read next to its first add inside the
// chain.
__device__ __forceinline__ void seg_read(f4 (&r)[kSegVec], const float *src) {
#pragma unroll
    for (int c = 0; c < kSegVec; ++c) r[c] = *reinterpret_cast<const f4 *>(src + 4 * c);
}

template <int C>
__device__ __forceinline__ void seg_held(f4 (&r)[kSegVec]) {
    if constexpr (C < kSegVec) {
        asm volatile(""
                     : "+v"(r[C]), "+v"(r[C + 1]), "+v"(r[C + 2]), "+v"(r[C + 3]), "+v"(r[C + 4]), "+v"(r[C + 5]),
                       "+v"(r[C + 6]), "+v"(r[C + 7]), "+v"(r[C + 8]), "+v"(r[C + 9]), "+v"(r[C + 10]),
                       "+v"(r[C + 11]), "+v"(r[C + 12]), "+v"(r[C + 13]), "+v"(r[C + 14]), "+v"(r[C + 15]));
        seg_held<C + 16>(r);
    }
}

// acc + r[0].x + r[0].y + ..., left to right, over the first cnt values
// rounded up to 16.  The values past cnt are -0.0f, which leaves any sum as
// it is (x + -0 = x for every x), so a partial segment needs no guards.
__device__ __forceinline__ float seg_chain(const f4 (&r)[kSegVec], int cnt, float acc) {
    if (cnt >= kSeg) {
#pragma unroll
        for (int i = 0; i < kSegVec; ++i) {
            acc = acc + r[i].x;
            acc = acc + r[i].y;
            acc = acc + r[i].z;
            acc = acc + r[i].w;
        }
        return acc;
    }
#pragma unroll
    for (int c = 0; c < kSegVec; c += 4) {
        if (4 * c < cnt) {
#pragma unroll
            for (int i = c; i < c + 4; ++i) {
                acc = acc + r[i].x;
                acc = acc + r[i].y;
                acc = acc + r[i].z;
                acc = acc + r[i].w;
            }
        }
    }
    return acc;
}

// The running sum entering segment k (0 for k = 0), from the chain's handoff
// word.  Only this workgroup writes the word, and every wave of it is
// resident, so the wait ends; the bound only guards against a broken caller.
__device__ __forceinline__ float take_turn(const uint64_t *word, int k) {
    if (k == 0) return 0.0f;
    uint64_t w;
    int spins = 0;
    do {
        w = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    } while (static_cast<int>(w >> 32) != k && ++spins < kTurnSpin);
    return __uint_as_float(static_cast<uint32_t>(w));
}

__device__ __forceinline__ void pass_turn(uint64_t *word, int k_next, float acc) {
    __hip_atomic_store(word, (static_cast<uint64_t>(k_next) << 32) | __float_as_uint(acc), __ATOMIC_RELAXED,
        __HIP_MEMORY_SCOPE_WORKGROUP);
}

// ------------------------------------------------- Z from candidate tables
// Z = e_0 + e_1 + ... left to right is one chain of n dependent adds.  The
// softmax kernel cuts it into kSeg-position segments and runs every segment
// in parallel from kZCand candidate starting sums: the consecutive floats
// around (float) of an estimate of the sum entering the segment (the
// double sum of a fast exp over the earlier positions; the true running sum
// differs from it by the chain's accumulated rounding, a few tens of ulps).
// Candidate c's chain over the segment's e values gives the entry T[c]; the
// workgroup also knows the next segment's window (its estimate is the same
// double sum, one segment longer) and stores, for every c, the index of T[c]
// among the next segment's candidates.  resolve_z() then walks the segments
// from candidate kZCand/2 of segment 0 (every candidate of segment 0 starts
// at exactly 0), one index per segment, and reads T of the last one: the
// chain's exact value.  When a running sum lies outside the next window that
// segment's chain is run from it over the stored e values, so the result is
// the left-to-right sum in every case.
constexpr int kZCand = 256;                // candidate starting sums per segment (one per thread)
static_assert((kZCand & (kZCand - 1)) == 0, "candidate indices are masked to a row");
constexpr int kZNext = kZCand;             // row offset of the next-segment indices
constexpr int kZCentre = 2 * kZCand;       // row offset of the centre's bits
constexpr int kZStride = 2 * kZCand + 2;   // row: T[kZCand] | next[kZCand] | centre | pad
__host__ __device__ constexpr int z_segments(int max_context) { return (max_context + kSeg - 1) / kSeg; }

// the index of s among the candidates around centre, or -1
__device__ __forceinline__ int z_index(float s, uint32_t centre) {
    const long long c = static_cast<long long>(__float_as_uint(s)) - static_cast<long long>(centre) + kZCand / 2;
    return c >= 0 && c < kZCand ? static_cast<int>(c) : -1;
}

// walk: the next indices of segment k (the last segment: its T bits) at
// walk + k * walk_stride, in LDS (compact, stride kZCand) or in the rows
// themselves (tab + kZNext, stride kZStride); tab: the full rows (global
// memory); ev: the n e values.
__device__ __forceinline__ float resolve_z(const int32_t *walk, int walk_stride, const float *tab, const float *ev,
    int n) {
    const int nseg = (n + kSeg - 1) / kSeg;
    // every running sum a candidate of its segment (the usual case): one
    // dependent LDS read per segment, an index outside a window (w < 0) only
    // noted, and the general walk below taken if one occurred
    {
        int idx = kZCand / 2, miss = 0;
#pragma unroll 4
        for (int k = 0; k + 1 < nseg; ++k) {
            const int w = walk[static_cast<size_t>(k) * walk_stride + idx];
            miss |= w;
            idx = w & (kZCand - 1);  // stays in the row when w < 0
        }
        if (miss >= 0) return __int_as_float(walk[static_cast<size_t>(nseg - 1) * walk_stride + idx]);
    }
    int idx = kZCand / 2;
    bool have = true;  // the running sum is candidate idx of segment k
    float s = 0.0f;
    for (int k = 0; k < nseg; ++k) {
        if (!have) {
            const int c = z_index(s, __float_as_uint(tab[static_cast<size_t>(k) * kZStride + kZCentre]));
            if (c < 0) {
                const int p0 = k * kSeg, cnt = min(kSeg, n - p0);
                for (int j = 0; j < cnt; ++j) s = s + ev[p0 + j];
                continue;
            }
            idx = c;
            have = true;
        }
        const int w = walk[static_cast<size_t>(k) * walk_stride + idx];
        if (k == nseg - 1) {
            s = __int_as_float(w);
        } else if (w >= 0) {
            idx = w;
        } else {
            s = tab[static_cast<size_t>(k) * kZStride + idx];
            have = false;
        }
    }
    return s;
}

// LDS of the output step, in floats: 8 reduction slots, kDims handoff words
// and one stage of kDims x kSeg values per wave (work_floats); a caller that
// keeps the scores in LDS adds sw_floats(max_context) in front.
__host__ __device__ constexpr size_t work_floats() {
    return 8 + 2 * kDims + static_cast<size_t>(kWaves) * kDims * kStagePitch;
}
__host__ __device__ constexpr size_t sw_floats(int max_context) {
    return static_cast<size_t>((max_context + 3) / 4 * 4);
}
__host__ __device__ constexpr size_t output_lds_floats(int max_context) {
    return sw_floats(max_context) + work_floats();
}

// The value pieces (kDims fp16 = 16 bytes) a lane multiplies for its wave's
// first segment: positions wave*kSeg + lane + 64 i.
constexpr int kPieces = kSeg / 64;
typedef uint4 ValuePieces[kPieces];

// Every load is unconditional, its position clamped to the first n (n >= 1):
// a per-lane condition around a load makes the compiler branch and wait for
// it on the spot.  The pieces of positions p >= n are never used (their
// products are staged as -0 by the callers).
__device__ __forceinline__ void value_fetch(const uint16_t *vbase, size_t vstride, int n, int k, ValuePieces &v) {
    const int lane = static_cast<int>(threadIdx.x) & 63;
#pragma unroll
    for (int i = 0; i < kPieces; ++i) {
        const int p = min(k * kSeg + lane + 64 * i, n - 1);
        v[i] = *reinterpret_cast<const uint4 *>(vbase + static_cast<size_t>(p) * vstride);
    }
}

__device__ __forceinline__ void value_prefetch(const uint16_t *vbase, size_t vstride, int n, ValuePieces &v) {
    value_fetch(vbase, vstride, n, static_cast<int>(threadIdx.x) >> 6, v);
}

// The e values of the wave's first segment (clamped to the first n).
__device__ __forceinline__ void e_prefetch(const float *ev, int n, float (&e4)[kPieces]) {
    const int lane = static_cast<int>(threadIdx.x) & 63, wave = static_cast<int>(threadIdx.x) >> 6;
#pragma unroll
    for (int i = 0; i < kPieces; ++i) e4[i] = ev[min(wave * kSeg + lane + 64 * i, n - 1)];
}

// P.V of kDims value dims with Z given (attention_softmax_kernel's e values
// and resolve_z): out_j = fl(e_0/Z v_0,j) + fl(e_1/Z v_1,j) + ... left to
// right.  ev: the n e values (global memory);
// v and e4: the value pieces and e values of the wave's first segment
// (value_prefetch, e_prefetch).  All threads call it; the result is valid in
// threads 0..kDims-1.
template <bool FINITE>
__device__ __forceinline__ float attend_given_z(const float *ev, float z, int n, const uint16_t *vbase,
    size_t vstride, float *work, ValuePieces &v, float (&e4)[kPieces]) {
    static_assert(kDims == 8, "one 16-byte value piece per position");
    const int tid = static_cast<int>(threadIdx.x), wave = tid >> 6, lane = tid & 63;
    uint64_t *hand = reinterpret_cast<uint64_t *>(work + 8);
    float *stage = work + 8 + 2 * kDims + wave * kDims * kStagePitch;
    const int nseg = (n + kSeg - 1) / kSeg;
    if (tid < kDims) hand[tid] = 0;
    auto load_e = [&](int k) {
#pragma unroll
        for (int i = 0; i < kPieces; ++i) e4[i] = ev[min(k * kSeg + lane + 64 * i, n - 1)];
    };
    __syncthreads();
    FORTAI_ATT_MARK(6);
    f4 r[kSegVec];
    float acc = 0.0f;
    for (int k = wave; k < nseg; k += kWaves) {
        const int p0 = k * kSeg, cnt = min(kSeg, n - p0);
#pragma unroll
        for (int i = 0; i < kPieces; ++i) {
            const int j = lane + 64 * i, p = p0 + j;
            if (p < n) {
                const float wp = e4[i] / z;
                const uint32_t hw[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    stage[(2 * q) * kStagePitch + j] = wp * kv<FINITE>(static_cast<uint16_t>(hw[q] & 0xffffu));
                    stage[(2 * q + 1) * kStagePitch + j] = wp * kv<FINITE>(static_cast<uint16_t>(hw[q] >> 16));
                }
            } else {
#pragma unroll
                for (int d = 0; d < kDims; ++d) stage[d * kStagePitch + j] = -0.0f;
            }
        }
        if (k + kWaves < nseg) {
            load_e(k + kWaves);
            value_fetch(vbase, vstride, n, k + kWaves, v);
        }
        if (lane < kDims) {
            seg_read(r, stage + lane * kStagePitch);
            seg_held<0>(r);
            float a = take_turn(hand + lane, k);
            a = seg_chain(r, cnt, a);
            pass_turn(hand + lane, k + 1, a);
        }
        if (k == 0) FORTAI_ATT_MARK(9);
    }
    __syncthreads();
    FORTAI_ATT_MARK(7);
    if (tid < kDims) acc = __uint_as_float(static_cast<uint32_t>(hand[tid]));
    __syncthreads();  // hand and stage are free again when this returns
    return acc;
}

}  // namespace exact_attention
}  // namespace fortai_hip
