// Persistent whole-token decode kernel for gfx950.
//
// One launch runs a complete Qwen3.5 decode step (fortai_qwen35_cpu.f90:591-711
// plus the greedy maxloc of app/fortai_cpu_run.f90:58) on one workgroup per
// CU.  The step is a fixed sequence of phases:
//   embed | per layer: projections, GDN or attention (+ chunk merge),
//   out projection + residual, gate/up (SiLU pair), down + residual |
//   LM head with per-workgroup argmax | final argmax.
// A phase's outputs reach the next phase's workgroups as 64-bit tagged words
// (tag << 32 | payload), written with device-scope atomic stores into a
// buffer that only this phase writes, and read with device-scope atomic loads
// until every word carries the current tag (the launch's sequence number,
// counted by the host and passed as an argument).
// Each word validates itself, so the handoff needs neither counters nor
// fences: measured on MI355X, a handoff costs about one load round trip
// (~1 us), against ~1.7 us for a dependent kernel boundary plus the reload of
// the activation that follows it.  A workgroup issues the weight loads of its
// next rows before it waits, so weight streaming overlaps the handoff.
//
// Every wait is bounded: a workgroup that waits too long (or sees another
// workgroup's timeout) records it in `status` and exits, so the grid always
// drains; the host reports the step as failed.  All workgroups must be
// co-resident: the grid is one workgroup per CU, and the kernel's register
// footprint (one wave per SIMD) admits exactly one workgroup per CU.
//
// Arithmetic is the same as the per-op kernels (bit-exact Q8_0 dots in the
// reference's AVX2 lane order, the reference quantizer, fp16 LM head chains,
// the GDN step) except where noted: reductions feeding a double sum may be
// grouped differently (double precision makes the float result the same in
// practice) and attention is split over chunks with an online softmax.
#include "fortai_hip_internal.h"
#include "fortai_hip_kernels.h"

namespace fortai_hip {
namespace {
__device__ __forceinline__ void mark(int i);
}
}  // namespace fortai_hip
#define FORTAI_ATT_MARK(i) mark(i)
#include "attention_exact.h"

namespace fortai_hip {

namespace {

constexpr int kT = 256;            // threads per workgroup
constexpr int kW = kT / 64;        // waves per workgroup
constexpr int kSpin = 1 << 21;     // polls before a wait is declared failed (~2 s)
constexpr int kMaxIter = 4;        // activation groups of 4 per thread: width <= 4096
constexpr int kMaxKernel = 8;      // conv1d taps
constexpr int kMaxGroup = 4;       // q heads per kv head
constexpr int kMaxHead = 256;      // head_dim / value_dim
constexpr size_t kLdsBytes = 64 * 1024;  // the largest phase (LM head tile, attention tiles) needs < 48 KiB

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------ tagged words

__device__ __forceinline__ uint64_t ll_load(const uint64_t *p) {
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_put(uint64_t *p, uint32_t v, uint32_t tag) {
    __hip_atomic_store(p, (static_cast<uint64_t>(tag) << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_putf(uint64_t *p, float v, uint32_t tag) { ll_put(p, __float_as_uint(v), tag); }
__device__ __forceinline__ float ll_f(uint64_t w) { return __uint_as_float(static_cast<uint32_t>(w)); }
__device__ __forceinline__ bool tagged(uint64_t w, uint32_t tag) { return static_cast<uint32_t>(w >> 32) == tag; }

// Phase being executed (diagnostics of a failed wait).
__shared__ int s_phase;
// optional timing marks of the matvec phases (FORTAI_HIP_PHASE_TIMES=2)
__shared__ uint64_t *g_marks;
__shared__ int g_mark_stride;
__device__ __forceinline__ void mark(int i) {
    if (g_marks && threadIdx.x == 0)
        g_marks[(static_cast<size_t>(blockIdx.x) * g_mark_stride + s_phase) * 4 + i] = wall_clock64();
}

// Load src[idx[k]] for every k (idx < 0: unused) and poll until all carry
// `tag`.  false: timed out, or another workgroup already failed.  The first
// timeout records status[1..5] = phase + 1, workgroup, word index, the tag
// found and the tag expected.
template <int N>
__device__ __forceinline__ bool ll_wait(const uint64_t *src, const int (&idx)[N], uint64_t (&v)[N], uint32_t tag, int *status) {
    const uint64_t ready = static_cast<uint64_t>(tag) << 32;
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = idx[k] >= 0 ? ll_load(src + idx[k]) : ready;
    for (int spin = 0;; ++spin) {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < N; ++k) ok = ok && tagged(v[k], tag);
        if (ok) return true;
        if (spin >= kSpin ||
            ((spin & 255) == 255 && __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0)) {
            int bad_idx = -1, bad_tag = 0;  // selected without indexing the arrays at run time
#pragma unroll
            for (int k = N - 1; k >= 0; --k)
                if (!tagged(v[k], tag)) { bad_idx = idx[k]; bad_tag = static_cast<int>(v[k] >> 32); }
            // per-workgroup record: the host reports the workgroup furthest behind
            status[8 + blockIdx.x] = s_phase + 1;
            status[8 + 256 + blockIdx.x] = bad_idx;
            if (spin >= kSpin && atomicCAS(status + 1, 0, s_phase + 1) == 0) {
                status[2] = static_cast<int>(blockIdx.x);
                status[3] = bad_idx;
                status[4] = bad_tag;
                status[5] = static_cast<int>(tag);
            }
            atomicOr(status, 1);
            return false;
        }
        __builtin_amdgcn_s_sleep(2);
#pragma unroll
        for (int k = 0; k < N; ++k)
            if (!tagged(v[k], tag)) v[k] = ll_load(src + idx[k]);
    }
}

// Two sources polled together (one round trip instead of two).
template <int N>
__device__ __forceinline__ bool ll_wait2(const uint64_t *a, const uint64_t *b, const int (&idx)[N], uint64_t (&va)[N],
    uint64_t (&vb)[N], uint32_t tag, int *status) {
    const uint64_t ready = static_cast<uint64_t>(tag) << 32;
#pragma unroll
    for (int k = 0; k < N; ++k) {
        va[k] = idx[k] >= 0 ? ll_load(a + idx[k]) : ready;
        vb[k] = idx[k] >= 0 ? ll_load(b + idx[k]) : ready;
    }
    bool ok = true;
#pragma unroll
    for (int k = 0; k < N; ++k) ok = ok && tagged(va[k], tag) && tagged(vb[k], tag);
    if (ok) return true;
    return ll_wait(a, idx, va, tag, status) && ll_wait(b, idx, vb, tag, status);
}

// every thread of the workgroup agrees on failure (and on LDS reuse)
__device__ __forceinline__ bool wg_ok(bool ok) { return __syncthreads_count(ok ? 0 : 1) == 0; }

// ------------------------------------------------- quantized activation

enum class Pro { RMS, F32, GATED };

// Build the LDS Q8L activation (aq: u32 lanes, as: block scales) of a tagged
// vector: RMS = rms_norm(x, norm) (fortai_qwen35_cpu.f90:1408-1432), F32 = x,
// GATED = per-head gated RMSNorm of the GDN output with z
// (fortai_qwen35_cpu.f90:907-915); then fortai_q8_quantize.  Thread t owns
// the 4-value groups t + 256 i, so an 8-lane group is one Q8_0 block.
template <Pro PRO>
__device__ __forceinline__ bool build_act(const uint64_t *x, const uint64_t *z, const float *norm, int width, int head, float eps,
    uint32_t tag, int *status, uint32_t *aq, float *as, double *red) {
    const int tid = static_cast<int>(threadIdx.x);
    const int groups = width / 4, blocks = width / kQ8Block, chunks = (blocks + 3) / 4;
    const int iters = (groups + kT - 1) / kT;
    constexpr int N = 4 * kMaxIter;
    int ix[N];
#pragma unroll
    for (int it = 0; it < kMaxIter; ++it) {
        const int g = tid + it * kT;
#pragma unroll
        for (int j = 0; j < 4; ++j) ix[4 * it + j] = (it < iters && g < groups) ? 4 * g + j : -1;
    }
    // weights first (independent of the handoff)
    float4 w[kMaxIter];
#pragma unroll
    for (int it = 0; it < kMaxIter; ++it) {
        const int g = tid + it * kT;
        w[it] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (PRO != Pro::F32 && it < iters && g < groups)
            w[it] = *reinterpret_cast<const float4 *>(norm + (PRO == Pro::GATED ? (4 * g) % head : 4 * g));
    }
    uint64_t v[N];
    uint64_t vz[PRO == Pro::GATED ? N : 1];
    bool ok;
    if constexpr (PRO == Pro::GATED) ok = ll_wait2(x, z, ix, v, vz, tag, status);
    else ok = ll_wait(x, ix, v, tag, status);
    if (!wg_ok(ok)) return false;
    for (int b = blocks + tid; b < chunks * 4; b += kT) {
        as[b] = 0.0f;
        for (int l = 0; l < kLanesPerRow; ++l) aq[((b >> 2) * 8 + l) * 4 + (b & 3)] = 0u;
    }
    float4 y[kMaxIter];
#pragma unroll
    for (int it = 0; it < kMaxIter; ++it)
        y[it] = make_float4(ll_f(v[4 * it]), ll_f(v[4 * it + 1]), ll_f(v[4 * it + 2]), ll_f(v[4 * it + 3]));
    if constexpr (PRO == Pro::RMS) {
        double ss = 0.0;
#pragma unroll
        for (int it = 0; it < kMaxIter; ++it) {
            ss += static_cast<double>(y[it].x) * static_cast<double>(y[it].x);
            ss += static_cast<double>(y[it].y) * static_cast<double>(y[it].y);
            ss += static_cast<double>(y[it].z) * static_cast<double>(y[it].z);
            ss += static_cast<double>(y[it].w) * static_cast<double>(y[it].w);
        }
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        double total = 0.0;
        for (int k = 0; k < kW; ++k) total += red[k];
        const float inv = 1.0f / sqrtf(static_cast<float>(total / static_cast<double>(width)) + eps);
#pragma unroll
        for (int it = 0; it < kMaxIter; ++it) {
            y[it].x = (y[it].x * inv) * w[it].x;
            y[it].y = (y[it].y * inv) * w[it].y;
            y[it].z = (y[it].z * inv) * w[it].z;
            y[it].w = (y[it].w * inv) * w[it].w;
        }
    } else if constexpr (PRO == Pro::GATED) {
#pragma unroll
        for (int it = 0; it < kMaxIter; ++it) {
            double ss = static_cast<double>(y[it].x) * static_cast<double>(y[it].x);
            ss += static_cast<double>(y[it].y) * static_cast<double>(y[it].y);
            ss += static_cast<double>(y[it].z) * static_cast<double>(y[it].z);
            ss += static_cast<double>(y[it].w) * static_cast<double>(y[it].w);
            for (int m = 1; m < head / 4; m <<= 1) ss += __shfl_xor(ss, m);
            const float nf = sqrtf(static_cast<float>(ss / static_cast<double>(head)) + eps);
            const float4 zz = make_float4(ll_f(vz[4 * it]), ll_f(vz[4 * it + 1]), ll_f(vz[4 * it + 2]),
                ll_f(vz[4 * it + 3]));
            y[it].x = ((y[it].x / nf) * w[it].x) * silu_poly(zz.x);
            y[it].y = ((y[it].y / nf) * w[it].y) * silu_poly(zz.y);
            y[it].z = ((y[it].z / nf) * w[it].z) * silu_poly(zz.z);
            y[it].w = ((y[it].w / nf) * w[it].w) * silu_poly(zz.w);
        }
    }
#pragma unroll
    for (int it = 0; it < kMaxIter; ++it) {
        if (it >= iters) break;
        const int g = tid + it * kT;
        float scale;
        uint16_t bits;
        const uint32_t packed = quantize_group(y[it], scale, bits);
        if (g < groups) {
            const int b = g >> 3, l = g & 7;
            aq[((b >> 2) * 8 + l) * 4 + (b & 3)] = packed;
            if (l == 0) as[b] = scale;
        }
    }
    __syncthreads();
    return true;
}

// -------------------------------------------------------------- Q8_0 matvec

enum class Epi { STORE, ADD, SILU };

struct MvSrc {
    const uint64_t *x;      // tagged activation (GATED: raw GDN output)
    const uint64_t *z;      // GATED: gate pre-activation
    const float *norm;      // RMS: [width]; GATED: [head]
    const uint64_t *resid;  // ADD: residual words
    int width, head;
    float eps;
};

// Rows of the phase are 8-row groups over all segments; wave w of workgroup b
// takes groups (4b + w) + j * (4 grid), j < MAXRG, and loads their weights
// (NREG 16-byte chunks per lane) before it waits for the activation.
template <int NREG, int MAXRG, Pro PRO, Epi EPI>
__device__ __forceinline__ bool mv_phase(const PersistentMatvec &m, const MvSrc &src, uint32_t tag, int *status, unsigned char *lds,
    double *red) {
    constexpr bool kPair = EPI == Epi::SILU;
    const int total = kPair ? m.first_rg[1] : m.first_rg[m.count];
    if (static_cast<int>(blockIdx.x) * kW >= total) return true;  // no rows here (uniform in the workgroup)
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63, wave = tid >> 6, r = lane >> 3, l = lane & 7;
    const int gw = static_cast<int>(blockIdx.x) * kW + wave, nw = static_cast<int>(gridDim.x) * kW;
    const int chunks = (src.width / kQ8Block + 3) / 4;

    uint4 q[MAXRG][NREG], q2[kPair ? MAXRG : 1][kPair ? NREG : 1];
    uint2 sc[MAXRG][NREG], sc2[kPair ? MAXRG : 1][kPair ? NREG : 1];
    int seg[MAXRG], lrg[MAXRG];
#pragma unroll
    for (int j = 0; j < MAXRG; ++j) {
        const int grg = gw + j * nw;
        int s = 0;
        if (!kPair)
            while (s + 1 < m.count && grg >= m.first_rg[s + 1]) ++s;
        seg[j] = grg < total ? s : -1;
        lrg[j] = grg - m.first_rg[s];
        if (seg[j] < 0) continue;
        const Q8Matrix &w = m.w[s];
        const uint4 *qp = w.quants + static_cast<size_t>(lrg[j]) * w.chunks * 64 + lane;
        const uint2 *sp = w.scales + static_cast<size_t>(lrg[j]) * w.chunks * 8 + r;
#pragma unroll
        for (int c = 0; c < NREG; ++c) {
            if (c < w.chunks) {
                q[j][c] = load_stream(qp + static_cast<size_t>(c) * 64);
                sc[j][c] = load_stream(sp + static_cast<size_t>(c) * 8);
            }
        }
        if constexpr (kPair) {
            const Q8Matrix &w2 = m.w[1];
            const uint4 *qp2 = w2.quants + static_cast<size_t>(lrg[j]) * w2.chunks * 64 + lane;
            const uint2 *sp2 = w2.scales + static_cast<size_t>(lrg[j]) * w2.chunks * 8 + r;
#pragma unroll
            for (int c = 0; c < NREG; ++c) {
                if (c < w2.chunks) {
                    q2[j][c] = load_stream(qp2 + static_cast<size_t>(c) * 64);
                    sc2[j][c] = load_stream(sp2 + static_cast<size_t>(c) * 8);
                }
            }
        }
    }
    mark(0);
    // residual words of this lane's rows (published phases ago): loaded now, checked later
    uint64_t rres[MAXRG];
#pragma unroll
    for (int j = 0; j < MAXRG; ++j) {
        rres[j] = 0;
        if constexpr (EPI == Epi::ADD) {
            const int row = lrg[j] * kRowsPerWave + r;
            if (seg[j] >= 0 && l == 0 && row < m.w[seg[j]].rows) rres[j] = ll_load(src.resid + row);
        }
    }
    uint32_t *aq = reinterpret_cast<uint32_t *>(lds);
    float *as = reinterpret_cast<float *>(lds + static_cast<size_t>(chunks) * 128);
    if (!build_act<PRO>(src.x, src.z, src.norm, src.width, src.head, src.eps, tag, status, aq, as, red))
        return false;
    mark(1);

    const uint4 *act4 = reinterpret_cast<const uint4 *>(aq);
    const float4 *as4 = reinterpret_cast<const float4 *>(as);
    bool ok = true;
#pragma unroll
    for (int j = 0; j < MAXRG; ++j) {
        if (seg[j] < 0) continue;
        const Q8Matrix &w = m.w[seg[j]];
        float acc = 0.0f, acc2 = 0.0f;
#pragma unroll
        for (int c = 0; c < NREG; ++c) {
            if (c < w.chunks) {
                const uint4 a = act4[c * 8 + l];
                const float4 s4 = as4[c];
                acc = dot_chunk(q[j][c], sc[j][c], a, s4, acc);
                if constexpr (kPair) acc2 = dot_chunk(q2[j][c], sc2[j][c], a, s4, acc2);
            }
        }
        acc = row_hsum8(acc);
        if constexpr (kPair) acc2 = row_hsum8(acc2);
        if (j == 0) mark(2);
        const int row = lrg[j] * kRowsPerWave + r;
        if (l != 0 || row >= w.rows) continue;
        if constexpr (EPI == Epi::STORE) {
            ll_putf(m.out[seg[j]] + row, acc, tag);
        } else if constexpr (EPI == Epi::ADD) {
            uint64_t rv[1] = {rres[j]};
            if (!tagged(rv[0], tag)) {
                const int ix[1] = {row};
                if (!ll_wait(src.resid, ix, rv, tag, status)) { ok = false; continue; }
            }
            const float y = acc + ll_f(rv[0]);
            ll_putf(m.out[seg[j]] + row, y, tag);
            if (m.plain) m.plain[row] = y;
        } else {
            // fortai_silu_product: vector lanes for the first rows/8*8 rows,
            // the libm expression for the tail (fortai_q8_dot.c:492-505)
            const int vector_rows = (w.rows / 8) * 8;
            const float h = row < vector_rows ? silu_poly(acc) * acc2 : acc / (1.0f + exp_rounded(-acc)) * acc2;
            ll_putf(m.out[0] + row, h, tag);
        }
    }
    const bool all = wg_ok(ok);
    mark(3);
    return all;
}

// ------------------------------------------------------------------- embed

__device__ __forceinline__ void embed_phase(const PersistentPlan &P, int64_t token, uint32_t tag) {
    const int i = static_cast<int>(blockIdx.x) * kT + static_cast<int>(threadIdx.x);
    if (i >= P.hidden) return;
    float v;
    if (P.emb16) {
        v = gguf_half_to_real(P.emb16[token * P.hidden + i]);  // fortai_gguf_runtime.f90:324 (value())
    } else {
        const Q8Matrix &w = P.emb8;
        const int g = static_cast<int>(token >> 3), r = static_cast<int>(token & 7);
        const int b = i / kQ8Block, within = i % kQ8Block, l = within >> 2, byte = within & 3;
        const int c = b >> 2, j = b & 3;
        const uint32_t *q32 = reinterpret_cast<const uint32_t *>(w.quants);
        const uint32_t word = q32[((static_cast<size_t>(g) * w.chunks + c) * 64 + r * 8 + l) * 4 + j];
        const int8_t q = static_cast<int8_t>((word >> (8 * byte)) & 0xffu);
        const uint16_t *s16 = reinterpret_cast<const uint16_t *>(w.scales);
        const uint16_t sb = s16[((static_cast<size_t>(g) * w.chunks + c) * 8 + r) * 4 + j];
        v = half_bits_to_float(sb) * static_cast<float>(q);  // fortai_q8_dequantize_row
    }
    ll_putf(P.ll_x0 + i, v, tag);
}

// --------------------------------------------------------- Gated DeltaNet

// One unit = 8 state rows of one value head: conv1d + SiLU of the head's q/k
// channels (recomputed by each unit of the key head) and of its 8 v channels,
// L2 norms, decay/beta, and the delta rule on wave 0 (fortai_qwen35_cpu.f90:
// 856-906, fortai_q8_dot.c:356-398).  The conv window is only read here; it
// is shifted in the next phase, after every unit has read it.
template <int D>
__device__ __forceinline__ bool gdn_phase(const PersistentPlan &P, const PersistentLayer &L, uint32_t tag, int *status,
    unsigned char *lds, double *red) {
    constexpr int kCols = D / 8;
    const int VH = P.value_heads, KH = P.key_heads, K = P.kernel, C = P.conv_size, I = P.inner;
    const int ratio = VH / KH, units = VH * (D / 8), nch = 2 * D + 8;
    const int tid = static_cast<int>(threadIdx.x), wave = tid >> 6, lane = tid & 63;
    float *sq = reinterpret_cast<float *>(lds);  // q | k | v(8), contiguous
    float *sk = sq + D;
    float *sv = sk + D;
    float *hs = sv + 8;                          // beta, decay
    for (int u = static_cast<int>(blockIdx.x); u < units; u += static_cast<int>(gridDim.x)) {
        const int h = u / (D / 8), r0 = (u % (D / 8)) * 8, kh = h / ratio;
        auto chan = [&](int i) {
            return i < D ? kh * D + i : (i < 2 * D ? D * KH + kh * D + (i - D) : 2 * D * KH + h * D + r0 + (i - 2 * D));
        };
        // independent loads first: state rows, conv windows and taps, head scalars
        const int rr = r0 + (lane >> 3), l8 = lane & 7;
        float s[kCols];
        float4 *srow = reinterpret_cast<float4 *>(L.state + ((static_cast<size_t>(h) * D + rr) * 8 + l8) * kCols);
        if (wave == 0) {
#pragma unroll
            for (int i = 0; i < kCols / 4; ++i) {
                const float4 f = srow[i];
                s[4 * i] = f.x; s[4 * i + 1] = f.y; s[4 * i + 2] = f.z; s[4 * i + 3] = f.w;
            }
        }
        float win[2][kMaxKernel], cw[2][kMaxKernel];
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
            const int i = tid + k2 * kT;
            const int ch = i < nch ? chan(i) : 0;
#pragma unroll
            for (int sl = 0; sl < kMaxKernel; ++sl) {
                win[k2][sl] = (i < nch && sl < K - 1) ? L.conv_state[static_cast<size_t>(sl) * C + ch] : 0.0f;
                cw[k2][sl] = (i < nch && sl < K) ? L.conv_w[static_cast<size_t>(ch) * K + sl] : 0.0f;
            }
        }
        float a_h = 0.0f, dt_h = 0.0f;
        if (tid == kT - 1) { a_h = L.ssm_a[h]; dt_h = L.ssm_dt[h]; }
        int ix[4];
        ix[0] = tid < nch ? chan(tid) : -1;
        ix[1] = tid + kT < nch ? chan(tid + kT) : -1;
        ix[2] = tid == kT - 1 ? C + I + h : -1;        // alpha
        ix[3] = tid == kT - 1 ? C + I + VH + h : -1;   // beta
        uint64_t v[4];
        if (!wg_ok(ll_wait(L.ll_proj, ix, v, tag, status))) return false;
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
            const int i = tid + k2 * kT;
            if (i < nch) {
                // oldest slot first, current value last (fortai_qwen35_cpu.f90:856-867)
                float acc = 0.0f;
                float last = 0.0f;
#pragma unroll
                for (int sl = 0; sl < kMaxKernel; ++sl) {
                    if (sl < K - 1) acc = acc + cw[k2][sl] * win[k2][sl];
                    if (sl == K - 1) last = cw[k2][sl];
                }
                acc = acc + last * ll_f(v[k2]);
                sq[i] = silu_poly(acc);
            }
        }
        if (tid == kT - 1) {
            hs[0] = sigmoid_ref(ll_f(v[3]));
            hs[1] = exp_rounded(a_h * softplus_ref(ll_f(v[2]) + dt_h));
        }
        __syncthreads();
        if (tid < 128) {  // L2 norms of q (wave 0) and k (wave 1), fortai_qwen35_cpu.f90:1455-1471
            const float *vv = tid < 64 ? sq : sk;
            double ss = 0.0;
            for (int i = lane; i < D; i += 64) ss += static_cast<double>(vv[i]) * static_cast<double>(vv[i]);
            ss = wave_sum(ss);
            if (lane == 0) red[tid >> 6] = ss;
        }
        __syncthreads();
        if (tid < 2 * D) {
            const float n = sqrtf(static_cast<float>(red[tid < D ? 0 : 1]));
            sq[tid] = sq[tid] * (1.0f / (n > P.eps ? n : P.eps));
        }
        __syncthreads();
        if (wave == 0) {
            const float beta = hs[0], decay = hs[1];
            float kd = 0.0f;
#pragma unroll
            for (int i = 0; i < kCols; ++i) {
                const float d = s[i] * decay;
                s[i] = d;
                kd = __builtin_fmaf(d, sk[8 * i + l8], kd);
            }
            kd = row_hsum8(kd);
            const float delta = (sv[lane >> 3] - kd) * beta;
            float qd = 0.0f;
#pragma unroll
            for (int i = 0; i < kCols; ++i) {
                const float uu = __builtin_fmaf(delta, sk[8 * i + l8], s[i]);
                s[i] = uu;
                qd = __builtin_fmaf(uu, sq[8 * i + l8], qd);
            }
            qd = row_hsum8(qd);
#pragma unroll
            for (int i = 0; i < kCols / 4; ++i) srow[i] = make_float4(s[4 * i], s[4 * i + 1], s[4 * i + 2], s[4 * i + 3]);
            if (l8 == 0) ll_putf(L.ll_mid + h * D + rr, qd * (1.0f / sqrtf(static_cast<float>(D))), tag);
        }
        __syncthreads();
    }
    return true;
}

// Shift the conv windows (fortai_qwen35_cpu.f90:870-879) once every GDN unit
// of the layer has finished reading them: run during the gate/up phase by
// the workgroups that have no rows there, after they see the mixer output
// x1 (published only after every GDN unit did).  Without idle workgroups,
// every workgroup shifts a share after its rows.
__device__ __forceinline__ bool conv_shift(const PersistentPlan &P, const PersistentLayer &L, int first, int count,
    uint32_t tag, int *status) {
    const int C = P.conv_size, K = P.kernel;
    const int tid = static_cast<int>(threadIdx.x);
    const int me = static_cast<int>(blockIdx.x) - first;
    if (me < 0 || me * kT >= C) return true;
    constexpr int N = 4;  // hidden <= 1024
    int ix[N];
#pragma unroll
    for (int k = 0; k < N; ++k) ix[k] = tid + k * kT < P.hidden ? tid + k * kT : -1;
    uint64_t v[N];
    if (!wg_ok(ll_wait(L.ll_x1, ix, v, tag, status))) return false;
    bool ok = true;
    for (int ch = me * kT + tid; ch < C; ch += count * kT) {
        const int one[1] = {ch};
        uint64_t xv[1];
        if (!ll_wait(L.ll_proj, one, xv, tag, status)) { ok = false; break; }
        for (int sl = 0; sl + 1 < K - 1; ++sl)
            L.conv_state[static_cast<size_t>(sl) * C + ch] = L.conv_state[static_cast<size_t>(sl + 1) * C + ch];
        L.conv_state[static_cast<size_t>(K - 2) * C + ch] = ll_f(xv[0]);
    }
    return wg_ok(ok);
}

// -------------------------------------------------------------- attention

namespace ea = exact_attention;

struct ScoreLds {
    float qh[kMaxGroup * kMaxHead];
    float kn[kMaxHead];
    float vn[kMaxHead];
    float qw[kMaxHead];
    float kw[kMaxHead];
    float2 rs[kMaxHead / 2];
    uint16_t ktile[ea::kPosBlock][kMaxHead + 8];
    int overflow;
};
constexpr int kKLoads = ea::kPosBlock * (kMaxHead / 8) / kT;  // 16-byte key loads per thread

// Scores of one kv head's GQA group over 64 positions (exact_attention::score);
// the unit that holds pos normalises, rotates and appends the new key and
// value (fortai_qwen35_cpu.f90:990-1004, 1584-1604, float_to_half with ties
// away from zero).  The new value row and the overflow flag are stored with
// device-scope stores before the scores are published, so the output phase
// (other CUs) reads them after its wait.
__device__ __forceinline__ bool att_scores_phase(const PersistentPlan &P, const PersistentLayer &L, int pos,
    uint32_t tag, int *status, unsigned char *lds) {
    const int NKV = P.kv_heads, NH = P.heads, group = NH / NKV, HD = P.head_dim, VD = P.value_dim;
    const int positions = pos + 1, nblk = (positions + ea::kPosBlock - 1) / ea::kPosBlock;
    const int units = NKV * nblk;
    ScoreLds &S = *reinterpret_cast<ScoreLds *>(lds);
    const int tid = static_cast<int>(threadIdx.x), wave = tid >> 6, lane = tid & 63;
    const int half = P.rope_dim / 2;
    const float sqrt_head = sqrtf(static_cast<float>(HD));
    for (int u = static_cast<int>(blockIdx.x); u < units; u += static_cast<int>(gridDim.x)) {
        const int kvh = u / nblk, b = u % nblk;
        const int p0 = b * ea::kPosBlock, n = min(ea::kPosBlock, positions - p0);
        const bool owns_new = pos >= p0 && pos < p0 + n;
        // independent loads: the key rows, norm weights, the RoPE row, the overflow flag
        v4u kr[kKLoads];
        const int segs = HD / 8;
#pragma unroll
        for (int i = 0; i < kKLoads; ++i) {
            const int li = tid + i * kT;
            const int j = min(li / segs, n - 1), sg = li % segs;  // rows past n re-read row n-1 (in bounds)
            kr[i] = reinterpret_cast<const v4u *>(L.kcache + (static_cast<size_t>(p0 + j) * NKV + kvh) * HD)[sg];
        }
        float qwv = 0.0f, kwv = 0.0f;
        float2 rv = make_float2(0.0f, 0.0f);
        if (tid < HD) { qwv = L.q_norm[tid]; kwv = L.k_norm[tid]; }
        if (tid < half) rv = L.rope[static_cast<size_t>(pos) * half + tid];
        const int flag = __hip_atomic_load(L.cache_flags + kvh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int koff = 2 * NH * HD, voff = koff + NKV * HD;
        int ix[6];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = tid + k * kT;
            ix[k] = i < group * HD ? (kvh * group + i / HD) * 2 * HD + i % HD : -1;
        }
        ix[4] = owns_new && tid < HD ? koff + kvh * HD + tid : -1;
        ix[5] = owns_new && tid < VD ? voff + kvh * VD + tid : -1;
        uint64_t v[6];
        if (!wg_ok(ll_wait(L.ll_proj, ix, v, tag, status))) return false;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = tid + k * kT;
            if (i < group * HD) S.qh[i] = ll_f(v[k]);
        }
        if (tid < HD) { S.kn[tid] = ll_f(v[4]); S.qw[tid] = qwv; S.kw[tid] = kwv; }
        if (tid < VD) S.vn[tid] = ll_f(v[5]);
        if (tid < half) S.rs[tid] = rv;
        if (tid == 0) S.overflow = 0;
#pragma unroll
        for (int i = 0; i < kKLoads; ++i) {
            const int li = tid + i * kT;
            const int j = li / segs, sg = li % segs;
            if (j < n) *reinterpret_cast<v4u *>(&S.ktile[j][sg * 8]) = kr[i];
        }
        __syncthreads();
        for (int sl = wave; sl < group + (owns_new ? 1 : 0); sl += kW) {
            if (sl < group) ea::norm_rope(S.qh + sl * HD, HD, S.qw, P.eps, S.rs, P.rope_dim, lane);
            else ea::norm_rope(S.kn, HD, S.kw, P.eps, S.rs, P.rope_dim, lane);
        }
        __syncthreads();
        if (owns_new) {
            if (tid < HD) {
                const uint16_t kb = float_to_half_kv(S.kn[tid]);
                L.kcache[(static_cast<size_t>(pos) * NKV + kvh) * HD + tid] = kb;
                S.ktile[pos - p0][tid] = kb;
                if ((kb & 0x7c00u) == 0x7c00u) S.overflow = 1;
            }
            if (2 * tid < VD) {  // value pairs, device-scope (read by other CUs in the next phase)
                const uint16_t a = float_to_half_kv(S.vn[2 * tid]), c = float_to_half_kv(S.vn[2 * tid + 1]);
                uint32_t *dst = reinterpret_cast<uint32_t *>(L.vcache + (static_cast<size_t>(pos) * NKV + kvh) * VD);
                __hip_atomic_store(dst + tid, static_cast<uint32_t>(a) | (static_cast<uint32_t>(c) << 16),
                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if ((a & 0x7c00u) == 0x7c00u || (c & 0x7c00u) == 0x7c00u) S.overflow = 1;
            }
            __syncthreads();
            if (tid == 0 && S.overflow)
                __hip_atomic_store(L.cache_flags + kvh, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // the stores above have completed
        }
        __syncthreads();
        const bool finite = flag == 0 && S.overflow == 0;
        const int gi = tid >> 6, j = tid & 63;
        if (gi < group && j < n) {
            const float sc = finite ? ea::score<true>(S.qh + gi * HD, &S.ktile[j][0], HD, sqrt_head)
                                    : ea::score<false>(S.qh + gi * HD, &S.ktile[j][0], HD, sqrt_head);
            ll_putf(L.ll_mid + static_cast<size_t>(kvh * group + gi) * P.max_context + p0 + j, sc, tag);
        }
        __syncthreads();
    }
    return true;
}

// Softmax weights and the P.V chains of one head x 8 value dims
// (exact_attention::softmax_weights / pv_chains), then the sigmoid gate
// (fortai_qwen35_cpu.f90:1030-1031).
__device__ __forceinline__ bool att_output_phase(const PersistentPlan &P, const PersistentLayer &L, int pos,
    uint32_t tag, int *status, unsigned char *lds) {
    const int NKV = P.kv_heads, NH = P.heads, group = NH / NKV, HD = P.head_dim, VD = P.value_dim;
    const int slices = VD / ea::kDims, units = NH * slices;
    const int positions = pos + 1;
    const int tid = static_cast<int>(threadIdx.x);
    float *sw = reinterpret_cast<float *>(lds);
    float *work = sw + ea::sw_floats(P.max_context);
    for (int u = static_cast<int>(blockIdx.x); u < units; u += static_cast<int>(gridDim.x)) {
        const int h = u / slices, d0 = (u % slices) * ea::kDims, kvh = h / group;
        constexpr int N = 24;  // positions <= 6144
        int ix[N];
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const int p = tid + k * kT;
            ix[k] = p < positions ? h * P.max_context + p : -1;
        }
        uint64_t v[N];
        bool ok = ll_wait(L.ll_mid, ix, v, tag, status);
        int gx[1] = {tid < ea::kDims ? h * 2 * HD + HD + d0 + tid : -1};
        uint64_t gv[1];
        if (ok) ok = ll_wait(L.ll_proj, gx, gv, tag, status);
        if (!wg_ok(ok)) return false;
#pragma unroll
        for (int k = 0; k < N; ++k)
            if (ix[k] >= 0) sw[tid + k * kT] = ll_f(v[k]);
        const int flag = __hip_atomic_load(L.cache_flags + kvh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint16_t *vbase = L.vcache + static_cast<size_t>(kvh) * VD + d0;
        const size_t vstride = static_cast<size_t>(NKV) * VD;
        ea::ValuePieces vp;
        ea::value_prefetch(vbase, vstride, positions, vp);
        __syncthreads();
        mark(0);
        const float acc = flag == 0 ? ea::attend<true>(sw, positions, vbase, vstride, work, vp)
                                    : ea::attend<false>(sw, positions, vbase, vstride, work, vp);
        mark(3);
        if (tid < ea::kDims) ll_putf(L.ll_ao + h * VD + d0 + tid, acc * sigmoid_ref(ll_f(gv[0])), tag);
        __syncthreads();
    }
    return true;
}

// ------------------------------------------------------------------ kernel

enum Op : int { EMBED, PROJ, GDN64, GDN128, GOUT, NOP, ATT, MERGE, AOUT, FFN1, FFN2 };

// The layers of one step as a flat list of phases (each case inlined, so only
// the loop state is live across phases).  The plan and the descriptor of the
// current layer live in LDS: layer li + 1's descriptor is fetched into a
// register while layer li runs and stored at its end.
__global__ __launch_bounds__(kT) void decode_persistent_kernel(const PersistentPlan *__restrict__ plan,
    const uint32_t tag) {
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ double red[kW];
    constexpr int kPlanWords = sizeof(PersistentPlan) / 4, kLayerWords = sizeof(PersistentLayer) / 4;
    static_assert(kPlanWords <= kT && kLayerWords <= kT, "one word per thread");
    __shared__ __align__(16) uint32_t s_plan_words[kPlanWords];
    __shared__ __align__(16) uint32_t s_layer_words[2][kLayerWords];
    PersistentPlan &s_plan = *reinterpret_cast<PersistentPlan *>(s_plan_words);
    PersistentLayer *s_layer = reinterpret_cast<PersistentLayer *>(&s_layer_words[0][0]);
    const int tid = static_cast<int>(threadIdx.x);
    if (tid < kPlanWords) reinterpret_cast<uint32_t *>(&s_plan)[tid] = reinterpret_cast<const uint32_t *>(plan)[tid];
    if (tid < kLayerWords)
        reinterpret_cast<uint32_t *>(&s_layer[0])[tid] = reinterpret_cast<const uint32_t *>(plan->layer)[tid];
    __syncthreads();
    const PersistentPlan &P = s_plan;
    int *status = P.status;
    const int pos = *P.position;
    const int64_t token = *P.token;
    const int vocab_in = P.emb16 ? P.vocab : P.emb8.rows;
    if (pos < 0 || pos >= P.max_context || token < 0 || token >= vocab_in) {
        if (blockIdx.x == 0 && tid == 0) atomicOr(status, 2);
        return;
    }
    const int ops = P.layers * 6 + 1;
    if (tid == 0) { g_marks = P.phase_marks; g_mark_stride = ops + 1; }
    __syncthreads();
    uint32_t next_word = 0;
    for (int k = 0; k < ops; ++k) {
        if (tid == 0) s_phase = k;
        // op k: 0 embed; then 6 slots per layer
        int op, li = 0, slot = 0;
        if (k == 0) {
            op = EMBED;
        } else {
            li = (k - 1) / 6;
            slot = (k - 1) % 6;
            const bool rec = s_layer[li & 1].recurrent != 0;
            switch (slot) {
            case 0: op = PROJ; break;
            case 1: op = rec ? (P.head == 64 ? GDN64 : GDN128) : ATT; break;
            case 2: op = rec ? GOUT : MERGE; break;
            case 3: op = rec ? NOP : AOUT; break;
            case 4: op = FFN1; break;
            default: op = FFN2; break;
            }
            if (slot == 0 && li + 1 < P.layers && tid < kLayerWords)
                next_word = reinterpret_cast<const uint32_t *>(P.layer + li + 1)[tid];
        }
        const PersistentLayer &L = s_layer[li & 1];
        const uint64_t *xin = li == 0 ? P.ll_x0 : s_layer[(li - 1) & 1].ll_x2;
        bool ok = true;
        switch (op) {
        case EMBED: embed_phase(P, token, tag); break;
        case PROJ: {
            MvSrc in{};
            in.x = xin; in.norm = L.attn_norm; in.width = P.hidden; in.eps = P.eps;
            ok = mv_phase<8, 2, Pro::RMS, Epi::STORE>(L.proj, in, tag, status, lds, red);
            break;
        }
        case GDN64: ok = gdn_phase<64>(P, L, tag, status, lds, red); break;
        case GDN128: ok = gdn_phase<128>(P, L, tag, status, lds, red); break;
        case GOUT: {
            MvSrc mix{};
            mix.x = L.ll_mid; mix.z = L.ll_proj + P.conv_size; mix.norm = L.ssm_norm; mix.resid = xin;
            mix.width = P.inner; mix.head = P.head; mix.eps = P.eps;
            ok = mv_phase<16, 1, Pro::GATED, Epi::ADD>(L.outp, mix, tag, status, lds, red);
            break;
        }
        case NOP: break;  // the conv shift runs inside FFN1 of the recurrent layer
        case ATT: ok = wg_ok(att_scores_phase(P, L, pos, tag, status, lds)); break;
        case MERGE: ok = wg_ok(att_output_phase(P, L, pos, tag, status, lds)); break;
        case AOUT: {
            MvSrc mix{};
            mix.x = L.ll_ao; mix.resid = xin; mix.width = P.heads * P.value_dim; mix.eps = P.eps;
            ok = mv_phase<16, 1, Pro::F32, Epi::ADD>(L.outp, mix, tag, status, lds, red);
            break;
        }
        case FFN1: {
            MvSrc f1{};
            f1.x = L.ll_x1; f1.norm = L.post_norm; f1.width = P.hidden; f1.eps = P.eps;
            ok = mv_phase<8, 1, Pro::RMS, Epi::SILU>(L.ffn1, f1, tag, status, lds, red);
            if (ok && L.recurrent) {
                const int busy = (L.ffn1.first_rg[1] + kW - 1) / kW;  // workgroups with gate/up rows
                const int G = static_cast<int>(gridDim.x);
                ok = busy < G ? conv_shift(P, L, busy, G - busy, tag, status) : conv_shift(P, L, 0, G, tag, status);
            }
            break;
        }
        default: {
            MvSrc f2{};
            f2.x = L.ll_h; f2.resid = L.ll_x1; f2.width = P.ffn; f2.eps = P.eps;
            ok = mv_phase<28, 1, Pro::F32, Epi::ADD>(L.ffn2, f2, tag, status, lds, red);
            break;
        }
        }
        if (!ok) return;
        if (slot == 5 && li + 1 < P.layers) {
            __syncthreads();  // every thread is done with the old descriptor slot
            if (tid < kLayerWords) reinterpret_cast<uint32_t *>(&s_layer[(li + 1) & 1])[tid] = next_word;
            __syncthreads();
        }
        if (P.phase_times && tid == 0) P.phase_times[static_cast<size_t>(blockIdx.x) * (ops + 1) + k] = wall_clock64();
    }
}

}  // namespace

size_t persistent_lds_bytes() { return kLdsBytes; }

int persistent_blocks_per_cu() {
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, decode_persistent_kernel, kT, kLdsBytes) != hipSuccess)
        return 0;
    return blocks;
}

const char *persistent_unsupported(const PersistentPlan &P, int grid) {
    if (grid <= 0 || grid > kT) return "grid must be 1..256 workgroups";
    if (P.hidden % 64 || P.hidden > 1024) return "hidden size must be a multiple of 64, at most 1024";
    if (P.ffn % kQ8Block || P.ffn > 3584 || P.ffn / 8 > grid * kW) return "FFN width out of range";
    if (P.hidden / 8 > grid * kW) return "hidden rows exceed one row group per wave";
    if (sizeof(ScoreLds) > kLdsBytes) return "attention LDS";
    if (P.heads > 0 && P.max_context > 24 * kT) return "context longer than the persistent output phase holds";
    if (P.heads > 0 && exact_attention::output_lds_floats(P.max_context) * sizeof(float) > kLdsBytes)
        return "attention output LDS";
    for (int li = 0; li < P.layers; ++li) {
        (void)li;
    }
    if (P.value_heads > 0) {
        if (P.head != 64 && P.head != 128) return "GDN head size must be 64 or 128";
        if (P.kernel < 2 || P.kernel > kMaxKernel) return "conv kernel out of range";
        if (P.inner % kQ8Block || P.inner > 2048 || P.inner != P.value_heads * P.head) return "GDN inner size";
        if (P.value_heads % P.key_heads) return "GDN head groups";
    }
    if (P.heads > 0) {
        const int group = P.heads / P.kv_heads;
        if (P.heads % P.kv_heads || group > kMaxGroup) return "GQA group out of range";
        if (P.kv_heads <= 0 || P.head_dim % 8 || P.head_dim > kMaxHead || P.value_dim % 64 || P.value_dim > kMaxHead ||
            P.value_dim > P.head_dim || P.value_dim > 2 * kT)
            return "head dims";
        if (P.heads * P.value_dim > 2048) return "attention output width";
        if (P.rope_dim > P.head_dim || P.rope_dim % 2) return "rope dimension";
        if (group * P.head_dim > 4 * kT) return "q words per unit";
    }
    return "";
}

hipError_t launch_decode_persistent(const PersistentPlan *plan_device, uint32_t tag, int grid, hipStream_t stream) {
    hipLaunchKernelGGL(decode_persistent_kernel, dim3(grid), dim3(kT), kLdsBytes, stream, plan_device, tag);
    note_launch("decode_persistent_kernel grid %d", grid);
    return hipGetLastError();
}

}  // namespace fortai_hip
