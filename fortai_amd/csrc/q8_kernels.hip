// Q8_0 matrix-vector kernels for gfx950 (wave64).
//
// Arithmetic contract (bit-exact with the reference's AVX2 CPU dot,
// src/backend/cpu/fortai_q8_dot.c:287-331): a row is owned by 8 lanes of a
// wave; lane l holds the fp32 accumulator of products 4l..4l+3 of every
// block and applies, block by block in order,
//     acc_l = fma(f32(w_scale_b) * a_scale_b, (float)dot4(w_b[4l..], a_b[4l..]), acc_l)
// with the int8 dot on v_dot4c_i32_i8 (exact; the reference's pmaddubsw can
// only saturate for activations of -128, which the quantizer never emits).
// The 8 lanes are then summed in the AVX2 horizontal-sum order.
//
// HBM layout (repacked once at upload, same 34 B per 32 values as GGUF):
//   quants[(g * chunks + c) * 64 + r * 8 + l]  (16 B) = for j = 0..3 the
//       bytes 4l..4l+3 of block 4c+j of row 8g+r;
//   scales[(g * chunks + c) * 8 + r]            (8 B) = the 4 fp16 scales.
// One 64-lane load instruction therefore reads 1 KiB of contiguous quants
// (8 full 128-byte lines) and 64 contiguous bytes of scales, and every lane
// receives exactly the operands of its own fp32 accumulator.
//
// Latency structure: a wave first issues every weight load of its 8 rows
// (the whole row slice, up to 32 chunks, held in VGPRs), then builds the
// quantized activation in LDS while those loads are in flight.  The
// activation comes from the producer already quantized (Q8L layout, a
// 16-byte copy), or is quantized in-workgroup from fp32 (fortai_q8_quantize,
// fortai_q8_dot.c:153-198), optionally after the RMSNorm of
// fortai_qwen35_cpu.f90:1408-1432.
#include "fortai_hip_internal.h"
#include "fortai_hip_kernels.h"

#include <algorithm>

#ifndef FORTAI_MV_MARK
#define FORTAI_MV_MARK(i)
#endif

namespace fortai_hip {

namespace {

struct MatvecArgs {
    MatvecSegment seg[4];
    int first_wg[5];
    int count;
    int chunks;            // activation chunks (ceil(blocks / 4))
    int pair_vector_rows;  // SILU_PAIR: rows below this use the vector SiLU lane
    MatvecInput in;
};

__device__ __forceinline__ uint32_t load_u32_unaligned(const int8_t *p) {
    const uint8_t *b = reinterpret_cast<const uint8_t *>(p);
    return static_cast<uint32_t>(b[0]) | (static_cast<uint32_t>(b[1]) << 8) |
        (static_cast<uint32_t>(b[2]) << 16) | (static_cast<uint32_t>(b[3]) << 24);
}

// Build the workgroup's LDS copy of the quantized activation (Q8L layout).
// The activation of a matvec is read before the weights, into registers
// (act_fetch), and stored to LDS after the weight loads are issued
// (act_store): the compiler's in-order vmcnt waits for the activation then do
// not wait for the weights.
constexpr int kMaxChunks = 96;  // Q8L activations up to 12288 wide

template <int THREADS, Prologue PRO>
struct ActShape {
    static constexpr int kQ8L = (kMaxChunks * 9 + THREADS - 1) / THREADS;  // 16-byte pieces per thread
    static constexpr int kPre = 8;                                          // float4 groups per thread
    static constexpr bool kF32 = PRO == Prologue::F32 || PRO == Prologue::RMSNORM || PRO == Prologue::GATED;
    static constexpr int kQ = PRO == Prologue::Q8L ? kQ8L : 1;
    static constexpr int kX = kF32 ? kPre : 1;
    static constexpr int kW = PRO == Prologue::RMSNORM || PRO == Prologue::GATED ? kPre : 1;
    static constexpr int kZ = PRO == Prologue::GATED ? kPre : 1;
};

template <int THREADS, Prologue PRO, int NQ, int NX, int NW, int NZ>
__device__ __forceinline__ void act_fetch(const MatvecInput &in, int chunks, u32x4_t (&q8l)[NQ], float4 (&xr)[NX],
    float4 (&wr)[NW], float4 (&zr)[NZ]) {
    using A = ActShape<THREADS, PRO>;
    const int tid = static_cast<int>(threadIdx.x);
    if constexpr (PRO == Prologue::Q8L) {
        const u32x4_t *src = reinterpret_cast<const u32x4_t *>(in.xq8l);
        // clamped: every load is in bounds; the trip count is uniform
        const int last = chunks * 9 - 1, iters = (last + THREADS) / THREADS;
#pragma unroll
        for (int k = 0; k < A::kQ8L; ++k)
            if (k < iters) q8l[k] = src[min(tid + k * THREADS, last)];
    } else if constexpr (A::kF32) {
        const int groups = in.width / 4;
        const float4 *x4 = reinterpret_cast<const float4 *>(in.x);
        const float4 *w4 = reinterpret_cast<const float4 *>(in.norm);
        const float4 *z4 = reinterpret_cast<const float4 *>(in.z);
        const int iters = (groups + THREADS - 1) / THREADS;  // uniform
#pragma unroll
        for (int k = 0; k < A::kPre; ++k) {
            if (k < iters) {
                const int g = min(tid + k * THREADS, groups - 1);  // clamped; duplicates are masked below
                xr[k] = x4[g];
                if constexpr (PRO == Prologue::RMSNORM) wr[k] = w4[g];
                if constexpr (PRO == Prologue::GATED) {
                    wr[k] = w4[g % (in.head / 4)];
                    zr[k] = z4[g];
                }
            }
        }
    }
}

template <int THREADS, Prologue PRO, int NQ, int NX, int NW, int NZ>
__device__ __forceinline__ void act_store(const MatvecInput &in, int chunks, const u32x4_t (&q8l)[NQ],
    const float4 (&xr)[NX], const float4 (&wr)[NW], const float4 (&zr)[NZ], uint32_t *act32, float *act_s,
    double *red) {
    using A = ActShape<THREADS, PRO>;
    const int tid = static_cast<int>(threadIdx.x);
    const int groups = in.width / 4;
    const int blocks = in.width / kQ8Block;
    if constexpr (PRO == Prologue::Q8L) {
        u32x4_t *dst = reinterpret_cast<u32x4_t *>(act32);
        const int iters = (chunks * 9 + THREADS - 1) / THREADS;
#pragma unroll
        for (int k = 0; k < A::kQ8L; ++k) {
            const int i = tid + k * THREADS;
            if (k < iters && i < chunks * 9) dst[i] = q8l[k];
        }
        __syncthreads();
        return;
    } else {
        for (int b = blocks + tid; b < chunks * 4; b += THREADS) {
            act_s[b] = 0.0f;
            for (int l = 0; l < kLanesPerRow; ++l) act32[((b >> 2) * 8 + l) * 4 + (b & 3)] = 0u;
        }
        if constexpr (PRO == Prologue::Q8) {
            for (int g = tid; g < groups; g += THREADS) {
                const int b = g >> 3, l = g & 7;
                const int8_t *block = in.xq + static_cast<size_t>(b) * kQ8Bytes;
                act32[((b >> 2) * 8 + l) * 4 + (b & 3)] = load_u32_unaligned(block + 2 + 4 * l);
                if (l == 0) {
                    const uint8_t *sb = reinterpret_cast<const uint8_t *>(block);
                    act_s[b] = half_bits_to_float(static_cast<uint16_t>(sb[0] | (sb[1] << 8)));
                }
            }
            __syncthreads();
            return;
        } else {
            // widths up to kPre * THREADS * 4 are held in registers
            float inverse_rms = 1.0f;
            if constexpr (PRO == Prologue::RMSNORM) {
                double ss = 0.0;
                const int iters = (groups + THREADS - 1) / THREADS;
#pragma unroll
                for (int k = 0; k < A::kPre; ++k) {
                    if (k >= iters) break;
                    double t = static_cast<double>(xr[k].x) * static_cast<double>(xr[k].x);
                    t += static_cast<double>(xr[k].y) * static_cast<double>(xr[k].y);
                    t += static_cast<double>(xr[k].z) * static_cast<double>(xr[k].z);
                    t += static_cast<double>(xr[k].w) * static_cast<double>(xr[k].w);
                    ss += tid + k * THREADS < groups ? t : 0.0;
                }
                ss = wave_sum(ss);
                if constexpr (THREADS > 64) {
                    if ((tid & 63) == 0) red[tid >> 6] = ss;
                    __syncthreads();
                    ss = 0.0;
                    for (int w = 0; w < THREADS / 64; ++w) ss += red[w];
                }
                const float mean = static_cast<float>(div_count(ss, in.width));
                inverse_rms = 1.0f / sqrtf(mean + in.eps);
            }
            const int iters = (groups + THREADS - 1) / THREADS;
#pragma unroll
            for (int k = 0; k < A::kPre; ++k) {
                if (k >= iters) break;
                const int g = tid + k * THREADS;
                float4 y = xr[k];
                if constexpr (PRO == Prologue::RMSNORM) {
                    y.x = (y.x * inverse_rms) * wr[k].x;
                    y.y = (y.y * inverse_rms) * wr[k].y;
                    y.z = (y.z * inverse_rms) * wr[k].z;
                    y.w = (y.w * inverse_rms) * wr[k].w;
                } else if constexpr (PRO == Prologue::GATED) {
                    // a head is head/4 consecutive lanes (aligned): its sum of
                    // squares in double over those lanes, then the gate
                    double ss = static_cast<double>(y.x) * static_cast<double>(y.x);
                    ss += static_cast<double>(y.y) * static_cast<double>(y.y);
                    ss += static_cast<double>(y.z) * static_cast<double>(y.z);
                    ss += static_cast<double>(y.w) * static_cast<double>(y.w);
                    ss = group_sum_up(ss, in.head / 4);
                    const float nf = sqrtf(static_cast<float>(div_count(ss, in.head)) + in.eps);
                    y.x = ((y.x / nf) * wr[k].x) * zr[k].x;
                    y.y = ((y.y / nf) * wr[k].y) * zr[k].y;
                    y.z = ((y.z / nf) * wr[k].z) * zr[k].z;
                    y.w = ((y.w / nf) * wr[k].w) * zr[k].w;
                }
                float scale;
                uint16_t bits;
                const uint32_t packed = quantize_group(y, scale, bits);
                if (g < groups) {
                    const int b = g >> 3, l = g & 7;
                    act32[((b >> 2) * 8 + l) * 4 + (b & 3)] = packed;
                    if (l == 0) act_s[b] = scale;
                }
            }
            __syncthreads();
        }
    }
}

// NREG > 0: every chunk of the row slice (<= NREG) is loaded into registers
// before the activation is built; NREG == 0 streams batches of 8 chunks.
template <int THREADS, Prologue PRO>
__device__ __forceinline__ void build_activation(const MatvecInput &in, int chunks, uint32_t *act32, float *act_s,
    double *red) {
    using A = ActShape<THREADS, PRO>;
    u32x4_t q8l[A::kQ];
    float4 xr[A::kX], wr[A::kW], zr[A::kZ];
    act_fetch<THREADS, PRO>(in, chunks, q8l, xr, wr, zr);
    act_store<THREADS, PRO>(in, chunks, q8l, xr, wr, zr, act32, act_s, red);
}

// One wave per 8-row group, eight lanes per row.
// NREG > 0: the matrix has exactly NREG chunks per row, all held in
// registers; NREG = 0: any width, weights streamed in batches of 8 chunks.
// MULTI: several segments share the activation (a workgroup finds its
// segment in first_wg); otherwise segment 0 only, so that every kernel
// argument the waves read has a fixed offset and all of them arrive in one
// scalar round trip.
// SPLIT: the four waves share one 8-row group, wave w loading chunks
// [w NREG/4, (w+1) NREG/4); waves 1..3 hand wave 0, through LDS, each of
// their blocks' scale product fl(f32(w_scale) * a_scale) and lane dot, and
// wave 0 runs every lane's fma chain over all blocks in order (the same
// operations as the unsplit chain).  A workgroup then moves a quarter of
// the bytes and a wave issues a quarter of the dot work.
template <int WAVES, int NREG, Prologue PRO, Epilogue EPI, bool MULTI, bool SPLIT>
__global__ __launch_bounds__(WAVES * 64) void q8_matvec_kernel(const MatvecArgs args) {
    FORTAI_TRACE_SCOPE(1);
    constexpr bool kPair = EPI == Epilogue::SILU_PAIR;
    static_assert(!SPLIT || (WAVES == 4 && NREG > 0 && NREG % 4 == 0 && !MULTI && !kPair), "split form");
    constexpr int kPer = SPLIT ? NREG / 4 : NREG;  // chunks this wave loads
    constexpr int kRegs = kPer > 0 ? kPer : 1;
    // unsplit, whole groups of 8 chunks: the weight scales come in one load
    // per 8 chunks (lane (r, l) takes chunk l of row r, 512 contiguous bytes)
    // instead of one 64-byte load per chunk, and go through the wave's own
    // LDS slice, from which the 8 lanes of a row read each chunk's scales
    // (split: the wave's kPer <= 8 chunks in one load, lanes past kPer clamped)
    constexpr bool kScLds = NREG > 0 && (SPLIT ? kPer <= 8 : NREG % 8 == 0);
    constexpr int kScLoads = kScLds ? (SPLIT ? 1 : NREG / 8) : 1;
    extern __shared__ __align__(16) unsigned char lds[];
    uint32_t *act32 = reinterpret_cast<uint32_t *>(lds);
    float *act_s = reinterpret_cast<float *>(lds + static_cast<size_t>(args.chunks) * 8 * 16);
    double *red = reinterpret_cast<double *>(lds + static_cast<size_t>(args.chunks) * 144);
    float *epi = reinterpret_cast<float *>(lds + static_cast<size_t>(args.chunks) * 144 + 8 * WAVES);
    // SPLIT: [wave - 1][chunk][scales, dots][lane], then (kScLds) each wave's
    // 512 scale bytes; unsplit kScLds: [wave][w, w2][chunk / 8][lane] scales
    float4 *handoff = reinterpret_cast<float4 *>(lds + static_cast<size_t>(args.chunks) * 144 + 40 * WAVES);

    FORTAI_MV_MARK(5);
    kernarg_warm<sizeof(MatvecArgs)>();
    const int wg = static_cast<int>(blockIdx.x);
    int s = 0;
    if constexpr (MULTI)
        while (s + 1 < args.count && wg >= args.first_wg[s + 1]) ++s;
    const MatvecSegment &seg = args.seg[s];
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int rg = SPLIT ? wg - args.first_wg[s] : (wg - args.first_wg[s]) * WAVES + wave;
    const bool active = rg < seg.w.row_groups;
    const int rgc = active ? rg : seg.w.row_groups - 1;  // excess waves re-read the last group, write nothing
    const int r = lane >> 3, l = lane & 7;
    const int chunks = seg.w.chunks;
    const int c_first = SPLIT ? wave * kPer : 0;
    const uint4 *qp = seg.w.quants + (static_cast<size_t>(rgc) * chunks + c_first) * 64 + lane;
    const uint2 *sp = seg.w.scales + (static_cast<size_t>(rgc) * chunks + c_first) * 8 + r;
    const uint4 *qp2 = kPair ? seg.w2.quants + static_cast<size_t>(rgc) * chunks * 64 + lane : nullptr;
    const uint2 *sp2 = kPair ? seg.w2.scales + static_cast<size_t>(rgc) * chunks * 8 + r : nullptr;

    FORTAI_MV_MARK(0);
    // The epilogue's own inputs first: the compiler's in-order load counter
    // cannot count loads under a condition, so one issued after the weights
    // would make the prologue's wait for the activation also wait for most
    // of the weights.  The residual is loaded by every lane (row clamped),
    // the conv window and taps by every lane of a conv wave.
    const int row = rg * kRowsPerWave + r;
    const int rowc = min(row, seg.w.rows - 1);
    const bool writer = active && l == 0 && row < seg.w.rows && (!SPLIT || wave == 0);
    float resid = 0.0f;  // used after the dot
    if constexpr (EPI == Epilogue::ADD) resid = seg.resid[rowc];
    float win[kConvMax - 1], taps[kConvMax];
    // (row groups are whole 8-row groups, so conv and SiLU are uniform per wave)
    const bool conv = EPI == Epilogue::STORE && seg.conv_w != nullptr && (seg.conv_rows == 0 || row < seg.conv_rows);
    const int ck = conv ? seg.kernel : 0;
    if (conv) {
#pragma unroll
        for (int t = 0; t < kConvMax; ++t) {
            if (t < ck - 1) win[t] = seg.conv_state[static_cast<size_t>(t) * seg.conv_size + rowc];
            if (t < ck) taps[t] = seg.conv_w[static_cast<size_t>(rowc) * ck + t];
        }
    }
    using AS = ActShape<WAVES * 64, PRO>;
    u32x4_t act_q[AS::kQ];
    float4 act_x[AS::kX], act_w[AS::kW], act_z[AS::kZ];
    act_fetch<WAVES * 64, PRO>(args.in, args.chunks, act_q, act_x, act_w, act_z);
    uint4 q[kRegs], q2[kPair ? kRegs : 1];
    uint2 sc[kScLds ? 1 : kRegs], sc2[kPair && !kScLds ? kRegs : 1];
    uint2 scw[kScLoads], scw2[kPair ? kScLoads : 1];
    if constexpr (kScLds) {
        const int lc = SPLIT ? c_first + min(l, kPer - 1) : l;
        const size_t sb = (static_cast<size_t>(rgc) * chunks + lc) * 8 + r;
#pragma unroll
        for (int k = 0; k < kScLoads; ++k) {
            scw[k] = load_stream(seg.w.scales + sb + k * 64);
            if constexpr (kPair) scw2[k] = load_stream(seg.w2.scales + sb + k * 64);
        }
    }
    if constexpr (NREG > 0) {
#pragma unroll
        for (int c = 0; c < kPer; ++c) {
            q[c] = load_stream(qp + static_cast<size_t>(c) * 64);
            if constexpr (!kScLds) sc[c] = load_stream(sp + static_cast<size_t>(c) * 8);
            if constexpr (kPair) {
                q2[c] = load_stream(qp2 + static_cast<size_t>(c) * 64);
                if constexpr (!kScLds) sc2[c] = load_stream(sp2 + static_cast<size_t>(c) * 8);
            }
        }
    }
    FORTAI_MV_MARK(1);
    act_store<WAVES * 64, PRO>(args.in, args.chunks, act_q, act_x, act_w, act_z, act32, act_s, red);
    FORTAI_MV_MARK(2);

    const uint4 *act4 = reinterpret_cast<const uint4 *>(act32);
    const float4 *as4 = reinterpret_cast<const float4 *>(act_s);
    float acc = 0.0f, acc2 = 0.0f;
    if constexpr (SPLIT) {
        uint2 *ws = reinterpret_cast<uint2 *>(handoff + 3 * kPer * 128) + wave * 64;
        auto wscale = [&](int c) {
            if constexpr (kScLds) return ws[r * 8 + c];
            else return sc[c];
        };
        if (active) {
            if constexpr (kScLds) {
                ws[lane] = scw[0];
                wave_lds_fence();  // the row's lanes read each other's scales
            }
            if (wave > 0) {
#pragma unroll
                for (int c = 0; c < kPer; ++c) {
                    const uint4 a = act4[(c_first + c) * 8 + l];
                    const float4 as = as4[c_first + c];
                    const float4 d = sdot4x4_f(q[c], a);
                    const uint2 sw = wscale(c);
                    const float4 sv = make_float4(half_times<false>(sw.x, as.x), half_times<true>(sw.x, as.y),
                        half_times<false>(sw.y, as.z), half_times<true>(sw.y, as.w));
                    float4 *h = handoff + ((wave - 1) * kPer + c) * 128 + lane;
                    h[0] = sv;
                    h[64] = d;
                }
            } else {
#pragma unroll
                for (int c = 0; c < kPer; ++c) acc = dot_chunk(q[c], wscale(c), act4[c * 8 + l], as4[c], acc);
            }
        }
        __syncthreads();
        if (wave > 0) return;
        if (active) {
#pragma unroll
            for (int c = 0; c < 3 * kPer; ++c) {
                const float4 sv = handoff[c * 128 + lane];
                const float4 d = handoff[c * 128 + 64 + lane];
                acc = __builtin_fmaf(sv.x, d.x, acc);
                acc = __builtin_fmaf(sv.y, d.y, acc);
                acc = __builtin_fmaf(sv.z, d.z, acc);
                acc = __builtin_fmaf(sv.w, d.w, acc);
            }
        }
    } else if (active) {
        if constexpr (kScLds) {
            uint2 *ws = reinterpret_cast<uint2 *>(handoff) + static_cast<size_t>(wave) * (kPair ? 2 : 1) * kScLoads * 64;
#pragma unroll
            for (int k = 0; k < kScLoads; ++k) {
                ws[k * 64 + lane] = scw[k];
                if constexpr (kPair) ws[(kScLoads + k) * 64 + lane] = scw2[k];
            }
            wave_lds_fence();  // the row's lanes read each other's scales
#pragma unroll
            for (int c = 0; c < NREG; ++c) {
                const uint4 a = act4[c * 8 + l];
                const float4 as = as4[c];
                const int si = (c >> 3) * 64 + r * 8 + (c & 7);
                acc = dot_chunk(q[c], ws[si], a, as, acc);
                if constexpr (kPair) acc2 = dot_chunk(q2[c], ws[kScLoads * 64 + si], a, as, acc2);
            }
        } else if constexpr (NREG > 0) {
#pragma unroll
            for (int c = 0; c < NREG; ++c) {
                const uint4 a = act4[c * 8 + l];
                const float4 as = as4[c];
                acc = dot_chunk(q[c], sc[c], a, as, acc);
                if constexpr (kPair) acc2 = dot_chunk(q2[c], sc2[c], a, as, acc2);
            }
        } else {
            for (int c0 = 0; c0 < chunks; c0 += 8) {
                uint4 qb[8], qb2[kPair ? 8 : 1];
                uint2 sb[8], sb2[kPair ? 8 : 1];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    if (c0 + i < chunks) {
                        qb[i] = load_stream(qp + static_cast<size_t>(c0 + i) * 64);
                        sb[i] = load_stream(sp + static_cast<size_t>(c0 + i) * 8);
                        if constexpr (kPair) {
                            qb2[i] = load_stream(qp2 + static_cast<size_t>(c0 + i) * 64);
                            sb2[i] = load_stream(sp2 + static_cast<size_t>(c0 + i) * 8);
                        }
                    }
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    if (c0 + i < chunks) {
                        const uint4 a = act4[(c0 + i) * 8 + l];
                        const float4 as = as4[c0 + i];
                        acc = dot_chunk(qb[i], sb[i], a, as, acc);
                        if constexpr (kPair) acc2 = dot_chunk(qb2[i], sb2[i], a, as, acc2);
                    }
                }
            }
        }
    }
    FORTAI_MV_MARK(3);
    acc = row_hsum8(acc);
    if constexpr (kPair) acc2 = row_hsum8(acc2);
    if constexpr (EPI == Epilogue::STORE) {
        if (conv && writer) {
            // the window then moves by one (only this thread touches it)
            seg.out[row] = conv_silu(win, taps, ck, acc);
#pragma unroll
            for (int t = 0; t + 1 < kConvMax - 1; ++t)
                if (t + 1 < ck - 1) seg.conv_state[static_cast<size_t>(t) * seg.conv_size + row] = win[t + 1];
            seg.conv_state[static_cast<size_t>(ck - 2) * seg.conv_size + row] = acc;
        } else if (writer) {
            const bool silu = seg.silu || (row >= seg.silu_begin && row < seg.silu_end);
            seg.out[row] = silu ? silu_poly(acc) : acc;
        }
    } else if constexpr (EPI == Epilogue::ADD) {
        if (writer) seg.out[row] = acc + resid;
    } else {
        // fortai_silu_product: vector lanes for the first count/8*8 rows, the
        // libm tail expression for the rest (fortai_q8_dot.c:492-505)
        const float h = row < args.pair_vector_rows ? silu_poly(acc) * acc2
                                                    : acc / (1.0f + exp_rounded(-acc)) * acc2;
        if (writer && seg.out) seg.out[row] = h;
        if (seg.out_q8l) {
            // the workgroup's 32 rows form one quantization block of h
            if (l == 0) epi[wave * 8 + r] = h;
            __syncthreads();
            if (threadIdx.x < 8) {
                const int t = static_cast<int>(threadIdx.x);
                const float4 y = make_float4(epi[4 * t], epi[4 * t + 1], epi[4 * t + 2], epi[4 * t + 3]);
                float scale;
                uint16_t bits;
                const uint32_t packed = quantize_group(y, scale, bits);
                const int b = wg - args.first_wg[s];
                const int hchunks = (seg.w.rows / kQ8Block + 3) / 4;
                uint32_t *dq = static_cast<uint32_t *>(seg.out_q8l);
                dq[((b >> 2) * 8 + t) * 4 + (b & 3)] = packed;
                if (t == 0) reinterpret_cast<float *>(dq + hchunks * 32)[b] = scale;
            }
        }
    }
    FORTAI_MV_MARK(4);
}

constexpr int kMatvecWaves = 4;  // large launches; small ones use one wave per workgroup

template <int WAVES, int NREG, Prologue PRO, Epilogue EPI, bool MULTI = false, bool SPLIT = false>
hipError_t launch_matvec_t(const MatvecArgs &args, int grid, hipStream_t stream) {
    constexpr bool kScLds = NREG > 0 && (SPLIT ? NREG / 4 <= 8 : NREG % 8 == 0);
    constexpr int kScLoads = SPLIT ? 1 : NREG / 8;
    const size_t lds = static_cast<size_t>(args.chunks) * 144 + 8 * WAVES + 4 * 8 * WAVES +
        (SPLIT ? static_cast<size_t>(3 * (NREG / 4)) * 128 * 16 : 0) +
        (kScLds ? static_cast<size_t>(WAVES) * (EPI == Epilogue::SILU_PAIR ? 2 : 1) * kScLoads * 64 * 8 : 0);
    hipLaunchKernelGGL((q8_matvec_kernel<WAVES, NREG, PRO, EPI, MULTI, SPLIT>), dim3(grid), dim3(WAVES * 64), lds,
        stream, args);
    note_launch("q8_matvec_kernel<waves=%d,regs=%d,%s,%s%s%s> grid %d", WAVES, NREG, prologue_name(PRO),
        epilogue_name(EPI), MULTI ? ",segments" : "", SPLIT ? ",split" : "", grid);
    return hipGetLastError();
}

// one 8-row group per workgroup, its chunks split over four waves
template <Prologue PRO, Epilogue EPI>
hipError_t launch_matvec_split(const MatvecArgs &args, int grid, int chunks, hipStream_t stream) {
    if (chunks == 8) return launch_matvec_t<4, 8, PRO, EPI, false, true>(args, grid, stream);
    if (chunks == 16) return launch_matvec_t<4, 16, PRO, EPI, false, true>(args, grid, stream);
    if (chunks == 28) return launch_matvec_t<4, 28, PRO, EPI, false, true>(args, grid, stream);
    if (chunks == 32) return launch_matvec_t<4, 32, PRO, EPI, false, true>(args, grid, stream);
    return hipErrorInvalidValue;
}

template <int WAVES, Prologue PRO, Epilogue EPI>
hipError_t launch_matvec_regs(const MatvecArgs &args, int grid, int chunks, hipStream_t stream) {
    constexpr bool kPair = EPI == Epilogue::SILU_PAIR;
    // several segments (the host-side pair/triplet products): the streamed form
    if constexpr (EPI == Epilogue::STORE)
        if (args.count > 1) return launch_matvec_t<WAVES, 0, PRO, EPI, true>(args, grid, stream);
    if (chunks == 8) return launch_matvec_t<WAVES, 8, PRO, EPI>(args, grid, stream);
    if (chunks == 16) return launch_matvec_t<WAVES, 16, PRO, EPI>(args, grid, stream);
    if (!kPair && chunks == 28) return launch_matvec_t<WAVES, kPair ? 0 : 28, PRO, EPI>(args, grid, stream);
    if (!kPair && chunks == 32) return launch_matvec_t<WAVES, kPair ? 0 : 32, PRO, EPI>(args, grid, stream);
    return launch_matvec_t<WAVES, 0, PRO, EPI>(args, grid, stream);
}

template <Prologue PRO>
hipError_t launch_matvec_pro(const MatvecArgs &args, int waves, int grid, int chunks, Epilogue epi,
    hipStream_t stream, bool split) {
    if (split) {
        if (epi == Epilogue::STORE) return launch_matvec_split<PRO, Epilogue::STORE>(args, grid, chunks, stream);
        if (epi == Epilogue::ADD) return launch_matvec_split<PRO, Epilogue::ADD>(args, grid, chunks, stream);
        return hipErrorInvalidValue;
    }
    if (epi == Epilogue::SILU_PAIR) return launch_matvec_regs<4, PRO, Epilogue::SILU_PAIR>(args, grid, chunks, stream);
    if (epi == Epilogue::STORE) {
        if (waves == 4) return launch_matvec_regs<4, PRO, Epilogue::STORE>(args, grid, chunks, stream);
        return launch_matvec_regs<1, PRO, Epilogue::STORE>(args, grid, chunks, stream);
    }
    if (epi == Epilogue::ADD) {
        if (waves == 4) return launch_matvec_regs<4, PRO, Epilogue::ADD>(args, grid, chunks, stream);
        return launch_matvec_regs<1, PRO, Epilogue::ADD>(args, grid, chunks, stream);
    }
    return hipErrorInvalidValue;
}

// ---- batches of sequences ----------------------------------------------------
// The activation of each sequence is built once per step by q8l_prep_kernel
// (one workgroup per sequence, the same code as the single-sequence
// prologues, into the Q8L layout in device memory); the batched matvec then
// streams every weight once for all sequences.  Per (row, sequence) it runs
// the single-sequence kernel's eight lane chains, horizontal sum and
// epilogue, so each sequence's outputs are bit-identical to batch 1.
constexpr int kMaxBatch = 8;
constexpr int kBatchThreads = 256;

constexpr int kPrepThreads = 512;  // activations up to 16384 wide

template <Prologue PRO>
__global__ __launch_bounds__(kPrepThreads) void q8l_prep_kernel(MatvecInput in, void *q8l) {
    FORTAI_TRACE_SCOPE(10);
    __shared__ double red[kPrepThreads / 64];
    const int seq = static_cast<int>(blockIdx.x);
    const int chunks = (in.width / kQ8Block + 3) / 4;
    in.x += static_cast<size_t>(seq) * in.width;
    if (in.z) in.z += static_cast<size_t>(seq) * in.width;
    unsigned char *base = static_cast<unsigned char *>(q8l) + static_cast<size_t>(seq) * q8l_bytes(in.width);
    build_activation<kPrepThreads, PRO>(in, chunks, reinterpret_cast<uint32_t *>(base),
        reinterpret_cast<float *>(base + static_cast<size_t>(chunks) * 128), red);
}

struct BatchMatvecArgs {
    MatvecSegment seg[4];  // outputs [batch][rows]; conv windows [batch][kernel-1][conv_size]
    int first_wg[5];
    int count;
    int chunks;            // activation chunks
    int batch;
    int split;             // waves sharing one row group (each takes every split-th sequence)
    int pair_vector_rows;
    const void *act;       // Q8L [batch][q8l_bytes(width)]
};

__device__ __forceinline__ float dot_chunk_f(uint4 q, const float (&ws)[4], uint4 a, float4 as, float acc) {
    const float4 d = sdot4x4_f(q, a);
    acc = __builtin_fmaf(ws[0] * as.x, d.x, acc);
    acc = __builtin_fmaf(ws[1] * as.y, d.y, acc);
    acc = __builtin_fmaf(ws[2] * as.z, d.z, acc);
    acc = __builtin_fmaf(ws[3] * as.w, d.w, acc);
    return acc;
}

__device__ __forceinline__ void scales_f(uint2 sc, float (&ws)[4]) {
    ws[0] = half_bits_to_float(static_cast<uint16_t>(sc.x));
    ws[1] = half_bits_to_float(static_cast<uint16_t>(sc.x >> 16));
    ws[2] = half_bits_to_float(static_cast<uint16_t>(sc.y));
    ws[3] = half_bits_to_float(static_cast<uint16_t>(sc.y >> 16));
}

// Four waves per workgroup; wave w takes row group slot w / SPLIT and the
// sequences w % SPLIT, w % SPLIT + SPLIT, ... (8 / SPLIT of them; indices past
// the batch repeat its last sequence and write nothing).  The activations of
// every sequence are copied to LDS by direct global-to-LDS loads; weights
// stream in groups of G chunks (G divides the chunk count), two groups in
// flight while one is consumed.  Every load is unconditional (clamped), so
// the compiler's in-order load counters never wait for a prefetch.
// CH > 0: exactly CH chunks, the group loop fully unrolled (a rolled loop
// makes the compiler wait for every prefetch at its head); CH == 0: any count.
template <Epilogue EPI, int SPLIT, int G, int WAVES, int CH>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(WAVES >= 16 ? 4 : WAVES / 2))) void q8_batch_matvec_kernel(const BatchMatvecArgs args) {
    FORTAI_TRACE_SCOPE(9);
    constexpr bool kPair = EPI == Epilogue::SILU_PAIR;
    constexpr int NS = kMaxBatch / SPLIT;
    extern __shared__ __align__(16) unsigned char lds[];
    const int seq_bytes = args.chunks * 144;
    const int act_bytes = (args.batch * seq_bytes + 1023) / 1024 * 1024;  // whole 1 KiB load blocks
    constexpr int kSlots = WAVES / SPLIT;                      // row groups per workgroup
    float *epi = reinterpret_cast<float *>(lds + act_bytes);  // [8][kSlots * 8]
    // the gate/up pair with one chunk per group: each wave forms the chunk's
    // scale products fl(f32(w_scale) * a_scale) once per (matrix, row,
    // sequence, block) -- four per lane -- into its own LDS table, instead of
    // every lane of a row forming all of them; LDS operations of one wave
    // read back after a wavefront-scope fence, without a workgroup barrier
    constexpr bool kTable = kPair && G == 1 && NS == 4;
    float *ptab = epi + kMaxBatch * kSlots * 8 + (static_cast<int>(threadIdx.x) >> 6) * 2 * 8 * NS * 4;  // [2][8][NS][4]

    const int wg = static_cast<int>(blockIdx.x);
    int sgi = 0;
    while (sgi + 1 < args.count && wg >= args.first_wg[sgi + 1]) ++sgi;
    const MatvecSegment &seg = args.seg[sgi];
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63, wave = tid >> 6;
    const int slot = wave / SPLIT, sub = wave % SPLIT;
    const int rg = (wg - args.first_wg[sgi]) * (WAVES / SPLIT) + slot;
    const bool active = rg < seg.w.row_groups;
    const int rgc = active ? rg : seg.w.row_groups - 1;
    const int r = lane >> 3, l = lane & 7;
    const int chunks = seg.w.chunks;
    const uint4 *qp = seg.w.quants + static_cast<size_t>(rgc) * chunks * 64 + lane;
    const uint2 *sp = seg.w.scales + static_cast<size_t>(rgc) * chunks * 8 + r;
    const uint4 *qp2 = kPair ? seg.w2.quants + static_cast<size_t>(rgc) * chunks * 64 + lane : nullptr;
    const uint2 *sp2 = kPair ? seg.w2.scales + static_cast<size_t>(rgc) * chunks * 8 + r : nullptr;
    int sq[NS];
#pragma unroll
    for (int k = 0; k < NS; ++k) sq[k] = min(sub + k * SPLIT, args.batch - 1);

    // a ring of three operand groups: two in flight while one is consumed
    uint4 qa[G], qa2[kPair ? G : 1], qb[G], qb2[kPair ? G : 1], qc[G], qc2[kPair ? G : 1];
    uint2 sa[G], sa2[kPair ? G : 1], sb[G], sb2[kPair ? G : 1], sc_[G], sc2_[kPair ? G : 1];
    auto fetch = [&](int c0, uint4 (&q)[G], uint2 (&sc)[G], uint4 (&q2)[kPair ? G : 1], uint2 (&sc2)[kPair ? G : 1]) {
        c0 = min(c0, chunks - G);  // past the end: the last group again (cached, unused)
#pragma unroll
        for (int i = 0; i < G; ++i) {
            q[i] = load_stream(qp + static_cast<size_t>(c0 + i) * 64);
            sc[i] = load_stream(sp + static_cast<size_t>(c0 + i) * 8);
            if constexpr (kPair) {
                q2[i] = load_stream(qp2 + static_cast<size_t>(c0 + i) * 64);
                sc2[i] = load_stream(sp2 + static_cast<size_t>(c0 + i) * 8);
            }
        }
    };
    fetch(0, qa, sa, qa2, sa2);
    fetch(G, qb, sb, qb2, sb2);
    {
        // activations of every sequence: 1 KiB blocks, wave w takes blocks w, w + 4, ...
        const int pieces = args.batch * seq_bytes / 16;
        const int blocks = act_bytes / 1024;
        const u32x4_t *src = static_cast<const u32x4_t *>(args.act);
        for (int b = wave; b < blocks; b += WAVES)
            __builtin_amdgcn_global_load_lds(src + min(b * 64 + lane, pieces - 1),
                reinterpret_cast<u32x4_t *>(lds) + b * 64, 16, 0, 0);
    }
    const int row = rg * kRowsPerWave + r;
    const int rowc = min(row, seg.w.rows - 1);
    const bool writer = active && l == 0 && row < seg.w.rows;
    // per-sequence residuals and conv windows, loaded now (clamped, unconditional)
    float resid[NS], win[NS][kConvMax - 1], taps[kConvMax];
    // (row groups are whole 8-row groups, so conv and SiLU are uniform per wave)
    const bool conv = EPI == Epilogue::STORE && seg.conv_w != nullptr && (seg.conv_rows == 0 || row < seg.conv_rows);
    const int ck = conv ? seg.kernel : 0;
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        resid[k] = 0.0f;
        if constexpr (EPI == Epilogue::ADD) resid[k] = seg.resid[static_cast<size_t>(sq[k]) * seg.w.rows + rowc];
    }
    if (conv) {
#pragma unroll
        for (int k = 0; k < NS; ++k)
#pragma unroll
            for (int t = 0; t < kConvMax - 1; ++t)
                win[k][t] = t < ck - 1
                    ? seg.conv_state[(static_cast<size_t>(sq[k]) * (ck - 1) + t) * seg.conv_size + rowc] : 0.0f;
#pragma unroll
        for (int t = 0; t < kConvMax; ++t) taps[t] = t < ck ? seg.conv_w[static_cast<size_t>(rowc) * ck + t] : 0.0f;
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's direct-to-LDS loads have landed
    __syncthreads();

    float acc[NS], acc2[NS];
#pragma unroll
    for (int k = 0; k < NS; ++k) { acc[k] = 0.0f; acc2[k] = 0.0f; }
    // per group: the weight scales once, then two sequences at a time with all
    // of their activation reads for the group issued before the dots (each
    // sequence's chain still runs chunk by chunk in order)
    auto consume = [&](int c0, const uint4 (&q)[G], const uint2 (&sc)[G], const uint4 (&q2)[kPair ? G : 1],
                       const uint2 (&sc2)[kPair ? G : 1]) {
        if constexpr (kTable) {
            // lane (r, l): sequence l / 2, blocks 2 (l % 2) and 2 (l % 2) + 1, both matrices
            {
                const int ks = l >> 1, j0 = (l & 1) * 2;
                const unsigned char *sb = lds + static_cast<size_t>(sq[ks]) * seq_bytes;
                const float4 a4 = reinterpret_cast<const float4 *>(sb + static_cast<size_t>(args.chunks) * 128)[c0];
                float ws[4], ws2[4];
                scales_f(sc[0], ws);
                scales_f(sc2[0], ws2);
                const float a0 = j0 == 0 ? a4.x : a4.z, a1 = j0 == 0 ? a4.y : a4.w;
                const float w0 = j0 == 0 ? ws[0] : ws[2], w1 = j0 == 0 ? ws[1] : ws[3];
                const float v0 = j0 == 0 ? ws2[0] : ws2[2], v1 = j0 == 0 ? ws2[1] : ws2[3];
                *reinterpret_cast<float2 *>(ptab + ((0 * 8 + r) * NS + ks) * 4 + j0) = make_float2(w0 * a0, w1 * a1);
                *reinterpret_cast<float2 *>(ptab + ((1 * 8 + r) * NS + ks) * 4 + j0) = make_float2(v0 * a0, v1 * a1);
            }
            wave_lds_fence();
#pragma unroll
            for (int k = 0; k < NS; ++k) {
                const unsigned char *sbase = lds + static_cast<size_t>(sq[k]) * seq_bytes;
                const uint4 a = reinterpret_cast<const uint4 *>(sbase)[c0 * 8 + l];
                const float4 p1 = *reinterpret_cast<const float4 *>(ptab + ((0 * 8 + r) * NS + k) * 4);
                const float4 p2 = *reinterpret_cast<const float4 *>(ptab + ((1 * 8 + r) * NS + k) * 4);
                const float4 d = sdot4x4_f(q[0], a);
                const float4 d2 = sdot4x4_f(q2[0], a);
                acc[k] = __builtin_fmaf(p1.x, d.x, acc[k]);
                acc[k] = __builtin_fmaf(p1.y, d.y, acc[k]);
                acc[k] = __builtin_fmaf(p1.z, d.z, acc[k]);
                acc[k] = __builtin_fmaf(p1.w, d.w, acc[k]);
                acc2[k] = __builtin_fmaf(p2.x, d2.x, acc2[k]);
                acc2[k] = __builtin_fmaf(p2.y, d2.y, acc2[k]);
                acc2[k] = __builtin_fmaf(p2.z, d2.z, acc2[k]);
                acc2[k] = __builtin_fmaf(p2.w, d2.w, acc2[k]);
            }
            wave_lds_fence();
            return;
        }
        float ws[G][4], ws2[kPair ? G : 1][4];
#pragma unroll
        for (int i = 0; i < G; ++i) {
            scales_f(sc[i], ws[i]);
            if constexpr (kPair) scales_f(sc2[i], ws2[i]);
        }
#pragma unroll
        for (int k0 = 0; k0 < NS; k0 += 2) {
            constexpr int kP = NS >= 2 ? 2 : 1;
            uint4 a[kP][G];
            float4 as[kP][G];
#pragma unroll
            for (int kk = 0; kk < kP; ++kk) {
                const unsigned char *sbase = lds + static_cast<size_t>(sq[k0 + kk]) * seq_bytes;
#pragma unroll
                for (int i = 0; i < G; ++i) {
                    a[kk][i] = reinterpret_cast<const uint4 *>(sbase)[(c0 + i) * 8 + l];
                    as[kk][i] = reinterpret_cast<const float4 *>(sbase + static_cast<size_t>(args.chunks) * 128)[c0 + i];
                }
            }
#pragma unroll
            for (int kk = 0; kk < kP; ++kk) {
#pragma unroll
                for (int i = 0; i < G; ++i) {
                    acc[k0 + kk] = dot_chunk_f(q[i], ws[i], a[kk][i], as[kk][i], acc[k0 + kk]);
                    if constexpr (kPair) acc2[k0 + kk] = dot_chunk_f(q2[i], ws2[i], a[kk][i], as[kk][i], acc2[k0 + kk]);
                }
            }
        }
    };
    if constexpr (CH > 0) {
        constexpr int NG = CH / G;
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
            // folded after unrolling: group gi in buffer gi % 3, group gi + 2 fetched
            if (gi % 3 == 0) {
                if (gi + 2 < NG) fetch((gi + 2) * G, qc, sc_, qc2, sc2_);
                consume(gi * G, qa, sa, qa2, sa2);
            } else if (gi % 3 == 1) {
                if (gi + 2 < NG) fetch((gi + 2) * G, qa, sa, qa2, sa2);
                consume(gi * G, qb, sb, qb2, sb2);
            } else {
                if (gi + 2 < NG) fetch((gi + 2) * G, qb, sb, qb2, sb2);
                consume(gi * G, qc, sc_, qc2, sc2_);
            }
        }
    } else {
        for (int c0 = 0;; c0 += 3 * G) {
            fetch(c0 + 2 * G, qc, sc_, qc2, sc2_);
            consume(c0, qa, sa, qa2, sa2);
            if (c0 + G >= chunks) break;
            fetch(c0 + 3 * G, qa, sa, qa2, sa2);
            consume(c0 + G, qb, sb, qb2, sb2);
            if (c0 + 2 * G >= chunks) break;
            fetch(c0 + 4 * G, qb, sb, qb2, sb2);
            consume(c0 + 2 * G, qc, sc_, qc2, sc2_);
            if (c0 + 3 * G >= chunks) break;
        }
    }
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        acc[k] = row_hsum8(acc[k]);
        if constexpr (kPair) acc2[k] = row_hsum8(acc2[k]);
    }
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const bool mine = sub + k * SPLIT < args.batch;
        float *out = seg.out ? seg.out + static_cast<size_t>(sq[k]) * seg.w.rows : nullptr;
        if constexpr (EPI == Epilogue::STORE) {
            if (conv && writer && mine) {
                float *cs = seg.conv_state + static_cast<size_t>(sq[k]) * (ck - 1) * seg.conv_size;
                out[row] = conv_silu(win[k], taps, ck, acc[k]);
#pragma unroll
                for (int t = 0; t + 1 < kConvMax - 1; ++t)
                    if (t + 1 < ck - 1) cs[static_cast<size_t>(t) * seg.conv_size + row] = win[k][t + 1];
                cs[static_cast<size_t>(ck - 2) * seg.conv_size + row] = acc[k];
            } else if (writer && mine) {
                out[row] = seg.silu ? silu_poly(acc[k]) : acc[k];
            }
        } else if constexpr (EPI == Epilogue::ADD) {
            if (writer && mine) out[row] = acc[k] + resid[k];
        } else {
            const float h = row < args.pair_vector_rows ? silu_poly(acc[k]) * acc2[k]
                                                        : acc[k] / (1.0f + exp_rounded(-acc[k])) * acc2[k];
            if (writer && mine && out) out[row] = h;
            if (seg.out_q8l && l == 0 && mine) epi[sq[k] * (kSlots * 8) + slot * 8 + r] = h;
        }
    }
    if constexpr (kPair) {
        if (seg.out_q8l) {
            // every 32 rows of the workgroup (4 row groups) form one
            // quantization block of every sequence's h
            static_assert(kSlots % 4 == 0, "whole quantization blocks per workgroup");
            constexpr int kBlocks = kSlots / 4;
            __syncthreads();
            const int t = tid & 7, q = tid >> 3;  // q: sequence + 8 * block
            const int qs = q & 7, qb = q >> 3;
            if (qs < args.batch && qb < kBlocks) {
                const float *e = epi + qs * (kSlots * 8) + qb * 32;
                const float4 y = make_float4(e[4 * t], e[4 * t + 1], e[4 * t + 2], e[4 * t + 3]);
                float scale;
                uint16_t bits;
                const uint32_t packed = quantize_group(y, scale, bits);
                const int b = (wg - args.first_wg[sgi]) * kBlocks + qb;
                const int hchunks = (seg.w.rows / kQ8Block + 3) / 4;
                uint32_t *dq = reinterpret_cast<uint32_t *>(static_cast<unsigned char *>(seg.out_q8l) +
                    static_cast<size_t>(qs) * q8l_bytes(seg.w.rows));
                dq[((b >> 2) * 8 + t) * 4 + (b & 3)] = packed;
                if (t == 0) reinterpret_cast<float *>(dq + hchunks * 32)[b] = scale;
            }
        }
    }
}

// vmcnt(n) with the other counters left alone (gfx9 s_waitcnt encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int waitcnt_vm(int n) { return (n & 15) | (((n >> 4) & 3) << 14) | (7 << 4) | (15 << 8); }

constexpr int kRingG = 4;  // chunks per ring group

// Store/add matvec of a batch with the weights fetched once per workgroup.
// One workgroup per 8-row group; its four waves take two sequences each
// (w and w + 4).  Every wave loads one chunk of each group of four (1 KiB) and
// the group's row scales into a register ring R groups deep, so R groups are
// in flight per wave; just before a group is consumed the four waves put it
// into one of two LDS slots and, after one barrier, all read it from there.
// With two sequences per wave (NS = 2) the scale products
// fl(f32(w_scale) * a_scale) of the group (4 blocks per chunk, row and
// sequence of the workgroup) are then formed once into an LDS table (one
// float4 per thread) instead of by each of the 8 lanes of a row, and after a
// second barrier every lane reads its four products with one 16-byte load
// (with NS = 1 half the threads would fill the table and the extra barrier
// costs more than the products: measured 18.4 -> 19.9 us).  Per (row, sequence) the chain is the
// single-sequence kernel's, rounding for rounding.
template <Epilogue EPI, int GROUPS, int NS>
__global__ __launch_bounds__(kBatchThreads) void q8_batch_ring_kernel(const BatchMatvecArgs args) {
    FORTAI_TRACE_SCOPE(8);
    constexpr int R = GROUPS < 8 ? GROUPS : 8;  // groups in flight per wave
    constexpr int kSlot = kRingG * 1024 + kRingG * 64;  // quants then scales of one group
    constexpr bool kTable = NS == 2;
    constexpr int kTab = kRingG * 4 * NS * 8;            // float4 products of one group [chunk][seq][row]
    extern __shared__ __align__(16) unsigned char lds[];
    const int seq_bytes = args.chunks * 144;
    // this workgroup's block of 4 NS sequences (blockIdx.y)
    const int base = static_cast<int>(blockIdx.y) * 4 * NS;
    const int nseq = min(4 * NS, args.batch - base);
    const int act_bytes = (nseq * seq_bytes + 1023) / 1024 * 1024;
    unsigned char *slots = lds + act_bytes;  // [2][kSlot]
    float4 *tabs = reinterpret_cast<float4 *>(slots + 2 * kSlot);  // [2][kTab]

    const int wg = static_cast<int>(blockIdx.x);
    int sgi = 0;
    while (sgi + 1 < args.count && wg >= args.first_wg[sgi + 1]) ++sgi;
    const MatvecSegment &seg = args.seg[sgi];
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63, wave = tid >> 6;
    const int rg = wg - args.first_wg[sgi];
    const int r = lane >> 3, l = lane & 7;
    constexpr int chunks = GROUPS * kRingG, groups = GROUPS;
    const u32x4_t *qsrc = reinterpret_cast<const u32x4_t *>(seg.w.quants) + static_cast<size_t>(rg) * chunks * 64;
    const uint32_t *ssrc = reinterpret_cast<const uint32_t *>(seg.w.scales) + static_cast<size_t>(rg) * chunks * 16;
    int sq[NS];  // sequences of this wave (clamped to the batch)
#pragma unroll
    for (int k = 0; k < NS; ++k) sq[k] = min(base + wave + 4 * k, args.batch - 1);

    u32x4_t rq[R];
    uint32_t rs[R];
    // group g -> register slot g % R: this wave's chunk and one scale word
    auto fetch = [&](int g, u32x4_t &q, uint32_t &sw) {
        const int gc = min(g, groups - 1);  // past the end: the last group again (never consumed)
        q = __builtin_nontemporal_load(qsrc + (static_cast<size_t>(gc) * kRingG + wave) * 64 + lane);
        sw = __builtin_nontemporal_load(ssrc + static_cast<size_t>(gc) * kRingG * 16 + lane);
    };
#pragma unroll
    for (int g = 0; g < R; ++g) fetch(g, rq[g], rs[g]);
    {
        const int pieces = nseq * seq_bytes / 16;
        const int blocks = act_bytes / 1024;
        const u32x4_t *src = static_cast<const u32x4_t *>(args.act) + static_cast<size_t>(base) * seq_bytes / 16;
        for (int b = wave; b < blocks; b += 4)
            __builtin_amdgcn_global_load_lds(src + min(b * 64 + lane, pieces - 1),
                reinterpret_cast<u32x4_t *>(lds) + b * 64, 16, 0, 0);
    }
    const int row = rg * kRowsPerWave + r;
    const int rowc = min(row, seg.w.rows - 1);
    const bool writer = l == 0 && row < seg.w.rows;
    float resid[NS], win[NS][kConvMax - 1], taps[kConvMax];
    // (row groups are whole 8-row groups, so conv and SiLU are uniform per wave)
    const bool conv = EPI == Epilogue::STORE && seg.conv_w != nullptr && (seg.conv_rows == 0 || row < seg.conv_rows);
    const int ck = conv ? seg.kernel : 0;
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        resid[k] = 0.0f;
        if constexpr (EPI == Epilogue::ADD) resid[k] = seg.resid[static_cast<size_t>(sq[k]) * seg.w.rows + rowc];
    }
    if (conv) {
#pragma unroll
        for (int k = 0; k < NS; ++k)
#pragma unroll
            for (int t = 0; t < kConvMax - 1; ++t)
                win[k][t] = t < ck - 1
                    ? seg.conv_state[(static_cast<size_t>(sq[k]) * (ck - 1) + t) * seg.conv_size + rowc] : 0.0f;
#pragma unroll
        for (int t = 0; t < kConvMax; ++t) taps[t] = t < ck ? seg.conv_w[static_cast<size_t>(rowc) * ck + t] : 0.0f;
    }

    float acc[NS];
#pragma unroll
    for (int k = 0; k < NS; ++k) acc[k] = 0.0f;
    // one group: into LDS slot g & 1, barrier, refill the register slot with
    // group g + R, then the dots from LDS
    auto step = [&](int g, u32x4_t &q, uint32_t &sw) {
        unsigned char *slot = slots + (g & 1) * kSlot;
        float4 *tab = tabs + (g & 1) * kTab;
        reinterpret_cast<u32x4_t *>(slot + wave * 1024)[lane] = q;
        if (wave == 0) reinterpret_cast<uint32_t *>(slot + kRingG * 1024)[lane] = sw;
        __syncthreads();  // the group is in LDS (and, the first time, the activations: see below)
        if (g + R < GROUPS) fetch(g + R, q, sw);
        if (kTable && tid < kTab) {
            // entry (chunk i, workgroup sequence kk, row rr): the four blocks' products
            const int rr = tid & 7, kk = (tid >> 3) % (4 * NS), i = tid / (8 * 4 * NS);
            const int sk = min(base + kk, args.batch - 1) - base;
            const uint2 sc = reinterpret_cast<const uint2 *>(slot + kRingG * 1024 + i * 64)[rr];
            float ws[4];
            scales_f(sc, ws);
            const float4 as = reinterpret_cast<const float4 *>(
                lds + static_cast<size_t>(sk) * seq_bytes + static_cast<size_t>(args.chunks) * 128)[g * kRingG + i];
            tab[tid] = make_float4(ws[0] * as.x, ws[1] * as.y, ws[2] * as.z, ws[3] * as.w);
        }
        if constexpr (kTable) __syncthreads();  // the products are in LDS
#pragma unroll
        for (int i = 0; i < kRingG; ++i) {
            const int c = g * kRingG + i;
            const uint4 qq = reinterpret_cast<const uint4 *>(slot + i * 1024)[lane];
            float ws[4];
            if constexpr (!kTable) scales_f(reinterpret_cast<const uint2 *>(slot + kRingG * 1024 + i * 64)[r], ws);
#pragma unroll
            for (int k = 0; k < NS; ++k) {
                const unsigned char *sbase = lds + static_cast<size_t>(sq[k] - base) * seq_bytes;
                const uint4 a = reinterpret_cast<const uint4 *>(sbase)[c * 8 + l];
                if constexpr (kTable) {
                    const float4 pr = tab[(i * 4 * NS + wave + 4 * k) * 8 + r];
                    const float4 d = sdot4x4_f(qq, a);
                    acc[k] = __builtin_fmaf(pr.x, d.x, acc[k]);
                    acc[k] = __builtin_fmaf(pr.y, d.y, acc[k]);
                    acc[k] = __builtin_fmaf(pr.z, d.z, acc[k]);
                    acc[k] = __builtin_fmaf(pr.w, d.w, acc[k]);
                } else {
                    const float4 as = reinterpret_cast<const float4 *>(sbase + static_cast<size_t>(args.chunks) * 128)[c];
                    acc[k] = dot_chunk_f(qq, ws, a, as, acc[k]);
                }
            }
        }
    };
    // the activations' direct-to-LDS copies were issued after the first R
    // groups: waiting for all of this wave's loads once covers both
    __builtin_amdgcn_s_waitcnt(0);
    FORTAI_MV_MARK(0);
    // fully unrolled (the group count is a template parameter): the compiler's
    // load counters then know that group g is the oldest load in flight
#pragma unroll
    for (int g = 0; g < GROUPS; ++g) {
        step(g, rq[g % R], rs[g % R]);
        if (g == 0) FORTAI_MV_MARK(1);
        if (g == GROUPS / 2) FORTAI_MV_MARK(2);
    }
    FORTAI_MV_MARK(3);
#pragma unroll
    for (int k = 0; k < NS; ++k) acc[k] = row_hsum8(acc[k]);
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const bool mine = base + wave + 4 * k < args.batch;
        if (!(writer && mine)) continue;
        float *out = seg.out + static_cast<size_t>(sq[k]) * seg.w.rows;
        if constexpr (EPI == Epilogue::STORE) {
            if (conv) {
                float *cs = seg.conv_state + static_cast<size_t>(sq[k]) * (ck - 1) * seg.conv_size;
                out[row] = conv_silu(win[k], taps, ck, acc[k]);
#pragma unroll
                for (int t = 0; t + 1 < kConvMax - 1; ++t)
                    if (t + 1 < ck - 1) cs[static_cast<size_t>(t) * seg.conv_size + row] = win[k][t + 1];
                cs[static_cast<size_t>(ck - 2) * seg.conv_size + row] = acc[k];
            } else {
                out[row] = seg.silu ? silu_poly(acc[k]) : acc[k];
            }
        } else {
            out[row] = acc[k] + resid[k];
        }
    }
}

template <Epilogue EPI, int SPLIT, int WAVES = 4>
hipError_t launch_batch_g(const BatchMatvecArgs &args, int grid, size_t lds, hipStream_t stream) {
    // groups of at most 4 chunks (with three groups in registers, larger
    // groups exceed the register budget of two workgroups per CU)
    const int c = args.chunks;
    // eight-wave workgroups run two per CU with single-chunk groups (larger
    // groups exceed that register budget)
    const int g = WAVES >= 8 ? 1 : (c % 4 == 0 ? 4 : (c % 2 == 0 ? 2 : 1));
    if constexpr (WAVES >= 8) {
        // the widths of the supported shapes unrolled exactly
#define FORTAI_PAIR(CHN) hipLaunchKernelGGL((q8_batch_matvec_kernel<EPI, SPLIT, 1, WAVES, CHN>), dim3(grid), \
        dim3(WAVES * 64), lds, stream, args)
        switch (c) {
        case 2: FORTAI_PAIR(2); break;
        case 8: FORTAI_PAIR(8); break;
        case 20: FORTAI_PAIR(20); break;
        default: FORTAI_PAIR(0); break;
        }
#undef FORTAI_PAIR
    } else {
        switch (g) {
        case 4: hipLaunchKernelGGL((q8_batch_matvec_kernel<EPI, SPLIT, 4, WAVES, 0>), dim3(grid), dim3(WAVES * 64), lds, stream, args); break;
        case 2: hipLaunchKernelGGL((q8_batch_matvec_kernel<EPI, SPLIT, 2, WAVES, 0>), dim3(grid), dim3(WAVES * 64), lds, stream, args); break;
        default: hipLaunchKernelGGL((q8_batch_matvec_kernel<EPI, SPLIT, 1, WAVES, 0>), dim3(grid), dim3(WAVES * 64), lds, stream, args); break;
        }
    }
    note_launch("q8_batch_matvec_kernel<%s,split=%d,group=%d,waves=%d> grid %d", epilogue_name(EPI), SPLIT, g, WAVES,
        grid);
    return hipGetLastError();
}

__global__ void q8_repack_kernel(const uint8_t *gguf, int rows, int blocks, int chunks,
    int row_groups, uint4 *quants, uint2 *scales) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t total = static_cast<size_t>(row_groups) * chunks * 64;
    if (idx >= total) return;
    const int lane = static_cast<int>(idx & 63);
    const size_t gc = idx >> 6;
    const int c = static_cast<int>(gc % chunks);
    const int g = static_cast<int>(gc / chunks);
    const int r = lane >> 3, l = lane & 7;
    const int row = g * kRowsPerWave + r;
    uint32_t v[4];
    uint32_t s[4];
    for (int j = 0; j < 4; ++j) {
        const int b = 4 * c + j;
        v[j] = 0u;
        s[j] = 0u;
        if (row < rows && b < blocks) {
            const uint8_t *p = gguf + (static_cast<size_t>(row) * blocks + b) * kQ8Bytes;
            s[j] = static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8);
            v[j] = static_cast<uint32_t>(p[2 + 4 * l]) | (static_cast<uint32_t>(p[3 + 4 * l]) << 8) |
                (static_cast<uint32_t>(p[4 + 4 * l]) << 16) | (static_cast<uint32_t>(p[5 + 4 * l]) << 24);
        }
    }
    quants[idx] = make_uint4(v[0], v[1], v[2], v[3]);
    if (l == 0) scales[gc * 8 + r] = make_uint2(s[0] | (s[1] << 16), s[2] | (s[3] << 16));
}

// fortai_q8_quantize on device: one block per 8 lanes, GGUF output bytes.
__global__ void q8_quantize_kernel(const float *x, int width, int8_t *out34, float *scales) {
    const int g = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
    const int groups = width / 4;
    const bool valid = g < groups;
    float4 y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (valid) y = reinterpret_cast<const float4 *>(x)[g];
    float scale;
    uint16_t bits;
    const uint32_t packed = quantize_group(y, scale, bits);
    if (!valid) return;
    const int b = g >> 3, l = g & 7;
    int8_t *block = out34 + static_cast<size_t>(b) * kQ8Bytes;
    for (int i = 0; i < 4; ++i) block[2 + 4 * l + i] = static_cast<int8_t>((packed >> (8 * i)) & 0xffu);
    if (l == 0) {
        block[0] = static_cast<int8_t>(bits & 0xffu);
        block[1] = static_cast<int8_t>(bits >> 8);
        scales[b] = scale;
    }
}

// Exact int32 block dots through the repacked layout (parity entry point).
__global__ void q8_block_dots_kernel(Q8Matrix w, const int8_t *xq, int32_t *out, int blocks) {
    extern __shared__ __align__(16) unsigned char lds[];
    uint32_t *act32 = reinterpret_cast<uint32_t *>(lds);
    float *act_s = reinterpret_cast<float *>(lds + static_cast<size_t>(w.chunks) * 8 * 16);
    MatvecInput in;
    in.xq = xq;
    in.width = blocks * kQ8Block;
    build_activation<64, Prologue::Q8>(in, w.chunks, act32, act_s, nullptr);
    const int lane = static_cast<int>(threadIdx.x);
    const int rg = static_cast<int>(blockIdx.x);
    const int r = lane >> 3, l = lane & 7;
    const int row = rg * kRowsPerWave + r;
    const uint4 *qp = w.quants + static_cast<size_t>(rg) * w.chunks * 64 + lane;
    const uint4 *act4 = reinterpret_cast<const uint4 *>(act32);
    for (int c = 0; c < w.chunks; ++c) {
        const uint4 q = qp[static_cast<size_t>(c) * 64];
        const uint4 a = act4[c * 8 + l];
        int d[4] = {sdot4(q.x, a.x),
            sdot4(q.y, a.y),
            sdot4(q.z, a.z),
            sdot4(q.w, a.w)};
        for (int j = 0; j < 4; ++j) {
            int v = d[j];
            v += xor_lane<4>(v);
            v += xor_lane<2>(v);
            v += xor_lane<1>(v);
            const int b = 4 * c + j;
            if (l == 0 && row < w.rows && b < blocks) out[static_cast<size_t>(row) * blocks + b] = v;
        }
    }
}

__global__ void q8_embedding_kernel(Q8Matrix w, const int64_t *token, int64_t token_value, float *out) {
    const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= w.blocks * kQ8Block) return;
    const int seq = static_cast<int>(blockIdx.y);  // batch: token[seq] -> row seq of out
    out += static_cast<size_t>(seq) * w.blocks * kQ8Block;
    int64_t t = token ? token[seq] : token_value;
    if (t < 0 || t >= w.rows) t = 0;  // a device-fed id is never trusted as an address
    const int g = static_cast<int>(t >> 3), r = static_cast<int>(t & 7);
    const int b = i / kQ8Block, within = i % kQ8Block, l = within >> 2, byte = within & 3;
    const int c = b >> 2, j = b & 3;
    const uint32_t *q32 = reinterpret_cast<const uint32_t *>(w.quants);
    const uint32_t word = q32[((static_cast<size_t>(g) * w.chunks + c) * 64 + r * 8 + l) * 4 + j];
    const int8_t q = static_cast<int8_t>((word >> (8 * byte)) & 0xffu);
    const uint16_t *s16 = reinterpret_cast<const uint16_t *>(w.scales);
    const uint16_t sb = s16[((static_cast<size_t>(g) * w.chunks + c) * 8 + r) * 4 + j];
    out[i] = half_bits_to_float(sb) * static_cast<float>(q);
}

__global__ void f16_embedding_kernel(const uint16_t *table, int rows, int width, const int64_t *token,
    int64_t token_value, float *out) {
    FORTAI_TRACE_SCOPE(15);
    const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= width) return;
    const int seq = static_cast<int>(blockIdx.y);  // batch: token[seq] -> row seq of out
    out += static_cast<size_t>(seq) * width;
    int64_t t = token ? token[seq] : token_value;
    if (t < 0 || t >= rows) t = 0;  // a device-fed id is never trusted as an address
    out[i] = gguf_half_to_real(table[t * width + i]);
}

__global__ void add_kernel(const float *a, const float *b, float *out, int n) {
    const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) out[i] = a[i] + b[i];
}

// fortai_qwen35_cpu.f90:1408-1432 on one workgroup (double sum of squares).
__global__ __launch_bounds__(256) void rms_norm_kernel(const float *x, const float *w, float *out,
    int n, float eps) {
    __shared__ double red[4];
    const int tid = static_cast<int>(threadIdx.x);
    double ss = 0.0;
    for (int i = tid; i < n; i += 256) ss += static_cast<double>(x[i]) * static_cast<double>(x[i]);
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const double total = (red[0] + red[1]) + (red[2] + red[3]);
    const float mean = static_cast<float>(div_count(total, n));
    const float inv = 1.0f / sqrtf(mean + eps);
    for (int i = tid; i < n; i += 256) out[i] = (x[i] * inv) * w[i];
}

}  // namespace

// Which launches take the split form: single matrices of whole register
// chunks that would otherwise run one-wave workgroups (their dot work then
// spreads over four SIMDs) or the gated prologue (32 four-wave workgroups
// would each move 70 KB for ssm_out).  The large four-wave projections keep
// the unsplit form (measured faster).  Both forms give the same bits.
bool matvec_split(int count, int chunks, Prologue prologue, Epilogue epilogue, int waves) {
    if (count != 1 || epilogue == Epilogue::SILU_PAIR) return false;
    if (chunks != 8 && chunks != 16 && chunks != 28 && chunks != 32) return false;
    return waves == 1 || prologue == Prologue::GATED;
}

hipError_t launch_q8_matvec(const MatvecSegment *segments, int count, const MatvecInput &in,
    Prologue prologue, Epilogue epilogue, hipStream_t stream) {
    if (count < 1 || count > 4 || in.width <= 0 || in.width % kQ8Block) return hipErrorInvalidValue;
    // activation widths the register prologues hold
    if (prologue == Prologue::Q8L && (in.width / kQ8Block + 3) / 4 > kMaxChunks) return hipErrorInvalidValue;
    constexpr int kPre = ActShape<64, Prologue::F32>::kPre;  // float4 groups per thread
    const bool f32_in = prologue == Prologue::F32 || prologue == Prologue::RMSNORM || prologue == Prologue::GATED;
    if (prologue == Prologue::GATED) {
        // a head must be an aligned power-of-two run of lanes
        const int hl = in.head / 4;
        if (in.head <= 0 || in.head % 4 || hl > 64 || (hl & (hl - 1)) || in.width % in.head || !in.z || !in.norm)
            return hipErrorInvalidValue;
    }
    for (int s = 0; s < count; ++s) {
        const MatvecSegment &g = segments[s];
        const int conv_rows = g.conv_rows > 0 ? g.conv_rows : g.w.rows;
        if (g.conv_w && (epilogue != Epilogue::STORE || g.kernel < 2 || g.kernel > kConvMax || g.conv_size < conv_rows ||
                            conv_rows > g.w.rows || (g.conv_rows > 0 && conv_rows % kRowsPerWave)))
            return hipErrorInvalidValue;
        if (g.silu_end > g.silu_begin && (epilogue != Epilogue::STORE || g.silu_begin % kRowsPerWave ||
                                             (g.silu_end % kRowsPerWave && g.silu_end != g.w.rows)))
            return hipErrorInvalidValue;
    }
    if (count > 1 && epilogue != Epilogue::STORE) return hipErrorInvalidValue;
    if (f32_in && in.width / 4 > kPre * kMatvecWaves * 64) return hipErrorInvalidValue;
    // small matrices: one wave per workgroup keeps their row groups spread
    // over many CUs (each CU's memory pipeline serves one wave's loads); large
    // multi-matrix launches use 4 (one activation per 32 rows)
    int total_groups = 0;
    for (int s = 0; s < count; ++s) total_groups += segments[s].w.row_groups;
    // (the gated prologue's per-value divisions are spread over 4 waves too)
    const int waves = (epilogue == Epilogue::SILU_PAIR || total_groups >= 1024 || prologue == Prologue::GATED ||
                          (f32_in && in.width / 4 > kPre * 64)) ? 4 : 1;
    if (epilogue == Epilogue::SILU_PAIR) {
        // one workgroup = 32 rows = one quantization block of h
        if (count != 1 || (segments[0].out_q8l && segments[0].w.rows % kQ8Block)) return hipErrorInvalidValue;
    }
    MatvecArgs args{};
    args.count = count;
    args.in = in;
    args.chunks = (in.width / kQ8Block + 3) / 4;
    const bool split = matvec_split(count, args.chunks, prologue, epilogue, waves);
    int grid = 0;
    for (int s = 0; s < count; ++s) {
        args.seg[s] = segments[s];
        args.first_wg[s] = grid;
        if (segments[s].w.chunks != args.chunks) return hipErrorInvalidValue;
        grid += split ? segments[s].w.row_groups : (segments[s].w.row_groups + waves - 1) / waves;
    }
    args.first_wg[count] = grid;
    const int rows = segments[0].w.rows;
    args.pair_vector_rows = rows >= 8 ? (rows / 8) * 8 : 0;
    if (grid == 0) return hipSuccess;
    switch (prologue) {
    case Prologue::Q8: return launch_matvec_pro<Prologue::Q8>(args, waves, grid, args.chunks, epilogue, stream, split);
    case Prologue::F32: return launch_matvec_pro<Prologue::F32>(args, waves, grid, args.chunks, epilogue, stream, split);
    case Prologue::RMSNORM:
        return launch_matvec_pro<Prologue::RMSNORM>(args, waves, grid, args.chunks, epilogue, stream, split);
    case Prologue::Q8L: return launch_matvec_pro<Prologue::Q8L>(args, waves, grid, args.chunks, epilogue, stream, split);
    case Prologue::GATED: return launch_matvec_pro<Prologue::GATED>(args, waves, grid, args.chunks, epilogue, stream, split);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_q8l_prep(const MatvecInput &in, Prologue prologue, void *q8l, int batch, hipStream_t stream) {
    constexpr int kPre = ActShape<kPrepThreads, Prologue::F32>::kPre;
    if (batch < 1 || batch > kMaxBatch || in.width <= 0 || in.width % kQ8Block || in.width / 4 > kPre * kPrepThreads ||
        (in.width / kQ8Block + 3) / 4 > kMaxChunks)
        return hipErrorInvalidValue;
    switch (prologue) {
    case Prologue::F32:
        hipLaunchKernelGGL(q8l_prep_kernel<Prologue::F32>, dim3(batch), dim3(kPrepThreads), 0, stream, in, q8l);
        break;
    case Prologue::RMSNORM:
        hipLaunchKernelGGL(q8l_prep_kernel<Prologue::RMSNORM>, dim3(batch), dim3(kPrepThreads), 0, stream, in, q8l);
        break;
    case Prologue::GATED: {
        const int hl = in.head / 4;
        if (in.head <= 0 || in.head % 4 || hl > 64 || (hl & (hl - 1)) || in.width % in.head || !in.z || !in.norm)
            return hipErrorInvalidValue;
        hipLaunchKernelGGL(q8l_prep_kernel<Prologue::GATED>, dim3(batch), dim3(kPrepThreads), 0, stream, in, q8l);
        break;
    }
    default: return hipErrorInvalidValue;
    }
    note_launch("q8l_prep_kernel<%s> grid %d", prologue_name(prologue), batch);
    return hipGetLastError();
}

hipError_t launch_q8_batch_matvec(const MatvecSegment *segments, int count, const void *q8l, int width, int batch,
    Epilogue epilogue, hipStream_t stream) {
    const int chunks = (width / kQ8Block + 3) / 4;
    if (count < 1 || count > 4 || width <= 0 || width % kQ8Block || batch < 1 || batch > kMaxBatch ||
        static_cast<size_t>(batch) * chunks * 144 > 120 * 1024)
        return hipErrorInvalidValue;
    int total_groups = 0;
    for (int s = 0; s < count; ++s) {
        if (segments[s].w.chunks != chunks) return hipErrorInvalidValue;
        if (segments[s].conv_w && (epilogue != Epilogue::STORE || segments[s].kernel < 2 ||
                                     segments[s].kernel > kConvMax || segments[s].conv_size < segments[s].w.rows))
            return hipErrorInvalidValue;
        total_groups += segments[s].w.row_groups;
    }
    // enough waves for the chip: sequences spread over up to 4 waves per row
    // group when the matrices are small (the quantized-h epilogue needs all
    // sequences of 32 rows in one workgroup)
    int split = total_groups >= 1024 ? 1 : (total_groups >= 512 ? 2 : 4);
    if (epilogue == Epilogue::SILU_PAIR) {
        if (count != 1 || (segments[0].out_q8l && segments[0].w.rows % kQ8Block)) return hipErrorInvalidValue;
        // one workgroup = 32 rows of every sequence (one quantization block of
        // h): eight waves, two per row group with four sequences each
        split = 2;
    }
    BatchMatvecArgs args{};
    args.count = count;
    args.chunks = chunks;
    args.batch = batch;
    args.split = split;
    args.act = q8l;
    int grid = 0;
    // the pair: one 32-row quantization block of h per eight-wave workgroup,
    // or two per sixteen-wave workgroup when the blocks outnumber the CUs (a
    // launch of, say, 288 blocks would give 32 CUs two workgroups each and
    // end with them; 144 workgroups of two blocks each end together)
    const bool pair_blocks2 = epilogue == Epilogue::SILU_PAIR && segments[0].w.row_groups > 4 * 256 &&
        segments[0].w.row_groups % 8 == 0;
    const int per_wg = epilogue == Epilogue::SILU_PAIR ? (pair_blocks2 ? 8 : 4) : 4 / split;
    for (int s = 0; s < count; ++s) {
        args.seg[s] = segments[s];
        args.first_wg[s] = grid;
        grid += (segments[s].w.row_groups + per_wg - 1) / per_wg;
    }
    args.first_wg[count] = grid;
    const int rows = segments[0].w.rows;
    args.pair_vector_rows = rows >= 8 ? (rows / 8) * 8 : 0;
    if (grid == 0) return hipSuccess;
    const size_t act = (static_cast<size_t>(batch) * chunks * 144 + 1023) / 1024 * 1024;
    const size_t lds = act + kMaxBatch * 32 * 4;
    const int ring_groups = chunks % kRingG == 0 ? chunks / kRingG : 0;
    const bool ring = epilogue != Epilogue::SILU_PAIR && (ring_groups == 2 || ring_groups == 4 || ring_groups == 5 ||
        ring_groups == 7 || ring_groups == 8 || ring_groups == 16 || ring_groups == 18);
    if (ring) {
        // weights fetched once per workgroup (a register ring of up to 8
        // groups per wave, shared through LDS): one workgroup per row group
        int ring_grid = 0;
        for (int s = 0; s < count; ++s) {
            args.first_wg[s] = ring_grid;
            ring_grid += segments[s].w.row_groups;
        }
        args.first_wg[count] = ring_grid;
        constexpr size_t kSlot = kRingG * 1024 + kRingG * 64;
        // two sequences per wave, or one when eight sequences' activations
        // would keep the workgroup at one per CU
        const int ns = static_cast<size_t>(std::min(batch, 8)) * chunks * 144 > 48 * 1024 ? 1 : 2;
        const int per_block = 4 * ns, seq_blocks = (batch + per_block - 1) / per_block;
        const size_t ring_lds = (static_cast<size_t>(std::min(batch, per_block)) * chunks * 144 + 1023) / 1024 * 1024 +
            2 * kSlot + (ns == 2 ? 2 * static_cast<size_t>(kRingG) * per_block * 8 * 16 : 0);
        if (ring_lds > 160 * 1024) return hipErrorInvalidValue;
#define FORTAI_RING(E, G)                                                                                          \
    do {                                                                                                          \
        if (ns == 1)                                                                                              \
            hipLaunchKernelGGL((q8_batch_ring_kernel<E, G, 1>), dim3(ring_grid, seq_blocks), dim3(kBatchThreads), \
                ring_lds, stream, args);                                                                          \
        else                                                                                                      \
            hipLaunchKernelGGL((q8_batch_ring_kernel<E, G, 2>), dim3(ring_grid, seq_blocks), dim3(kBatchThreads), \
                ring_lds, stream, args);                                                                          \
    } while (0)
#define FORTAI_RING_E(E)                                 \
        switch (ring_groups) {                           \
        case 2: FORTAI_RING(E, 2); break;                \
        case 4: FORTAI_RING(E, 4); break;                \
        case 5: FORTAI_RING(E, 5); break;                \
        case 7: FORTAI_RING(E, 7); break;                \
        case 8: FORTAI_RING(E, 8); break;                \
        case 16: FORTAI_RING(E, 16); break;              \
        default: FORTAI_RING(E, 18); break;              \
        }
        if (epilogue == Epilogue::STORE) { FORTAI_RING_E(Epilogue::STORE) }
        else { FORTAI_RING_E(Epilogue::ADD) }
#undef FORTAI_RING_E
#undef FORTAI_RING
        note_launch("q8_batch_ring_kernel<%s,groups=%d,seqs/wave=%d> grid %dx%d", epilogue_name(epilogue), ring_groups,
            ns, ring_grid, seq_blocks);
        return hipGetLastError();
    }
    // the pair's per-wave scale-product tables: waves x [2][8][4][4] floats
    if (epilogue == Epilogue::SILU_PAIR) {
        if (pair_blocks2)
            return launch_batch_g<Epilogue::SILU_PAIR, 2, 16>(args, grid, lds + kMaxBatch * 32 * 4 +
                16 * 2 * 8 * 4 * 4 * sizeof(float), stream);
        return launch_batch_g<Epilogue::SILU_PAIR, 2, 8>(args, grid, lds + 8 * 2 * 8 * 4 * 4 * sizeof(float), stream);
    }
    if (epilogue == Epilogue::STORE) {
        if (split == 1) return launch_batch_g<Epilogue::STORE, 1>(args, grid, lds, stream);
        if (split == 2) return launch_batch_g<Epilogue::STORE, 2>(args, grid, lds, stream);
        return launch_batch_g<Epilogue::STORE, 4>(args, grid, lds, stream);
    }
    if (epilogue == Epilogue::ADD) {
        if (split == 1) return launch_batch_g<Epilogue::ADD, 1>(args, grid, lds, stream);
        if (split == 2) return launch_batch_g<Epilogue::ADD, 2>(args, grid, lds, stream);
        return launch_batch_g<Epilogue::ADD, 4>(args, grid, lds, stream);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_q8_repack(const uint8_t *gguf, int rows, int blocks, uint4 *quants, uint2 *scales,
    hipStream_t stream) {
    const int chunks = (blocks + 3) / 4;
    const int row_groups = (rows + kRowsPerWave - 1) / kRowsPerWave;
    const size_t total = static_cast<size_t>(row_groups) * chunks * 64;
    const int threads = 256;
    const size_t grid = (total + threads - 1) / threads;
    hipLaunchKernelGGL(q8_repack_kernel, dim3(static_cast<unsigned>(grid)), dim3(threads), 0, stream,
        gguf, rows, blocks, chunks, row_groups, quants, scales);
    return hipGetLastError();
}

hipError_t launch_q8_quantize(const float *x, int width, int8_t *out34, float *scales, hipStream_t stream) {
    if (width <= 0 || width % kQ8Block) return hipErrorInvalidValue;
    const int groups = width / 4;
    hipLaunchKernelGGL(q8_quantize_kernel, dim3((groups + 255) / 256), dim3(256), 0, stream, x, width, out34, scales);
    return hipGetLastError();
}

hipError_t launch_q8_block_dots(const Q8Matrix &w, const int8_t *xq34, int32_t *out, hipStream_t stream) {
    const size_t lds = static_cast<size_t>(w.chunks) * 144;
    hipLaunchKernelGGL(q8_block_dots_kernel, dim3(w.row_groups), dim3(64), lds, stream, w, xq34, out, w.blocks);
    return hipGetLastError();
}

hipError_t launch_q8_embedding(const Q8Matrix &w, const int64_t *token, int64_t token_value, float *out,
    hipStream_t stream, int batch) {
    if (batch < 1 || (batch > 1 && !token)) return hipErrorInvalidValue;
    const int n = w.blocks * kQ8Block;
    hipLaunchKernelGGL(q8_embedding_kernel, dim3((n + 255) / 256, batch), dim3(256), 0, stream, w, token, token_value, out);
    note_launch("q8_embedding_kernel grid %dx%d", (n + 255) / 256, batch);
    return hipGetLastError();
}

hipError_t launch_f16_embedding(const uint16_t *table, int rows, int width, const int64_t *token,
    int64_t token_value, float *out, hipStream_t stream, int batch) {
    if (batch < 1 || (batch > 1 && !token)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(f16_embedding_kernel, dim3((width + 255) / 256, batch), dim3(256), 0, stream, table, rows, width,
        token, token_value, out);
    note_launch("f16_embedding_kernel grid %dx%d", (width + 255) / 256, batch);
    return hipGetLastError();
}

hipError_t launch_add(const float *a, const float *b, float *out, int n, hipStream_t stream) {
    hipLaunchKernelGGL(add_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, a, b, out, n);
    return hipGetLastError();
}

hipError_t launch_rms_norm(const float *x, const float *w, float *out, int n, float eps, hipStream_t stream) {
    hipLaunchKernelGGL(rms_norm_kernel, dim3(1), dim3(256), 0, stream, x, w, out, n, eps);
    return hipGetLastError();
}

}  // namespace fortai_hip
