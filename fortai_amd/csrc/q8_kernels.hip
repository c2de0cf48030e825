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
// The activation is quantized inside every workgroup (fortai_q8_quantize,
// fortai_q8_dot.c:153-198) from the producer's fp32 vector, optionally after
// the RMSNorm of fortai_qwen35_cpu.f90:1408-1432 or the gated norm of
// :907-915, and kept in LDS as [chunk][lane][4 blocks] 4-byte groups.
#include "fortai_hip_internal.h"
#include "fortai_hip_kernels.h"

namespace fortai_hip {

namespace {

struct MatvecArgs {
    MatvecSegment seg[4];
    int first_wg[5];
    int count;
    int chunks;  // activation chunks (ceil(blocks / 4))
    int pair_vector_rows;  // SILU_PAIR: rows below this use the vector SiLU lane
    MatvecInput in;
};

__device__ __forceinline__ uint32_t load_u32_unaligned(const int8_t *p) {
    const uint8_t *b = reinterpret_cast<const uint8_t *>(p);
    return static_cast<uint32_t>(b[0]) | (static_cast<uint32_t>(b[1]) << 8) |
        (static_cast<uint32_t>(b[2]) << 16) | (static_cast<uint32_t>(b[3]) << 24);
}

__device__ __forceinline__ int8_t sat8_rne(float v) {
    const float r = rintf(v);
    // cvtps_epi32 gives INT32_MIN for NaN/out of range, which packs to -128
    if (!(r >= -2147483648.0f && r < 2147483648.0f)) return -128;
    return static_cast<int8_t>(r < -128.0f ? -128.0f : (r > 127.0f ? 127.0f : r));
}

// Quantize one 4-value group of a 32-value block held by 8 consecutive
// lanes (lane l of the block holds values 4l..4l+3).  Returns the packed
// int8x4 and the block's fp32 scale (f32 of the fp16 RNE scale).
__device__ __forceinline__ uint32_t quantize_group(float4 y, float &scale_out, uint16_t &scale_bits) {
    float amax = fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    amax = fmaxf(amax, __shfl_xor(amax, 4));
    const float scale = amax / 127.0f;
    const float inverse = amax != 0.0f ? 127.0f / amax : 0.0f;
    scale_bits = float_to_half_rne(scale);
    scale_out = half_bits_to_float(scale_bits);
    const uint32_t q0 = static_cast<uint8_t>(sat8_rne(y.x * inverse));
    const uint32_t q1 = static_cast<uint8_t>(sat8_rne(y.y * inverse));
    const uint32_t q2 = static_cast<uint8_t>(sat8_rne(y.z * inverse));
    const uint32_t q3 = static_cast<uint8_t>(sat8_rne(y.w * inverse));
    return q0 | (q1 << 8) | (q2 << 16) | (q3 << 24);
}

// Build the workgroup's LDS copy of the quantized activation.
//   act32[(c * 8 + l) * 4 + j] = int8x4 of lane l of block 4c+j
//   act_s[b] = fp32 activation scale of block b
template <int THREADS, Prologue PRO>
__device__ __forceinline__ void build_activation(const MatvecInput &in, int chunks, uint32_t *act32,
    float *act_s, double *red) {
    const int tid = static_cast<int>(threadIdx.x);
    const int groups = in.width / 4;
    const int blocks = in.width / kQ8Block;
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
        const float4 *x4 = reinterpret_cast<const float4 *>(in.x);
        float inverse_rms = 1.0f;
        if constexpr (PRO == Prologue::RMSNORM) {
            double ss = 0.0;
            for (int g = tid; g < groups; g += THREADS) {
                const float4 v = x4[g];
                ss += static_cast<double>(v.x) * static_cast<double>(v.x);
                ss += static_cast<double>(v.y) * static_cast<double>(v.y);
                ss += static_cast<double>(v.z) * static_cast<double>(v.z);
                ss += static_cast<double>(v.w) * static_cast<double>(v.w);
            }
            ss = wave_sum(ss);
            if ((tid & 63) == 0) red[tid >> 6] = ss;
            __syncthreads();
            double total = 0.0;
            for (int w = 0; w < THREADS / 64; ++w) total += red[w];
            const float mean = static_cast<float>(total / static_cast<double>(in.width));
            inverse_rms = 1.0f / sqrtf(mean + in.eps);
        }
        const int iterations = (groups + THREADS - 1) / THREADS;
        for (int it = 0; it < iterations; ++it) {
            const int g = tid + it * THREADS;
            const bool valid = g < groups;
            float4 y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (valid) y = x4[g];
            if constexpr (PRO == Prologue::RMSNORM) {
                if (valid) {
                    const float4 w = reinterpret_cast<const float4 *>(in.norm)[g];
                    y.x = (y.x * inverse_rms) * w.x;
                    y.y = (y.y * inverse_rms) * w.y;
                    y.z = (y.z * inverse_rms) * w.z;
                    y.w = (y.w * inverse_rms) * w.w;
                }
            } else if constexpr (PRO == Prologue::GATED) {
                // rms over the head (head/4 consecutive lanes), double sum
                double ss = static_cast<double>(y.x) * static_cast<double>(y.x);
                ss += static_cast<double>(y.y) * static_cast<double>(y.y);
                ss += static_cast<double>(y.z) * static_cast<double>(y.z);
                ss += static_cast<double>(y.w) * static_cast<double>(y.w);
                for (int m = 1; m < in.head / 4; m <<= 1) ss += __shfl_xor(ss, m);
                if (valid) {
                    const float nf = sqrtf(static_cast<float>(ss / static_cast<double>(in.head)) + in.eps);
                    const float4 z = reinterpret_cast<const float4 *>(in.gate)[g];
                    const int j = (4 * g) % in.head;
                    const float4 w = *reinterpret_cast<const float4 *>(in.norm + j);
                    y.x = ((y.x / nf) * w.x) * silu_poly(z.x);
                    y.y = ((y.y / nf) * w.y) * silu_poly(z.y);
                    y.z = ((y.z / nf) * w.z) * silu_poly(z.z);
                    y.w = ((y.w / nf) * w.w) * silu_poly(z.w);
                }
            }
            float scale;
            uint16_t bits;
            const uint32_t packed = quantize_group(y, scale, bits);
            if (valid) {
                const int b = g >> 3, l = g & 7;
                act32[((b >> 2) * 8 + l) * 4 + (b & 3)] = packed;
                if (l == 0) act_s[b] = scale;
            }
        }
        __syncthreads();
    }
}

template <int WAVES, Prologue PRO, Epilogue EPI>
__global__ __launch_bounds__(WAVES * 64) void q8_matvec_kernel(const MatvecArgs args) {
    extern __shared__ __align__(16) unsigned char lds[];
    uint32_t *act32 = reinterpret_cast<uint32_t *>(lds);
    float *act_s = reinterpret_cast<float *>(lds + static_cast<size_t>(args.chunks) * 8 * 16);
    double *red = reinterpret_cast<double *>(lds + static_cast<size_t>(args.chunks) * (8 * 16 + 16));
    build_activation<WAVES * 64, PRO>(args.in, args.chunks, act32, act_s, red);

    const int wg = static_cast<int>(blockIdx.x);
    int s = 0;
    while (s + 1 < args.count && wg >= args.first_wg[s + 1]) ++s;
    const MatvecSegment &seg = args.seg[s];
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int rg = (wg - args.first_wg[s]) * WAVES + wave;
    if (rg >= seg.w.row_groups) return;
    const int r = lane >> 3, l = lane & 7;
    const int chunks = seg.w.chunks;
    const uint4 *qp = seg.w.quants + static_cast<size_t>(rg) * chunks * 64 + lane;
    const uint2 *sp = seg.w.scales + static_cast<size_t>(rg) * chunks * 8 + r;
    const uint4 *qp2 = nullptr;
    const uint2 *sp2 = nullptr;
    if constexpr (EPI == Epilogue::SILU_PAIR) {
        qp2 = seg.w2.quants + static_cast<size_t>(rg) * chunks * 64 + lane;
        sp2 = seg.w2.scales + static_cast<size_t>(rg) * chunks * 8 + r;
    }
    const uint4 *act4 = reinterpret_cast<const uint4 *>(act32);
    const float4 *as4 = reinterpret_cast<const float4 *>(act_s);
    float acc = 0.0f, acc2 = 0.0f;
#pragma unroll 4
    for (int c = 0; c < chunks; ++c) {
        const uint4 q = load_stream(qp + static_cast<size_t>(c) * 64);
        const uint2 sc = load_stream(sp + static_cast<size_t>(c) * 8);
        const uint4 a = act4[c * 8 + l];
        const float4 as = as4[c];
        acc = __builtin_fmaf(half_bits_to_float(static_cast<uint16_t>(sc.x)) * as.x,
            static_cast<float>(__builtin_amdgcn_sdot4(static_cast<int>(q.x), static_cast<int>(a.x), 0, false)), acc);
        acc = __builtin_fmaf(half_bits_to_float(static_cast<uint16_t>(sc.x >> 16)) * as.y,
            static_cast<float>(__builtin_amdgcn_sdot4(static_cast<int>(q.y), static_cast<int>(a.y), 0, false)), acc);
        acc = __builtin_fmaf(half_bits_to_float(static_cast<uint16_t>(sc.y)) * as.z,
            static_cast<float>(__builtin_amdgcn_sdot4(static_cast<int>(q.z), static_cast<int>(a.z), 0, false)), acc);
        acc = __builtin_fmaf(half_bits_to_float(static_cast<uint16_t>(sc.y >> 16)) * as.w,
            static_cast<float>(__builtin_amdgcn_sdot4(static_cast<int>(q.w), static_cast<int>(a.w), 0, false)), acc);
        if constexpr (EPI == Epilogue::SILU_PAIR) {
            const uint4 q2 = load_stream(qp2 + static_cast<size_t>(c) * 64);
            const uint2 sc2 = load_stream(sp2 + static_cast<size_t>(c) * 8);
            acc2 = __builtin_fmaf(half_bits_to_float(static_cast<uint16_t>(sc2.x)) * as.x,
                static_cast<float>(__builtin_amdgcn_sdot4(static_cast<int>(q2.x), static_cast<int>(a.x), 0, false)), acc2);
            acc2 = __builtin_fmaf(half_bits_to_float(static_cast<uint16_t>(sc2.x >> 16)) * as.y,
                static_cast<float>(__builtin_amdgcn_sdot4(static_cast<int>(q2.y), static_cast<int>(a.y), 0, false)), acc2);
            acc2 = __builtin_fmaf(half_bits_to_float(static_cast<uint16_t>(sc2.y)) * as.z,
                static_cast<float>(__builtin_amdgcn_sdot4(static_cast<int>(q2.z), static_cast<int>(a.z), 0, false)), acc2);
            acc2 = __builtin_fmaf(half_bits_to_float(static_cast<uint16_t>(sc2.y >> 16)) * as.w,
                static_cast<float>(__builtin_amdgcn_sdot4(static_cast<int>(q2.w), static_cast<int>(a.w), 0, false)), acc2);
        }
    }
    acc = row_hsum8(acc);
    if constexpr (EPI == Epilogue::SILU_PAIR) acc2 = row_hsum8(acc2);
    const int row = rg * kRowsPerWave + r;
    if (l != 0 || row >= seg.w.rows) return;
    if constexpr (EPI == Epilogue::STORE) {
        seg.out[row] = acc;
    } else if constexpr (EPI == Epilogue::ADD) {
        seg.out[row] = acc + seg.resid[row];
    } else {
        // fortai_silu_product: vector lanes for the first count/8*8 rows, the
        // libm tail expression for the rest (fortai_q8_dot.c:492-505)
        if (row < args.pair_vector_rows) seg.out[row] = silu_poly(acc) * acc2;
        else seg.out[row] = acc / (1.0f + exp_rounded(-acc)) * acc2;
    }
}

template <int WAVES, Prologue PRO, Epilogue EPI>
hipError_t launch_matvec_t(const MatvecArgs &args, int grid, hipStream_t stream) {
    const size_t lds = static_cast<size_t>(args.chunks) * (8 * 16 + 16) + 8 * WAVES;
    hipLaunchKernelGGL((q8_matvec_kernel<WAVES, PRO, EPI>), dim3(grid), dim3(WAVES * 64), lds, stream, args);
    return hipGetLastError();
}

template <int WAVES, Prologue PRO>
hipError_t launch_matvec_epi(const MatvecArgs &args, int grid, Epilogue epi, hipStream_t stream) {
    switch (epi) {
    case Epilogue::STORE: return launch_matvec_t<WAVES, PRO, Epilogue::STORE>(args, grid, stream);
    case Epilogue::ADD: return launch_matvec_t<WAVES, PRO, Epilogue::ADD>(args, grid, stream);
    case Epilogue::SILU_PAIR: return launch_matvec_t<WAVES, PRO, Epilogue::SILU_PAIR>(args, grid, stream);
    }
    return hipErrorInvalidValue;
}

constexpr int kMatvecWaves = 2;

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
        int d[4] = {__builtin_amdgcn_sdot4(static_cast<int>(q.x), static_cast<int>(a.x), 0, false),
            __builtin_amdgcn_sdot4(static_cast<int>(q.y), static_cast<int>(a.y), 0, false),
            __builtin_amdgcn_sdot4(static_cast<int>(q.z), static_cast<int>(a.z), 0, false),
            __builtin_amdgcn_sdot4(static_cast<int>(q.w), static_cast<int>(a.w), 0, false)};
        for (int j = 0; j < 4; ++j) {
            int v = d[j];
            v += __shfl_xor(v, 4);
            v += __shfl_xor(v, 2);
            v += __shfl_xor(v, 1);
            const int b = 4 * c + j;
            if (l == 0 && row < w.rows && b < blocks) out[static_cast<size_t>(row) * blocks + b] = v;
        }
    }
}

__global__ void q8_embedding_kernel(Q8Matrix w, const int64_t *token, int64_t token_value, float *out) {
    const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= w.blocks * kQ8Block) return;
    const int64_t t = token ? *token : token_value;
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

__global__ void f16_embedding_kernel(const uint16_t *table, int width, const int64_t *token,
    int64_t token_value, float *out) {
    const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= width) return;
    const int64_t t = token ? *token : token_value;
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
    const float mean = static_cast<float>(total / static_cast<double>(n));
    const float inv = 1.0f / sqrtf(mean + eps);
    for (int i = tid; i < n; i += 256) out[i] = (x[i] * inv) * w[i];
}

}  // namespace

hipError_t launch_q8_matvec(const MatvecSegment *segments, int count, const MatvecInput &in,
    Prologue prologue, Epilogue epilogue, hipStream_t stream) {
    if (count < 1 || count > 4 || in.width <= 0 || in.width % kQ8Block) return hipErrorInvalidValue;
    MatvecArgs args{};
    args.count = count;
    args.in = in;
    args.chunks = (in.width / kQ8Block + 3) / 4;
    int grid = 0;
    for (int s = 0; s < count; ++s) {
        args.seg[s] = segments[s];
        args.first_wg[s] = grid;
        if (segments[s].w.chunks != args.chunks) return hipErrorInvalidValue;
        grid += (segments[s].w.row_groups + kMatvecWaves - 1) / kMatvecWaves;
    }
    args.first_wg[count] = grid;
    const int rows = segments[0].w.rows;
    args.pair_vector_rows = rows >= 8 ? (rows / 8) * 8 : 0;
    if (grid == 0) return hipSuccess;
    switch (prologue) {
    case Prologue::Q8: return launch_matvec_epi<kMatvecWaves, Prologue::Q8>(args, grid, epilogue, stream);
    case Prologue::F32: return launch_matvec_epi<kMatvecWaves, Prologue::F32>(args, grid, epilogue, stream);
    case Prologue::RMSNORM: return launch_matvec_epi<kMatvecWaves, Prologue::RMSNORM>(args, grid, epilogue, stream);
    case Prologue::GATED:
        if (in.head < 4 || in.head > 256 || (in.head & (in.head - 1)) || in.width % in.head) return hipErrorInvalidValue;
        return launch_matvec_epi<kMatvecWaves, Prologue::GATED>(args, grid, epilogue, stream);
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
    const size_t lds = static_cast<size_t>(w.chunks) * (8 * 16 + 16);
    hipLaunchKernelGGL(q8_block_dots_kernel, dim3(w.row_groups), dim3(64), lds, stream, w, xq34, out, w.blocks);
    return hipGetLastError();
}

hipError_t launch_q8_embedding(const Q8Matrix &w, const uint8_t *, const int64_t *token, int64_t token_value,
    float *out, hipStream_t stream) {
    const int n = w.blocks * kQ8Block;
    hipLaunchKernelGGL(q8_embedding_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, w, token, token_value, out);
    return hipGetLastError();
}

hipError_t launch_f16_embedding(const uint16_t *table, int width, const int64_t *token, int64_t token_value,
    float *out, hipStream_t stream) {
    hipLaunchKernelGGL(f16_embedding_kernel, dim3((width + 255) / 256), dim3(256), 0, stream, table, width, token,
        token_value, out);
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
