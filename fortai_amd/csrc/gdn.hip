// Gated DeltaNet decode step for gfx950, one workgroup per key head:
// causal conv1d + SiLU, L2 norm of q and k, decay/beta, the delta-rule state
// update, and the gated RMSNorm of the output with its Q8_0 quantisation for
// the ssm_out projection -- fused in one launch with no cross-workgroup
// traffic (a workgroup owns every conv channel and state row it touches).
//
// Reference: the recurrent branch of fortai_qwen35_cpu.f90:856-916 and the
// AVX2 state step fortai_q8_dot.c:356-398.  A state row r of value head h only
// depends on S[h][r][:], k, q, v[r], beta and the decay, so 8 lanes of a wave
// own one row and lane l owns columns l, l+8, l+16, ... -- exactly the fp32
// lane of the reference's 8-wide vector loop -- with the same fma chains and
// the same horizontal-sum tree: the state and raw output are bit-identical to
// the CPU step.
//
// Layouts (backend-owned, persistent):
//  * state[((h * head + r) * 8 + l) * (head / 8) + i] = S[h][r][8 i + l]
//    (a lane's head/8 floats are contiguous: 16-byte loads and stores);
//  * conv_state[slot][conv_size], oldest slot first, shifted in place by the
//    channel's owner (fortai_qwen35_cpu.f90:870-879).
#include "fortai_hip_internal.h"
#include "fortai_hip_kernels.h"

namespace fortai_hip {

namespace {

constexpr int kThreads = 1024;
constexpr int kMaxKernel = 8;

template <int HEAD>
__global__ __launch_bounds__(kThreads) void gdn_group_kernel(const GdnParams p) {
    constexpr int kCols = HEAD / 8;  // columns per lane
    extern __shared__ __align__(16) float smem[];
    const int ratio = p.value_heads / p.key_heads;
    const int rows = ratio * HEAD;   // state rows of this workgroup
    float *qs = smem;                // [HEAD]
    float *ks = qs + HEAD;           // [HEAD]
    float *vs = ks + HEAD;           // [rows]
    float *os = vs + rows;           // [rows]
    float *hs = os + rows;           // [ratio][2]: beta, decay factor
    double *red = reinterpret_cast<double *>(hs + 2 * ratio + (ratio & 1) * 2);  // [2]
    const int tid = static_cast<int>(threadIdx.x);
    const int kh = static_cast<int>(blockIdx.x);
    const int h0 = kh * ratio;       // first value head of the group
    const int K = p.kernel;

    // state rows of the first pass: issue the loads before anything else
    const int r8 = tid >> 3, l = tid & 7;
    const int passes = (rows * 8 + kThreads - 1) / kThreads;
    float s[kCols];
    auto state_ptr = [&](int row) {
        const int h = h0 + row / HEAD, rr = row % HEAD;
        return reinterpret_cast<float4 *>(p.state + ((static_cast<size_t>(h) * HEAD + rr) * 8 + l) * kCols);
    };
    auto load_state = [&](int row) {
        const float4 *src = state_ptr(row);
#pragma unroll
        for (int i = 0; i < kCols / 4; ++i) {
            const float4 f = src[i];
            s[4 * i] = f.x; s[4 * i + 1] = f.y; s[4 * i + 2] = f.z; s[4 * i + 3] = f.w;
        }
    };
    if (r8 < rows) load_state(r8);
    // operands of the gated norm, also fetched up front (4 values per thread)
    const int groups = rows / 4;
    float4 zpre = make_float4(0.0f, 0.0f, 0.0f, 0.0f), npre = zpre;
    if (p.out_q8l && tid < groups) {
        zpre = reinterpret_cast<const float4 *>(p.z + static_cast<size_t>(h0) * HEAD)[tid];
        npre = *reinterpret_cast<const float4 *>(p.ssm_norm + (4 * tid) % HEAD);
    }

    // conv + SiLU over every channel of the group, then shift the window
    const int qk_base = kh * HEAD;
    const int k_base = p.state_size * p.key_heads + kh * HEAD;
    const int v_base = 2 * p.state_size * p.key_heads + h0 * HEAD;
    const int nch = 2 * HEAD + rows;
    for (int i = tid; i < nch; i += kThreads) {
        const int ch = i < HEAD ? qk_base + i : (i < 2 * HEAD ? k_base + (i - HEAD) : v_base + (i - 2 * HEAD));
        float window[kMaxKernel];
        for (int slot = 0; slot < K - 1; ++slot) window[slot] = p.conv_state[static_cast<size_t>(slot) * p.conv_size + ch];
        const float x = p.qkv[ch];
        const float *w = p.conv_w + static_cast<size_t>(ch) * K;
        // fortai_qwen35_cpu.f90:856-867: oldest slot first, current value last
        float acc = 0.0f;
        for (int slot = 0; slot < K - 1; ++slot) acc = acc + w[slot] * window[slot];
        acc = acc + w[K - 1] * x;
        smem[i] = silu_poly(acc);  // qs | ks | vs are contiguous
        for (int slot = 0; slot + 1 < K - 1; ++slot)
            p.conv_state[static_cast<size_t>(slot) * p.conv_size + ch] = window[slot + 1];
        p.conv_state[static_cast<size_t>(K - 2) * p.conv_size + ch] = x;
    }
    // per value head scalars (fortai_qwen35_cpu.f90:890-894), by otherwise idle threads
    if (tid >= kThreads - ratio) {
        const int hl = tid - (kThreads - ratio), h = h0 + hl;
        hs[2 * hl] = sigmoid_ref(p.beta[h]);
        hs[2 * hl + 1] = exp_rounded(p.ssm_a[h] * softplus_ref(p.alpha[h] + p.ssm_dt[h]));
    }
    __syncthreads();
    // L2 norms of q (wave 0) and k (wave 1), fortai_qwen35_cpu.f90:1455-1471
    if (tid < 128) {
        const float *v = (tid < 64) ? qs : ks;
        double ss = 0.0;
        for (int i = tid & 63; i < HEAD; i += 64) ss += static_cast<double>(v[i]) * static_cast<double>(v[i]);
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
    }
    __syncthreads();
    if (tid < 2 * HEAD) {
        const float n = sqrtf(static_cast<float>(red[tid < HEAD ? 0 : 1]));
        const float inv = 1.0f / (n > p.eps ? n : p.eps);
        smem[tid] = smem[tid] * inv;
    }
    __syncthreads();

    // delta rule, one row per 8 lanes (fortai_q8_dot.c:363-396)
    const float output_scale = 1.0f / sqrtf(static_cast<float>(HEAD));
    for (int pass = 0; pass < passes; ++pass) {
        const int row = pass * (kThreads / 8) + r8;
        if (row >= rows) break;
        if (pass > 0) load_state(row);
        const int hl = row / HEAD;
        const float beta = hs[2 * hl], decay = hs[2 * hl + 1];
        float kd = 0.0f;
#pragma unroll
        for (int i = 0; i < kCols; ++i) {
            const float d = s[i] * decay;
            s[i] = d;
            kd = __builtin_fmaf(d, ks[8 * i + l], kd);
        }
        kd = row_hsum8(kd);
        const float delta = (vs[row] - kd) * beta;
        float qd = 0.0f;
#pragma unroll
        for (int i = 0; i < kCols; ++i) {
            const float u = __builtin_fmaf(delta, ks[8 * i + l], s[i]);
            s[i] = u;
            qd = __builtin_fmaf(u, qs[8 * i + l], qd);
        }
        qd = row_hsum8(qd);
        float4 *dst = state_ptr(row);
#pragma unroll
        for (int i = 0; i < kCols / 4; ++i) dst[i] = make_float4(s[4 * i], s[4 * i + 1], s[4 * i + 2], s[4 * i + 3]);
        if (l == 0) {
            const float o = qd * output_scale;
            os[row] = o;
            if (p.out) p.out[h0 * HEAD + row] = o;
        }
    }
    __syncthreads();

    // gated RMSNorm per value head (fortai_qwen35_cpu.f90:907-915), then the
    // Q8_0 quantisation of the ssm_out input: 4 values per thread, a head is
    // HEAD/4 consecutive lanes of one wave
    if (!p.out_q8l) return;
    if (tid < ((groups + 63) / 64) * 64) {
        const bool valid = tid < groups;
        float4 y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (valid) y = reinterpret_cast<const float4 *>(os)[tid];
        double ss = static_cast<double>(y.x) * static_cast<double>(y.x);
        ss += static_cast<double>(y.y) * static_cast<double>(y.y);
        ss += static_cast<double>(y.z) * static_cast<double>(y.z);
        ss += static_cast<double>(y.w) * static_cast<double>(y.w);
        for (int m = 1; m < HEAD / 4; m <<= 1) ss += __shfl_xor(ss, m);
        if (valid) {
            const float nf = sqrtf(static_cast<float>(ss / static_cast<double>(HEAD)) + p.eps);
            const float4 w = npre, z = zpre;
            y.x = ((y.x / nf) * w.x) * silu_poly(z.x);
            y.y = ((y.y / nf) * w.y) * silu_poly(z.y);
            y.z = ((y.z / nf) * w.z) * silu_poly(z.z);
            y.w = ((y.w / nf) * w.w) * silu_poly(z.w);
        }
        float scale;
        uint16_t bits;
        const uint32_t packed = quantize_group(y, scale, bits);
        if (valid) {
            const int g = h0 * HEAD / 4 + tid;  // group index in the inner vector
            const int b = g >> 3, ll = g & 7;
            const int chunks = (p.value_heads * HEAD / kQ8Block + 3) / 4;
            uint32_t *dq = static_cast<uint32_t *>(p.out_q8l);
            dq[((b >> 2) * 8 + ll) * 4 + (b & 3)] = packed;
            if (ll == 0) reinterpret_cast<float *>(dq + chunks * 32)[b] = scale;
        }
    }
}

// The delta rule of 16 state rows of one value head per workgroup (128
// threads, 8 lanes per row): the L2 norms of the head's q and k (waves 0 and
// 1, the same sums as gdn_group_kernel), beta and the decay, the row updates
// and the raw output.  qkv already holds conv + SiLU.
constexpr int kDeltaRows = 16;
constexpr int kDeltaThreads = kDeltaRows * 8;

template <int HEAD>
__global__ __launch_bounds__(kDeltaThreads) void gdn_delta_kernel(const GdnParams p) {
    constexpr int kCols = HEAD / 8;
    __shared__ __align__(16) float qs[HEAD];
    __shared__ __align__(16) float ks[HEAD];
    __shared__ double red[2];
    __shared__ float hs[2];
    const int tid = static_cast<int>(threadIdx.x);
    const int blocks_per_head = HEAD / kDeltaRows;
    const int h = static_cast<int>(blockIdx.x) / blocks_per_head;
    const int r0 = (static_cast<int>(blockIdx.x) % blocks_per_head) * kDeltaRows;
    const int kh = h / (p.value_heads / p.key_heads);
    const int r8 = tid >> 3, l = tid & 7, row = r0 + r8;
    // every load first: the state row, q and k of the key head, v, the scalars
    float s[kCols];
    float4 *srow = reinterpret_cast<float4 *>(p.state + ((static_cast<size_t>(h) * HEAD + row) * 8 + l) * kCols);
#pragma unroll
    for (int i = 0; i < kCols / 4; ++i) {
        const float4 f = srow[i];
        s[4 * i] = f.x; s[4 * i + 1] = f.y; s[4 * i + 2] = f.z; s[4 * i + 3] = f.w;
    }
    constexpr int kPer = (2 * HEAD + kDeltaThreads - 1) / kDeltaThreads;  // q|k values per thread
    float qk[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = min(tid + k * kDeltaThreads, 2 * HEAD - 1);
        qk[k] = p.qkv[i < HEAD ? kh * HEAD + i : p.state_size * p.key_heads + kh * HEAD + (i - HEAD)];
    }
    const float vrow = p.qkv[2 * p.state_size * p.key_heads + h * HEAD + row];
    float beta = 0.0f, decay = 0.0f;
    if (tid == 0) {
        // fortai_qwen35_cpu.f90:890-894
        beta = sigmoid_ref(p.beta[h]);
        decay = exp_rounded(p.ssm_a[h] * softplus_ref(p.alpha[h] + p.ssm_dt[h]));
        hs[0] = beta;
        hs[1] = decay;
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = tid + k * kDeltaThreads;
        if (i < HEAD) qs[i] = qk[k];
        else if (i < 2 * HEAD) ks[i - HEAD] = qk[k];
    }
    __syncthreads();
    // L2 norms of q (wave 0) and k (wave 1), fortai_qwen35_cpu.f90:1455-1471
    {
        const float *v = (tid < 64) ? qs : ks;
        double ss = 0.0;
        for (int i = tid & 63; i < HEAD; i += 64) ss += static_cast<double>(v[i]) * static_cast<double>(v[i]);
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
    }
    __syncthreads();
    const float qinv = 1.0f / fmaxf(sqrtf(static_cast<float>(red[0])), p.eps);
    const float kinv = 1.0f / fmaxf(sqrtf(static_cast<float>(red[1])), p.eps);
    beta = hs[0];
    decay = hs[1];
    // delta rule (fortai_q8_dot.c:363-396), the normalized q and k read from LDS
    float kd = 0.0f;
#pragma unroll
    for (int i = 0; i < kCols; ++i) {
        const float d = s[i] * decay;
        s[i] = d;
        kd = __builtin_fmaf(d, ks[8 * i + l] * kinv, kd);
    }
    kd = row_hsum8(kd);
    const float delta = (vrow - kd) * beta;
    float qd = 0.0f;
#pragma unroll
    for (int i = 0; i < kCols; ++i) {
        const float u = __builtin_fmaf(delta, ks[8 * i + l] * kinv, s[i]);
        s[i] = u;
        qd = __builtin_fmaf(u, qs[8 * i + l] * qinv, qd);
    }
    qd = row_hsum8(qd);
#pragma unroll
    for (int i = 0; i < kCols / 4; ++i) srow[i] = make_float4(s[4 * i], s[4 * i + 1], s[4 * i + 2], s[4 * i + 3]);
    if (l == 0) p.out[h * HEAD + row] = qd * (1.0f / sqrtf(static_cast<float>(HEAD)));
}

}  // namespace

hipError_t launch_gdn_step(const GdnParams &p, hipStream_t stream) {
    if (p.key_heads <= 0 || p.value_heads % p.key_heads || p.kernel < 2 || p.kernel > kMaxKernel ||
        p.state_size != p.head)
        return hipErrorInvalidValue;
    const int ratio = p.value_heads / p.key_heads;
    const int rows = ratio * p.head;
    if (2 * p.head > kThreads || rows > 4 * kThreads) return hipErrorInvalidValue;
    const size_t lds = (2 * static_cast<size_t>(p.head) + 2 * rows + 2 * ratio + 4) * sizeof(float) + 2 * sizeof(double);
    switch (p.head) {
    case 64: hipLaunchKernelGGL(gdn_group_kernel<64>, dim3(p.key_heads), dim3(kThreads), lds, stream, p); break;
    case 128: hipLaunchKernelGGL(gdn_group_kernel<128>, dim3(p.key_heads), dim3(kThreads), lds, stream, p); break;
    case 256: hipLaunchKernelGGL(gdn_group_kernel<256>, dim3(p.key_heads), dim3(kThreads), lds, stream, p); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gdn_delta(const GdnParams &p, hipStream_t stream) {
    if (p.key_heads <= 0 || p.value_heads % p.key_heads || p.state_size != p.head || !p.out) return hipErrorInvalidValue;
    const dim3 grid(p.value_heads * (p.head / kDeltaRows));
    switch (p.head) {
    case 64: hipLaunchKernelGGL(gdn_delta_kernel<64>, grid, dim3(kDeltaThreads), 0, stream, p); break;
    case 128: hipLaunchKernelGGL(gdn_delta_kernel<128>, grid, dim3(kDeltaThreads), 0, stream, p); break;
    case 256: hipLaunchKernelGGL(gdn_delta_kernel<256>, grid, dim3(kDeltaThreads), 0, stream, p); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace fortai_hip
