// Gated DeltaNet decode step for gfx950: causal conv1d + SiLU + L2 norm of q
// and k + decay/beta + the delta-rule state update, fused in one launch.
//
// Reference: the recurrent branch of fortai_qwen35_cpu.f90:856-906 and the
// AVX2 state step fortai_q8_dot.c:356-398.  A state row r of value head h only
// depends on S[h][r][:], k, q, v[r], beta and the decay, so one wave handles 8
// rows x 8 lanes and lane l owns columns l, l+8, l+16, ... -- exactly the
// fp32 lane of the reference's 8-wide vector loop -- with the same fma chains
// and the same horizontal-sum tree.  The per-row results are therefore
// bit-identical to the CPU step.
//
// Layouts (backend-owned, persistent):
//  * state[((h * head + r) * 8 + l) * (head / 8) + i] = S[h][r][8 i + l]
//    (a lane's 16 floats are contiguous: four 16-byte loads and stores);
//  * conv_ring[slot][conv_size] holds x_t in slot t % kernel, so the step
//    reads slots t-(kernel-1) .. t-1 and writes slot t, which no workgroup of
//    the same step reads (the reference shifts a [kernel-1][C] window,
//    fortai_qwen35_cpu.f90:870-879; the ring has the same contents without
//    moving data);
//  * step: the layer's own device step counter t, advanced by the last
//    workgroup, so graph replays need no host update.
#include "fortai_hip_internal.h"
#include "fortai_hip_kernels.h"

namespace fortai_hip {

namespace {

constexpr int kMaxHead = 256;

__device__ __forceinline__ float conv_channel(const GdnParams &p, int ch, int t) {
    // fortai_qwen35_cpu.f90:856-867: slots 1..K-1 oldest first, then the
    // current value, accumulated left to right.
    const int K = p.kernel;
    float acc = 0.0f;
    for (int slot = 0; slot < K - 1; ++slot) {
        int ring = (t - (K - 1) + slot) % K;
        if (ring < 0) ring += K;
        acc = acc + p.conv_w[static_cast<size_t>(ch) * K + slot] * p.conv_ring[static_cast<size_t>(ring) * p.conv_size + ch];
    }
    acc = acc + p.conv_w[static_cast<size_t>(ch) * K + K - 1] * p.qkv[ch];
    return silu_poly(acc);
}

template <int HEAD>
__global__ __launch_bounds__(64) void gdn_step_kernel(const GdnParams p) {
    constexpr int kCols = HEAD / 8;  // columns per lane
    __shared__ float qs[HEAD];
    __shared__ float ks[HEAD];
    const int lane = static_cast<int>(threadIdx.x);
    const int chunks = HEAD / kRowsPerWave;
    const int h = static_cast<int>(blockIdx.x) / chunks;
    const int chunk = static_cast<int>(blockIdx.x) % chunks;
    const int ratio = p.value_heads / p.key_heads;
    const int kh = h / ratio;
    const int t = *p.step;
    const int q_base = kh * HEAD;
    const int k_base = p.state_size * p.key_heads + kh * HEAD;
    const int v_base = 2 * p.state_size * p.key_heads + h * HEAD;

    // conv + SiLU of this key head's q and k, then their L2 norms
    double sq = 0.0, sk = 0.0;
    for (int i = lane; i < HEAD; i += 64) {
        const float qv = conv_channel(p, q_base + i, t);
        const float kv = conv_channel(p, k_base + i, t);
        qs[i] = qv;
        ks[i] = kv;
        sq += static_cast<double>(qv) * static_cast<double>(qv);
        sk += static_cast<double>(kv) * static_cast<double>(kv);
    }
    sq = wave_sum(sq);
    sk = wave_sum(sk);
    // fortai_qwen35_cpu.f90:1455-1471
    const float nq = sqrtf(static_cast<float>(sq));
    const float nk = sqrtf(static_cast<float>(sk));
    const float iq = 1.0f / (nq > p.eps ? nq : p.eps);
    const float ik = 1.0f / (nk > p.eps ? nk : p.eps);
    __syncthreads();
    for (int i = lane; i < HEAD; i += 64) {
        qs[i] = qs[i] * iq;
        ks[i] = ks[i] * ik;
    }

    const int r = lane >> 3, l = lane & 7;
    const int row = chunk * kRowsPerWave + r;
    const float v = conv_channel(p, v_base + row, t);

    // per-head scalars (fortai_qwen35_cpu.f90:890-894)
    const float beta = sigmoid_ref(p.beta[h]);
    const float decay = p.ssm_a[h] * softplus_ref(p.alpha[h] + p.ssm_dt[h]);
    const float decay_factor = exp_rounded(decay);
    const float output_scale = 1.0f / sqrtf(static_cast<float>(HEAD));
    __syncthreads();

    float4 *srow = reinterpret_cast<float4 *>(p.state + ((static_cast<size_t>(h) * HEAD + row) * 8 + l) * kCols);
    float s[kCols];
#pragma unroll
    for (int i = 0; i < kCols / 4; ++i) {
        const float4 f = srow[i];
        s[4 * i] = f.x; s[4 * i + 1] = f.y; s[4 * i + 2] = f.z; s[4 * i + 3] = f.w;
    }
    float kd = 0.0f;
#pragma unroll
    for (int i = 0; i < kCols; ++i) {
        const float d = s[i] * decay_factor;
        s[i] = d;
        kd = __builtin_fmaf(d, ks[8 * i + l], kd);
    }
    kd = row_hsum8(kd);
    const float delta = (v - kd) * beta;
    float qd = 0.0f;
#pragma unroll
    for (int i = 0; i < kCols; ++i) {
        const float u = __builtin_fmaf(delta, ks[8 * i + l], s[i]);
        s[i] = u;
        qd = __builtin_fmaf(u, qs[8 * i + l], qd);
    }
    qd = row_hsum8(qd);
#pragma unroll
    for (int i = 0; i < kCols / 4; ++i) srow[i] = make_float4(s[4 * i], s[4 * i + 1], s[4 * i + 2], s[4 * i + 3]);
    if (l == 0) p.out[h * HEAD + row] = qd * output_scale;

    // append x_t to the conv ring: v channels of these rows; q/k channels of
    // the key head by the first row chunk of its first value head
    const int slot = t % p.kernel;
    float *ring = p.conv_ring + static_cast<size_t>(slot) * p.conv_size;
    if (l == 0) ring[v_base + row] = p.qkv[v_base + row];
    if (chunk == 0 && h % ratio == 0)
        for (int i = lane; i < HEAD; i += 64) {
            ring[q_base + i] = p.qkv[q_base + i];
            ring[k_base + i] = p.qkv[k_base + i];
        }

    // the last workgroup advances the layer's step counter
    __threadfence();
    if (lane == 0) {
        const unsigned prev = atomicAdd(p.done, 1u);
        if (prev == gridDim.x - 1) {
            *p.step = t + 1;
            __hip_atomic_store(p.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

}  // namespace

hipError_t launch_gdn_step(const GdnParams &p, hipStream_t stream) {
    if (p.key_heads <= 0 || p.value_heads % p.key_heads || p.kernel < 2 || p.state_size != p.head)
        return hipErrorInvalidValue;
    const int grid = p.value_heads * (p.head / kRowsPerWave);
    switch (p.head) {
    case 64: hipLaunchKernelGGL(gdn_step_kernel<64>, dim3(grid), dim3(64), 0, stream, p); break;
    case 128: hipLaunchKernelGGL(gdn_step_kernel<128>, dim3(grid), dim3(64), 0, stream, p); break;
    case 256: hipLaunchKernelGGL(gdn_step_kernel<256>, dim3(grid), dim3(64), 0, stream, p); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace fortai_hip
