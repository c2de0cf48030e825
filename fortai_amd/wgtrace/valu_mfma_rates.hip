// valu_mfma_rates.hip -- issue cost of the instructions the exact Q8_0
// kernels are made of, on one MI355X:
//   * a wave64 fp32 fma on the vector ALUs (independent chains, 8 waves per
//     SIMD), against the matrix-core shapes that can form 4-byte lane dots
//     (K = 4: 32x32x4 x2, 16x16x4 x4, 4x4x4 x16 blocks, fp16 and int8) and the
//     wide-K shapes (32x32x8/16 fp16, 32x32x32 int8);
//   * the fma rate per SIMD with 1, 2, 4 and 8 waves on it (one wave alone
//     issues a vector instruction only about every other slot);
//   * how far the two overlap when one wave stream issues both;
//   * whether the diagonal of v_mfma_f32_4x4x1f32 is a fused multiply-add
//     (lane l's own a * b + c lands in its output register l % 4) bit for bit
//     against v_fma_f32, on arbitrary bit patterns, cancellations, subnormal
//     and overflow ranges, and over a 4096-step accumulation chain.
// build: hipcc --offload-arch=gfx950 -O3 -ffp-contract=off \
//            -Xclang -target-feature -Xclang -packed-fp32-ops valu_mfma_rates.hip -o valu_mfma_rates
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("ERR %s line %d: %s\n", #x, __LINE__, hipGetErrorString(e_)); fflush(stdout); exit(1); } } while (0)

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f32v __attribute__((ext_vector_type(32)));
typedef int i4 __attribute__((ext_vector_type(4)));
typedef int i16v __attribute__((ext_vector_type(16)));
typedef int i32v __attribute__((ext_vector_type(32)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

// ------------------------------------------------------------ exactness
__global__ void diag_fma(const float *a, const float *b, const float *c, float *by_mfma, float *by_valu) {
    const int i = static_cast<int>(blockIdx.x) * 64 + static_cast<int>(threadIdx.x), l = threadIdx.x & 3;
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    acc[0] = l == 0 ? c[i] : 0.0f;
    acc[1] = l == 1 ? c[i] : 0.0f;
    acc[2] = l == 2 ? c[i] : 0.0f;
    acc[3] = l == 3 ? c[i] : 0.0f;
    const f4 d = __builtin_amdgcn_mfma_f32_4x4x1f32(a[i], b[i], acc, 0, 0, 0);
    by_mfma[i] = l == 0 ? d[0] : l == 1 ? d[1] : l == 2 ? d[2] : d[3];
    by_valu[i] = __builtin_fmaf(a[i], b[i], c[i]);
}

__global__ void diag_chain(const float *a, const float *b, int steps, float *by_mfma, float *by_valu) {
    const int t = threadIdx.x, l = t & 3;
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    float v = 0.0f;
    for (int k = 0; k < steps; ++k) {
        acc = __builtin_amdgcn_mfma_f32_4x4x1f32(a[k * 64 + t], b[k * 64 + t], acc, 0, 0, 0);
        v = __builtin_fmaf(a[k * 64 + t], b[k * 64 + t], v);
    }
    by_mfma[t] = l == 0 ? acc[0] : l == 1 ? acc[1] : l == 2 ? acc[2] : acc[3];
    by_valu[t] = v;
}

// ------------------------------------------------------------ rates
enum Shape { NONE, F16_32x32x4, I8_32x32x4, F16_16x16x4, I8_16x16x4, F16_4x4x4, I8_4x4x4, F16_32x32x8, F16_32x32x16,
             I8_32x32x32, F32_4x4x1 };

// NV fmas on 8 independent chains and NM matrix ops on 2 independent
// accumulators per step, 4 steps per iteration; nothing depends on the
// other unit's results.
template <int NV, int NM, Shape S>
__global__ __launch_bounds__(256) void rate_kernel(float s, int iters, float *sink) {
    float v[8];
    for (int j = 0; j < 8; ++j) v[j] = static_cast<float>(threadIdx.x) * 1e-3f + static_cast<float>(j);
    const float x = s + static_cast<float>(threadIdx.x), y = 0.5f * s;
    const h4 a4 = {(_Float16)x, (_Float16)y, (_Float16)1.0f, (_Float16)2.0f};
    const h8 a8 = {(_Float16)x, (_Float16)y, (_Float16)1.0f, (_Float16)2.0f, (_Float16)y, (_Float16)x, (_Float16)3.0f, (_Float16)1.0f};
    const i4 q4 = {static_cast<int>(threadIdx.x), 3, 5, 7};
    f32v m32[2] = {};
    f16v m16[2] = {};
    f4 m4[2] = {};
    i32v n32[2] = {};
    i16v n16[2] = {};
    i4 n4[2] = {};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
            for (int j = 0; j < NV; ++j) v[j & 7] = __builtin_fmaf(x, v[j & 7], y);
#pragma unroll
            for (int j = 0; j < NM; ++j) {
                const int u = j & 1;
                if constexpr (S == F16_32x32x4) m32[u] = __builtin_amdgcn_mfma_f32_32x32x4f16(a4, a4, m32[u], 0, 0, 0);
                if constexpr (S == I8_32x32x4) n32[u] = __builtin_amdgcn_mfma_i32_32x32x4i8(q4[0], q4[1], n32[u], 0, 0, 0);
                if constexpr (S == F16_16x16x4) m16[u] = __builtin_amdgcn_mfma_f32_16x16x4f16(a4, a4, m16[u], 0, 0, 0);
                if constexpr (S == I8_16x16x4) n16[u] = __builtin_amdgcn_mfma_i32_16x16x4i8(q4[0], q4[1], n16[u], 0, 0, 0);
                if constexpr (S == F16_4x4x4) m4[u] = __builtin_amdgcn_mfma_f32_4x4x4f16(a4, a4, m4[u], 0, 0, 0);
                if constexpr (S == I8_4x4x4) n4[u] = __builtin_amdgcn_mfma_i32_4x4x4i8(q4[0], q4[1], n4[u], 0, 0, 0);
                if constexpr (S == F16_32x32x8) m16[u] = __builtin_amdgcn_mfma_f32_32x32x8f16(a4, a4, m16[u], 0, 0, 0);
                if constexpr (S == F16_32x32x16) m16[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a8, a8, m16[u], 0, 0, 0);
                if constexpr (S == I8_32x32x32) n16[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(q4, q4, n16[u], 0, 0, 0);
                if constexpr (S == F32_4x4x1) m4[u] = __builtin_amdgcn_mfma_f32_4x4x1f32(x, y, m4[u], 0, 0, 0);
            }
        }
    }
    float acc = 0.0f;
    for (int j = 0; j < 8; ++j) acc += v[j];
    for (int u = 0; u < 2; ++u) {
        for (int j = 0; j < 32; ++j) acc += m32[u][j] + static_cast<float>(n32[u][j]);
        for (int j = 0; j < 16; ++j) acc += m16[u][j] + static_cast<float>(n16[u][j]);
        for (int j = 0; j < 4; ++j) acc += m4[u][j] + static_cast<float>(n4[u][j]);
    }
    sink[blockIdx.x * 256 + threadIdx.x] = acc;
}

template <int NV, int NM, Shape S>
void rate(const char *name, float *sink, int kBlocks = 2048) {  // 2048: 8 waves per SIMD on 256 CUs
    constexpr int kIters = 1000;
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    hipLaunchKernelGGL((rate_kernel<NV, NM, S>), dim3(kBlocks), dim3(256), 0, 0, 1.0f, kIters, sink);
    CK(hipEventRecord(e0));
    hipLaunchKernelGGL((rate_kernel<NV, NM, S>), dim3(kBlocks), dim3(256), 0, 0, 1.0f, kIters, sink);
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    float ms = 0.0f;
    CK(hipEventElapsedTime(&ms, e0, e1));
    const double per_simd = kBlocks * 4.0 / 1024.0 * kIters * 4;  // steps per SIMD
    printf("%-34s %d waves/SIMD %7.3f ms", name, kBlocks / 256, ms);
    if (NV) printf("  %.3f ns per fma", ms * 1e6 / (per_simd * NV));
    if (NM && !NV) printf("  %.2f ns per matrix op", ms * 1e6 / (per_simd * NM));
    printf("\n");
    fflush(stdout);
    CK(hipEventDestroy(e0));
    CK(hipEventDestroy(e1));
}

static uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

int main() {
    // exactness of the 4x4x1 diagonal
    const int n = 64 * 20000;
    std::mt19937 g(7);
    std::uniform_int_distribution<uint32_t> U;
    std::uniform_real_distribution<float> R(-1.0f, 1.0f);
    std::vector<float> a(n), b(n), c(n);
    for (int i = 0; i < n; ++i) {
        switch (i % 8) {
        case 0: a[i] = from_bits(U(g)); b[i] = from_bits(U(g)); c[i] = from_bits(U(g)); break;
        case 1: a[i] = R(g); b[i] = R(g); c[i] = -(a[i] * b[i]) * (1.0f + R(g) * 1e-6f); break;
        case 2: a[i] = R(g) * 1e-20f; b[i] = R(g) * 1e-20f; c[i] = R(g) * 1e-38f; break;
        case 3: a[i] = static_cast<float>(static_cast<int>(U(g) % 1024) - 512); b[i] = R(g) * 1e-3f; c[i] = R(g) * 100.0f; break;
        case 4: a[i] = R(g) * 1e19f; b[i] = R(g) * 1e19f; c[i] = R(g) * 3e38f; break;
        case 5: a[i] = R(g); b[i] = R(g); c[i] = -static_cast<float>(static_cast<double>(a[i]) * b[i]); break;
        case 6: a[i] = 1.0f + R(g) * 1e-7f; b[i] = 1.0f + R(g) * 1e-7f; c[i] = -1.0f; break;
        default: a[i] = R(g); b[i] = R(g); c[i] = R(g); break;
        }
    }
    float *da, *db, *dc, *dm, *dv;
    CK(hipMalloc(&da, n * 4));
    CK(hipMalloc(&db, n * 4));
    CK(hipMalloc(&dc, n * 4));
    CK(hipMalloc(&dm, n * 4));
    CK(hipMalloc(&dv, n * 4));
    CK(hipMemcpy(da, a.data(), n * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(db, b.data(), n * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(dc, c.data(), n * 4, hipMemcpyHostToDevice));
    hipLaunchKernelGGL(diag_fma, dim3(n / 64), dim3(64), 0, 0, da, db, dc, dm, dv);
    CK(hipDeviceSynchronize());
    std::vector<float> om(n), ov(n);
    CK(hipMemcpy(om.data(), dm, n * 4, hipMemcpyDeviceToHost));
    CK(hipMemcpy(ov.data(), dv, n * 4, hipMemcpyDeviceToHost));
    int differ = 0, nan_both = 0;
    for (int i = 0; i < n; ++i) {
        if (om[i] != om[i] && ov[i] != ov[i]) { ++nan_both; continue; }
        if (bits_of(om[i]) != bits_of(ov[i])) ++differ;
    }
    printf("4x4x1 diagonal vs v_fma_f32: %d of %d differ (%d NaN in both)\n", differ, n, nan_both);
    const int steps = 4096;
    std::vector<float> ca(steps * 64), cb(steps * 64);
    for (int i = 0; i < steps * 64; ++i) {
        ca[i] = static_cast<float>(static_cast<int>(U(g) % 1024) - 512);
        cb[i] = R(g) * 1e-3f;
    }
    float *dca, *dcb;
    CK(hipMalloc(&dca, steps * 256));
    CK(hipMalloc(&dcb, steps * 256));
    CK(hipMemcpy(dca, ca.data(), steps * 256, hipMemcpyHostToDevice));
    CK(hipMemcpy(dcb, cb.data(), steps * 256, hipMemcpyHostToDevice));
    hipLaunchKernelGGL(diag_chain, dim3(1), dim3(64), 0, 0, dca, dcb, steps, dm, dv);
    CK(hipDeviceSynchronize());
    CK(hipMemcpy(om.data(), dm, 256, hipMemcpyDeviceToHost));
    CK(hipMemcpy(ov.data(), dv, 256, hipMemcpyDeviceToHost));
    int chain_differ = 0;
    for (int t = 0; t < 64; ++t) chain_differ += bits_of(om[t]) != bits_of(ov[t]);
    printf("%d-step accumulation, 64 lanes: %d differ\n", steps, chain_differ);

    float *sink;
    CK(hipMalloc(&sink, 2048 * 256 * 4));
    for (int blocks : {256, 512, 1024, 2048}) rate<16, 0, NONE>("fma x16", sink, blocks);
    rate<8, 0, NONE>("fma x8", sink);
    rate<0, 2, F16_32x32x4>("32x32x4 f16 (2 blocks)", sink);
    rate<0, 2, I8_32x32x4>("32x32x4 i8 (2 blocks)", sink);
    rate<0, 2, F16_16x16x4>("16x16x4 f16 (4 blocks)", sink);
    rate<0, 2, I8_16x16x4>("16x16x4 i8 (4 blocks)", sink);
    rate<0, 8, F16_4x4x4>("4x4x4 f16 (16 blocks)", sink);
    rate<0, 8, I8_4x4x4>("4x4x4 i8 (16 blocks)", sink);
    rate<0, 2, F16_32x32x8>("32x32x8 f16", sink);
    rate<0, 2, F16_32x32x16>("32x32x16 f16", sink);
    rate<0, 2, I8_32x32x32>("32x32x32 i8", sink);
    rate<0, 8, F32_4x4x1>("4x4x1 f32 (16 blocks)", sink);
    rate<8, 1, F16_32x32x4>("fma x8 + 32x32x4 f16 x1", sink);
    rate<16, 1, F16_32x32x4>("fma x16 + 32x32x4 f16 x1", sink);
    rate<32, 1, F16_32x32x4>("fma x32 + 32x32x4 f16 x1", sink);
    rate<16, 1, F16_32x32x16>("fma x16 + 32x32x16 f16 x1", sink);
    rate<8, 2, F32_4x4x1>("fma x8 + 4x4x1 f32 x2", sink);
    printf("done\n");
    return 0;
}
