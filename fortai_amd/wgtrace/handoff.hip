// handoff.hip -- what a persistent (one-launch) decode would pay per phase:
// chained phases in one cooperative launch, P = 128 producer workgroups each
// publishing 8 words, every consumer (or only those of the producer's XCD)
// waiting for them: 64-bit tagged words at agent scope, or data plus a flag
// behind a release fence; idle and with the other waves streaming HBM.
// build: hipcc --offload-arch=gfx950 -O3 handoff.hip -o handoff
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <cstdint>
#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("ERR %s line %d: %s\n", #x, __LINE__, hipGetErrorString(e)); fflush(stdout); exit(1);} } while (0)

typedef unsigned int u4 __attribute__((ext_vector_type(4)));
constexpr int kSpin = 1 << 16;
constexpr int P = 128;      // producers (first P workgroups), 8 words each
constexpr int WORDS = P * 8;

__device__ __forceinline__ uint64_t ld_agent(const uint64_t *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_agent(uint64_t *p, uint64_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// MODE 0: all->all tagged words, agent scope.  1: XCD-local tagged words, agent scope.
// MODE 3: all->all flags + data (fence).
template <int MODE, bool BG>
__global__ __launch_bounds__(256) void phases(uint64_t *buf, uint32_t *flags, const uint4 *bg, size_t bg_n, int nphase, int *err, float *sink) {
    const int b = blockIdx.x, t = threadIdx.x, G = gridDim.x;
    __shared__ int done;
    if (t == 0) done = 0;
    __syncthreads();
    if (BG && t >= 64) {
        // background stream: waves 1-3 read bg until done
        const size_t per = bg_n / G;
        const uint4 *p = bg + (size_t)b * per;
        uint32_t acc = 0; size_t i = t - 64;
        while (true) {
            for (int k = 0; k < 16; ++k) { u4 v = __builtin_nontemporal_load((const u4 *)(p + i)); acc ^= v.x + v.w; i += 192; if (i >= per) i = t - 64; }
            if (__hip_atomic_load(&done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) break;
        }
        if (acc == 0x1234567u) sink[0] = 1.f;
        return;
    }
    if (t >= 64) return;
    int bad = 0, tmo = 0;
    for (int ph = 0; ph < nphase; ++ph) {
        uint64_t *d = buf + (size_t)(ph & 1) * WORDS;
        const uint64_t tag = (uint64_t)(ph + 1) << 32;
        // produce
        if (b < P && t < 8) {
            const uint64_t v = tag | (uint32_t)(b * 8 + t + ph);
            if (MODE == 3) d[b * 8 + t] = v;
            else st_agent(&d[b * 8 + t], v);
        }
        if (MODE == 3) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            if (b < P && t == 0) __hip_atomic_store(&flags[b], (uint32_t)(ph + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // consume
        if (MODE == 0 || MODE == 3) {
            if (MODE == 3) {
                for (int q = t; q < P; q += 64) {
                    int s = 0;
                    while (__hip_atomic_load(&flags[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (uint32_t)(ph + 1) && s < kSpin) ++s;
                    if (s >= kSpin) ++tmo;
                }
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            }
            if (MODE == 3) {
                for (int q = t; q < WORDS; q += 64) { uint64_t v = d[q]; if ((uint32_t)v != (uint32_t)(q + ph)) ++bad; }
            } else {
                uint64_t v[WORDS / 64]; int s = 0; bool ok;
                do {
#pragma unroll
                    for (int k = 0; k < WORDS / 64; ++k) v[k] = ld_agent(&d[t + 64 * k]);
                    ok = true;
#pragma unroll
                    for (int k = 0; k < WORDS / 64; ++k) ok &= (v[k] >> 32) == (uint64_t)(ph + 1);
                } while (!ok && ++s < kSpin);
                if (!ok) ++tmo;
#pragma unroll
                for (int k = 0; k < WORDS / 64; ++k) if ((uint32_t)v[k] != (uint32_t)(t + 64 * k + ph)) ++bad;
            }
        } else {
            // XCD-local: producers q with q % 8 == b % 8
            for (int i = t; i < (P / 8) * 8; i += 64) {
                const int q = ((i >> 3) * 8 + (b & 7)) * 8 + (i & 7);
                uint64_t v; int s = 0;
                do { v = ld_agent(&d[q]); } while ((v >> 32) != (uint64_t)(ph + 1) && ++s < kSpin);
                if (s >= kSpin) ++tmo;
                if ((uint32_t)v != (uint32_t)(q + ph)) ++bad;
            }
        }
        if (tmo) break;
        __builtin_amdgcn_wave_barrier();
    }
    if (t == 0) __hip_atomic_store(&done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (bad) atomicAdd(&err[0], bad);
    if (tmo) atomicAdd(&err[1], tmo);
}

template <int MODE, bool BG>
void run(const char *name, uint64_t *buf, uint32_t *flags, const uint4 *bg, size_t bg_n, int *err, float *sink, hipStream_t s, hipEvent_t e0, hipEvent_t e1, int G) {
    CK(hipMemset(buf, 0, 2 * WORDS * 8)); CK(hipMemset(flags, 0, 4096)); CK(hipMemset(err, 0, 8));
    CK(hipDeviceSynchronize());
    int nphase = 2000;
    void *args[] = {&buf, &flags, (void *)&bg, &bg_n, &nphase, &err, &sink};
    CK(hipEventRecord(e0, s));
    CK(hipLaunchCooperativeKernel((void *)phases<MODE, BG>, dim3(G), dim3(256), args, 0, s));
    CK(hipEventRecord(e1, s)); CK(hipEventSynchronize(e1));
    float ms; CK(hipEventElapsedTime(&ms, e0, e1));
    int h[2]; CK(hipMemcpy(h, err, 8, hipMemcpyDeviceToHost));
    printf("%-44s bg=%d: %.3f us per phase, bad %d, timeouts %d\n", name, (int)BG, ms * 1000 / nphase, h[0], h[1]);
    fflush(stdout);
    if (h[1]) { printf("timeouts: stop\n"); exit(2); }
}

int main() {
    hipDeviceProp_t prop; CK(hipGetDeviceProperties(&prop, 0));
    const int G = prop.multiProcessorCount;
    printf("device %s CUs %d\n", prop.gcnArchName, G); fflush(stdout);
    hipStream_t s; CK(hipStreamCreate(&s));
    hipEvent_t e0, e1; CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
    uint64_t *buf; CK(hipMalloc(&buf, 2 * WORDS * 8));
    uint32_t *flags; CK(hipMalloc(&flags, 4096));
    const size_t bg_bytes = (size_t)2 << 30; uint4 *bg; CK(hipMalloc(&bg, bg_bytes)); CK(hipMemset(bg, 1, bg_bytes));
    const size_t bg_n = bg_bytes / 16;
    int *err; CK(hipMalloc(&err, 8)); float *sink; CK(hipMalloc(&sink, 4));
    run<0, false>("all->all tagged, agent (batched loads)", buf, flags, bg, bg_n, err, sink, s, e0, e1, G);
    run<3, false>("all->all flags+fence", buf, flags, bg, bg_n, err, sink, s, e0, e1, G);
    run<1, false>("xcd-local tagged, agent", buf, flags, bg, bg_n, err, sink, s, e0, e1, G);
    run<0, true>("all->all tagged, agent (batched loads)", buf, flags, bg, bg_n, err, sink, s, e0, e1, G);
    run<3, true>("all->all flags+fence", buf, flags, bg, bg_n, err, sink, s, e0, e1, G);
    run<1, true>("xcd-local tagged, agent", buf, flags, bg, bg_n, err, sink, s, e0, e1, G);
    printf("probe done\n");
    return 0;
}
