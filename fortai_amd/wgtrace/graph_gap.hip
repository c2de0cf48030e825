// graph_gap.hip -- the cost of one kernel boundary in a captured HIP graph: 200
// empty kernels chained, replayed 20 times, per kernel, for 8- and 600-byte
// arguments, 0-44 KB dynamic LDS and 128 / 256 workgroups.
// build: hipcc --offload-arch=gfx950 -O3 graph_gap.hip -o graph_gap
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("ERR %s %d %s\n", #x, __LINE__, hipGetErrorString(e)); exit(1);} } while (0)
template <int N> struct Args { int v[N]; };
template <int N>
__global__ void k_args(Args<N> a, float *x) {
    extern __shared__ float s[];
    if (threadIdx.x == 0 && a.v[N - 1] == 12345) { s[0] = 1; x[blockIdx.x] = s[0]; }
}
__global__ void k_ptr(const int *a, float *x) { if (threadIdx.x == 0 && a[0] == 12345) x[blockIdx.x] = 1; }
template <typename F>
float chain(F launch, hipStream_t s) {
    hipGraph_t g; hipGraphExec_t ge;
    CK(hipStreamBeginCapture(s, hipStreamCaptureModeGlobal));
    for (int i = 0; i < 200; ++i) launch();
    CK(hipStreamEndCapture(s, &g)); CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    CK(hipGraphLaunch(ge, s)); CK(hipStreamSynchronize(s));
    hipEvent_t e0, e1; CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
    CK(hipEventRecord(e0, s));
    for (int r = 0; r < 20; ++r) CK(hipGraphLaunch(ge, s));
    CK(hipEventRecord(e1, s)); CK(hipEventSynchronize(e1));
    float ms; CK(hipEventElapsedTime(&ms, e0, e1));
    return ms * 1000 / 4000;
}
int main() {
    hipStream_t s; CK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    float *x; CK(hipMalloc(&x, 1 << 20)); int *p; CK(hipMalloc(&p, 4096)); CK(hipMemset(p, 0, 4096));
    for (int grid : {128, 256}) for (int lds : {0, 16384, 45056}) {
        Args<2> a2{}; Args<150> a150{};
        printf("grid %d lds %5d: args 8B %.3f us  args 600B %.3f us  ptr %.3f us\n", grid, lds,
            chain([&] { hipLaunchKernelGGL(k_args<2>, dim3(grid), dim3(256), lds, s, a2, x); }, s),
            chain([&] { hipLaunchKernelGGL(k_args<150>, dim3(grid), dim3(256), lds, s, a150, x); }, s),
            chain([&] { hipLaunchKernelGGL(k_ptr, dim3(grid), dim3(256), 0, s, p, x); }, s));
        fflush(stdout);
    }
    return 0;
}
