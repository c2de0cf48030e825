// trace.h -- per-workgroup timing build of libfortai_hip (profiling only).
//
// Force-included (-include) before the kernel sources: it defines the
// FORTAI_TRACE_SCOPE hook that the decode kernels place as their first
// statement (empty in the library) and the matvec's FORTAI_MV_MARK phase
// marks.  Thread 0 of every workgroup records, with the 100 MHz
// s_memrealtime clock (one clock for the whole device): its start, the end,
// the kernel kind, the XCD it ran on and up to four phase marks.  Records go
// to per-(kind, workgroup) rings, so no two workgroups of a launch contend for
// one counter.  Each translation unit has its own buffer, read by
// fortai_wgtrace_<unit>().
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define FORTAI_WGTRACE_DEPTH 512                       // launches per (kind, workgroup) slot
#define FORTAI_WGTRACE_SLOTS (8 * 1024)                // 8 kinds x 1024 workgroup indices
struct WgTraceRec {
    uint64_t t0, t1;   // start, end (10 ns ticks)
    uint32_t kind;     // kernel kind | XCD << 8
    uint32_t block;    // blockIdx.x | blockIdx.y << 20
    uint32_t mark[4];  // low 32 bits of the phase marks
};
static __device__ WgTraceRec g_wgtrace[FORTAI_WGTRACE_SLOTS * FORTAI_WGTRACE_DEPTH];
static __device__ unsigned int g_wgtrace_count[FORTAI_WGTRACE_SLOTS];
static __device__ __shared__ uint32_t g_wgtrace_mark[4];

#define FORTAI_MV_MARK(i) \
    do { if (threadIdx.x == 0 && (i) < 4) g_wgtrace_mark[(i) & 3] = (uint32_t)__builtin_amdgcn_s_memrealtime(); } while (0)

struct WgTraceScope {
    uint64_t t0;
    uint32_t kind;
    __device__ explicit WgTraceScope(uint32_t k) : kind(k) { t0 = __builtin_amdgcn_s_memrealtime(); }
    __device__ ~WgTraceScope() {
        if (threadIdx.x != 0) return;
        const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
        const unsigned slot = (kind & 7) * 1024 + (blockIdx.x & 1023);
        const unsigned k = atomicAdd(&g_wgtrace_count[slot], 1u) % FORTAI_WGTRACE_DEPTH;
        const uint32_t xcc = __builtin_amdgcn_s_getreg((20) | (0 << 6) | (3 << 11));  // HW_REG_XCC_ID
        g_wgtrace[slot * FORTAI_WGTRACE_DEPTH + k] = WgTraceRec{t0, t1, kind | (xcc << 8),
            blockIdx.x | (blockIdx.y << 20),
            {g_wgtrace_mark[0], g_wgtrace_mark[1], g_wgtrace_mark[2], g_wgtrace_mark[3]}};
    }
};
#define FORTAI_TRACE_SCOPE(id) WgTraceScope fortai_wgtrace_scope_(id)

// host side: reset the ring counters, or read one unit's records (records of
// earlier launches stay until overwritten; the reader keeps the latest ones)
#define FORTAI_WGTRACE_EXPORT_(n)                                                                            \
    extern "C" int fortai_wgtrace_##n(void *host, int reset) {                                              \
        if (reset) {                                                                                        \
            static unsigned zero[FORTAI_WGTRACE_SLOTS];                                                     \
            return hipMemcpyToSymbol(HIP_SYMBOL(g_wgtrace_count), zero, sizeof(zero)) == hipSuccess ? 0 : 1; \
        }                                                                                                   \
        return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_wgtrace), sizeof(g_wgtrace)) == hipSuccess ? 0 : 1;  \
    }
#define FORTAI_WGTRACE_EXPORT(n) FORTAI_WGTRACE_EXPORT_(n)
