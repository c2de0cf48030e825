// Gated GQA decode attention for gfx950 (per-op path): per-head RMSNorm of q
// and k, RoPE, the fp16 KV append, and the reference's two-pass softmax with
// its summation orders kept (attention_exact.h), so the output is
// bit-identical to the CPU path (fortai_qwen35_cpu.f90:990-1033).
//
// Two kernels: scores (one workgroup per kv head x 64 positions; the one
// that holds the new position also appends it) and output (one workgroup per
// head x 8 value dims: softmax weights, the P.V chains and the sigmoid gate).
#include "attention_exact.h"
#include "fortai_hip_internal.h"
#include "fortai_hip_kernels.h"

namespace fortai_hip {

namespace {

namespace ea = exact_attention;

constexpr int kMaxGroup = 4;
constexpr int kMaxHead = 256;
constexpr int kLoads = ea::kPosBlock * (kMaxHead / 8) / ea::kThreads;
constexpr int kQLoads = kMaxGroup * kMaxHead / ea::kThreads;

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(ea::kThreads) void attention_scores_kernel(const AttentionParams p) {
    __shared__ __align__(16) float qh[kMaxGroup * kMaxHead];
    __shared__ __align__(16) float kn[kMaxHead];
    __shared__ __align__(16) float vn[kMaxHead];
    __shared__ __align__(16) float qw[kMaxHead];
    __shared__ __align__(16) float kw[kMaxHead];
    __shared__ __align__(16) float2 rs[kMaxHead / 2];
    __shared__ __align__(16) uint16_t ktile[ea::kPosBlock][kMaxHead + 8];
    __shared__ int overflow;
    const int tid = static_cast<int>(threadIdx.x), wave = tid >> 6, lane = tid & 63;
    FORTAI_ATT_MARK(8);
    const int pos = *p.position;
    if (pos < 0 || pos >= p.max_context) return;  // never index past the cache
    const int positions = pos + 1, nblk_max = (p.max_context + ea::kPosBlock - 1) / ea::kPosBlock;
    const int kvh = static_cast<int>(blockIdx.x) / nblk_max, b = static_cast<int>(blockIdx.x) % nblk_max;
    const int p0 = b * ea::kPosBlock;
    if (p0 >= positions) return;
    const int n = min(ea::kPosBlock, positions - p0);
    const bool owns_new = pos >= p0 && pos < p0 + n;
    const int group = p.heads / p.kv_heads, HD = p.head, VD = p.value, NKV = p.kv_heads;
    const int half = p.rope_dim / 2, segs = HD / 8;

    v4u kr[kLoads];  // key rows first: the only HBM stream of this kernel
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int li = tid + i * ea::kThreads;
        const int j = min(li / segs, n - 1), sg = li % segs;  // rows past n re-read row n-1 (in bounds)
        kr[i] = reinterpret_cast<const v4u *>(p.kcache + (static_cast<size_t>(p0 + j) * NKV + kvh) * HD)[sg];
    }
    // every other input in the same round trip (indices clamped in bounds),
    // then the LDS stores
    float qv[kQLoads];
#pragma unroll
    for (int i = 0; i < kQLoads; ++i) {
        const int e = min(tid + i * ea::kThreads, group * HD - 1);
        qv[i] = p.q[static_cast<size_t>(kvh * group + e / HD) * 2 * HD + e % HD];
    }
    const int th = min(tid, HD - 1), tv = min(tid, VD - 1);
    const float qwv = p.q_norm[th], kwv = p.k_norm[th];
    const float knv = p.k[static_cast<size_t>(kvh) * HD + th];
    const float vnv = p.v[static_cast<size_t>(kvh) * VD + tv];
    const float2 rsv = half > 0 ? p.rope[static_cast<size_t>(pos) * half + min(tid, half - 1)] : make_float2(0.0f, 0.0f);
    const int flag = p.cache_flags[kvh];
#pragma unroll
    for (int i = 0; i < kQLoads; ++i)
        if (tid + i * ea::kThreads < group * HD) qh[tid + i * ea::kThreads] = qv[i];
    if (tid < HD) {
        qw[tid] = qwv;
        kw[tid] = kwv;
        kn[tid] = knv;
    }
    if (tid < VD) vn[tid] = vnv;
    if (tid < half) rs[tid] = rsv;
    if (tid == 0) overflow = 0;
    FORTAI_ATT_MARK(9);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int li = tid + i * ea::kThreads;
        const int j = li / segs, sg = li % segs;
        if (j < n) *reinterpret_cast<v4u *>(&ktile[j][sg * 8]) = kr[i];
    }
    __syncthreads();
    for (int sl = wave; sl < group + (owns_new ? 1 : 0); sl += ea::kThreads / 64) {
        if (sl < group) ea::norm_rope(qh + sl * HD, HD, qw, p.eps, rs, p.rope_dim, lane);
        else ea::norm_rope(kn, HD, kw, p.eps, rs, p.rope_dim, lane);
    }
    __syncthreads();
    FORTAI_ATT_MARK(10);
    if (owns_new) {
        // append at pos (fortai_qwen35_cpu.f90:1594-1601)
        if (tid < HD) {
            const uint16_t kb = float_to_half_kv(kn[tid]);
            p.kcache[(static_cast<size_t>(pos) * NKV + kvh) * HD + tid] = kb;
            ktile[pos - p0][tid] = kb;
            if ((kb & 0x7c00u) == 0x7c00u) overflow = 1;
        }
        if (tid < VD) {
            const uint16_t vb = float_to_half_kv(vn[tid]);
            p.vcache[(static_cast<size_t>(pos) * NKV + kvh) * VD + tid] = vb;
            if ((vb & 0x7c00u) == 0x7c00u) overflow = 1;
        }
        __syncthreads();
        if (tid == 0 && overflow) p.cache_flags[kvh] = 1;
    }
    const bool finite = flag == 0 && overflow == 0;
    const float sqrt_head = sqrtf(static_cast<float>(HD));
    const int gi = tid >> 6, j = tid & 63;
    if (gi < group && j < n) {
        const float sc = finite ? ea::score<true>(qh + gi * HD, &ktile[j][0], HD, sqrt_head)
                                : ea::score<false>(qh + gi * HD, &ktile[j][0], HD, sqrt_head);
        p.partial[static_cast<size_t>(kvh * group + gi) * p.max_context + p0 + j] = sc;
    }
    FORTAI_ATT_MARK(11);
}

__global__ __launch_bounds__(ea::kThreads) void attention_output_kernel(const AttentionParams p) {
    extern __shared__ __align__(16) float lds[];
    const int tid = static_cast<int>(threadIdx.x);
    FORTAI_ATT_MARK(0);
    const int pos = *p.position;
    if (pos < 0 || pos >= p.max_context) return;
    const int positions = pos + 1;
    const int group = p.heads / p.kv_heads, HD = p.head, VD = p.value, NKV = p.kv_heads;
    const int slices = VD / ea::kDims;
    const int h = static_cast<int>(blockIdx.x) / slices, d0 = (static_cast<int>(blockIdx.x) % slices) * ea::kDims;
    const int kvh = h / group;
    float *work = lds;
    const uint16_t *vbase = p.vcache + static_cast<size_t>(kvh) * VD + d0;
    const size_t vstride = static_cast<size_t>(NKV) * VD;
    ea::ValuePieces v;
    ea::value_prefetch(vbase, vstride, positions, v);
    const float gate = tid < ea::kDims ? p.q[static_cast<size_t>(h) * 2 * HD + HD + d0 + tid] : 0.0f;
    const int flag = p.cache_flags[kvh];
    const float *sc = p.partial + static_cast<size_t>(h) * p.max_context;  // read in place
    FORTAI_ATT_MARK(3);
    const float acc = flag == 0 ? ea::attend<true>(sc, positions, vbase, vstride, work, v)
                                : ea::attend<false>(sc, positions, vbase, vstride, work, v);
    if (tid < ea::kDims) p.out[static_cast<size_t>(h) * VD + d0 + tid] = acc * sigmoid_ref(gate);
    FORTAI_ATT_MARK(4);
}

size_t output_lds_bytes() { return ea::work_floats() * sizeof(float); }

}  // namespace

size_t attention_scores_floats(int heads, int max_context) { return static_cast<size_t>(heads) * max_context; }

hipError_t launch_attention(const AttentionParams &p, hipStream_t stream) {
    const int group = p.kv_heads > 0 ? p.heads / p.kv_heads : 0;
    if (group < 1 || group > kMaxGroup || p.heads % p.kv_heads || p.head > kMaxHead || p.head % 8 ||
        p.value % ea::kDims || p.value > p.head || p.rope_dim > p.head || p.rope_dim % 2 || !p.out || !p.partial)
        return hipErrorInvalidValue;
    const size_t lds = output_lds_bytes();  // independent of the context length
    const int nblk_max = (p.max_context + ea::kPosBlock - 1) / ea::kPosBlock;
    hipLaunchKernelGGL(attention_scores_kernel, dim3(p.kv_heads * nblk_max), dim3(ea::kThreads), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attention_output_kernel, dim3(p.heads * (p.value / ea::kDims)), dim3(ea::kThreads), lds, stream, p);
    return hipGetLastError();
}

}  // namespace fortai_hip
