// Gated DeltaNet decode step for gfx950 (the recurrent branch of
// fortai_qwen35_cpu.f90:856-916, the AVX2 state step fortai_q8_dot.c:356-398),
// in three parts that each run where they are cheapest:
//  * conv1d + SiLU of each channel and the window shift: one thread per
//    channel (conv_silu_kernel, or the qkv projection's epilogue);
//  * the delta rule: 16 state rows per workgroup (gdn_delta_kernel).  A state
//    row r of value head h only depends on S[h][r][:], q, k, v[r], beta and
//    the decay, so 8 lanes own one row and lane l owns columns l, l+8, ... --
//    exactly the fp32 lane of the reference's 8-wide vector loop -- with the
//    same fma chains and the same horizontal-sum tree: the state and raw
//    output are bit-identical to the CPU step;
//  * the gated RMSNorm: the ssm_out matvec's prologue (q8_kernels.hip).
//
// Layouts (backend-owned, persistent):
//  * state[((h * head + r) * 8 + l) * (head / 8) + i] = S[h][r][8 i + l]
//    (a lane's head/8 floats are contiguous: 16-byte loads and stores);
//  * conv_state[slot][conv_size], oldest slot first (the reference layout).
#include "fortai_hip_internal.h"
#include "fortai_hip_kernels.h"

namespace fortai_hip {

namespace {

// Causal conv1d + SiLU over every channel, one thread per channel, which then
// shifts that channel's window (fortai_qwen35_cpu.f90:856-879).  (In the
// decoder the same step runs in the qkv projection's epilogue.)
__global__ __launch_bounds__(256) void conv_silu_kernel(const float *__restrict__ x, const float *__restrict__ conv_w,
    float *__restrict__ conv_state, float *__restrict__ out, int channels, int K) {
    const int c = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
    if (c >= channels) return;
    float win[kConvMax - 1], taps[kConvMax];
#pragma unroll
    for (int t = 0; t < kConvMax; ++t) {
        if (t < K - 1) win[t] = conv_state[static_cast<size_t>(t) * channels + c];
        if (t < K) taps[t] = conv_w[static_cast<size_t>(c) * K + t];
    }
    const float v = x[c];
    out[c] = conv_silu(win, taps, K, v);
#pragma unroll
    for (int t = 0; t + 1 < kConvMax - 1; ++t)
        if (t + 1 < K - 1) conv_state[static_cast<size_t>(t) * channels + c] = win[t + 1];
    conv_state[static_cast<size_t>(K - 2) * channels + c] = v;
}

// The delta rule of 16 state rows of one value head per workgroup (128
// threads, 8 lanes per row): the L2 norms of the head's q and k (waves 0 and
// 1, the same sums as gdn_group_kernel), beta and the decay, the row updates
// and the raw output.  qkv already holds conv + SiLU.
constexpr int kDeltaRows = 16;
constexpr int kDeltaThreads = kDeltaRows * 8;

// Sequence s of a batch (blockIdx.y): buffers laid out [batch][...] with the
// single-sequence sizes.
__device__ __forceinline__ GdnParams gdn_seq(GdnParams p, int s) {
    const size_t conv = static_cast<size_t>(2) * p.state_size * p.key_heads + static_cast<size_t>(p.value_heads) * p.head;
    p.qkv += s * conv;
    p.alpha += static_cast<size_t>(s) * p.value_heads;
    p.beta += static_cast<size_t>(s) * p.value_heads;
    p.state += static_cast<size_t>(s) * p.value_heads * p.head * p.head;
    p.out += static_cast<size_t>(s) * p.value_heads * p.head;
    return p;
}

// Workgroup b runs on XCD b % 8.  The logical (head, row block) index of b
// is chosen so that a head's row blocks are consecutive on one XCD, whose L2
// then serves the head's q and k to all of them.
__device__ __forceinline__ int xcd_grouped(int b, int n) { return n % 8 == 0 ? (b % 8) * (n / 8) + b / 8 : b; }

template <int HEAD>
__global__ __launch_bounds__(kDeltaThreads) void gdn_delta_kernel(const GdnParams p_batch) {
    FORTAI_TRACE_SCOPE(2);
    const GdnParams p = gdn_seq(p_batch, static_cast<int>(blockIdx.y));
    constexpr int kCols = HEAD / 8;
    __shared__ __align__(16) float qs[HEAD];
    __shared__ __align__(16) float ks[HEAD];
    __shared__ double red[2];
    __shared__ float hs[2];
    __shared__ MathTables mt;
    const uint64_t mt_word = MathTables::fetch();  // stored after the other loads are issued
    const int tid = static_cast<int>(threadIdx.x);
    const int blocks_per_head = HEAD / kDeltaRows;
    const int wg = xcd_grouped(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
    const int h = wg / blocks_per_head;
    const int r0 = (wg % blocks_per_head) * kDeltaRows;
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
    const float beta_in = p.beta[h], alpha_in = p.alpha[h], ssm_a = p.ssm_a[h], ssm_dt = p.ssm_dt[h];
    mt.put(mt_word);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = tid + k * kDeltaThreads;
        if (i < HEAD) qs[i] = qk[k];
        else if (i < 2 * HEAD) ks[i - HEAD] = qk[k];
    }
    __syncthreads();
    if (tid == 0) {
        // fortai_qwen35_cpu.f90:890-894 (the tables in LDS since the barrier)
        hs[0] = mt.sigmoid(beta_in);
        hs[1] = mt.expf(ssm_a * mt.softplus(alpha_in + ssm_dt));
    }
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
    const float beta = hs[0];
    const float decay = hs[1];
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

// The batch decode's delta rule with the ssm_out projection's input built in
// the same launch: one workgroup per (value head, sequence) runs every state
// row of the head (HEAD x 8 threads, the row code of gdn_delta_kernel above,
// operation for operation), collects the head's raw output in LDS, and then
// wave 0 forms the head's gated RMSNorm and Q8_0 quantization with the
// matvec's gated-prologue code (a lane per 4 values, the double sum of
// squares by the same butterfly over the head's lanes, the same per-value
// expression and quantizer) into the Q8L activation [batch][q8l_bytes(width)]
// that the batched ssm_out projection reads -- the bits the separate
// normalise-and-quantize launch would write.  width = value_heads * HEAD, a
// multiple of 128 (no padding blocks); z: the SiLU'd gate [batch][width];
// norm: the per-head weights [HEAD]; eps: the gated norm's epsilon.
template <int HEAD>
__global__ __launch_bounds__(HEAD * 8) void gdn_delta_gated_kernel(const GdnParams p_batch, const float *z_batch,
    const float *norm, float eps, void *q8l, int width) {
    FORTAI_TRACE_SCOPE(11);
    const int seq = static_cast<int>(blockIdx.y);
    const GdnParams p = gdn_seq(p_batch, seq);
    constexpr int kThreads = HEAD * 8;
    constexpr int kCols = HEAD / 8;
    constexpr int kGroups = HEAD / 4;  // 4-value groups (lanes of wave 0) per head
    static_assert(kGroups <= 64 && kGroups % 8 == 0, "one head's groups in whole blocks of wave 0");
    __shared__ __align__(16) float qs[HEAD];
    __shared__ __align__(16) float ks[HEAD];
    __shared__ __align__(16) float os[HEAD];
    __shared__ double red[2];
    __shared__ float hs[2];
    __shared__ MathTables mt;
    const uint64_t mt_word = MathTables::fetch();  // stored after the other loads are issued
    const int tid = static_cast<int>(threadIdx.x), lane = tid & 63, wave = tid >> 6;
    const int h = static_cast<int>(blockIdx.x);
    const int kh = h / (p.value_heads / p.key_heads);
    const int row = tid >> 3, l = tid & 7;
    float s[kCols];
    float4 *srow = reinterpret_cast<float4 *>(p.state + ((static_cast<size_t>(h) * HEAD + row) * 8 + l) * kCols);
#pragma unroll
    for (int i = 0; i < kCols / 4; ++i) {
        const float4 f = srow[i];
        s[4 * i] = f.x; s[4 * i + 1] = f.y; s[4 * i + 2] = f.z; s[4 * i + 3] = f.w;
    }
    const int iq = min(tid, 2 * HEAD - 1);
    const float qk = p.qkv[iq < HEAD ? kh * HEAD + iq : p.state_size * p.key_heads + kh * HEAD + (iq - HEAD)];
    const float vrow = p.qkv[2 * p.state_size * p.key_heads + h * HEAD + row];
    const float beta_in = p.beta[h], alpha_in = p.alpha[h], ssm_a = p.ssm_a[h], ssm_dt = p.ssm_dt[h];
    // the gated norm's inputs (wave 0; lanes past the head's groups re-read its last)
    const int t = min(lane, kGroups - 1);
    float4 zr = make_float4(0.0f, 0.0f, 0.0f, 0.0f), wr = zr;
    if (wave == 0) {
        zr = reinterpret_cast<const float4 *>(z_batch + static_cast<size_t>(seq) * width)[h * kGroups + t];
        wr = reinterpret_cast<const float4 *>(norm)[t];
    }
    mt.put(mt_word);
    if (tid < HEAD) qs[tid] = qk;
    else if (tid < 2 * HEAD) ks[tid - HEAD] = qk;
    __syncthreads();
    if (tid == 0) {
        // fortai_qwen35_cpu.f90:890-894 (the tables in LDS since the barrier)
        hs[0] = mt.sigmoid(beta_in);
        hs[1] = mt.expf(ssm_a * mt.softplus(alpha_in + ssm_dt));
    }
    // L2 norms of q (wave 0) and k (wave 1), fortai_qwen35_cpu.f90:1455-1471
    if (tid < 128) {
        const float *v = (tid < 64) ? qs : ks;
        double ss = 0.0;
        for (int i = tid & 63; i < HEAD; i += 64) ss += static_cast<double>(v[i]) * static_cast<double>(v[i]);
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
    }
    __syncthreads();
    const float qinv = 1.0f / fmaxf(sqrtf(static_cast<float>(red[0])), p.eps);
    const float kinv = 1.0f / fmaxf(sqrtf(static_cast<float>(red[1])), p.eps);
    const float beta = hs[0];
    const float decay = hs[1];
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
    if (l == 0) os[row] = qd * (1.0f / sqrtf(static_cast<float>(HEAD)));
    __syncthreads();
    if (wave != 0) return;
    // gated RMSNorm of the head, fortai_qwen35_cpu.f90:907-915, then Q8_0
    float4 y = reinterpret_cast<const float4 *>(os)[t];
    double ss = static_cast<double>(y.x) * static_cast<double>(y.x);
    ss += static_cast<double>(y.y) * static_cast<double>(y.y);
    ss += static_cast<double>(y.z) * static_cast<double>(y.z);
    ss += static_cast<double>(y.w) * static_cast<double>(y.w);
    ss = group_sum_up(ss, kGroups);
    const float nf = sqrtf(static_cast<float>(div_count(ss, HEAD)) + eps);
    y.x = ((y.x / nf) * wr.x) * zr.x;
    y.y = ((y.y / nf) * wr.y) * zr.y;
    y.z = ((y.z / nf) * wr.z) * zr.z;
    y.w = ((y.w / nf) * wr.w) * zr.w;
    float scale;
    uint16_t bits;
    const uint32_t packed = quantize_group(y, scale, bits);
    if (lane < kGroups) {
        const int g = h * kGroups + lane, b = g >> 3, lb = g & 7;
        unsigned char *base = static_cast<unsigned char *>(q8l) + static_cast<size_t>(seq) * q8l_bytes(width);
        reinterpret_cast<uint32_t *>(base)[((b >> 2) * 8 + lb) * 4 + (b & 3)] = packed;
        const int chunks = width / 128;
        if (lb == 0) reinterpret_cast<float *>(base + static_cast<size_t>(chunks) * 128)[b] = scale;
    }
}

// ------------------------------------------------------- state-resident
// `steps` autoregressive steps of the recurrent core in one launch: each
// workgroup keeps its 16 state rows in registers across every step, and the
// conv1d window of each channel it reads in registers too.  Per step it
// runs the conv1d + SiLU of the channels it needs (the key head's q and k,
// its own v rows; the q / k channels are computed by every workgroup of the
// key head, redundantly and identically), then the same delta-rule code as
// gdn_delta_kernel.  Bit-identical to `steps` calls of conv_silu_kernel +
// gdn_delta_kernel.  At the end the state rows go back, and each conv
// window is written by the one workgroup that owns the channel: v channels
// by their row's workgroup, q / k channels by row block 0 of the first value
// head of the key head.  The windows are read from conv_in, a copy taken
// before the launch, so no workgroup can read a window another has already
// advanced.
// qkv [steps][conv_size] (projection outputs), alpha / beta [steps][value_heads],
// out [steps][value_heads * head].
template <int HEAD>
__global__ __launch_bounds__(kDeltaThreads) void gdn_recurrence_kernel(const GdnParams p, const float *__restrict__ conv_w,
    const float *__restrict__ conv_in, float *__restrict__ conv_state, int conv_size, int K, int steps) {
    static_assert(HEAD == kDeltaThreads, "one q and one k channel per thread");
    constexpr int kCols = HEAD / 8;
    __shared__ __align__(16) float qs[HEAD];
    __shared__ __align__(16) float ks[HEAD];
    __shared__ float vs[kDeltaRows];
    __shared__ double red[2];
    __shared__ float hs[2];
    __shared__ MathTables mt;  // written and read by wave 0 (thread 0 uses it)
    const uint64_t mt_word = MathTables::fetch();  // stored after the other loads are issued
    const int tid = static_cast<int>(threadIdx.x);
    const int blocks_per_head = HEAD / kDeltaRows;
    const int wg = xcd_grouped(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
    const int h = wg / blocks_per_head;
    const int rb = wg % blocks_per_head, r0 = rb * kDeltaRows;
    const int group = p.value_heads / p.key_heads, kh = h / group;
    const int r8 = tid >> 3, l = tid & 7, row = r0 + r8;
    const int inner = p.value_heads * HEAD;
    // this thread's channels: q and k of the key head, v of row r0 + tid (tid < 16)
    const int cq = kh * HEAD + tid, ck = p.state_size * p.key_heads + kh * HEAD + tid;
    const int cv = 2 * p.state_size * p.key_heads + h * HEAD + r0 + min(tid, kDeltaRows - 1);
    const int chans[3] = {cq, ck, cv};
    float win[3][kConvMax - 1], taps[3][kConvMax];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
#pragma unroll
        for (int t = 0; t < kConvMax; ++t) {
            if (t < K - 1) win[c][t] = conv_in[static_cast<size_t>(t) * conv_size + chans[c]];
            if (t < K) taps[c][t] = conv_w[static_cast<size_t>(chans[c]) * K + t];
        }
    }
    float s[kCols];
    float4 *srow = reinterpret_cast<float4 *>(p.state + ((static_cast<size_t>(h) * HEAD + row) * 8 + l) * kCols);
#pragma unroll
    for (int i = 0; i < kCols / 4; ++i) {
        const float4 f = srow[i];
        s[4 * i] = f.x; s[4 * i + 1] = f.y; s[4 * i + 2] = f.z; s[4 * i + 3] = f.w;
    }
    mt.put(mt_word);
    wave_lds_fence();
    const float inv_sqrt = 1.0f / sqrtf(static_cast<float>(HEAD));
    // the next step's inputs are loaded while the current one runs
    float xn[3], an = 0.0f, bn = 0.0f;
    auto fetch = [&](int t) {
        const float *x = p.qkv + static_cast<size_t>(t) * conv_size;
#pragma unroll
        for (int c = 0; c < 3; ++c) xn[c] = x[chans[c]];
        if (tid == 0) {
            an = p.alpha[static_cast<size_t>(t) * p.value_heads + h];
            bn = p.beta[static_cast<size_t>(t) * p.value_heads + h];
        }
    };
    fetch(0);
    for (int t = 0; t < steps; ++t) {
        float x[3] = {xn[0], xn[1], xn[2]};
        const float a = an, b = bn;
        if (t + 1 < steps) fetch(t + 1);
        // conv1d + SiLU of the three channels, then the windows move by one
        float y[3];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            y[c] = conv_silu(win[c], taps[c], K, x[c]);
#pragma unroll
            for (int u = 0; u + 1 < kConvMax - 1; ++u)
                if (u + 1 < K - 1) win[c][u] = win[c][u + 1];
#pragma unroll
            for (int u = 0; u < kConvMax - 1; ++u)
                if (u == K - 2) win[c][u] = x[c];
        }
        qs[tid] = y[0];
        ks[tid] = y[1];
        if (tid < kDeltaRows) vs[tid] = y[2];
        if (tid == 0) {
            // fortai_qwen35_cpu.f90:890-894
            hs[0] = mt.sigmoid(b);
            hs[1] = mt.expf(p.ssm_a[h] * mt.softplus(a + p.ssm_dt[h]));
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
        const float beta = hs[0], decay = hs[1];
        const float vrow = vs[r8];
        // delta rule (fortai_q8_dot.c:363-396)
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
        if (l == 0) p.out[static_cast<size_t>(t) * inner + h * HEAD + row] = qd * inv_sqrt;
        __syncthreads();  // qs / ks / vs / hs / red are rewritten by the next step
    }
#pragma unroll
    for (int i = 0; i < kCols / 4; ++i) srow[i] = make_float4(s[4 * i], s[4 * i + 1], s[4 * i + 2], s[4 * i + 3]);
    const bool qk_owner = rb == 0 && h % group == 0;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const bool owner = c < 2 ? qk_owner : tid < kDeltaRows;
        if (!owner) continue;
#pragma unroll
        for (int u = 0; u < kConvMax - 1; ++u)
            if (u < K - 1) conv_state[static_cast<size_t>(u) * conv_size + chans[c]] = win[c][u];
    }
}

}  // namespace

hipError_t launch_conv_silu(const float *x, const float *conv_w, float *conv_state, float *out, int channels, int K,
    hipStream_t stream) {
    if (channels <= 0 || K < 2 || K > kConvMax) return hipErrorInvalidValue;
    hipLaunchKernelGGL(conv_silu_kernel, dim3((channels + 255) / 256), dim3(256), 0, stream, x, conv_w, conv_state, out,
        channels, K);
    note_launch("conv_silu_kernel grid %d", (channels + 255) / 256);
    return hipGetLastError();
}

hipError_t launch_gdn_delta(const GdnParams &p, hipStream_t stream, int batch) {
    if (batch < 1 || p.key_heads <= 0 || p.value_heads % p.key_heads || p.state_size != p.head || !p.out) return hipErrorInvalidValue;
    const dim3 grid(p.value_heads * (p.head / kDeltaRows), batch);
    switch (p.head) {
    case 64: hipLaunchKernelGGL(gdn_delta_kernel<64>, grid, dim3(kDeltaThreads), 0, stream, p); break;
    case 128: hipLaunchKernelGGL(gdn_delta_kernel<128>, grid, dim3(kDeltaThreads), 0, stream, p); break;
    case 256: hipLaunchKernelGGL(gdn_delta_kernel<256>, grid, dim3(kDeltaThreads), 0, stream, p); break;
    default: return hipErrorInvalidValue;
    }
    note_launch("gdn_delta_kernel<%d> grid %dx%d", p.head, grid.x, batch);
    return hipGetLastError();
}

hipError_t launch_gdn_delta_gated(const GdnParams &p, const float *z, const float *norm, float eps, void *q8l,
    hipStream_t stream, int batch) {
    const int width = p.value_heads * p.head;
    if (batch < 1 || p.key_heads <= 0 || p.value_heads % p.key_heads || p.state_size != p.head || width % 128 || !q8l)
        return hipErrorInvalidValue;
    const dim3 grid(p.value_heads, batch);
    switch (p.head) {
    case 64: hipLaunchKernelGGL(gdn_delta_gated_kernel<64>, grid, dim3(64 * 8), 0, stream, p, z, norm, eps, q8l, width); break;
    case 128: hipLaunchKernelGGL(gdn_delta_gated_kernel<128>, grid, dim3(128 * 8), 0, stream, p, z, norm, eps, q8l, width); break;
    default: return hipErrorInvalidValue;
    }
    note_launch("gdn_delta_gated_kernel<%d> grid %dx%d", p.head, grid.x, batch);
    return hipGetLastError();
}

}  // namespace fortai_hip

namespace fortai_hip {
hipError_t launch_gdn_recurrence(const GdnParams &p, const float *conv_w, const float *conv_in, float *conv_state,
    int conv_size, int K, int steps, hipStream_t stream) {
    if (steps < 1 || p.key_heads <= 0 || p.value_heads % p.key_heads || p.state_size != p.head || !p.out ||
        K < 2 || K > kConvMax || p.head != kDeltaThreads ||
        conv_size != 2 * p.state_size * p.key_heads + p.value_heads * p.head)
        return hipErrorInvalidValue;
    const dim3 grid(p.value_heads * (p.head / kDeltaRows));
    hipLaunchKernelGGL(gdn_recurrence_kernel<kDeltaThreads>, grid, dim3(kDeltaThreads), 0, stream, p, conv_w, conv_in,
        conv_state, conv_size, K, steps);
    note_launch("gdn_recurrence_kernel<%d> grid %d, %d steps", p.head, grid.x, steps);
    return hipGetLastError();
}
}  // namespace fortai_hip
