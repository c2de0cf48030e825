// Prompt prefill of a batch of sequences: T tokens per sequence in one pass.
//
// The reference has no prefill: it runs every prompt token through the decode
// step (fortai_qwen35_cpu.f90:591-711).  Here the projections of all
// batch x T tokens are token-block products on the i8 matrix cores
// (mmq.hip), and the parts that are sequential in time run as one kernel per
// layer that loops over the tokens: the causal conv1d (per channel,
// :856-879), the delta rule (per value head and 16 state rows, :880-906) and
// causal attention (per query block, online softmax).  Results agree with the
// per-token decode within fp32 rounding (the block dots are exact; the fp32
// accumulation orders differ), not bit for bit.  Rows are token-major: row
// n = s * T + t is token t of sequence s, at position t.
#include "attention_exact.h"
#include "fortai_hip_internal.h"
#include "fortai_hip_kernels.h"

namespace fortai_hip {

namespace {

namespace ea = exact_attention;

constexpr int kRowThreads = 256;

// x [rows][width] (row pitch ld_x) -> optional RMSNorm (fortai_qwen35_cpu.f90:
// 1408-1432) -> fortai_q8_quantize of every row into X8.  One workgroup per row.
__global__ __launch_bounds__(kRowThreads) void rms_quantize_tokens_kernel(const float *__restrict__ x, int ld_x,
    int width, const float *__restrict__ norm, float eps, int ld, int blocks_pad, int8_t *__restrict__ xq,
    float *__restrict__ xs) {
    __shared__ double red[kRowThreads / 64];
    const int n = static_cast<int>(blockIdx.x), tid = static_cast<int>(threadIdx.x);
    const float *row = x + static_cast<size_t>(n) * ld_x;
    float inv = 1.0f;
    if (norm) {
        double ss = 0.0;
        for (int i = tid; i < width; i += kRowThreads) ss += static_cast<double>(row[i]) * static_cast<double>(row[i]);
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        double total = 0.0;
        for (int w = 0; w < kRowThreads / 64; ++w) total += red[w];
        inv = 1.0f / sqrtf(static_cast<float>(div_count(total, width)) + eps);
    }
    for (int g = tid; g < blocks_pad * 8; g += kRowThreads) {
        float4 y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (g < width / 4) {
            y = reinterpret_cast<const float4 *>(row)[g];
            if (norm) {
                const float4 w4 = reinterpret_cast<const float4 *>(norm)[g];
                y.x = (y.x * inv) * w4.x; y.y = (y.y * inv) * w4.y; y.z = (y.z * inv) * w4.z; y.w = (y.w * inv) * w4.w;
            }
        }
        float scale;
        uint16_t bits;
        const uint32_t packed = quantize_group(y, scale, bits);
        const int b = g >> 3, l = g & 7;
        reinterpret_cast<uint32_t *>(xq + (static_cast<size_t>(b) * ld + n) * 32)[l] = packed;
        if (l == 0) xs[static_cast<size_t>(b) * ld + n] = scale;
    }
}

// GDN output o with the gate: per head ((o / rms(o)) * ssm_norm) * silu(z)
// (fortai_qwen35_cpu.f90:907-915), quantized into X8.  One workgroup per row;
// a head is head/4 consecutive threads (aligned power of two).
__global__ __launch_bounds__(kRowThreads) void gated_quantize_tokens_kernel(const float *__restrict__ o,
    const float *__restrict__ z, const float *__restrict__ norm, float eps, int width, int head, int ld,
    int blocks_pad, int8_t *__restrict__ xq, float *__restrict__ xs) {
    const int n = static_cast<int>(blockIdx.x), tid = static_cast<int>(threadIdx.x);
    const float *orow = o + static_cast<size_t>(n) * width;
    const float *zrow = z + static_cast<size_t>(n) * width;
    const int hl = head / 4;
    for (int g0 = 0; g0 < blocks_pad * 8; g0 += kRowThreads) {
        const int g = g0 + tid;
        const bool in = g < width / 4;
        float4 y = in ? reinterpret_cast<const float4 *>(orow)[g] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        double ss = static_cast<double>(y.x) * y.x + static_cast<double>(y.y) * y.y +
            static_cast<double>(y.z) * y.z + static_cast<double>(y.w) * y.w;
        ss = group_sum_up(ss, hl);
        if (in) {
            const float nf = sqrtf(static_cast<float>(div_count(ss, head)) + eps);
            const float4 w4 = reinterpret_cast<const float4 *>(norm)[g % hl];
            const float4 z4 = reinterpret_cast<const float4 *>(zrow)[g];
            y.x = ((y.x / nf) * w4.x) * silu_poly(z4.x);
            y.y = ((y.y / nf) * w4.y) * silu_poly(z4.y);
            y.z = ((y.z / nf) * w4.z) * silu_poly(z4.z);
            y.w = ((y.w / nf) * w4.w) * silu_poly(z4.w);
        }
        float scale;
        uint16_t bits;
        const uint32_t packed = quantize_group(y, scale, bits);
        if (g < blocks_pad * 8) {
            const int b = g >> 3, l = g & 7;
            reinterpret_cast<uint32_t *>(xq + (static_cast<size_t>(b) * ld + n) * 32)[l] = packed;
            if (l == 0) xs[static_cast<size_t>(b) * ld + n] = scale;
        }
    }
}

// FFN hidden silu(gate) * up (fortai_silu_product) quantized into X8.
__global__ __launch_bounds__(kRowThreads) void silu_product_quantize_kernel(const float *__restrict__ gate,
    const float *__restrict__ up, int width, int ld, int blocks_pad, int8_t *__restrict__ xq, float *__restrict__ xs) {
    const int n = static_cast<int>(blockIdx.x), tid = static_cast<int>(threadIdx.x);
    const float4 *g4 = reinterpret_cast<const float4 *>(gate + static_cast<size_t>(n) * width);
    const float4 *u4 = reinterpret_cast<const float4 *>(up + static_cast<size_t>(n) * width);
    for (int g = tid; g < blocks_pad * 8; g += kRowThreads) {
        float4 y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (g < width / 4) {
            const float4 a = g4[g], b = u4[g];
            y = make_float4(silu_poly(a.x) * b.x, silu_poly(a.y) * b.y, silu_poly(a.z) * b.z, silu_poly(a.w) * b.w);
        }
        float scale;
        uint16_t bits;
        const uint32_t packed = quantize_group(y, scale, bits);
        const int b = g >> 3, l = g & 7;
        reinterpret_cast<uint32_t *>(xq + (static_cast<size_t>(b) * ld + n) * 32)[l] = packed;
        if (l == 0) xs[static_cast<size_t>(b) * ld + n] = scale;
    }
}

// Causal conv1d + SiLU over the prompt (fortai_qwen35_cpu.f90:856-879).  The
// conv has no recurrence: output t reads the inputs t-K+1..t, those before
// the prompt from conv_state [batch][K-1][C] (oldest first).  One thread per
// (sequence, channel, kConvTokens consecutive tokens) computes each output
// with the decode's conv_silu (same window, same order), reading the old
// state only; conv_state_advance_kernel then stores the last K-1 inputs.
// x: raw projections [batch*T][C].
constexpr int kConvTokens = 8;

__global__ __launch_bounds__(256) void conv_silu_tokens_kernel(const float *__restrict__ x,
    const float *__restrict__ conv_w, const float *__restrict__ conv_state, float *__restrict__ out, int T, int C,
    int K) {
    const int c = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
    const int t0 = static_cast<int>(blockIdx.y) * kConvTokens;
    const int s = static_cast<int>(blockIdx.z);
    if (c >= C) return;
    float taps[kConvMax];
#pragma unroll
    for (int i = 0; i < kConvMax; ++i) taps[i] = i < K ? conv_w[static_cast<size_t>(c) * K + i] : 0.0f;
    const float *cs = conv_state + static_cast<size_t>(s) * (K - 1) * C + c;
    const float *xs = x + static_cast<size_t>(s) * T * C + c;
    float *os = out + static_cast<size_t>(s) * T * C + c;
    // inputs t0-K+1 .. t0+kConvTokens-1 (kConvMax-1 window slots, then the tokens)
    float in[kConvMax - 1 + kConvTokens];
#pragma unroll
    for (int i = 0; i < kConvMax - 1 + kConvTokens; ++i) {
        const int u = t0 - (kConvMax - 1) + i;  // input index; < 0: from the state
        float v = 0.0f;
        if (u >= 0 && u < T) v = xs[static_cast<size_t>(u) * C];
        else if (u < 0 && u >= -(K - 1)) v = cs[static_cast<size_t>(K - 1 + u) * C];
        in[i] = v;
    }
#pragma unroll
    for (int j = 0; j < kConvTokens; ++j) {
        const int t = t0 + j;
        if (t >= T) break;
        float win[kConvMax - 1];
#pragma unroll
        for (int i = 0; i < kConvMax - 1; ++i) win[i] = i < K - 1 ? in[j + (kConvMax - K) + i] : 0.0f;
        os[static_cast<size_t>(t) * C] = conv_silu(win, taps, K, in[j + kConvMax - 1]);
    }
}

// conv_state <- the last K-1 inputs of the prompt (older state entries when
// the prompt is shorter than K-1); each thread reads its channel's old state
// before writing it.
__global__ __launch_bounds__(256) void conv_state_advance_kernel(const float *__restrict__ x, float *conv_state, int T,
    int C, int K) {
    const int c = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
    const int s = static_cast<int>(blockIdx.y);
    if (c >= C) return;
    float *cs = conv_state + static_cast<size_t>(s) * (K - 1) * C + c;
    const float *xs = x + static_cast<size_t>(s) * T * C + c;
    float nw[kConvMax - 1];
#pragma unroll
    for (int i = 0; i < kConvMax - 1; ++i) {
        if (i >= K - 1) break;
        const int u = T - (K - 1) + i;
        nw[i] = u >= 0 ? xs[static_cast<size_t>(u) * C] : cs[static_cast<size_t>(i + T) * C];
    }
#pragma unroll
    for (int i = 0; i < kConvMax - 1; ++i)
        if (i < K - 1) cs[static_cast<size_t>(i) * C] = nw[i];
}

// Per token: the L2 norms of every key head's q and k (1 / max(|x|, eps),
// fortai_qwen35_cpu.f90:1455-1471) and every value head's beta and decay
// (:890-894).  One workgroup per token; wave w takes key heads w, w + 4, ...
__global__ __launch_bounds__(256) void gdn_token_prep_kernel(const float *__restrict__ qkv, const float *__restrict__ alpha,
    const float *__restrict__ beta, const float *__restrict__ ssm_a, const float *__restrict__ ssm_dt, int C,
    int key_heads, int value_heads, int head, int state_size, float eps, float *__restrict__ qinv,
    float *__restrict__ kinv, float *__restrict__ beta_out, float *__restrict__ decay_out) {
    const int n = static_cast<int>(blockIdx.x), tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63, wave = tid >> 6;
    const float *row = qkv + static_cast<size_t>(n) * C;
    for (int kh = wave; kh < key_heads; kh += 4) {
        const float *q = row + kh * head, *k = row + state_size * key_heads + kh * head;
        double sq = 0.0, sk = 0.0;
        for (int i = lane; i < head; i += 64) {
            sq += static_cast<double>(q[i]) * q[i];
            sk += static_cast<double>(k[i]) * k[i];
        }
        sq = wave_sum(sq);
        sk = wave_sum(sk);
        if (lane == 0) {
            qinv[static_cast<size_t>(n) * key_heads + kh] = 1.0f / fmaxf(sqrtf(static_cast<float>(sq)), eps);
            kinv[static_cast<size_t>(n) * key_heads + kh] = 1.0f / fmaxf(sqrtf(static_cast<float>(sk)), eps);
        }
    }
    for (int h = tid; h < value_heads; h += 256) {
        const size_t i = static_cast<size_t>(n) * value_heads + h;
        beta_out[i] = sigmoid_ref(beta[i]);
        decay_out[i] = exp_rounded(ssm_a[h] * softplus_ref(alpha[i] + ssm_dt[h]));
    }
}

// The delta rule over time (fortai_q8_dot.c:356-398) for 16 state rows of one
// value head of one sequence (blockIdx.y), the state in registers in the
// decode kernel's layout: S[row][8 i + l] at
// state[((h * HEAD + row) * 8 + l) * HEAD/8 + i].  Normalized q and k of
// kStage tokens are staged in LDS at a time.
constexpr int kGdnRows = 16;
constexpr int kStage = 16;

template <int HEAD>
__global__ __launch_bounds__(kGdnRows * 8) void gdn_prefill_kernel(const float *__restrict__ qkv,
    const float *__restrict__ qinv, const float *__restrict__ kinv, const float *__restrict__ beta,
    const float *__restrict__ decay, float *__restrict__ state, float *__restrict__ out, int T, int C, int key_heads,
    int value_heads, int state_size) {
    constexpr int kCols = HEAD / 8;
    __shared__ __align__(16) float qs[kStage][HEAD];
    __shared__ __align__(16) float ks[kStage][HEAD];
    __shared__ float vs[kStage][kGdnRows];
    __shared__ float bs[kStage], ds[kStage];
    const int tid = static_cast<int>(threadIdx.x);
    const int s = static_cast<int>(blockIdx.y);
    const int bph = HEAD / kGdnRows;
    const int h = static_cast<int>(blockIdx.x) / bph, r0 = (static_cast<int>(blockIdx.x) % bph) * kGdnRows;
    const int kh = h / (value_heads / key_heads);
    const int r8 = tid >> 3, l = tid & 7, row = r0 + r8;
    const int inner = value_heads * HEAD;
    float *sp = state + static_cast<size_t>(s) * value_heads * HEAD * HEAD + ((static_cast<size_t>(h) * HEAD + row) * 8 + l) * kCols;
    float st[kCols];
#pragma unroll
    for (int i = 0; i < kCols; ++i) st[i] = sp[i];
    const float scale = 1.0f / sqrtf(static_cast<float>(HEAD));
    for (int t0 = 0; t0 < T; t0 += kStage) {
        const int steps = min(kStage, T - t0);
        __syncthreads();  // the previous stage is consumed
#pragma unroll
        for (int e = tid; e < kStage * HEAD; e += kGdnRows * 8) {
            const int j = e / HEAD, i = e % HEAD;
            const size_t n = static_cast<size_t>(s) * T + t0 + min(j, steps - 1);
            const float *rowp = qkv + n * C;
            qs[j][i] = rowp[kh * HEAD + i] * qinv[n * key_heads + kh];
            ks[j][i] = rowp[state_size * key_heads + kh * HEAD + i] * kinv[n * key_heads + kh];
        }
#pragma unroll
        for (int e = tid; e < kStage * kGdnRows; e += kGdnRows * 8) {
            const int j = e / kGdnRows, rr = e % kGdnRows;
            const size_t n = static_cast<size_t>(s) * T + t0 + min(j, steps - 1);
            vs[j][rr] = qkv[n * C + 2 * state_size * key_heads + h * HEAD + r0 + rr];
        }
        if (tid < kStage) {
            const size_t n = static_cast<size_t>(s) * T + t0 + min(tid, steps - 1);
            bs[tid] = beta[n * value_heads + h];
            ds[tid] = decay[n * value_heads + h];
        }
        __syncthreads();
        for (int j = 0; j < steps; ++j) {
            const float dec = ds[j];
            float kd = 0.0f;
#pragma unroll
            for (int i = 0; i < kCols; ++i) {
                const float d = st[i] * dec;
                st[i] = d;
                kd = __builtin_fmaf(d, ks[j][8 * i + l], kd);
            }
            kd = row_hsum8(kd);
            const float delta = (vs[j][r8] - kd) * bs[j];
            float qd = 0.0f;
#pragma unroll
            for (int i = 0; i < kCols; ++i) {
                const float u = __builtin_fmaf(delta, ks[j][8 * i + l], st[i]);
                st[i] = u;
                qd = __builtin_fmaf(u, qs[j][8 * i + l], qd);
            }
            qd = row_hsum8(qd);
            if (l == 0) out[(static_cast<size_t>(s) * T + t0 + j) * inner + h * HEAD + row] = qd * scale;
        }
    }
#pragma unroll
    for (int i = 0; i < kCols; ++i) sp[i] = st[i];
}

// Per token: q and k per-head RMSNorm + RoPE at the token's position
// (fortai_qwen35_cpu.f90:990-999, 1473-1497), q in place; k and v appended to
// the fp16 caches [batch][max_context][kv_heads][head] with the reference's
// float_to_half (:1594-1601); cache_flags [batch][kv_heads] set when an
// exponent-31 half is stored.  One workgroup per token, one wave per head.
__global__ __launch_bounds__(256) void qk_rope_append_kernel(float *__restrict__ q, const float *__restrict__ k,
    const float *__restrict__ v, const float *__restrict__ q_norm, const float *__restrict__ k_norm,
    const float2 *__restrict__ rope, uint16_t *__restrict__ kcache, uint16_t *__restrict__ vcache,
    int *__restrict__ flags, int T, int heads, int kv_heads, int head, int value, int rope_dim, int max_context,
    float eps) {
    __shared__ __align__(16) float buf[4][256];
    __shared__ __align__(16) float wq[256], wk[256];
    const int n = static_cast<int>(blockIdx.x), tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63, wave = tid >> 6;
    const int s = n / T, pos = n % T;
    for (int i = tid; i < head; i += 256) {
        wq[i] = q_norm[i];
        wk[i] = k_norm[i];
    }
    __syncthreads();
    const float2 *rp = rope + static_cast<size_t>(pos) * (rope_dim / 2);
    // q heads then k heads, one wave each
    for (int j = wave; j < heads + kv_heads; j += 4) {
        float *b = buf[wave];
        const bool isq = j < heads;
        const float *src = isq ? q + (static_cast<size_t>(n) * heads + j) * 2 * head
                               : k + (static_cast<size_t>(n) * kv_heads + (j - heads)) * head;
        for (int i = lane; i < head; i += 64) b[i] = src[i];
        wave_lds_fence();
        ea::norm_rope(b, head, isq ? wq : wk, eps, rp, rope_dim, lane);
        if (isq) {
            float *dst = q + (static_cast<size_t>(n) * heads + j) * 2 * head;
            for (int i = lane; i < head; i += 64) dst[i] = b[i];
        } else {
            const int kvh = j - heads;
            uint16_t *dst = kcache + ((static_cast<size_t>(s) * max_context + pos) * kv_heads + kvh) * head;
            int over = 0;
            for (int i = lane; i < head; i += 64) {
                const uint16_t hb = float_to_half_kv(b[i]);
                dst[i] = hb;
                over |= (hb & 0x7c00u) == 0x7c00u;
            }
            if (__any(over) && lane == 0) flags[static_cast<size_t>(s) * kv_heads + kvh] = 1;
        }
        wave_lds_fence();
    }
    for (int e = tid; e < kv_heads * value; e += 256) {
        const int kvh = e / value, i = e % value;
        const uint16_t hb = float_to_half_kv(v[(static_cast<size_t>(n) * kv_heads + kvh) * value + i]);
        vcache[((static_cast<size_t>(s) * max_context + pos) * kv_heads + kvh) * value + i] = hb;
        if ((hb & 0x7c00u) == 0x7c00u) flags[static_cast<size_t>(s) * kv_heads + kvh] = 1;
    }
}

// Causal attention of every prompt token with the reference's arithmetic
// and summation orders (fortai_qwen35_cpu.f90:1006-1031), so every output is
// bit-identical to the decode step's exact attention at that position:
//   s_j = (q . k_j, left to right, separately rounded) / sqrt(head)
//   m = max s_j;  e_j = expf(s_j - m);  Z = e_0 + e_1 + ... (left to right)
//   out_d = fl(e_0/Z v_0,d) + fl(e_1/Z v_1,d) + ... (left to right) * sigmoid(gate_d)
// One workgroup per (block of qb queries, head, sequence).  The scores of
// the block's keys stay in LDS (qb is chosen so that they fit); keys and
// values pass through LDS 64 positions at a time.  A query's masked keys
// (past its position) get e = +0 and weight +0: adding +0 or -0 to a running
// sum leaves it unchanged, so every chain can run to the block's last key.
constexpr int kXKeys = 64;  // keys per staged tile

template <int HEAD>
__global__ __launch_bounds__(256) void attention_prefill_exact_kernel(const float *__restrict__ q,
    const uint16_t *__restrict__ kcache, const uint16_t *__restrict__ vcache, float *__restrict__ out, int T,
    int heads, int kv_heads, int max_context, int qb, int kcap) {
    static_assert(HEAD % 64 == 0 && HEAD <= 256, "head 64, 128 or 256");
    extern __shared__ __align__(16) unsigned char lds_raw[];
    float *qs = reinterpret_cast<float *>(lds_raw);                  // [qb][HEAD] normalized q
    uint16_t *kv = reinterpret_cast<uint16_t *>(qs + qb * HEAD);    // K: [HEAD/8][kXKeys][8]; V: [kXKeys][HEAD]
    float *sc = reinterpret_cast<float *>(kv + kXKeys * HEAD);       // [qb][kcap] scores, then e, then weights
    const int tid = static_cast<int>(threadIdx.x), lane = tid & 63, wave = tid >> 6;
    const int h = static_cast<int>(blockIdx.y), s = static_cast<int>(blockIdx.z);
    const int q0 = static_cast<int>(blockIdx.x) * qb;
    const int nq = min(qb, T - q0);
    const int keys = q0 + nq;  // keys 0..keys-1 cover the block
    const int kvh = h / (heads / kv_heads);
    const float sqrt_head = sqrtf(static_cast<float>(HEAD));
    for (int e = tid; e < qb * HEAD; e += 256) {
        const int qi = e / HEAD, d = e % HEAD;
        qs[e] = qi < nq ? q[((static_cast<size_t>(s) * T + q0 + qi) * heads + h) * 2 * HEAD + d] : 0.0f;
    }
    // ---- scores: thread (key j = lane, query group = wave), queries wave + 4 r
    for (int j0 = 0; j0 < keys; j0 += kXKeys) {
        __syncthreads();
        for (int e = tid; e < kXKeys * (HEAD / 8); e += 256) {
            const int j = e / (HEAD / 8), piece = e % (HEAD / 8);
            const int p = min(j0 + j, keys - 1);
            const uint4 v8 = *reinterpret_cast<const uint4 *>(
                kcache + ((static_cast<size_t>(s) * max_context + p) * kv_heads + kvh) * HEAD + piece * 8);
            *reinterpret_cast<uint4 *>(kv + (piece * kXKeys + j) * 8) = v8;
        }
        __syncthreads();
        const int j = j0 + lane;
        for (int r0 = 0; r0 < qb; r0 += 16) {  // up to 4 queries of this wave at a time
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int d = 0; d < HEAD; d += 8) {
                const uint4 k8 = *reinterpret_cast<const uint4 *>(kv + ((d / 8) * kXKeys + lane) * 8);
                const uint32_t kw[4] = {k8.x, k8.y, k8.z, k8.w};
                float kf[8];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    kf[2 * u] = gguf_half_to_real(static_cast<uint16_t>(kw[u] & 0xffffu));
                    kf[2 * u + 1] = gguf_half_to_real(static_cast<uint16_t>(kw[u] >> 16));
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int qi = r0 + wave + 4 * r;
                    if (qi >= qb) break;
                    const float4 qa = *reinterpret_cast<const float4 *>(qs + qi * HEAD + d);
                    const float4 qc = *reinterpret_cast<const float4 *>(qs + qi * HEAD + d + 4);
                    float a = acc[r];
                    a = a + qa.x * kf[0];
                    a = a + qa.y * kf[1];
                    a = a + qa.z * kf[2];
                    a = a + qa.w * kf[3];
                    a = a + qc.x * kf[4];
                    a = a + qc.y * kf[5];
                    a = a + qc.z * kf[6];
                    a = a + qc.w * kf[7];
                    acc[r] = a;
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int qi = r0 + wave + 4 * r;
                if (qi < qb && j < keys) sc[qi * kcap + j] = acc[r] / sqrt_head;
            }
        }
    }
    __syncthreads();
    // ---- softmax weights: queries wave, wave + 4, ...; lanes over keys
    constexpr float kLowest = -3.402823466e38f;  // -huge(1.0_real32)
    for (int qi = wave; qi < nq; qi += 4) {
        const int n = q0 + qi + 1;  // this query's keys
        float *row = sc + qi * kcap;
        float m = kLowest;
        for (int j = lane; j < n; j += 64) m = fmaxf(m, row[j]);
        m = wave_max(m);
        for (int j = lane; j < keys; j += 64) row[j] = j < n ? expf_libm(row[j] - m) : 0.0f;
    }
    __syncthreads();
    // Z of each query by one lane, left to right (masked keys add +0)
    if (lane < 4) {
        const int qi = wave + 4 * lane;
        float z = 0.0f;
        if (qi < nq) {
            const float *row = sc + qi * kcap;
            int j = 0;
            for (; j + 4 <= keys; j += 4) {
                const float4 e4 = *reinterpret_cast<const float4 *>(row + j);
                z = z + e4.x;
                z = z + e4.y;
                z = z + e4.z;
                z = z + e4.w;
            }
            for (; j < keys; ++j) z = z + row[j];
        }
        // the weights e_j / Z (lanes of this wave finish the row below)
        if (qi < nq) qs[qi * HEAD] = z;  // q is no longer needed: slot 0 of the row holds Z
    }
    __syncthreads();
    for (int qi = wave; qi < nq; qi += 4) {
        const float z = qs[qi * HEAD];
        float *row = sc + qi * kcap;
        for (int j = lane; j < keys; j += 64) row[j] = row[j] / z;
    }
    // ---- P.V: thread = (dim d, queries qd, qd + QS, ...)
    constexpr int kQS = 256 / HEAD;  // query phases per dim
    const int d = tid % HEAD, qd = tid / HEAD;
    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    for (int j0 = 0; j0 < keys; j0 += kXKeys) {
        __syncthreads();
        for (int e = tid; e < kXKeys * (HEAD / 8); e += 256) {
            const int j = e / (HEAD / 8), piece = e % (HEAD / 8);
            const int p = min(j0 + j, keys - 1);
            *reinterpret_cast<uint4 *>(kv + j * HEAD + piece * 8) = *reinterpret_cast<const uint4 *>(
                vcache + ((static_cast<size_t>(s) * max_context + p) * kv_heads + kvh) * HEAD + piece * 8);
        }
        __syncthreads();
        const int jn = min(kXKeys, keys - j0);
        for (int jj = 0; jj < jn; jj += 4) {
            float vf[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) vf[u] = gguf_half_to_real(kv[min(jj + u, jn - 1) * HEAD + d]);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int qi = qd + kQS * r;
                if (qi >= nq) break;
                const float *w = sc + qi * kcap + j0 + jj;
                if (jj + 4 <= jn) {
                    const float4 w4 = *reinterpret_cast<const float4 *>(w);
                    float a = acc[r];
                    a = a + w4.x * vf[0];
                    a = a + w4.y * vf[1];
                    a = a + w4.z * vf[2];
                    a = a + w4.w * vf[3];
                    acc[r] = a;
                } else {
                    for (int u = 0; u < jn - jj; ++u) acc[r] = acc[r] + w[u] * vf[u];
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int qi = qd + kQS * r;
        if (qi >= nq) break;
        const size_t row = (static_cast<size_t>(s) * T + q0 + qi) * heads + h;
        const float gate = q[row * 2 * HEAD + HEAD + d];
        out[row * HEAD + d] = acc[r] * sigmoid_ref(gate);
    }
}

// The same arithmetic and orders with fixed trip counts: 16 queries per
// workgroup (rows past the prompt are zero and never stored), keys clamped
// into the cache and masked through zero weights, K / V tiles loaded one
// ahead into registers, and (FINITE, no exponent-31 half in this cache) each
// product fl(a * f32(h)) taken straight from the fp16 half by v_fma_mix_f32.
// A workgroup whose cache is flagged returns unless !FINITE, and the !FINITE
// instance serves only flagged caches, so the two launches split the work.
constexpr int kXQ = 16;  // queries per workgroup

template <bool FINITE>
__device__ __forceinline__ float times_half(uint32_t h2, bool hi, float a) {
    if constexpr (FINITE) return hi ? half_times<true>(h2, a) : half_times<false>(h2, a);
    return a * gguf_half_to_real(static_cast<uint16_t>(hi ? h2 >> 16 : h2 & 0xffffu));
}

template <int HEAD, bool FINITE>
__global__ __launch_bounds__(256, 2) void attention_prefill_exact16_kernel(const float *__restrict__ q,
    const uint16_t *__restrict__ kcache, const uint16_t *__restrict__ vcache, const int *__restrict__ flags,
    float *__restrict__ out, int T, int heads, int kv_heads, int max_context, int kcap) {
    static_assert(HEAD % 64 == 0 && HEAD <= 256, "head 64, 128 or 256");
    constexpr int kPieces = kXKeys * HEAD / 8 / 256;  // 16-byte tile pieces per thread
    constexpr int kQS = 256 / HEAD;                   // P.V: query phases per dim
    constexpr int kQPT = kXQ / kQS;                   // P.V: queries per thread
    extern __shared__ __align__(16) unsigned char lds_raw[];
    float *qs = reinterpret_cast<float *>(lds_raw);                   // [16][HEAD] normalized q
    uint16_t *kv = reinterpret_cast<uint16_t *>(qs + kXQ * HEAD);      // K: [HEAD/8][kXKeys][8]; V: [kXKeys][HEAD]
    float *sc = reinterpret_cast<float *>(kv + kXKeys * HEAD);          // [16][kcap] scores, then e, then weights
    const int tid = static_cast<int>(threadIdx.x), lane = tid & 63, wave = tid >> 6;
    const int h = static_cast<int>(blockIdx.y), s = static_cast<int>(blockIdx.z);
    const int kvh = h / (heads / kv_heads);
    if ((flags[static_cast<size_t>(s) * kv_heads + kvh] != 0) == FINITE) return;
    const int q0 = static_cast<int>(blockIdx.x) * kXQ;
    const int nq = min(kXQ, T - q0);
    const int keys = q0 + nq;                                       // keys 0..keys-1 cover the block
    const int tiles = (keys + kXKeys - 1) / kXKeys, kpad = tiles * kXKeys;
    const float sqrt_head = sqrtf(static_cast<float>(HEAD));
    const uint16_t *kbase = kcache + (static_cast<size_t>(s) * max_context * kv_heads + kvh) * HEAD;
    const uint16_t *vbase = vcache + (static_cast<size_t>(s) * max_context * kv_heads + kvh) * HEAD;
    const size_t kvstride = static_cast<size_t>(kv_heads) * HEAD;
    u32x4_t tile[kPieces];  // plain vectors (an array of the uint4 class would live in scratch)
    // K tile piece e: key e / (HEAD/8), 8 dims (e % (HEAD/8)) of it; V tile piece e: the same key and dims
    auto fetch = [&](const uint16_t *base, int j0) {
#pragma unroll
        for (int i = 0; i < kPieces; ++i) {
            const int e = tid + 256 * i, j = e / (HEAD / 8), piece = e % (HEAD / 8);
            tile[i] = *reinterpret_cast<const u32x4_t *>(base + static_cast<size_t>(min(j0 + j, keys - 1)) * kvstride +
                piece * 8);
        }
    };
    fetch(kbase, 0);
    for (int e = tid; e < kXQ * HEAD; e += 256) {
        const int qi = e / HEAD, d = e % HEAD;
        qs[e] = qi < nq ? q[((static_cast<size_t>(s) * T + q0 + qi) * heads + h) * 2 * HEAD + d] : 0.0f;
    }

    // ---- scores: lane = key, wave = queries wave + 4 r
    for (int t = 0; t < tiles; ++t) {
        __syncthreads();  // the previous tile is consumed (and q is in place)
#pragma unroll
        for (int i = 0; i < kPieces; ++i) {
            const int e = tid + 256 * i, j = e / (HEAD / 8), piece = e % (HEAD / 8);
            *reinterpret_cast<u32x4_t *>(kv + (piece * kXKeys + j) * 8) = tile[i];
        }
        __syncthreads();
        if (t + 1 < tiles) fetch(kbase, (t + 1) * kXKeys);
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int d = 0; d < HEAD; d += 8) {
            const uint4 k8 = *reinterpret_cast<const uint4 *>(kv + ((d / 8) * kXKeys + lane) * 8);
            const uint32_t kw[4] = {k8.x, k8.y, k8.z, k8.w};
            float qv[4][8];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float4 qa = *reinterpret_cast<const float4 *>(qs + (wave + 4 * r) * HEAD + d);
                const float4 qc = *reinterpret_cast<const float4 *>(qs + (wave + 4 * r) * HEAD + d + 4);
                qv[r][0] = qa.x; qv[r][1] = qa.y; qv[r][2] = qa.z; qv[r][3] = qa.w;
                qv[r][4] = qc.x; qv[r][5] = qc.y; qv[r][6] = qc.z; qv[r][7] = qc.w;
            }
            // the four queries' chains interleaved (each chain's order unchanged),
            // so consecutive adds do not wait on each other
#pragma unroll
            for (int k = 0; k < 8; ++k)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[r] = acc[r] + times_half<FINITE>(kw[k >> 1], (k & 1) != 0, qv[r][k]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[(wave + 4 * r) * kcap + t * kXKeys + lane] = acc[r] / sqrt_head;
    }
    fetch(vbase, 0);  // the first value tile, while the weights are formed
    __syncthreads();
    // ---- softmax weights: query wave + 4 r, lanes over keys; e = +0 past the query's keys
    constexpr float kLowest = -3.402823466e38f;  // -huge(1.0_real32)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int qi = wave + 4 * r, n = min(q0 + qi + 1, keys);
        float *row = sc + qi * kcap;
        float m = kLowest;
        for (int j = lane; j < n; j += 64) m = fmaxf(m, row[j]);
        m = wave_max(m);
        for (int j = lane; j < kpad; j += 64) row[j] = j < n ? expf_libm(row[j] - m) : 0.0f;
    }
    __syncthreads();
    // Z of each query by one lane, left to right (the masked keys add +0)
    if (lane < 4) {
        const int qi = wave + 4 * lane;
        const float *row = sc + qi * kcap;
        float z = 0.0f;
        for (int j = 0; j < kpad; j += 4) {
            const float4 e4 = *reinterpret_cast<const float4 *>(row + j);
            z = z + e4.x;
            z = z + e4.y;
            z = z + e4.z;
            z = z + e4.w;
        }
        qs[qi * HEAD] = z;  // q is no longer needed: slot 0 of the row holds Z
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int qi = wave + 4 * r;
        const float z = qs[qi * HEAD];
        float *row = sc + qi * kcap;
        for (int j = lane; j < kpad; j += 64) row[j] = row[j] / z;
    }

    // ---- P.V: thread = (dim d, queries qd + kQS r), keys left to right
    const int d = tid % HEAD, qd = tid / HEAD;
    float acc[kQPT];
#pragma unroll
    for (int r = 0; r < kQPT; ++r) acc[r] = 0.0f;
    for (int t = 0; t < tiles; ++t) {
        __syncthreads();  // the weights are complete / the previous tile is consumed
#pragma unroll
        for (int i = 0; i < kPieces; ++i) {
            const int e = tid + 256 * i, j = e / (HEAD / 8), piece = e % (HEAD / 8);
            *reinterpret_cast<u32x4_t *>(kv + j * HEAD + piece * 8) = tile[i];
        }
        __syncthreads();
        if (t + 1 < tiles) fetch(vbase, (t + 1) * kXKeys);
        for (int jj = 0; jj < kXKeys; jj += 4) {
            uint32_t vh[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) vh[u] = kv[(jj + u) * HEAD + d];
            float4 w4[kQPT];
#pragma unroll
            for (int r = 0; r < kQPT; ++r)
                w4[r] = *reinterpret_cast<const float4 *>(sc + (qd + kQS * r) * kcap + t * kXKeys + jj);
            // the queries' chains interleaved key by key (each chain's order unchanged)
#pragma unroll
            for (int r = 0; r < kQPT; ++r) acc[r] = acc[r] + times_half<FINITE>(vh[0], false, w4[r].x);
#pragma unroll
            for (int r = 0; r < kQPT; ++r) acc[r] = acc[r] + times_half<FINITE>(vh[1], false, w4[r].y);
#pragma unroll
            for (int r = 0; r < kQPT; ++r) acc[r] = acc[r] + times_half<FINITE>(vh[2], false, w4[r].z);
#pragma unroll
            for (int r = 0; r < kQPT; ++r) acc[r] = acc[r] + times_half<FINITE>(vh[3], false, w4[r].w);
        }
    }
#pragma unroll
    for (int r = 0; r < kQPT; ++r) {
        const int qi = qd + kQS * r;
        if (qi >= nq) continue;
        const size_t row = (static_cast<size_t>(s) * T + q0 + qi) * heads + h;
        const float gate = q[row * 2 * HEAD + HEAD + d];
        out[row * HEAD + d] = acc[r] * sigmoid_ref(gate);
    }
}

// Causal attention of every prompt token (fortai_qwen35_cpu.f90:1006-1033
// with an online softmax): one workgroup per (query block of 64, head,
// sequence); four threads per query, each with a quarter of the head dims;
// keys and values staged through LDS 32 positions at a time.  out =
// softmax(q k / sqrt(head)) v * sigmoid(gate).
constexpr int kQBlock = 64;
constexpr int kKTile = 32;

template <int HEAD>
__global__ __launch_bounds__(256) void attention_prefill_kernel(const float *__restrict__ q,
    const uint16_t *__restrict__ kcache, const uint16_t *__restrict__ vcache, const int *__restrict__ flags,
    int only_flagged, float *__restrict__ out, int T, int heads, int kv_heads, int max_context) {
    constexpr int kPart = HEAD / 4;
    constexpr int kPartPitch = kPart + 4;  // the four quarters of a row on different banks
    __shared__ __align__(16) float kt[kKTile][4 * kPartPitch];
    __shared__ __align__(16) float vt[kKTile][4 * kPartPitch];
    const int tid = static_cast<int>(threadIdx.x);
    const int qi = tid >> 2, part = tid & 3;
    const int h = static_cast<int>(blockIdx.y), s = static_cast<int>(blockIdx.z);
    const int q0 = static_cast<int>(blockIdx.x) * kQBlock;
    const int t = min(q0 + qi, T - 1);
    const int kvh = h / (heads / kv_heads);
    // after the matrix-core kernel: only the (sequence, kv head) pairs whose
    // cache holds exponent-31 halves, which that kernel leaves to this one
    if (only_flagged && flags[static_cast<size_t>(s) * kv_heads + kvh] == 0) return;
    const float *qrow = q + ((static_cast<size_t>(s) * T + t) * heads + h) * 2 * HEAD;
    float qv[kPart], o[kPart];
#pragma unroll
    for (int d = 0; d < kPart; ++d) {
        qv[d] = qrow[part * kPart + d];
        o[d] = 0.0f;
    }
    const float scale = 1.0f / sqrtf(static_cast<float>(HEAD));
    float m = -__builtin_inff(), z = 0.0f;
    const int last = min(q0 + kQBlock, T) - 1;  // keys 0..last cover the block
    for (int j0 = 0; j0 <= last; j0 += kKTile) {
        __syncthreads();
        for (int e = tid; e < kKTile * HEAD; e += 256) {
            const int j = e / HEAD, d = e % HEAD;
            const int p = min(j0 + j, last);
            const size_t off = ((static_cast<size_t>(s) * max_context + p) * kv_heads + kvh) * HEAD + d;
            const int dd = (d / kPart) * kPartPitch + d % kPart;
            kt[j][dd] = gguf_half_to_real(kcache[off]);
            vt[j][dd] = gguf_half_to_real(vcache[off]);
        }
        __syncthreads();
        const int jn = min(kKTile, t - j0 + 1);  // keys of this query in the tile
        for (int j = 0; j < kKTile; ++j) {
            float sc = 0.0f;
#pragma unroll
            for (int d = 0; d < kPart; ++d) sc = __builtin_fmaf(qv[d], kt[j][part * kPartPitch + d], sc);
            sc += __shfl_xor(sc, 1);
            sc += __shfl_xor(sc, 2);
            if (j >= jn) continue;  // masked (uniform per query: the 4 threads agree)
            sc *= scale;
            // online softmax; the running sums are rescaled only when the
            // maximum grows (within the fp32 tolerance of this path)
            if (sc > m) {
                const float corr = __expf(m - sc);
                z *= corr;
#pragma unroll
                for (int d = 0; d < kPart; ++d) o[d] *= corr;
                m = sc;
            }
            const float p = __expf(sc - m);
            z += p;
#pragma unroll
            for (int d = 0; d < kPart; ++d) o[d] = __builtin_fmaf(p, vt[j][part * kPartPitch + d], o[d]);
        }
    }
    if (q0 + qi >= T) return;
    const float *gate = qrow + HEAD;
    float *orow = out + ((static_cast<size_t>(s) * T + t) * heads + h) * HEAD;
#pragma unroll
    for (int d = 0; d < kPart; ++d) {
        const int dd = part * kPart + d;
        orow[dd] = (o[d] / z) * sigmoid_ref(gate[dd]);
    }
}

// The same causal attention on the fp16 matrix cores (the default prefill
// mode, within its tolerance): one workgroup per (32-query block, kv head,
// sequence), wave w taking q head kvh * group + w.  Per 32-key tile,
//   S^T = K Q^T  (v_mfma_f32_32x32x16_f16, keys x queries, q pre-scaled by
//                 1/sqrt(head) and rounded to fp16; K is the fp16 cache),
// an online softmax in fp32 (__expf; the running sums rescaled when a
// query's reference maximum moves, which it does only by jumps of more than
// 8), and
//   O^T += V^T P^T (the same instruction, dims x queries, P rounded to fp16).
// The accumulator of a 32x32 MFMA holds, in element i of lane l, row
// 8*(i/4) + 4*(l/32) + i%4 and column l%32: with keys and dims as rows and
// queries as columns, every value of a query stays in lanes l%32 == query,
// so the softmax rescale is a per-lane scalar, and the 16 probabilities of a
// lane are the B operand of the two P.V instructions of the tile as they are
// (A and B present the same keys in the same slots; which k the instruction
// assigns to a slot does not change the sum).  K reaches LDS key-major (the
// A operand of S^T: 16 bytes of one key per lane), V dim-major (the A operand
// of O^T: two 8-byte runs of keys per lane).  A (sequence, kv head) whose
// cache holds exponent-31 halves is left to attention_prefill_kernel.
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
constexpr int kMfmaQ = 32;  // queries per workgroup (one MFMA column block)
constexpr int kMfmaK = 32;  // keys per tile

template <int HEAD>
__global__ __launch_bounds__(256) void attention_prefill_mfma_kernel(const float *__restrict__ q,
    const uint16_t *__restrict__ kcache, const uint16_t *__restrict__ vcache, const int *__restrict__ flags,
    float *__restrict__ out, int T, int heads, int kv_heads, int max_context) {
    static_assert(HEAD % 64 == 0, "whole 16-byte pieces per thread and tile");
    constexpr int kKPitch = HEAD + 8;             // halves per K row (key-major)
    constexpr int kVPitch = kMfmaK + 8;           // halves per V^T row (dim-major)
    constexpr int kSteps = HEAD / 16;             // k-steps of S^T
    constexpr int kDT = HEAD / 32;                // 32-dim tiles of O^T
    constexpr int kPieces = HEAD / 8;             // 16-byte pieces of a key row
    constexpr int kLoads = kMfmaK * kPieces / 256;  // pieces per thread and tile (K and V each)
    extern __shared__ __align__(16) _Float16 mfma_lds[];
    _Float16 *kt = mfma_lds;                                   // [kMfmaK][kKPitch]
    _Float16 *vt = kt + kMfmaK * kKPitch;                      // [HEAD][kVPitch]
    _Float16 *qs = vt + HEAD * kVPitch;                        // [4 waves][kMfmaQ][kKPitch]
    const int tid = static_cast<int>(threadIdx.x), wave = tid >> 6, lane = tid & 63;
    const int col = lane & 31, g = lane >> 5;
    const int kvh = static_cast<int>(blockIdx.y), s = static_cast<int>(blockIdx.z);
    const int q0 = static_cast<int>(blockIdx.x) * kMfmaQ;
    if (flags[static_cast<size_t>(s) * kv_heads + kvh] != 0) return;
    const int group = heads / kv_heads;
    const bool active = wave < group;
    const int h = kvh * group + (active ? wave : 0);
    const int qq = q0 + col;                       // this lane's query
    const int qt = min(qq, T - 1);
    const float *qrow = q + ((static_cast<size_t>(s) * T + qt) * heads + h) * 2 * HEAD;
    // the wave's 32 query rows, scaled by 1/sqrt(head), in fp16 (the B
    // operand of S^T, read from LDS each tile): lane l writes dims
    // 4 * (l % kPieces4) .. of rows l / kPieces4, l / kPieces4 + 64 / kPieces4, ...
    _Float16 *qw = qs + wave * kMfmaQ * kKPitch;
    {
        const float scale = 1.0f / sqrtf(static_cast<float>(HEAD));
        constexpr int kPieces4 = HEAD / 4;  // float4 pieces of a q row
        for (int e = lane; e < kMfmaQ * kPieces4; e += 64) {
            const int r = e / kPieces4, c4 = e % kPieces4;
            const int t = min(q0 + r, T - 1);
            const float4 a = *reinterpret_cast<const float4 *>(
                q + ((static_cast<size_t>(s) * T + t) * heads + h) * 2 * HEAD + c4 * 4);
            const half4_t v = {static_cast<_Float16>(a.x * scale), static_cast<_Float16>(a.y * scale),
                static_cast<_Float16>(a.z * scale), static_cast<_Float16>(a.w * scale)};
            *reinterpret_cast<half4_t *>(qw + r * kKPitch + c4 * 4) = v;
        }
    }
    const int last = min(q0 + kMfmaQ, T) - 1;      // keys 0..last cover the block
    const int ntiles = last / kMfmaK + 1;
    u32x4_t kr[kLoads], vr[kLoads];
    // K pieces key-major (consecutive lanes: consecutive 16 bytes of a key
    // row); V pieces key-minor (consecutive lanes: consecutive keys), so that
    // each transposed 2-byte LDS store of a wave covers 32 consecutive keys
    // of one dim row (no bank conflicts)
    auto fetch = [&](int j0) {
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int li = tid + 256 * j;
            const int kkey = li / kPieces, kpc = li % kPieces;
            const int vkey = li % kMfmaK, vpc = li / kMfmaK;
            const size_t base = (static_cast<size_t>(s) * max_context) * kv_heads + kvh;
            kr[j] = *reinterpret_cast<const u32x4_t *>(
                kcache + (base + static_cast<size_t>(min(j0 + kkey, last)) * kv_heads) * HEAD + kpc * 8);
            vr[j] = *reinterpret_cast<const u32x4_t *>(
                vcache + (base + static_cast<size_t>(min(j0 + vkey, last)) * kv_heads) * HEAD + vpc * 8);
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int li = tid + 256 * j;
            const int kkey = li / kPieces, kpc = li % kPieces;
            const int vkey = li % kMfmaK, vpc = li / kMfmaK;
            *reinterpret_cast<u32x4_t *>(kt + kkey * kKPitch + kpc * 8) = kr[j];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                vt[(vpc * 8 + 2 * e) * kVPitch + vkey] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(vr[j][e] & 0xffffu));
                vt[(vpc * 8 + 2 * e + 1) * kVPitch + vkey] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(vr[j][e] >> 16));
            }
        }
    };
    float16_t o[kDT];
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt) o[dt] = float16_t{};
    float m = -__builtin_inff(), zl = 0.0f;
    fetch(0);
    for (int t = 0; t < ntiles; ++t) {
        const int j0 = t * kMfmaK;
        __syncthreads();  // every wave is done with the previous tile
        stash();
        __syncthreads();
        if (t + 1 < ntiles) fetch(j0 + kMfmaK);
        if (!active) continue;
        float16_t sc = float16_t{};
#pragma unroll
        for (int kk = 0; kk < kSteps; ++kk) {
            const half8_t a = *reinterpret_cast<const half8_t *>(kt + col * kKPitch + kk * 16 + g * 8);
            const half8_t b = *reinterpret_cast<const half8_t *>(qw + col * kKPitch + kk * 16 + g * 8);
            sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, sc, 0, 0, 0);
        }
        // element i: key j0 + 8 * (i / 4) + 4 * g + i % 4 of query qq
        float tmax = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int key = j0 + 8 * (i / 4) + 4 * g + (i % 4);
            if (key > qq || key >= T) sc[i] = -__builtin_inff();
            tmax = fmaxf(tmax, sc[i]);
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        // the reference maximum m of a query moves only when a score exceeds
        // it by more than 8 (probabilities stay <= e^8, well inside fp16), so
        // the sums are rescaled on few tiles: the first, and big jumps
        const bool grow = tmax > m + 8.0f;
        if (__any(grow)) {
            const float mnew = grow ? tmax : m;
            const float corr = __expf(m - mnew);  // 0 on the first tile (m = -inf), 1 where m stays
            m = mnew;
            zl *= corr;
#pragma unroll
            for (int dt = 0; dt < kDT; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[dt][i] *= corr;
        }
        // the denominator sums the same fp16-rounded probabilities the P.V
        // products use, so numerator and denominator round alike
        float pl[16];
        float zt = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            pl[i] = sc[i] == -__builtin_inff() ? 0.0f : __expf(sc[i] - m);
            zt += static_cast<float>(static_cast<_Float16>(pl[i]));
        }
        zl += zt;
        const half8_t pb0 = {static_cast<_Float16>(pl[0]), static_cast<_Float16>(pl[1]), static_cast<_Float16>(pl[2]),
            static_cast<_Float16>(pl[3]), static_cast<_Float16>(pl[4]), static_cast<_Float16>(pl[5]),
            static_cast<_Float16>(pl[6]), static_cast<_Float16>(pl[7])};
        const half8_t pb1 = {static_cast<_Float16>(pl[8]), static_cast<_Float16>(pl[9]), static_cast<_Float16>(pl[10]),
            static_cast<_Float16>(pl[11]), static_cast<_Float16>(pl[12]), static_cast<_Float16>(pl[13]),
            static_cast<_Float16>(pl[14]), static_cast<_Float16>(pl[15])};
#pragma unroll
        for (int dt = 0; dt < kDT; ++dt) {
            const _Float16 *vrow = vt + (dt * 32 + col) * kVPitch + 4 * g;
            const half4_t v0 = *reinterpret_cast<const half4_t *>(vrow);
            const half4_t v1 = *reinterpret_cast<const half4_t *>(vrow + 8);
            const half4_t v2 = *reinterpret_cast<const half4_t *>(vrow + 16);
            const half4_t v3 = *reinterpret_cast<const half4_t *>(vrow + 24);
            const half8_t va0 = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
            const half8_t va1 = {v2[0], v2[1], v2[2], v2[3], v3[0], v3[1], v3[2], v3[3]};
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va0, pb0, o[dt], 0, 0, 0);
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va1, pb1, o[dt], 0, 0, 0);
        }
    }
    if (!active || qq >= T) return;
    // the gate: 1 / (1 + e^-g) with the hardware exp and reciprocal (this
    // mode's tolerance; the exact mode's kernel uses the reference sigmoid),
    // and one reciprocal of Z per query
    const float zi = __builtin_amdgcn_rcpf(zl + __shfl_xor(zl, 32));
    const float *gate = qrow + HEAD;
    float *orow = out + ((static_cast<size_t>(s) * T + qq) * heads + h) * HEAD;
    auto sig = [](float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); };
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int d = dt * 32 + 8 * r + 4 * g;
            const float4 gt = *reinterpret_cast<const float4 *>(gate + d);
            float4 v;
            v.x = (o[dt][4 * r + 0] * zi) * sig(gt.x);
            v.y = (o[dt][4 * r + 1] * zi) * sig(gt.y);
            v.z = (o[dt][4 * r + 2] * zi) * sig(gt.z);
            v.w = (o[dt][4 * r + 3] * zi) * sig(gt.w);
            *reinterpret_cast<float4 *>(orow + d) = v;
        }
    }
}

// Rows [r0, r0 + count) of X8 -> the matvec's Q8L layout [count][q8l_bytes]
// (the same quantized values: used by the exact prefill mode).
__global__ __launch_bounds__(256) void x8_to_q8l_kernel(const int8_t *__restrict__ xq, const float *__restrict__ xs,
    int ld, int chunks, int r0, uint32_t *__restrict__ q8l) {
    const int rr = static_cast<int>(blockIdx.y), n = r0 + rr;
    uint32_t *dst = q8l + static_cast<size_t>(rr) * chunks * 36;
    for (int e = static_cast<int>(threadIdx.x); e < chunks * 36; e += 256) {
        if (e < chunks * 32) {
            const int c = e >> 5, l = (e >> 2) & 7, j = e & 3, b = 4 * c + j;
            dst[e] = reinterpret_cast<const uint32_t *>(xq + (static_cast<size_t>(b) * ld + n) * 32)[l];
        } else {
            const int b = e - chunks * 32;
            reinterpret_cast<float *>(dst)[e] = xs[static_cast<size_t>(b) * ld + n];
        }
    }
}

void x8_planes(void *x8, int tokens, int width, int8_t *&xq, float *&xs, int &ld, int &blocks_pad) {
    ld = q8_tokens_ld(tokens);
    blocks_pad = (width / kQ8Block + 3) / 4 * 4;
    xq = static_cast<int8_t *>(x8);
    xs = reinterpret_cast<float *>(xq + static_cast<size_t>(ld) * blocks_pad * 32);
}

}  // namespace

hipError_t launch_x8_to_q8l(const void *x8, int tokens, int width, int r0, int count, void *q8l, hipStream_t stream) {
    if (r0 < 0 || count < 1 || r0 + count > tokens || width % kQ8Block) return hipErrorInvalidValue;
    int8_t *xq; float *xs; int ld, bp;
    x8_planes(const_cast<void *>(x8), tokens, width, xq, xs, ld, bp);
    hipLaunchKernelGGL(x8_to_q8l_kernel, dim3(1, count), dim3(256), 0, stream, xq, xs, ld, bp / 4, r0,
        static_cast<uint32_t *>(q8l));
    note_launch("x8_to_q8l_kernel grid 1x%d", count);
    return hipGetLastError();
}

hipError_t launch_rms_quantize_tokens(const float *x, int rows, int width, const float *norm, float eps, void *x8,
    hipStream_t stream) {
    if (rows <= 0 || width <= 0 || width % kQ8Block) return hipErrorInvalidValue;
    int8_t *xq; float *xs; int ld, bp;
    x8_planes(x8, rows, width, xq, xs, ld, bp);
    hipLaunchKernelGGL(rms_quantize_tokens_kernel, dim3(rows), dim3(kRowThreads), 0, stream, x, width, width, norm, eps,
        ld, bp, xq, xs);
    note_launch("rms_quantize_tokens_kernel<%s> grid %d", norm ? "rmsnorm" : "f32", rows);
    return hipGetLastError();
}

hipError_t launch_gated_quantize_tokens(const float *o, const float *z, const float *norm, float eps, int rows,
    int width, int head, void *x8, hipStream_t stream) {
    const int hl = head / 4;
    if (rows <= 0 || width % kQ8Block || head % 4 || hl > 64 || (hl & (hl - 1)) || width % head) return hipErrorInvalidValue;
    int8_t *xq; float *xs; int ld, bp;
    x8_planes(x8, rows, width, xq, xs, ld, bp);
    hipLaunchKernelGGL(gated_quantize_tokens_kernel, dim3(rows), dim3(kRowThreads), 0, stream, o, z, norm, eps, width,
        head, ld, bp, xq, xs);
    note_launch("gated_quantize_tokens_kernel grid %d", rows);
    return hipGetLastError();
}

hipError_t launch_silu_product_quantize(const float *gate, const float *up, int rows, int width, void *x8,
    hipStream_t stream) {
    if (rows <= 0 || width % kQ8Block) return hipErrorInvalidValue;
    int8_t *xq; float *xs; int ld, bp;
    x8_planes(x8, rows, width, xq, xs, ld, bp);
    hipLaunchKernelGGL(silu_product_quantize_kernel, dim3(rows), dim3(kRowThreads), 0, stream, gate, up, width, ld, bp,
        xq, xs);
    note_launch("silu_product_quantize_kernel grid %d", rows);
    return hipGetLastError();
}

hipError_t launch_conv_silu_tokens(const float *x, const float *conv_w, float *conv_state, float *out, int batch, int T,
    int C, int K, hipStream_t stream) {
    if (batch < 1 || T < 1 || C < 1 || K < 2 || K > kConvMax) return hipErrorInvalidValue;
    const int cb = (C + 255) / 256, tb = (T + kConvTokens - 1) / kConvTokens;
    hipLaunchKernelGGL(conv_silu_tokens_kernel, dim3(cb, tb, batch), dim3(256), 0, stream, x, conv_w, conv_state, out,
        T, C, K);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(conv_state_advance_kernel, dim3(cb, batch), dim3(256), 0, stream, x, conv_state, T, C, K);
    note_launch("conv_silu_tokens_kernel grid %dx%dx%d + conv_state_advance_kernel grid %dx%d", cb, tb, batch, cb, batch);
    return hipGetLastError();
}

hipError_t launch_gdn_prefill(const GdnParams &p, int batch, int T, float *qinv, float *kinv, float *beta_t,
    float *decay_t, hipStream_t stream) {
    if (batch < 1 || T < 1 || p.key_heads <= 0 || p.value_heads % p.key_heads || p.state_size != p.head)
        return hipErrorInvalidValue;
    const int C = 2 * p.state_size * p.key_heads + p.value_heads * p.head;
    const int rows = batch * T;
    hipLaunchKernelGGL(gdn_token_prep_kernel, dim3(rows), dim3(256), 0, stream, p.qkv, p.alpha, p.beta, p.ssm_a,
        p.ssm_dt, C, p.key_heads, p.value_heads, p.head, p.state_size, p.eps, qinv, kinv, beta_t, decay_t);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 grid(p.value_heads * (p.head / kGdnRows), batch);
    switch (p.head) {
    case 64:
        hipLaunchKernelGGL(gdn_prefill_kernel<64>, grid, dim3(kGdnRows * 8), 0, stream, p.qkv, qinv, kinv, beta_t,
            decay_t, p.state, p.out, T, C, p.key_heads, p.value_heads, p.state_size);
        break;
    case 128:
        hipLaunchKernelGGL(gdn_prefill_kernel<128>, grid, dim3(kGdnRows * 8), 0, stream, p.qkv, qinv, kinv, beta_t,
            decay_t, p.state, p.out, T, C, p.key_heads, p.value_heads, p.state_size);
        break;
    default: return hipErrorInvalidValue;
    }
    note_launch("gdn_token_prep_kernel grid %d + gdn_prefill_kernel<%d> grid %dx%d", rows, p.head, grid.x, batch);
    return hipGetLastError();
}

hipError_t launch_attention_prefill(const AttentionParams &p, int batch, int T, float *out, hipStream_t stream,
    bool matrix_cores) {
    // every head width a kernel below is instantiated for; checked before
    // anything is enqueued, so an unsupported layer launches nothing
    if (batch < 1 || T < 1 || T > p.max_context || p.heads % p.kv_heads || p.head != p.value ||
        p.rope_dim > p.head || (p.head != 64 && p.head != 128 && p.head != 256))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(qk_rope_append_kernel, dim3(batch * T), dim3(256), 0, stream, const_cast<float *>(p.q), p.k,
        p.v, p.q_norm, p.k_norm, p.rope, p.kcache, p.vcache, p.cache_flags, T, p.heads, p.kv_heads, p.head, p.value,
        p.rope_dim, p.max_context, p.eps);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // the matrix-core kernel: head 64, 128 or 256, a GQA group of <= 4
    // (one wave per q head); it leaves the flagged (sequence, kv head) pairs
    // to the fp32 kernel below
    const bool mfma = matrix_cores && p.heads / p.kv_heads <= 4;
    if (mfma) {
        const dim3 mgrid((T + kMfmaQ - 1) / kMfmaQ, p.kv_heads, batch);
        // K tile, V^T tile and four waves' q rows, fp16
        const size_t mlds = static_cast<size_t>(kMfmaK * (p.head + 8) + p.head * (kMfmaK + 8) + 4 * kMfmaQ * (p.head + 8)) *
            sizeof(_Float16);
        switch (p.head) {
        case 64:
            hipLaunchKernelGGL(attention_prefill_mfma_kernel<64>, mgrid, dim3(256), mlds, stream, p.q, p.kcache, p.vcache,
                p.cache_flags, out, T, p.heads, p.kv_heads, p.max_context);
            break;
        case 128:
            hipLaunchKernelGGL(attention_prefill_mfma_kernel<128>, mgrid, dim3(256), mlds, stream, p.q, p.kcache,
                p.vcache, p.cache_flags, out, T, p.heads, p.kv_heads, p.max_context);
            break;
        case 256:
            hipLaunchKernelGGL(attention_prefill_mfma_kernel<256>, mgrid, dim3(256), mlds, stream, p.q, p.kcache,
                p.vcache, p.cache_flags, out, T, p.heads, p.kv_heads, p.max_context);
            break;
        }
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (!matrix_cores) {
        // 16 queries per workgroup when the block's scores fit in LDS (two
        // launches: caches without and with exponent-31 halves)
        const int kpad = (T + kXKeys - 1) / kXKeys * kXKeys;
        const size_t lds16 = static_cast<size_t>(kXQ) * p.head * 4 + static_cast<size_t>(kXKeys) * p.head * 2 +
            static_cast<size_t>(kXQ) * kpad * 4;
        if (lds16 <= 80 * 1024) {
            const dim3 xgrid((T + kXQ - 1) / kXQ, p.heads, batch);
#define FORTAI_PREX(H)                                                                                              \
    do {                                                                                                            \
        hipLaunchKernelGGL((attention_prefill_exact16_kernel<H, true>), xgrid, dim3(256), lds16, stream, p.q,       \
            p.kcache, p.vcache, p.cache_flags, out, T, p.heads, p.kv_heads, p.max_context, kpad);                   \
        hipLaunchKernelGGL((attention_prefill_exact16_kernel<H, false>), xgrid, dim3(256), lds16, stream, p.q,      \
            p.kcache, p.vcache, p.cache_flags, out, T, p.heads, p.kv_heads, p.max_context, kpad);                   \
    } while (0)
            switch (p.head) {
            case 64: FORTAI_PREX(64); break;
            case 128: FORTAI_PREX(128); break;
            case 256: FORTAI_PREX(256); break;
            default: return hipErrorInvalidValue;
            }
#undef FORTAI_PREX
            note_launch("qk_rope_append_kernel grid %d + attention_prefill_exact16_kernel<%d> grid %dx%dx%d (x2)",
                batch * T, p.head, xgrid.x, xgrid.y, xgrid.z);
            return hipGetLastError();
        }
        // longer prompts: queries per workgroup so that the block's scores fit in LDS
        const int kcap = (T + 3) / 4 * 4;
        int qb = 16;
        auto lds_of = [&](int b) {
            return static_cast<size_t>(b) * p.head * 4 + static_cast<size_t>(kXKeys) * p.head * 2 +
                static_cast<size_t>(b) * kcap * 4;
        };
        while (qb > 1 && lds_of(qb) > 150 * 1024) qb /= 2;
        if (lds_of(qb) > 150 * 1024) return hipErrorInvalidValue;
        const dim3 xgrid((T + qb - 1) / qb, p.heads, batch);
        switch (p.head) {
        case 64:
            hipLaunchKernelGGL(attention_prefill_exact_kernel<64>, xgrid, dim3(256), lds_of(qb), stream, p.q, p.kcache,
                p.vcache, out, T, p.heads, p.kv_heads, p.max_context, qb, kcap);
            break;
        case 128:
            hipLaunchKernelGGL(attention_prefill_exact_kernel<128>, xgrid, dim3(256), lds_of(qb), stream, p.q, p.kcache,
                p.vcache, out, T, p.heads, p.kv_heads, p.max_context, qb, kcap);
            break;
        case 256:
            hipLaunchKernelGGL(attention_prefill_exact_kernel<256>, xgrid, dim3(256), lds_of(qb), stream, p.q, p.kcache,
                p.vcache, out, T, p.heads, p.kv_heads, p.max_context, qb, kcap);
            break;
        default: return hipErrorInvalidValue;
        }
        note_launch("qk_rope_append_kernel grid %d + attention_prefill_exact_kernel<%d> grid %dx%dx%d", batch * T, p.head,
            xgrid.x, xgrid.y, xgrid.z);
        return hipGetLastError();
    }
    const int only_flagged = mfma ? 1 : 0;
    const dim3 grid((T + kQBlock - 1) / kQBlock, p.heads, batch);
    switch (p.head) {
    case 64:
        hipLaunchKernelGGL(attention_prefill_kernel<64>, grid, dim3(256), 0, stream, p.q, p.kcache, p.vcache,
            p.cache_flags, only_flagged, out, T, p.heads, p.kv_heads, p.max_context);
        break;
    case 128:
        hipLaunchKernelGGL(attention_prefill_kernel<128>, grid, dim3(256), 0, stream, p.q, p.kcache, p.vcache,
            p.cache_flags, only_flagged, out, T, p.heads, p.kv_heads, p.max_context);
        break;
    case 256:
        hipLaunchKernelGGL(attention_prefill_kernel<256>, grid, dim3(256), 0, stream, p.q, p.kcache, p.vcache,
            p.cache_flags, only_flagged, out, T, p.heads, p.kv_heads, p.max_context);
        break;
    default: return hipErrorInvalidValue;
    }
    if (mfma)
        note_launch("qk_rope_append_kernel grid %d + attention_prefill_mfma_kernel<%d> grid %dx%dx%d + "
            "attention_prefill_kernel<%d> (exponent-31 caches only) grid %dx%dx%d", batch * T, p.head,
            (T + kMfmaQ - 1) / kMfmaQ, p.kv_heads, batch, p.head, grid.x, grid.y, grid.z);
    else
        note_launch("qk_rope_append_kernel grid %d + attention_prefill_kernel<%d> grid %dx%dx%d", batch * T, p.head,
            grid.x, grid.y, grid.z);
    return hipGetLastError();
}

}  // namespace fortai_hip
