/*
 * fortai_oracle.c -- CPU restatement of FortAI's Qwen3.5 Q8_0 decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline); the product path (libfortai_hip.so) never
 * links or calls it.
 *
 * It restates, operation for operation, the reference CPU path as the
 * reference dispatches it on an AVX2+F16C host:
 *   src/backend/cpu/fortai_q8_dot.c        (quantize, dot, GDN step, SiLU, fp16)
 *   src/fortai_gguf_runtime.f90            (GGUF load, value(), matvec_q8, F16 dot)
 *   src/models/qwen35/fortai_qwen35_cpu.f90 (the decode step)
 * Vector lanes are emulated with scalar arrays in the same lane order and the
 * same reduction tree, so results are bit-identical to the reference built by
 * oracle/Makefile (-O2 -ffp-contract=off, no -march: multiply and add are
 * separately rounded except where the reference calls an FMA intrinsic).
 *
 * Parity pinning of every function is listed in the header comment of
 * oracle/oracle.py.
 */
#define _GNU_SOURCE
#include <fcntl.h>
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define Q8_BLOCK 32
#define Q8_BYTES 34

static inline float f_from_bits(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t bits_from_f(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* ------------------------------------------------------------------ fp16 -- */

/* fortai_q8_dot.c:53-83 (exact widening; exp 31 keeps inf/NaN) */
float orc_half_to_float(uint16_t h)
{
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    const uint32_t m = (uint32_t)h & 0x3ffu;
    if (e == 0u) {
        if (m == 0u) return f_from_bits(sign);
        /* subnormal half: m * 2^-24 is exact in float */
        float v = (float)m * 0x1p-24f;
        return sign ? -v : v;
    }
    if (e == 31u) return f_from_bits(sign | 0x7f800000u | (m << 13));
    return f_from_bits(sign | ((e + 112u) << 23) | (m << 13));
}

/* fortai_q8_dot.c:85-113: truncating conversion that adds one half-ulp when
 * bit 12 of the float fraction is set (ties and above round away from zero);
 * the subnormal branch tests bit 12 of the *unshifted* fraction; overflow
 * gives inf and NaN inputs also map to inf. */
uint16_t orc_float_to_half(float value)
{
    const uint32_t bits = bits_from_f(value);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    int32_t exponent = (int32_t)((bits >> 23) & 0xffu) - 127 + 15;
    uint32_t fraction = bits & 0x007fffffu;
    if (exponent <= 0) {
        if (exponent < -10) return (uint16_t)sign;
        fraction = (fraction | 0x00800000u) >> (uint32_t)(1 - exponent);
        if (bits & 0x00001000u) fraction += 0x00002000u;
        return (uint16_t)(sign | (fraction >> 13));
    }
    if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
    if (fraction & 0x00001000u) {
        fraction += 0x00002000u;
        if (fraction & 0x00800000u) {
            fraction = 0;
            if (++exponent >= 31) return (uint16_t)(sign | 0x7c00u);
        }
    }
    return (uint16_t)(sign | ((uint32_t)exponent << 10) | (fraction >> 13));
}

/* IEEE binary32 -> binary16, round to nearest even, as F16C vcvtps2ph with
 * _MM_FROUND_TO_NEAREST_INT (used by the AVX2 quantizer, fortai_q8_dot.c:176). */
uint16_t orc_f32_to_f16_rne(float f)
{
    const uint32_t x = bits_from_f(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    const uint32_t e = ax >> 23;
    if (e < 113u) { /* result is a half subnormal (or rounds up to the smallest normal) */
        const uint64_t m = (ax & 0x7fffffu) | (e ? 0x800000u : 0u);
        const uint32_t s = (e ? 126u - e : 125u);
        if (s > 40u) return (uint16_t)sign;
        uint64_t q = m >> s;
        const uint64_t r = m & ((1ull << s) - 1ull);
        const uint64_t half = 1ull << (s - 1u);
        if (r > half || (r == half && (q & 1u))) ++q;
        return (uint16_t)(sign | (uint32_t)q);
    }
    if (e > 142u) return (uint16_t)(sign | 0x7c00u);
    uint32_t q = (ax & 0x7fffffu) >> 13;
    const uint32_t r = ax & 0x1fffu;
    uint32_t h = ((e - 112u) << 10);
    if (r > 0x1000u || (r == 0x1000u && (q & 1u))) ++q;
    h += q; /* a carry out of the mantissa increments the exponent; 31 is inf */
    if (h >= 0x7c00u) h = 0x7c00u;
    return (uint16_t)(sign | h);
}

/* fortai_gguf_runtime.f90:770-788: subnormals as fraction/1024*2^-14, exponent
 * 31 decodes to +-huge (no inf/NaN). */
float orc_gguf_fp16_to_real(uint16_t h)
{
    const uint32_t e = ((uint32_t)h >> 10) & 31u;
    const uint32_t m = (uint32_t)h & 1023u;
    float v;
    if (e == 0u) v = ((float)m / 1024.0f) * 0x1p-14f;
    else if (e == 31u) v = FLT_MAX;
    else v = (1.0f + (float)m / 1024.0f) * ldexpf(1.0f, (int)e - 15);
    return (h & 0x8000u) ? -v : v;
}

/* ------------------------------------------------------------ Q8_0 ops -- */

static inline int8_t sat8(int32_t v) { return (int8_t)(v < -128 ? -128 : (v > 127 ? 127 : v)); }
static inline int32_t cvt_rne_i32(float v)
{
    /* _mm256_cvtps_epi32(_mm256_round_ps(v, nearest)): out of range or NaN
     * gives INT32_MIN ("integer indefinite"). */
    const float r = rintf(v);
    if (!(r >= -2147483648.0f && r < 2147483648.0f)) return INT32_MIN;
    return (int32_t)r;
}
static inline int16_t sat16(int32_t v) { return (int16_t)(v < -32768 ? -32768 : (v > 32767 ? 32767 : v)); }

/* fortai_q8_dot.c:153-198 (AVX2 path, the one fortai_q8_quantize dispatches
 * at :200-213 on AVX2+F16C hosts).  Output: count/32 blocks of
 * [fp16 scale][32 x int8]; scales[b] = float(fp16 scale). */
void orc_q8_quantize(const float *input, int8_t *output, float *scales, int64_t count)
{
    if (count <= 0 || count % 32 != 0) return;
    for (int64_t offset = 0; offset < count; offset += 32) {
        int8_t *out = output + (offset / 32) * Q8_BYTES;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) {
            const float a = fabsf(input[offset + i]);
            amax = (amax > a) ? amax : a; /* max_ps(amax, a) */
        }
        const float scale = amax / 127.0f;
        const float inverse = amax != 0.0f ? 127.0f / amax : 0.0f;
        const uint16_t sb = orc_f32_to_f16_rne(scale);
        scales[offset / 32] = orc_half_to_float(sb);
        memcpy(out, &sb, 2);
        for (int i = 0; i < 32; ++i)
            out[2 + i] = sat8(sat16(cvt_rne_i32(input[offset + i] * inverse)));
    }
}

/* fortai_q8_dot.c:230-248 */
void orc_q8_dequantize_row(const int8_t *weights, float *output, int64_t block_count)
{
    for (int64_t b = 0; b < block_count; ++b) {
        uint16_t sb;
        memcpy(&sb, weights + b * Q8_BYTES, 2);
        const float s = orc_half_to_float(sb);
        for (int i = 0; i < 32; ++i)
            output[b * 32 + i] = s * (float)weights[b * Q8_BYTES + 2 + i];
    }
}

/* One 32-bit lane of maddubs(|w|, sign(a,w)) + madd(.,1): the int32 sum of
 * products 4l..4l+3 with the int16 pair saturation of vpmaddubsw
 * (fortai_q8_dot.c:313-318). */
static inline int32_t lane_dot(const int8_t *w, const int8_t *a, int l)
{
    int32_t lane = 0;
    for (int p = 0; p < 2; ++p) {
        int32_t pair = 0;
        for (int j = 0; j < 2; ++j) {
            const int8_t wv = w[4 * l + 2 * p + j], av = a[4 * l + 2 * p + j];
            const uint8_t absw = (uint8_t)(wv < 0 ? (int8_t)(-(int32_t)wv) : wv); /* psignb(w,w) */
            const int8_t sa = wv > 0 ? av : (wv < 0 ? (int8_t)(-(int32_t)av) : 0); /* psignb(a,w) */
            pair += (int32_t)absw * (int32_t)sa;
        }
        lane += sat16(pair);
    }
    return lane;
}

/* fortai_q8_dot.c:287-331: 8 fp32 lane accumulators, acc = fma(sw*sa, lane, acc)
 * per block, then the fixed horizontal sum (lo+hi, +movehl, +movehdup). */
float orc_q8_dot(const int8_t *weights, const int8_t *quantized, const float *scales,
    int64_t row, int64_t block_count)
{
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const int8_t *rs = weights + row * block_count * Q8_BYTES;
    for (int64_t b = 0; b < block_count; ++b) {
        uint16_t sb;
        memcpy(&sb, rs + b * Q8_BYTES, 2);
        const float sc = orc_half_to_float(sb) * scales[b];
        for (int l = 0; l < 8; ++l)
            acc[l] = fmaf(sc, (float)lane_dot(rs + b * Q8_BYTES + 2, quantized + b * Q8_BYTES + 2, l), acc[l]);
    }
    const float s0 = acc[0] + acc[4], s1 = acc[1] + acc[5], s2 = acc[2] + acc[6], s3 = acc[3] + acc[7];
    return (s0 + s2) + (s1 + s3);
}

/* Per-block int32 dots sum_i w_i*a_i (the quantity the parity gate requires
 * bit-exact), out[row*block_count + b]. */
void orc_q8_block_dots(const int8_t *weights, const int8_t *quantized, int64_t rows,
    int64_t block_count, int32_t *out)
{
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < block_count; ++b) {
            const int8_t *w = weights + (r * block_count + b) * Q8_BYTES + 2;
            const int8_t *a = quantized + b * Q8_BYTES + 2;
            int32_t d = 0;
            for (int i = 0; i < 32; ++i) d += (int32_t)w[i] * (int32_t)a[i];
            out[r * block_count + b] = d;
        }
}

/* fortai_gguf_runtime.f90:424-465: quantize x once, then every row's dot
 * (OpenMP row-parallel; the per-row result does not depend on threads). */
void orc_q8_matvec(const int8_t *weights, int64_t rows, int64_t width, const float *x,
    float *out, int8_t *qscratch, float *sscratch)
{
    const int64_t nb = width / 32;
    orc_q8_quantize(x, qscratch, sscratch, width);
    #pragma omp parallel for schedule(static) if (rows >= 128)
    for (int64_t r = 0; r < rows; ++r)
        out[r] = orc_q8_dot(weights, qscratch, sscratch, r, nb);
}

/* ----------------------------------------------------- SiLU / exp poly -- */

/* fortai_q8_dot.c:10-51, one lane (mul and add separately rounded). */
float orc_expf_poly(float value)
{
    value = (value < 88.3762626647949f) ? value : 88.3762626647949f;   /* min_ps */
    value = (value > -88.3762626647949f) ? value : -88.3762626647949f; /* max_ps */
    float fx = value * 1.44269504088896341f + 0.5f;
    int32_t e = (int32_t)fx; /* cvttps (fx is in range here) */
    if ((float)e > fx) e -= 1;
    fx = (float)e;
    value = value - fx * 0.693359375f;
    value = value - fx * -2.12194440e-4f;
    const float z = value * value;
    float p = 1.9875691500e-4f;
    p = p * value + 1.3981999507e-3f;
    p = p * value + 8.3334519073e-3f;
    p = p * value + 4.1665795894e-2f;
    p = p * value + 1.6666665459e-1f;
    p = p * value + 5.0000001201e-1f;
    p = p * z + value;
    p = p + 1.0f;
    return p * f_from_bits((uint32_t)(e + 0x7f) << 23);
}

static inline float silu_lane(float x)
{
    float r = x / (1.0f + orc_expf_poly(0.0f - x));
    if (x < -20.0f) r = 0.0f;
    if (x > 20.0f) r = x;
    return r;
}

/* fortai_q8_dot.c:442-482 (AVX2 for count >= 8; libm expf for the tail and
 * for count < 8). */
void orc_silu(float *values, int64_t count)
{
    int64_t i = 0;
    if (count >= 8)
        for (; i + 8 <= count; i += 8)
            for (int l = 0; l < 8; ++l) values[i + l] = silu_lane(values[i + l]);
    for (; i < count; ++i) values[i] = values[i] / (1.0f + expf(-values[i]));
}

/* fortai_q8_dot.c:484-525 */
void orc_silu_product(float *left, const float *right, int64_t count)
{
    int64_t i = 0;
    if (count >= 8)
        for (; i + 8 <= count; i += 8)
            for (int l = 0; l < 8; ++l) left[i + l] = silu_lane(left[i + l]) * right[i + l];
    for (; i < count; ++i) left[i] = left[i] / (1.0f + expf(-left[i])) * right[i];
}

/* ------------------------------------------------------------ GDN step -- */

static inline float hsum8(const float *a)
{
    const float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    return (s0 + s2) + (s1 + s3);
}

/* fortai_q8_dot.c:356-398 (AVX2, used when head_size % 8 == 0) and :400-425
 * (scalar otherwise). */
void orc_gdn_step(float *state, const float *key, const float *value, const float *query,
    float decay, float beta, int64_t head_size, float output_scale, float *output)
{
    if (head_size >= 8 && head_size % 8 == 0) {
        for (int64_t row = 0; row < head_size; ++row) {
            float *s = state + row * head_size;
            float kd[8] = {0, 0, 0, 0, 0, 0, 0, 0}, qd[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int64_t c = 0; c < head_size; c += 8)
                for (int l = 0; l < 8; ++l) {
                    const float d = s[c + l] * decay;
                    s[c + l] = d;
                    kd[l] = fmaf(d, key[c + l], kd[l]);
                }
            const float delta = (value[row] - hsum8(kd)) * beta;
            for (int64_t c = 0; c < head_size; c += 8)
                for (int l = 0; l < 8; ++l) {
                    const float u = fmaf(delta, key[c + l], s[c + l]);
                    s[c + l] = u;
                    qd[l] = fmaf(u, query[c + l], qd[l]);
                }
            output[row] = hsum8(qd) * output_scale;
        }
        return;
    }
    for (int64_t row = 0; row < head_size; ++row) {
        float dot = 0.0f;
        for (int64_t c = 0; c < head_size; ++c) {
            float *e = state + row * head_size + c;
            *e *= decay;
            dot += *e * key[c];
        }
        const float delta = (value[row] - dot) * beta;
        float qd = 0.0f;
        for (int64_t c = 0; c < head_size; ++c) {
            float *e = state + row * head_size + c;
            *e += delta * key[c];
            qd += *e * query[c];
        }
        output[row] = qd * output_scale;
    }
}

/* ------------------------------------------------- Fortran-side helpers -- */

/* fortai_qwen35_cpu.f90:1408-1432 */
void orc_rms_norm(const float *x, const float *w, float eps, float *out, int64_t n)
{
    double ss = 0.0;
    for (int64_t i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
    const float mean = (float)(ss / (double)n);
    const float inv = 1.0f / sqrtf(mean + eps);
    for (int64_t i = 0; i < n; ++i) {
        const float t = x[i] * inv;
        out[i] = t * w[i];
    }
}

/* fortai_qwen35_cpu.f90:1434-1453 (in place) */
void orc_normalize_slice(float *v, int64_t n, float eps, const float *w)
{
    double ss = 0.0;
    for (int64_t i = 0; i < n; ++i) ss += (double)v[i] * (double)v[i];
    const float mean = (float)(ss / (double)n);
    const float inv = 1.0f / sqrtf(mean + eps);
    for (int64_t i = 0; i < n; ++i) {
        const float t = v[i] * inv;
        v[i] = t * w[i];
    }
}

/* fortai_qwen35_cpu.f90:1455-1471 */
void orc_l2_normalize_slice(float *v, int64_t n, float eps)
{
    double ss = 0.0;
    for (int64_t i = 0; i < n; ++i) ss += (double)v[i] * (double)v[i];
    const float nrm = sqrtf((float)ss);
    const float inv = 1.0f / (nrm > eps ? nrm : eps);
    for (int64_t i = 0; i < n; ++i) v[i] = v[i] * inv;
}

/* fortai_qwen35_cpu.f90:1528-1539 */
float orc_rms_slice(const float *v, int64_t n, float eps)
{
    double ss = 0.0;
    for (int64_t i = 0; i < n; ++i) ss += (double)v[i] * (double)v[i];
    return sqrtf((float)(ss / (double)n) + eps);
}

/* fortai_qwen35_cpu.f90:1506-1526 */
float orc_sigmoid(float v) { return v >= 0.0f ? 1.0f / (1.0f + expf(-v)) : expf(v) / (1.0f + expf(v)); }
float orc_softplus(float v) { return v > 20.0f ? v : (v < -20.0f ? expf(v) : logf(1.0f + expf(v))); }

/* The RoPE angle table entry of fortai_qwen35_cpu.f90:1487-1490:
 * angle = real(pos)/base**(real(2i)/real(dim)); cos(angle), sin(angle). */
void orc_rope_cos_sin(int64_t position, int64_t i, int64_t dim, float base, float *c, float *s)
{
    const float angle = (float)position / powf(base, (float)(2 * i) / (float)dim);
    *c = cosf(angle);
    *s = sinf(angle);
}

/* fortai_qwen35_cpu.f90:1473-1497 (NeoX half pairs over the first dim values
 * of each head; heads are stride floats apart). */
void orc_apply_rope(float *values, int64_t heads, int64_t stride, int64_t position,
    int64_t dim, float base)
{
    const int64_t half = dim / 2;
    for (int64_t h = 0; h < heads; ++h)
        for (int64_t i = 0; i < half; ++i) {
            float c, s;
            orc_rope_cos_sin(position, i, dim, base, &c, &s);
            const float a = values[h * stride + i], b = values[h * stride + i + half];
            values[h * stride + i] = a * c - b * s;
            values[h * stride + i + half] = a * s + b * c;
        }
}

/* The attention part of fortai_qwen35_cpu.f90:1006-1033 over positions
 * 0..position, with caches stored as fp16 bits [pos][kv_head][dim] and read
 * through gguf_fp16_to_real (the f32 value the reference's cache holds,
 * :1594-1601, :1606-1623).  q_work is [heads][q(head_size) | gate(head_size)]. */
void orc_attention_apply(const float *q_work, const uint16_t *kcache, const uint16_t *vcache,
    int64_t heads, int64_t kv_heads, int64_t head_size, int64_t value_size, int64_t position,
    float *scores, float *out)
{
    const float inv_sqrt = sqrtf((float)head_size);
    for (int64_t h = 0; h < heads; ++h) {
        const int64_t kv = h / (heads / kv_heads);
        const float *q = q_work + h * 2 * head_size;
        float maximum = -FLT_MAX;
        for (int64_t p = 0; p <= position; ++p) {
            float score = 0.0f;
            const uint16_t *k = kcache + (p * kv_heads + kv) * head_size;
            for (int64_t i = 0; i < head_size; ++i) score = score + q[i] * orc_gguf_fp16_to_real(k[i]);
            scores[p] = score / inv_sqrt;
            maximum = maximum > scores[p] ? maximum : scores[p];
        }
        float normalizer = 0.0f;
        for (int64_t p = 0; p <= position; ++p) {
            scores[p] = expf(scores[p] - maximum);
            normalizer = normalizer + scores[p];
        }
        const float *gate = q_work + h * 2 * head_size + head_size;
        for (int64_t i = 0; i < value_size; ++i) {
            float acc = 0.0f;
            for (int64_t p = 0; p <= position; ++p)
                acc = acc + scores[p] / normalizer * orc_gguf_fp16_to_real(vcache[(p * kv_heads + kv) * value_size + i]);
            out[h * value_size + i] = acc * orc_sigmoid(gate[i]);
        }
    }
}

/* Attention core of one step (fortai_qwen35_cpu.f90:990-1033 without the
 * projections): per-head RMSNorm of q and k with q_norm/k_norm, RoPE, fp16
 * append at `position` (float_to_half, :1594-1601), then apply.  q_work and
 * k are modified in place. */
void orc_attention_core_step(float *q_work, float *k, const float *v, const float *q_norm,
    const float *k_norm, uint16_t *kcache, uint16_t *vcache, int64_t heads, int64_t kv_heads,
    int64_t head_size, int64_t value_size, int64_t position, int64_t rope_dim, float rope_base,
    float eps, float *scores, float *out)
{
    for (int64_t h = 0; h < heads; ++h) orc_normalize_slice(q_work + h * 2 * head_size, head_size, eps, q_norm);
    for (int64_t h = 0; h < kv_heads; ++h) orc_normalize_slice(k + h * head_size, head_size, eps, k_norm);
    orc_apply_rope(q_work, heads, 2 * head_size, position, rope_dim, rope_base);
    orc_apply_rope(k, kv_heads, head_size, position, rope_dim, rope_base);
    for (int64_t h = 0; h < kv_heads; ++h) {
        for (int64_t i = 0; i < head_size; ++i)
            kcache[(position * kv_heads + h) * head_size + i] = orc_float_to_half(k[h * head_size + i]);
        for (int64_t i = 0; i < value_size; ++i)
            vcache[(position * kv_heads + h) * value_size + i] = orc_float_to_half(v[h * value_size + i]);
    }
    orc_attention_apply(q_work, kcache, vcache, heads, kv_heads, head_size, value_size, position, scores, out);
}

/* The recurrent core of one step (fortai_qwen35_cpu.f90:856-906 without the
 * projections and the gated norm): causal conv1d over conv_state [K-1][C] and
 * the current qkv, SiLU, state shift, L2 normalisation of q and k per key
 * head, then per value head the decay/beta and fortai_gdn_step.
 * conv_w is [C][K] (K fastest).  out is [value_heads*head_size]. */
void orc_gdn_core_step(const float *qkv, const float *alpha, const float *beta_raw,
    const float *ssm_a, const float *ssm_dt, const float *conv_w, float *conv_state,
    float *gdn_state, int64_t conv_size, int64_t conv_kernel, int64_t state_size,
    int64_t key_heads, int64_t value_heads, int64_t head_size, float eps, float *conv_work,
    float *out)
{
    for (int64_t ch = 0; ch < conv_size; ++ch) {
        float acc = 0.0f;
        for (int64_t slot = 0; slot < conv_kernel - 1; ++slot)
            acc = acc + conv_w[ch * conv_kernel + slot] * conv_state[slot * conv_size + ch];
        acc = acc + conv_w[ch * conv_kernel + conv_kernel - 1] * qkv[ch];
        conv_work[ch] = acc;
    }
    orc_silu(conv_work, conv_size);
    for (int64_t slot = 0; slot + 1 < conv_kernel - 1; ++slot)
        memcpy(conv_state + slot * conv_size, conv_state + (slot + 1) * conv_size, (size_t)conv_size * 4);
    memcpy(conv_state + (conv_kernel - 2) * conv_size, qkv, (size_t)conv_size * 4);
    for (int64_t h = 0; h < key_heads; ++h) {
        orc_l2_normalize_slice(conv_work + h * head_size, head_size, eps);
        orc_l2_normalize_slice(conv_work + state_size * key_heads + h * head_size, head_size, eps);
    }
    for (int64_t h = 0; h < value_heads; ++h) {
        const int64_t kh = h / (value_heads / key_heads);
        const float b = orc_sigmoid(beta_raw[h]);
        const float decay = ssm_a[h] * orc_softplus(alpha[h] + ssm_dt[h]);
        const float decay_factor = expf(decay);
        orc_gdn_step(gdn_state + h * head_size * head_size,
            conv_work + state_size * key_heads + kh * head_size,
            conv_work + 2 * state_size * key_heads + h * head_size,
            conv_work + kh * head_size, decay_factor, b, head_size,
            1.0f / sqrtf((float)head_size), out + h * head_size);
    }
}

/* ---------------------------------------------------------- GGUF model -- */

enum { T_F32 = 0, T_F16 = 1, T_Q8 = 8 };

typedef struct {
    char name[96];
    int rank;
    int64_t shape[4];
    uint32_t type;
    const uint8_t *data;
    int64_t nbytes;
} orc_tensor;

typedef struct {
    int recurrent;
    const orc_tensor *attn_norm, *post_norm, *ffn_gate, *ffn_up, *ffn_down;
    const orc_tensor *qkv, *gate, *ssm_a, *alpha, *beta, *conv, *dt, *ssm_norm, *ssm_out;
    const orc_tensor *q, *k, *v, *o, *q_norm, *k_norm;
    float *conv_state, *gdn_state;
    uint16_t *kcache, *vcache;
} orc_layer;

typedef struct orc_model {
    void *map;
    size_t map_bytes;
    orc_tensor *tensors;
    int64_t n_tensors;
    int64_t hidden, vocab, layers, ffn, heads, kv_heads, head_size, value_size, rope_dim;
    int64_t conv_kernel, state_size, key_heads, value_heads, inner, gdn_head, conv_size;
    int64_t interval, max_context;
    float eps, rope_base;
    const orc_tensor *embd, *out_norm, *output;
    orc_layer *layer;
    float *x, *residual, *normalized, *hidden_work, *qkv_work, *gate_work, *q_work, *k_work,
        *v_work, *attn_work, *scores, *ffn_g, *ffn_u, *conv_work, *alpha_w, *beta_w;
    int8_t *qin;
    float *qsc;
} orc_model;

typedef struct { const uint8_t *p, *end; int ok; } rd;
static uint64_t rd_u(rd *r, int n)
{
    uint64_t v = 0;
    if (r->p + n > r->end) { r->ok = 0; return 0; }
    memcpy(&v, r->p, (size_t)n);
    r->p += n;
    return v;
}
typedef struct { char key[128]; uint32_t type; int64_t i; double f; } meta_kv;

static int skip_value(rd *r, uint32_t t, meta_kv *m)
{
    switch (t) {
    case 0: case 1: case 7: m->i = (t == 1) ? (int8_t)rd_u(r, 1) : (int64_t)rd_u(r, 1); break;
    case 2: case 3: m->i = (t == 3) ? (int16_t)rd_u(r, 2) : (int64_t)rd_u(r, 2); break;
    case 4: m->i = (int64_t)(uint32_t)rd_u(r, 4); break;
    case 5: m->i = (int32_t)rd_u(r, 4); break;
    case 6: { uint32_t b = (uint32_t)rd_u(r, 4); m->f = f_from_bits(b); break; }
    case 10: case 11: m->i = (int64_t)rd_u(r, 8); break;
    case 12: { uint64_t b = rd_u(r, 8); double d; memcpy(&d, &b, 8); m->f = d; break; }
    case 8: { uint64_t n = rd_u(r, 8); if (r->p + n > r->end) return 0; r->p += n; break; }
    case 9: {
        uint32_t et = (uint32_t)rd_u(r, 4);
        uint64_t n = rd_u(r, 8);
        meta_kv tmp;
        for (uint64_t j = 0; j < n && r->ok; ++j) if (!skip_value(r, et, &tmp)) return 0;
        break;
    }
    default: return 0;
    }
    return r->ok;
}

static int64_t tensor_bytes(uint32_t type, const int64_t *shape, int rank)
{
    int64_t el = 1;
    for (int i = 0; i < rank; ++i) el *= shape[i];
    if (type == T_F32) return 4 * el;
    if (type == T_F16) return 2 * el;
    if (type == T_Q8) return (shape[0] % 32) ? -1 : (el / shape[0]) * (shape[0] / 32) * 34;
    return -1;
}

static const orc_tensor *find_tensor(const orc_model *m, const char *name)
{
    for (int64_t i = 0; i < m->n_tensors; ++i)
        if (strcmp(m->tensors[i].name, name) == 0) return &m->tensors[i];
    return NULL;
}
static const orc_tensor *layer_tensor(const orc_model *m, int64_t l, const char *suffix)
{
    char name[128];
    snprintf(name, sizeof(name), "blk.%lld.%s", (long long)l, suffix);
    return find_tensor(m, name);
}

void orc_model_close(orc_model *m);
void orc_model_reset(orc_model *m);

/* Loader: fortai_gguf_runtime.f90:106-197; config: fortai_qwen35_cpu.f90:163-285. */
orc_model *orc_model_open(const char *path, int64_t max_context)
{
    orc_model *m = calloc(1, sizeof(*m));
    if (!m) return NULL;
    int fd = open(path, O_RDONLY);
    if (fd < 0) { free(m); return NULL; }
    struct stat st;
    fstat(fd, &st);
    m->map_bytes = (size_t)st.st_size;
    m->map = mmap(NULL, m->map_bytes, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m->map == MAP_FAILED) { free(m); return NULL; }
    rd r = {(const uint8_t *)m->map, (const uint8_t *)m->map + m->map_bytes, 1};
    if (memcmp(r.p, "GGUF", 4) != 0) goto fail;
    r.p += 4;
    if ((uint32_t)rd_u(&r, 4) != 3u) goto fail;
    const int64_t nt = (int64_t)rd_u(&r, 8), nm = (int64_t)rd_u(&r, 8);
    if (nt < 0 || nm < 0) goto fail;
    meta_kv *meta = calloc((size_t)nm + 1, sizeof(meta_kv));
    for (int64_t i = 0; i < nm; ++i) {
        uint64_t len = rd_u(&r, 8);
        size_t cp = len < 127 ? (size_t)len : 127;
        memcpy(meta[i].key, r.p, cp);
        r.p += len;
        meta[i].type = (uint32_t)rd_u(&r, 4);
        if (!skip_value(&r, meta[i].type, &meta[i])) { free(meta); goto fail; }
    }
#define META_I(k, d) ({ int64_t _v = (d); for (int64_t _i = 0; _i < nm; ++_i) \
        if (!strcmp(meta[_i].key, k) && meta[_i].type != 6 && meta[_i].type != 12 && meta[_i].type != 8 && meta[_i].type != 9) _v = meta[_i].i; _v; })
#define META_F(k, d) ({ float _v = (d); for (int64_t _i = 0; _i < nm; ++_i) \
        if (!strcmp(meta[_i].key, k) && (meta[_i].type == 6 || meta[_i].type == 12)) _v = (float)meta[_i].f; _v; })
    int64_t alignment = META_I("general.alignment", 32);
    if (alignment <= 0) alignment = 32;
    m->n_tensors = nt;
    m->tensors = calloc((size_t)nt + 1, sizeof(orc_tensor));
    for (int64_t i = 0; i < nt; ++i) {
        orc_tensor *t = &m->tensors[i];
        uint64_t len = rd_u(&r, 8);
        size_t cp = len < 95 ? (size_t)len : 95;
        memcpy(t->name, r.p, cp);
        r.p += len;
        t->rank = (int)rd_u(&r, 4);
        if (t->rank <= 0 || t->rank > 4) { free(meta); goto fail; }
        for (int j = 0; j < t->rank; ++j) t->shape[j] = (int64_t)rd_u(&r, 8);
        t->type = (uint32_t)rd_u(&r, 4);
        t->data = (const uint8_t *)(uintptr_t)rd_u(&r, 8); /* offset for now */
        t->nbytes = tensor_bytes(t->type, t->shape, t->rank);
        if (t->nbytes < 0 || !r.ok) { free(meta); goto fail; }
    }
    const size_t hdr = (size_t)(r.p - (const uint8_t *)m->map);
    const size_t data_start = ((hdr + (size_t)alignment - 1) / (size_t)alignment) * (size_t)alignment;
    for (int64_t i = 0; i < nt; ++i) {
        const size_t off = data_start + (size_t)(uintptr_t)m->tensors[i].data;
        if (off + (size_t)m->tensors[i].nbytes > m->map_bytes) { free(meta); goto fail; }
        m->tensors[i].data = (const uint8_t *)m->map + off;
    }
    m->hidden = META_I("qwen35.embedding_length", 0);
    m->vocab = META_I("qwen35.vocab_size", 0);
    m->layers = META_I("qwen35.block_count", 0);
    m->ffn = META_I("qwen35.feed_forward_length", 0);
    m->heads = META_I("qwen35.attention.head_count", 0);
    m->kv_heads = META_I("qwen35.attention.head_count_kv", 0);
    m->head_size = META_I("qwen35.attention.key_length", 0);
    m->value_size = META_I("qwen35.attention.value_length", 0);
    m->rope_dim = META_I("qwen35.rope.dimension_count", 0);
    m->conv_kernel = META_I("qwen35.ssm.conv_kernel", 0);
    m->state_size = META_I("qwen35.ssm.state_size", 0);
    m->key_heads = META_I("qwen35.ssm.group_count", 0);
    m->value_heads = META_I("qwen35.ssm.time_step_rank", 0);
    m->inner = META_I("qwen35.ssm.inner_size", 0);
    m->eps = META_F("qwen35.attention.layer_norm_rms_epsilon", 1.0e-6f);
    m->rope_base = META_F("qwen35.rope.freq_base", 10000000.0f);
    m->interval = META_I("qwen35.full_attention_interval", 4);
    free(meta);
    m->max_context = max_context;
    m->embd = find_tensor(m, "token_embd.weight");
    m->out_norm = find_tensor(m, "output_norm.weight");
    m->output = find_tensor(m, "output.weight");
    if (!m->output) m->output = m->embd;
    if (m->embd && m->embd->rank == 2) { m->hidden = m->embd->shape[0]; m->vocab = m->embd->shape[1]; }
    if (m->hidden <= 0 || m->vocab <= 0 || m->layers <= 0 || m->ffn <= 0 || m->heads <= 0 ||
        m->kv_heads <= 0 || m->head_size <= 0 || m->state_size <= 0 || m->inner <= 0 ||
        m->interval <= 0 || max_context <= 0 || !m->embd || !m->out_norm ||
        m->inner % m->value_heads || m->value_heads % m->key_heads || m->heads % m->kv_heads)
        goto fail;
    m->gdn_head = m->inner / m->value_heads;
    m->conv_size = 2 * m->state_size * m->key_heads + m->inner;
    m->layer = calloc((size_t)m->layers, sizeof(orc_layer));
    for (int64_t l = 0; l < m->layers; ++l) {
        orc_layer *L = &m->layer[l];
        L->recurrent = ((l + 1) % m->interval) != 0;
        L->attn_norm = layer_tensor(m, l, "attn_norm.weight");
        L->post_norm = layer_tensor(m, l, "post_attention_norm.weight");
        L->ffn_gate = layer_tensor(m, l, "ffn_gate.weight");
        L->ffn_up = layer_tensor(m, l, "ffn_up.weight");
        L->ffn_down = layer_tensor(m, l, "ffn_down.weight");
        if (!L->attn_norm || !L->post_norm || !L->ffn_gate || !L->ffn_up || !L->ffn_down) goto fail;
        if (L->recurrent) {
            L->qkv = layer_tensor(m, l, "attn_qkv.weight");
            L->gate = layer_tensor(m, l, "attn_gate.weight");
            L->ssm_a = layer_tensor(m, l, "ssm_a");
            L->alpha = layer_tensor(m, l, "ssm_alpha.weight");
            L->beta = layer_tensor(m, l, "ssm_beta.weight");
            L->conv = layer_tensor(m, l, "ssm_conv1d.weight");
            L->dt = layer_tensor(m, l, "ssm_dt.bias");
            L->ssm_norm = layer_tensor(m, l, "ssm_norm.weight");
            L->ssm_out = layer_tensor(m, l, "ssm_out.weight");
            if (!L->qkv || !L->gate || !L->ssm_a || !L->alpha || !L->beta || !L->conv || !L->dt ||
                !L->ssm_norm || !L->ssm_out) goto fail;
            L->conv_state = calloc((size_t)((m->conv_kernel - 1) * m->conv_size), 4);
            L->gdn_state = calloc((size_t)(m->gdn_head * m->gdn_head * m->value_heads), 4);
        } else {
            L->q = layer_tensor(m, l, "attn_q.weight");
            L->k = layer_tensor(m, l, "attn_k.weight");
            L->v = layer_tensor(m, l, "attn_v.weight");
            L->o = layer_tensor(m, l, "attn_output.weight");
            L->q_norm = layer_tensor(m, l, "attn_q_norm.weight");
            L->k_norm = layer_tensor(m, l, "attn_k_norm.weight");
            if (!L->q || !L->k || !L->v || !L->o || !L->q_norm || !L->k_norm) goto fail;
            L->kcache = calloc((size_t)(m->head_size * m->kv_heads * max_context), 2);
            L->vcache = calloc((size_t)(m->value_size * m->kv_heads * max_context), 2);
        }
    }
    int64_t ws = m->ffn > m->conv_size ? m->ffn : m->conv_size;
    if (2 * m->heads * m->head_size > ws) ws = 2 * m->heads * m->head_size;
    if (m->hidden > ws) ws = m->hidden;
    if (m->inner > ws) ws = m->inner;
    if (m->heads * m->value_size > ws) ws = m->heads * m->value_size;
    m->x = calloc((size_t)m->hidden, 4);
    m->residual = calloc((size_t)m->hidden, 4);
    m->normalized = calloc((size_t)m->hidden, 4);
    m->hidden_work = calloc((size_t)m->hidden, 4);
    m->qkv_work = calloc((size_t)ws, 4);
    m->gate_work = calloc((size_t)ws, 4);
    m->q_work = calloc((size_t)(2 * m->heads * m->head_size), 4);
    m->k_work = calloc((size_t)(m->kv_heads * m->head_size), 4);
    m->v_work = calloc((size_t)(m->kv_heads * m->value_size), 4);
    m->attn_work = calloc((size_t)ws, 4);
    m->scores = calloc((size_t)max_context, 4);
    m->ffn_g = calloc((size_t)m->ffn, 4);
    m->ffn_u = calloc((size_t)m->ffn, 4);
    m->conv_work = calloc((size_t)m->conv_size, 4);
    m->alpha_w = calloc((size_t)m->value_heads, 4);
    m->beta_w = calloc((size_t)m->value_heads, 4);
    m->qin = calloc((size_t)(ws + 2 * ((ws + 31) / 32)), 1);
    m->qsc = calloc((size_t)((ws + 31) / 32), 4);
    orc_model_reset(m);
    return m;
fail:
    orc_model_close(m);
    return NULL;
}

void orc_model_close(orc_model *m)
{
    if (!m) return;
    if (m->layer) {
        for (int64_t l = 0; l < m->layers; ++l) {
            free(m->layer[l].conv_state); free(m->layer[l].gdn_state);
            free(m->layer[l].kcache); free(m->layer[l].vcache);
        }
        free(m->layer);
    }
    free(m->x); free(m->residual); free(m->normalized); free(m->hidden_work); free(m->qkv_work);
    free(m->gate_work); free(m->q_work); free(m->k_work); free(m->v_work); free(m->attn_work);
    free(m->scores); free(m->ffn_g); free(m->ffn_u); free(m->conv_work); free(m->alpha_w);
    free(m->beta_w); free(m->qin); free(m->qsc); free(m->tensors);
    if (m->map && m->map != MAP_FAILED) munmap(m->map, m->map_bytes);
    free(m);
}

/* fortai_qwen35_cpu.f90:573-589 */
void orc_model_reset(orc_model *m)
{
    memset(m->x, 0, (size_t)m->hidden * 4);
    for (int64_t l = 0; l < m->layers; ++l) {
        orc_layer *L = &m->layer[l];
        if (L->conv_state) memset(L->conv_state, 0, (size_t)((m->conv_kernel - 1) * m->conv_size) * 4);
        if (L->gdn_state) memset(L->gdn_state, 0, (size_t)(m->gdn_head * m->gdn_head * m->value_heads) * 4);
        if (L->kcache) memset(L->kcache, 0, (size_t)(m->head_size * m->kv_heads * m->max_context) * 2);
        if (L->vcache) memset(L->vcache, 0, (size_t)(m->value_size * m->kv_heads * m->max_context) * 2);
    }
}

static const float *f32(const orc_tensor *t) { return (const float *)t->data; }

/* value(i) of an F32/F16 vector tensor (fortai_gguf_runtime.f90:290-322) */
static float tval(const orc_tensor *t, int64_t i)
{
    if (t->type == T_F32) return f32(t)[i];
    if (t->type == T_F16) return orc_gguf_fp16_to_real(((const uint16_t *)t->data)[i]);
    const int64_t b = i / 32, w = i % 32;
    uint16_t sb;
    memcpy(&sb, t->data + b * 34, 2);
    return orc_gguf_fp16_to_real(sb) * (float)(int32_t)((const int8_t *)t->data)[b * 34 + 2 + w];
}

/* model_matvec (fortai_qwen35_cpu.f90:1109-1137): Q8_0 -> matvec_q8; F32/F16
 * -> gguf_tensor_matvec with the sequential fp32 dot (fortai_gguf_runtime.f90:382-422). */
static void model_matvec(orc_model *m, const orc_tensor *t, const float *x, float *out)
{
    const int64_t width = t->shape[0], rows = t->rank > 1 ? t->shape[1] : 1;
    if (t->type == T_Q8) {
        orc_q8_matvec((const int8_t *)t->data, rows, width, x, out, m->qin, m->qsc);
        return;
    }
    #pragma omp parallel for schedule(static) if (rows >= 128)
    for (int64_t r = 0; r < rows; ++r) {
        float acc = 0.0f;
        if (t->type == T_F16) {
            const uint16_t *row = (const uint16_t *)t->data + r * width;
            for (int64_t i = 0; i < width; ++i) acc = acc + orc_gguf_fp16_to_real(row[i]) * x[i];
        } else {
            const float *row = f32(t) + r * width;
            for (int64_t i = 0; i < width; ++i) acc = acc + row[i] * x[i];
        }
        out[r] = acc;
    }
}

/* forward_recurrent, CPU branch (fortai_qwen35_cpu.f90:841-917) */
static void forward_recurrent(orc_model *m, orc_layer *L)
{
    model_matvec(m, L->qkv, m->normalized, m->qkv_work);
    model_matvec(m, L->gate, m->normalized, m->gate_work);
    model_matvec(m, L->alpha, m->normalized, m->alpha_w);
    model_matvec(m, L->beta, m->normalized, m->beta_w);
    orc_silu(m->gate_work, m->inner);
    float conv_w[64];
    for (int64_t ch = 0; ch < m->conv_size; ++ch) {
        for (int64_t s = 0; s < m->conv_kernel && s < 64; ++s) conv_w[s] = tval(L->conv, ch * m->conv_kernel + s);
        float acc = 0.0f;
        for (int64_t slot = 0; slot < m->conv_kernel - 1; ++slot)
            acc = acc + conv_w[slot] * L->conv_state[slot * m->conv_size + ch];
        acc = acc + conv_w[m->conv_kernel - 1] * m->qkv_work[ch];
        m->conv_work[ch] = acc;
    }
    orc_silu(m->conv_work, m->conv_size);
    for (int64_t slot = 0; slot + 1 < m->conv_kernel - 1; ++slot)
        memcpy(L->conv_state + slot * m->conv_size, L->conv_state + (slot + 1) * m->conv_size, (size_t)m->conv_size * 4);
    memcpy(L->conv_state + (m->conv_kernel - 2) * m->conv_size, m->qkv_work, (size_t)m->conv_size * 4);
    for (int64_t h = 0; h < m->key_heads; ++h) {
        orc_l2_normalize_slice(m->conv_work + h * m->gdn_head, m->gdn_head, m->eps);
        orc_l2_normalize_slice(m->conv_work + m->state_size * m->key_heads + h * m->gdn_head, m->gdn_head, m->eps);
    }
    const int64_t hs = m->gdn_head;
    for (int64_t h = 0; h < m->value_heads; ++h) {
        const int64_t kh = h / (m->value_heads / m->key_heads);
        const float beta = orc_sigmoid(m->beta_w[h]);
        const float decay = tval(L->ssm_a, h) * orc_softplus(m->alpha_w[h] + tval(L->dt, h));
        const float decay_factor = expf(decay);
        orc_gdn_step(L->gdn_state + h * hs * hs,
            m->conv_work + m->state_size * m->key_heads + kh * hs,
            m->conv_work + 2 * m->state_size * m->key_heads + h * hs,
            m->conv_work + kh * hs, decay_factor, beta, hs, 1.0f / sqrtf((float)hs),
            m->attn_work + h * hs);
        const float nf = orc_rms_slice(m->attn_work + h * hs, hs, m->eps);
        for (int64_t j = 0; j < hs; ++j) {
            float v = m->attn_work[h * hs + j] / nf;
            v = v * tval(L->ssm_norm, j);
            m->attn_work[h * hs + j] = v * m->gate_work[h * hs + j];
        }
    }
    model_matvec(m, L->ssm_out, m->attn_work, m->hidden_work);
}

/* forward_attention (fortai_qwen35_cpu.f90:978-1035) */
static void forward_attention(orc_model *m, orc_layer *L, int64_t position)
{
    model_matvec(m, L->q, m->normalized, m->q_work);
    model_matvec(m, L->k, m->normalized, m->k_work);
    model_matvec(m, L->v, m->normalized, m->v_work);
    float qn[1024], kn[1024];
    for (int64_t i = 0; i < m->head_size && i < 1024; ++i) { qn[i] = tval(L->q_norm, i); kn[i] = tval(L->k_norm, i); }
    orc_attention_core_step(m->q_work, m->k_work, m->v_work, qn, kn, L->kcache, L->vcache,
        m->heads, m->kv_heads, m->head_size, m->value_size, position, m->rope_dim, m->rope_base,
        m->eps, m->scores, m->attn_work);
    model_matvec(m, L->o, m->attn_work, m->hidden_work);
}

/* qwen35_cpu_forward, CPU branch (fortai_qwen35_cpu.f90:591-711).  Returns 0
 * on success, 1 on an invalid token/position. */
int orc_model_forward(orc_model *m, int64_t token, int64_t position, float *logits)
{
    if (token < 0 || token >= m->vocab || position < 0 || position >= m->max_context) return 1;
    if (m->embd->type == T_Q8)
        orc_q8_dequantize_row((const int8_t *)m->embd->data + token * (m->hidden / 32) * 34, m->x, m->hidden / 32);
    else
        for (int64_t i = 0; i < m->hidden; ++i) m->x[i] = tval(m->embd, token * m->hidden + i);
    for (int64_t l = 0; l < m->layers; ++l) {
        orc_layer *L = &m->layer[l];
        memcpy(m->residual, m->x, (size_t)m->hidden * 4);
        orc_rms_norm(m->x, f32(L->attn_norm), m->eps, m->normalized, m->hidden);
        if (L->recurrent) forward_recurrent(m, L);
        else forward_attention(m, L, position);
        for (int64_t i = 0; i < m->hidden; ++i) m->x[i] = m->hidden_work[i] + m->residual[i];
        memcpy(m->residual, m->x, (size_t)m->hidden * 4);
        orc_rms_norm(m->x, f32(L->post_norm), m->eps, m->normalized, m->hidden);
        model_matvec(m, L->ffn_gate, m->normalized, m->ffn_g);
        model_matvec(m, L->ffn_up, m->normalized, m->ffn_u);
        orc_silu_product(m->ffn_g, m->ffn_u, m->ffn);
        model_matvec(m, L->ffn_down, m->ffn_g, m->hidden_work);
        for (int64_t i = 0; i < m->hidden; ++i) m->x[i] = m->hidden_work[i] + m->residual[i];
    }
    orc_rms_norm(m->x, f32(m->out_norm), m->eps, m->normalized, m->hidden);
    model_matvec(m, m->output, m->normalized, logits);
    return 0;
}

/* maxloc (first maximum), app/fortai_cpu_run.f90:58; returns the 0-based id. */
int64_t orc_argmax(const float *v, int64_t n)
{
    int64_t best = 0;
    for (int64_t i = 1; i < n; ++i) if (v[i] > v[best]) best = i;
    return best;
}

/* Introspection for tests. */
int64_t orc_model_dims(const orc_model *m, int64_t *out, int64_t n)
{
    const int64_t d[] = {m->hidden, m->vocab, m->layers, m->ffn, m->heads, m->kv_heads,
        m->head_size, m->value_size, m->rope_dim, m->conv_kernel, m->state_size, m->key_heads,
        m->value_heads, m->inner, m->gdn_head, m->conv_size, m->interval, m->max_context};
    const int64_t k = (int64_t)(sizeof(d) / sizeof(d[0]));
    for (int64_t i = 0; i < n && i < k; ++i) out[i] = d[i];
    return k;
}
const float *orc_model_hidden(const orc_model *m) { return m->x; }
const float *orc_model_gdn_state(const orc_model *m, int64_t l) { return m->layer[l].gdn_state; }
const float *orc_model_conv_state(const orc_model *m, int64_t l) { return m->layer[l].conv_state; }
const uint16_t *orc_model_kcache(const orc_model *m, int64_t l) { return m->layer[l].kcache; }
const uint16_t *orc_model_vcache(const orc_model *m, int64_t l) { return m->layer[l].vcache; }
int orc_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------- parity helpers -- */

/* Exhaustive comparison of orc_float_to_half against another implementation
 * (the compiled reference's fortai_float_to_half) over the bit patterns
 * [begin, end); returns the number of mismatches. */
typedef uint16_t (*f2h_fn)(float);
int64_t orc_float_to_half_mismatches(void *other, uint64_t begin, uint64_t end)
{
    f2h_fn fn = (f2h_fn)other;
    int64_t bad = 0;
    #pragma omp parallel for reduction(+ : bad) schedule(static)
    for (int64_t i = (int64_t)begin; i < (int64_t)end; ++i) {
        const float f = f_from_bits((uint32_t)i);
        bad += orc_float_to_half(f) != fn(f);
    }
    return bad;
}

void orc_float_to_half_array(const float *in, uint16_t *out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = orc_float_to_half(in[i]);
}

void orc_f32_to_f16_rne_array(const float *in, uint16_t *out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16_rne(in[i]);
}

void orc_half_to_float_array(const uint16_t *in, float *out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = orc_half_to_float(in[i]);
}

void orc_gguf_fp16_to_real_array(const uint16_t *in, float *out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = orc_gguf_fp16_to_real(in[i]);
}

/* The expf sequence the GPU kernels use (fortai_amd/csrc/fortai_hip_internal.h,
 * expf_libm): glibc's ARM optimized-routines algorithm of
 * sysdeps/ieee754/flt-32/e_expf.c in its FMA form.  Test infrastructure: it is
 * compared with the host expf (the function the reference calls) in
 * tests/test_oracle.py. */
float orc_expf_restated(float x)
{
    static uint64_t tab[32];
    static int ready = 0;
    if (!ready) {
        for (int i = 0; i < 32; ++i) {
            const double t = (double)exp2l((long double)i / 32.0L);
            uint64_t b;
            memcpy(&b, &t, 8);
            tab[i] = b - ((uint64_t)i << 47);
        }
        ready = 1;
    }
    if (x != x) return x + x;
    if (x > 0x1.62e42ep6f) return INFINITY;
    if (x < -0x1.9fe368p6f) return 0.0f;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0), c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0),
                 c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x, z = inv_ln2_n * xd;
    double kd = z + shift;
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = fma(inv_ln2_n, xd, -kd);
    const uint64_t t = tab[ki % 32] + (ki << 47);
    double s;
    memcpy(&s, &t, 8);
    const double zz = fma(c0, r, c1), r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(zz, r2, y);
    return (float)(y * s);
}

/* mismatches of orc_expf_restated against the host expf over every float
 * bit pattern in [begin, end) */
int64_t orc_expf_restated_mismatches(uint32_t begin, uint32_t end)
{
    int64_t bad = 0;
    #pragma omp parallel for reduction(+ : bad) schedule(static)
    for (int64_t b = begin; b < (int64_t)end; ++b) {
        const float x = f_from_bits((uint32_t)b);
        const float a = expf(x), c = orc_expf_restated(x);
        bad += memcmp(&a, &c, 4) != 0;
    }
    return bad;
}
