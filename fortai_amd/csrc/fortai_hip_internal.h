// Internal types and device helpers of the gfx950 FortAI backend.
//
// Numerics conventions (all kernels are compiled with -ffp-contract=off):
//  * multiply and add are separately rounded unless a fused multiply-add is
//    written explicitly with __builtin_fmaf, mirroring where the reference CPU
//    path uses FMA intrinsics (src/backend/cpu/fortai_q8_dot.c:320,377,391,393);
//  * division and sqrtf are the correctly rounded IEEE operations (HIP's
//    default for fp32), never the approximate reciprocal;
//  * reductions that feed a float32 result through a double sum keep the double
//    accumulator (src/models/qwen35/fortai_qwen35_cpu.f90:1414-1427).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

// Per-workgroup timing hook of the decode kernels (first statement of each):
// empty in the library; a timing build defines it to record when each
// workgroup starts and ends.
#ifndef FORTAI_TRACE_SCOPE
#define FORTAI_TRACE_SCOPE(id)
#endif

namespace fortai_hip {

constexpr int kQ8Block = 32;       // values per Q8_0 block
constexpr int kQ8Bytes = 34;       // GGUF bytes per block: fp16 scale + 32 x int8
constexpr int kRowsPerWave = 8;    // a wave64 holds 8 rows x 8 lanes
constexpr int kLanesPerRow = 8;    // the 8 fp32 lanes of the reference's AVX2 dot

// ---------------------------------------------------------------- fp16 ----

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// gguf_fp16_to_real (src/fortai_gguf_runtime.f90:770-788): exact for finite
// halves, exponent 31 decodes to +-huge instead of inf/NaN.
__device__ __forceinline__ float gguf_half_to_real(uint16_t h) {
    if ((h & 0x7c00u) == 0x7c00u) return (h & 0x8000u) ? -3.402823466e38f : 3.402823466e38f;
    return half_bits_to_float(h);
}

// IEEE round-to-nearest-even binary32 -> binary16 (the F16C conversion the
// AVX2 quantizer uses for its scale, src/backend/cpu/fortai_q8_dot.c:176).
__device__ __forceinline__ uint16_t float_to_half_rne(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// The reference's float_to_half (src/backend/cpu/fortai_q8_dot.c:85-113),
// used for the KV cache store (fortai_qwen35_cpu.f90:1594-1601): it adds one
// half-ulp whenever bit 12 of the float fraction is set (ties round away from
// zero); its subnormal branch tests bit 12 of the unshifted fraction.
__device__ __forceinline__ uint16_t float_to_half_kv(float value) {
    const uint32_t bits = __builtin_bit_cast(uint32_t, value);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    int32_t exponent = static_cast<int32_t>((bits >> 23) & 0xffu) - 127 + 15;
    uint32_t fraction = bits & 0x007fffffu;
    if (exponent <= 0) {
        if (exponent < -10) return static_cast<uint16_t>(sign);
        fraction = (fraction | 0x00800000u) >> static_cast<uint32_t>(1 - exponent);
        if (bits & 0x00001000u) fraction += 0x00002000u;
        return static_cast<uint16_t>(sign | (fraction >> 13));
    }
    if (exponent >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
    if (fraction & 0x00001000u) {
        fraction += 0x00002000u;
        if (fraction & 0x00800000u) {
            fraction = 0;
            if (++exponent >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
        }
    }
    return static_cast<uint16_t>(sign | (static_cast<uint32_t>(exponent) << 10) | (fraction >> 13));
}

// ------------------------------------------------------------- scalars ----

// The vector exp polynomial of the reference SiLU (fortai_q8_dot.c:10-51):
// Cody-Waite reduction by ln2 (hi/lo split) and a degree-6 Cephes-style
// polynomial, evaluated with separately rounded multiply and add.
__device__ __forceinline__ float expf_poly(float value) {
    value = (value < 88.3762626647949f) ? value : 88.3762626647949f;
    value = (value > -88.3762626647949f) ? value : -88.3762626647949f;
    float fx = value * 1.44269504088896341f + 0.5f;
    int32_t e = static_cast<int32_t>(fx);
    if (static_cast<float>(e) > fx) e -= 1;
    fx = static_cast<float>(e);
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
    return p * __builtin_bit_cast(float, static_cast<uint32_t>(e + 0x7f) << 23);
}

// One lane of the reference's vector SiLU (fortai_q8_dot.c:450-459).
__device__ __forceinline__ float silu_poly(float x) {
    float r = x / (1.0f + expf_poly(0.0f - x));
    if (x < -20.0f) r = 0.0f;
    if (x > 20.0f) r = x;
    return r;
}

// Causal conv1d + SiLU of one channel (fortai_qwen35_cpu.f90:856-867): the
// window's K-1 values oldest first, then the current value x last, each
// product added in order; slots at or past K-1 (window) or K (taps) are
// unused.  The caller shifts the window (:870-879).
constexpr int kConvMax = 8;
__device__ __forceinline__ float conv_silu(const float (&win)[kConvMax - 1], const float (&taps)[kConvMax], int K,
    float x) {
    float a = 0.0f;
#pragma unroll
    for (int t = 0; t < kConvMax - 1; ++t)
        if (t < K - 1) a = a + taps[t] * win[t];
    float last = 0.0f;
#pragma unroll
    for (int t = 0; t < kConvMax; ++t)
        if (t == K - 1) last = taps[t];
    a = a + last * x;
    return silu_poly(a);
}

// expf of the C library the reference CPU path links (the Fortran real32
// exp intrinsic calls it): glibc's algorithm from ARM optimized-routines
// (sysdeps/ieee754/flt-32/e_expf.c, x86-64 FMA build).  x * 32/ln2 = k + r,
// 2^(k/32) from a 32-entry table of 2^(i/32) (exponent field pre-shifted),
// a cubic for 2^(r/32), all in double with fused multiply-adds, rounded once
// to float.  glibc's expf is not correctly rounded (about 1 input in 10^4
// differs from the rounded exact value), so only this sequence reproduces
// it; on every float of [-103.5, 88] it equals the host expf bit for bit.
// 2^(i/32) with the exponent field pre-shifted: bits(2^(i/32)) - (i << 47)
static __constant__ const uint64_t kExpf2Table[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};
// tab: kExpf2Table, or a copy of it in LDS (a lookup in the constant table
// is a memory round trip that depends on x; see MathTables)
template <typename TAB>
__device__ __forceinline__ float expf_libm_t(float x, const TAB *tab) {
    if (x != x) return x + x;
    if (x > 0x1.62e42ep6f) return __builtin_inff();
    if (x < -0x1.9fe368p6f) return 0.0f;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0), c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0),
                 c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = static_cast<double>(x);
    const double z = inv_ln2_n * xd;
    double kd = z + shift;
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const uint64_t t = static_cast<uint64_t>(tab[ki % 32]) + (ki << 47);
    const double s = __builtin_bit_cast(double, t);
    const double zz = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(zz, r2, y);
    return static_cast<float>(y * s);
}
__device__ __forceinline__ float expf_libm(float x) { return expf_libm_t(x, kExpf2Table); }
__device__ __forceinline__ float exp_rounded(float v) { return expf_libm(v); }

// logf of the same C library (the Fortran real32 log intrinsic calls it):
// glibc's algorithm from ARM optimized-routines (sysdeps/ieee754/flt-32/
// e_logf.c).  x = 2^k z with z in [0x1.66p-1, 0x1.66p0); the top 4 mantissa
// bits of z pick a table centre c, log(x) = k ln2 + log(c) + log1p(r) with
// r = z/c - 1 = z * invc - 1 exact in double, log1p(r) by a cubic; all in
// double, rounded once to float.  Like expf it is not correctly rounded
// (170327 of the 241653829 floats in [1, 1 + expf(20)], the softplus
// domain, differ from the rounded exact value), so only this sequence
// reproduces it; on every positive normal float it equals glibc 2.35's logf
// bit for bit.  Entry i: {invc, log(c)} with c near the centre of the i-th
// subinterval, chosen in the library so that 1/invc and log(c) are exact
// enough for the error bound; the values are the library's.
static __constant__ const double kLogfTable[16][2] = {
    {0x1.661ec79f8f3bep+0, -0x1.57bf7808caadep-2}, {0x1.571ed4aaf883dp+0, -0x1.2bef0a7c06ddbp-2},
    {0x1.49539f0f010bp+0, -0x1.01eae7f513a67p-2},  {0x1.3c995b0b80385p+0, -0x1.b31d8a68224e9p-3},
    {0x1.30d190c8864a5p+0, -0x1.6574f0ac07758p-3}, {0x1.25e227b0b8eap+0, -0x1.1aa2bc79c81p-3},
    {0x1.1bb4a4a1a343fp+0, -0x1.a4e76ce8c0e5ep-4}, {0x1.12358f08ae5bap+0, -0x1.1973c5a611cccp-4},
    {0x1.0953f419900a7p+0, -0x1.252f438e10c1ep-5}, {0x1p+0, 0x0p+0},
    {0x1.e608cfd9a47acp-1, 0x1.aa5aa5df25984p-5},  {0x1.ca4b31f026aap-1, 0x1.c5e53aa362eb4p-4},
    {0x1.b2036576afce6p-1, 0x1.526e57720db08p-3}, {0x1.9c2d163a1aa2dp-1, 0x1.bc2860d22477p-3},
    {0x1.886e6037841edp-1, 0x1.1058bc8a07ee1p-2}, {0x1.767dcf5534862p-1, 0x1.4043057b6ee09p-2}};
// positive normal finite x only (softplus passes 1 + expf(v) > 1); tab:
// kLogfTable or a copy of it in LDS
template <typename TAB>
__device__ __forceinline__ float logf_libm_t(float x, const TAB (*tab)[2]) {
    const uint32_t ix = __float_as_uint(x);
    if (ix == 0x3f800000u) return 0.0f;
    const uint32_t tmp = ix - 0x3f330000u;  // offset so that z lands in [0x1.66p-1, 0x1.66p0)
    const uint32_t i = (tmp >> 19) & 15u;
    const int k = static_cast<int32_t>(tmp) >> 23;
    const double z = static_cast<double>(__uint_as_float(ix - (tmp & 0xff800000u)));
    const double r = __builtin_fma(z, static_cast<double>(tab[i][0]), -1.0);
    const double y0 = static_cast<double>(tab[i][1]) + static_cast<double>(k) * 0x1.62e42fefa39efp-1;
    const double r2 = r * r;
    double y = __builtin_fma(0x1.5575b0be00b6ap-2, r, -0x1.ffffef20a4123p-2);
    y = __builtin_fma(-0x1.00ea348b88334p-2, r2, y);
    y = __builtin_fma(y, r2, y0 + r);
    return static_cast<float>(y);
}
__device__ __forceinline__ float logf_libm(float x) { return logf_libm_t(x, kLogfTable); }

// fortai_qwen35_cpu.f90:1506-1514
__device__ __forceinline__ float sigmoid_ref(float v) {
    if (v >= 0.0f) return 1.0f / (1.0f + exp_rounded(-v));
    const float e = exp_rounded(v);
    return e / (1.0f + e);
}

// fortai_qwen35_cpu.f90:1516-1526
__device__ __forceinline__ float softplus_ref(float v) {
    if (v > 20.0f) return v;
    if (v < -20.0f) return exp_rounded(v);
    return logf_libm(1.0f + exp_rounded(v));
}

// The expf and logf tables in LDS: a kernel whose critical path runs through
// those functions keeps them there, so that each lookup is an LDS read
// instead of a data-dependent memory round trip.  Same values, so the same
// results.  fetch() issues the table word of threads 0..63 as the kernel's
// first load (into a register, no wait); put() stores it once the kernel has
// issued its own loads, so that the wait for the table word does not hold
// them back (a load from memory followed by an LDS store of it waits for the
// load on the spot).  The stored tables are visible after the next barrier
// (or, for wave 0's own reads, after wave_lds_fence).
// x / n for a double x and a count n > 0, correctly rounded.  When n = 2^k
// the quotient is x scaled by 2^-k: ldexp rounds that same exact value the
// same way (bit-identical, subnormal results included) in one instruction
// instead of the division's dependent sequence.
__device__ __forceinline__ double div_count(double x, int n) {
    if ((n & (n - 1)) == 0) return __builtin_ldexp(x, -__builtin_ctz(static_cast<unsigned>(n)));
    return x / static_cast<double>(n);
}

// Cross-lane exchange through LDS within one wave: the writes of every lane
// are ordered before the reads that follow (no workgroup barrier needed).
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

struct MathTables {
    uint64_t exp2[32];
    double logc[16][2];
    __device__ __forceinline__ void load() { put(fetch()); }
    // word threadIdx.x of the tables (exp2 then logc; threads past 63 re-read word 63, unused)
    static __device__ __forceinline__ uint64_t fetch() {
        const int t = min(static_cast<int>(threadIdx.x), 63);
        const uint64_t *src = t < 32 ? kExpf2Table + t : reinterpret_cast<const uint64_t *>(&kLogfTable[0][0]) + (t - 32);
        return *src;
    }
    __device__ __forceinline__ void put(uint64_t word) {
        static_assert(sizeof(exp2) + sizeof(logc) == 64 * sizeof(uint64_t), "64 table words");
        const int t = static_cast<int>(threadIdx.x);
        if (t < 64) reinterpret_cast<uint64_t *>(this)[t] = word;
    }
    __device__ __forceinline__ float expf(float x) const { return expf_libm_t(x, exp2); }
    __device__ __forceinline__ float logf(float x) const { return logf_libm_t(x, logc); }
    // sigmoid_ref and softplus_ref with these tables
    __device__ __forceinline__ float sigmoid(float v) const {
        if (v >= 0.0f) return 1.0f / (1.0f + expf(-v));
        const float e = expf(v);
        return e / (1.0f + e);
    }
    __device__ __forceinline__ float softplus(float v) const {
        if (v > 20.0f) return v;
        if (v < -20.0f) return expf(v);
        return logf(1.0f + expf(v));
    }
};

// ------------------------------------------------------ streaming loads ----

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// Non-temporal 16/8-byte loads for weights that are streamed exactly once.
__device__ __forceinline__ uint4 load_stream(const uint4 *p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 load_stream(const uint2 *p) {
    const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t *>(p));
    return make_uint2(v.x, v.y);
}

// ------------------------------------------------------ kernel arguments ----

// Fetch every 64-byte line of the first BYTES of the kernel-argument segment
// into the scalar cache with one round trip.  A kernel's argument reads are
// scalar loads, and the compiler issues them where their values are first
// needed, so a prologue that reads a pointer, waits, loads through it and
// then reads the next argument pays one memory round trip per step; after
// this every later argument read hits the scalar cache.
// (One asm statement: the loads land in its own early-clobber register
// before the statement ends, so no later instruction can be handed that
// register while a load into it is still in flight.)
#define FORTAI_KW1 "s_load_dword %0, %1, 0x0\n"
#define FORTAI_KW2 FORTAI_KW1 "s_load_dword %0, %1, 0x40\n"
#define FORTAI_KW3 FORTAI_KW2 "s_load_dword %0, %1, 0x80\n"
#define FORTAI_KW4 FORTAI_KW3 "s_load_dword %0, %1, 0xc0\n"
#define FORTAI_KW5 FORTAI_KW4 "s_load_dword %0, %1, 0x100\n"
#define FORTAI_KW6 FORTAI_KW5 "s_load_dword %0, %1, 0x140\n"
#define FORTAI_KW7 FORTAI_KW6 "s_load_dword %0, %1, 0x180\n"
#define FORTAI_KW8 FORTAI_KW7 "s_load_dword %0, %1, 0x1c0\n"
#define FORTAI_KW9 FORTAI_KW8 "s_load_dword %0, %1, 0x200\n"
#define FORTAI_KW10 FORTAI_KW9 "s_load_dword %0, %1, 0x240\n"
#define FORTAI_KW11 FORTAI_KW10 "s_load_dword %0, %1, 0x280\n"
#define FORTAI_KW12 FORTAI_KW11 "s_load_dword %0, %1, 0x2c0\n"
template <int BYTES>
__device__ __forceinline__ void kernarg_warm() {
    constexpr int kLines = (BYTES + 63) / 64;
    static_assert(kLines >= 1 && kLines <= 12, "at most 12 lines");
    const auto k = __builtin_amdgcn_kernarg_segment_ptr();
    uint32_t t;
#define FORTAI_KW_CASE(n) \
    if constexpr (kLines == n) asm volatile(FORTAI_KW##n "s_waitcnt lgkmcnt(0)" : "=&s"(t) : "s"(k) : "memory");
    FORTAI_KW_CASE(1) FORTAI_KW_CASE(2) FORTAI_KW_CASE(3) FORTAI_KW_CASE(4) FORTAI_KW_CASE(5) FORTAI_KW_CASE(6)
    FORTAI_KW_CASE(7) FORTAI_KW_CASE(8) FORTAI_KW_CASE(9) FORTAI_KW_CASE(10) FORTAI_KW_CASE(11) FORTAI_KW_CASE(12)
#undef FORTAI_KW_CASE
}

// --------------------------------------------------------- reductions ----

// The value lane (lane ^ M) holds, M a power of two up to 32, in VALU
// operations only (a ds_bpermute costs an LDS round trip per exchange):
// DPP within 16-lane rows -- quad permutes for 1 and 2, the quad reversal
// then the half-row mirror for 4 ((l ^ 3) ^ 7 = l ^ 4), the row rotation by 8
// for 8 -- and the gfx950 permlane swaps across rows (16) and wave halves
// (32).  A swap of v with itself leaves {v.row0, v.row0, v.row2, v.row2} in
// its first result and {v.row1, v.row1, v.row3, v.row3} in its second (rows
// of 16 or 32 lanes), so a lane picks the one that is not its own row.
// Every lane of the wave must be active.
template <int M>
__device__ __forceinline__ uint32_t xor_lane_u32(uint32_t v) {
    static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "M: a power of two <= 32");
    const int x = static_cast<int>(v);
    if constexpr (M == 1) {
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));  // quad [1,0,3,2]
    } else if constexpr (M == 2) {
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false));  // quad [2,3,0,1]
    } else if constexpr (M == 4) {
        const int t = __builtin_amdgcn_update_dpp(0, x, 0x1B, 0xF, 0xF, false);          // quad [3,2,1,0]
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, t, 0x141, 0xF, 0xF, false));  // half-row mirror
    } else if constexpr (M == 8) {
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false));  // row rotate 8
    } else if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (__lane_id() & 16) ? r[0] : r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (__lane_id() & 32) ? r[0] : r[1];
    }
}

template <int M, typename T>
__device__ __forceinline__ T xor_lane(T v) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, xor_lane_u32<M>(__builtin_bit_cast(uint32_t, v)));
    } else {
        static_assert(sizeof(T) == 8, "4- or 8-byte values");
        const uint2 u = __builtin_bit_cast(uint2, v);
        return __builtin_bit_cast(T, make_uint2(xor_lane_u32<M>(u.x), xor_lane_u32<M>(u.y)));
    }
}

// Butterfly over the wave: v + v[lane ^ m] for m = 32, 16, ..., 1; every
// lane ends with the same value.
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
    v += xor_lane<32>(v);
    v += xor_lane<16>(v);
    v += xor_lane<8>(v);
    v += xor_lane<4>(v);
    v += xor_lane<2>(v);
    v += xor_lane<1>(v);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, xor_lane<32>(v));
    v = fmaxf(v, xor_lane<16>(v));
    v = fmaxf(v, xor_lane<8>(v));
    v = fmaxf(v, xor_lane<4>(v));
    v = fmaxf(v, xor_lane<2>(v));
    v = fmaxf(v, xor_lane<1>(v));
    return v;
}

// The butterfly sum over aligned groups of n lanes (n a power of two <= 64,
// uniform): m = 1, 2, ..., n / 2.
template <typename T>
__device__ __forceinline__ T group_sum_up(T v, int n) {
    if (n > 1) v += xor_lane<1>(v);
    if (n > 2) v += xor_lane<2>(v);
    if (n > 4) v += xor_lane<4>(v);
    if (n > 8) v += xor_lane<8>(v);
    if (n > 16) v += xor_lane<16>(v);
    if (n > 32) v += xor_lane<32>(v);
    return v;
}

// Horizontal sum of the 8 row lanes in the AVX2 order of
// fortai_q8_dot.c:323-330 / :345-353: (l + l^4), then (+ ^2), then (+ ^1).
// fp32 addition is commutative, so every lane of the group ends with the
// bit pattern lane 0 of the reference produces.
__device__ __forceinline__ float row_hsum8(float v) {
    v = v + xor_lane<4>(v);
    v = v + xor_lane<2>(v);
    v = v + xor_lane<1>(v);
    return v;
}

// ------------------------------------------------------- quantization ----

__device__ __forceinline__ int8_t sat8_rne(float v) {
    const float r = rintf(v);
    // cvtps_epi32 gives INT32_MIN for NaN/out of range, which packs to -128
    if (!(r >= -2147483648.0f && r < 2147483648.0f)) return -128;
    return static_cast<int8_t>(r < -128.0f ? -128.0f : (r > 127.0f ? 127.0f : r));
}


// Quantize one 4-value group of a 32-value block held by 8 consecutive lanes
// (lane l of the block holds values 4l..4l+3).  Returns the packed int8x4 and
// the block's fp32 scale (f32 of the fp16 RNE scale).
__device__ __forceinline__ uint32_t quantize_group(float4 y, float &scale_out, uint16_t &scale_bits) {
    float amax = fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w)));
    amax = fmaxf(amax, xor_lane<1>(amax));
    amax = fmaxf(amax, xor_lane<2>(amax));
    amax = fmaxf(amax, xor_lane<4>(amax));
    const float scale = amax / 127.0f;
    const float inverse = amax != 0.0f ? 127.0f / amax : 0.0f;
    scale_bits = float_to_half_rne(scale);
    scale_out = half_bits_to_float(scale_bits);
    const uint32_t q0 = static_cast<uint8_t>(sat8_rne(y.x * inverse));
    const uint32_t q1 = static_cast<uint8_t>(sat8_rne(y.y * inverse));
    const uint32_t q2 = static_cast<uint8_t>(sat8_rne(y.z * inverse));
    const uint32_t q3 = static_cast<uint8_t>(sat8_rne(y.w * inverse));
    return q0 | (q1 << 8) | (q2 << 16) | (q3 << 24);
}

// One 16-byte Q8L chunk (4 blocks) of a row lane: the reference's per-block
// acc = fma(f32(w_scale) * a_scale, (float)dot4(w, a), acc), block by block.
// sum of the four int8 products of a and b.  Kept on the builtin: the
// compiler then knows the result comes from a DOT instruction and pads the
// DOT-write -> other-VALU-read hazard (three wait states on gfx950), which
// it cannot do for an inline-asm dot.
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), 0, false);
}

// (float)sdot4 of four word pairs.  The three-operand dot with an inline
// zero addend saves the v_mov of a zero accumulator that the builtin's
// two-operand form needs (a fifth of the VALU work of the lane-exact
// matvecs).  A DOT result read by another VALU needs three wait states on
// gfx950, which the compiler inserts only for dots it emits itself: here the
// four dots come first, so three instructions separate each dot from its
// convert, and the early-clobber outputs keep every result register apart
// from the inputs of the later dots.
__device__ __forceinline__ float4 sdot4x4_f(uint4 q, uint4 a) {
    float4 r;
    asm("v_dot4_i32_i8 %0, %4, %8, 0\n\t"
        "v_dot4_i32_i8 %1, %5, %9, 0\n\t"
        "v_dot4_i32_i8 %2, %6, %10, 0\n\t"
        "v_dot4_i32_i8 %3, %7, %11, 0\n\t"
        "v_cvt_f32_i32 %0, %0\n\t"
        "v_cvt_f32_i32 %1, %1\n\t"
        "v_cvt_f32_i32 %2, %2\n\t"
        "v_cvt_f32_i32 %3, %3"
        : "=&v"(r.x), "=&v"(r.y), "=&v"(r.z), "=&v"(r.w)
        : "v"(q.x), "v"(q.y), "v"(q.z), "v"(q.w), "v"(a.x), "v"(a.y), "v"(a.z), "v"(a.w));
    return r;
}

// -0.0f that the compiler cannot see as a constant (so that an fma with it is
// not folded into a multiply); no inputs and no side effects, so it is
// computed once and hoisted
__device__ __forceinline__ float opaque_negzero() {
    float z;
    asm("v_mov_b32 %0, 0x80000000" : "=v"(z));
    return z;
}

// fl(f32(h) * a) for the low (HI = false) or high half h of a packed pair of
// fp16 bits: fma(f32(h), a, -0) widens exactly, multiplies and adds -0 (which
// leaves every product, zero or not, as it is) with one rounding -- the value
// of the convert-then-multiply.  The compiler selects v_fma_mix_f32 for it
// (one instruction) and, unlike for inline asm, knows its latencies.
template <bool HI>
__device__ __forceinline__ float half_times(uint32_t h2, float a) {
    typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
    const half2_t v = __builtin_bit_cast(half2_t, h2);
    return __builtin_fmaf(static_cast<float>(HI ? v.y : v.x), a, opaque_negzero());
}

__device__ __forceinline__ float dot_chunk(uint4 q, uint2 sc, uint4 a, float4 as, float acc) {
    const float4 d = sdot4x4_f(q, a);
    acc = __builtin_fmaf(half_times<false>(sc.x, as.x), d.x, acc);
    acc = __builtin_fmaf(half_times<true>(sc.x, as.y), d.y, acc);
    acc = __builtin_fmaf(half_times<false>(sc.y, as.z), d.z, acc);
    acc = __builtin_fmaf(half_times<true>(sc.y, as.w), d.w, acc);
    return acc;
}


}  // namespace fortai_hip
