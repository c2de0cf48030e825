// Q8_0 x Q8_0 matrix-matrix product on the i8 matrix cores (prefill / batched
// token blocks).
//
// The reference has no prefill: every token runs the matvec of
// fortai_gguf_runtime.f90:424-465, i.e. per row and block the exact int32 dot
// of 32 int8 products, scaled by f32(w_scale) * a_scale and accumulated in
// fp32 (fortai_q8_dot.c:262-284 scalar, :287-331 AVX2).  Here the int32 block
// dot of 32 tokens x 32 rows is one v_mfma_i32_32x32x32_i8 (exact: integer
// arithmetic), and the scale-and-accumulate of every (token, row, block) runs
// on the vector ALUs: acc = fma(f32(w_scale) * x_scale, f32(dot), acc), the
// scalar reference's form.  The AVX2 reference splits each block dot into
// eight 4-product lane partials before the fp32 accumulation, so results
// agree with it to fp32 rounding (relative 1e-5 class), not bit for bit; the
// per-block int32 dots are bit-exact and exported for testing.
//
// Token activations ("X8", written by q8_quantize_tokens_kernel):
//   q[(b * ld + t) * 32 + k]   int8 value k of block b of token t
//   s[b * ld + t]              f32 scale (the fp16-rounded reference scale)
// with ld = tokens rounded up to 128 and blocks padded to a multiple of 4;
// padding holds zeros.  The int8 part precedes the scales in one buffer of
// q8_tokens_bytes() bytes.
//
// Weights stay in the decode layout (q8_kernels.hip): lanes 4h..4h+3 of a
// row's 16-byte pieces hold its bytes 16h..16h+15 of four consecutive blocks,
// so a lane that loads those four pieces holds the B operand of four MFMAs
// with no shuffling.  Both operands present their 16 bytes in natural order,
// so the products pair up whatever k order the instruction uses internally.
#include "fortai_hip_internal.h"
#include "fortai_hip_kernels.h"


namespace fortai_hip {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kTokTile = 128;  // tokens per workgroup
constexpr int kRowTile = 128;  // rows per workgroup
constexpr int kMmqThreads = 256;

__device__ __forceinline__ v4i as_v4i(uint4 u) {
    v4i r;
    r.x = static_cast<int>(u.x); r.y = static_cast<int>(u.y);
    r.z = static_cast<int>(u.z); r.w = static_cast<int>(u.w);
    return r;
}

__device__ __forceinline__ uint32_t comp(const uint4 &u, int j) {
    return j == 0 ? u.x : (j == 1 ? u.y : (j == 2 ? u.z : u.w));
}

// LDS stage of one chunk (four blocks) of a 128-token x 128-row tile.
// Operand rows are 32 bytes; the two 16-byte halves of row n are stored
// swapped when bit 3 of n is set, so the 16-byte reads of 16 consecutive
// rows fall on distinct banks.
struct MmqStage {
    uint4 a[4][kTokTile][2];   // token bytes per block
    uint4 b[4][kRowTile][2];   // row bytes per block
    float as[4][kTokTile];     // token scales
    float bs[4][kRowTile];     // row scales (f32 of the fp16)
};

__device__ __forceinline__ int half_slot(int n, int h) { return h ^ ((n >> 3) & 1); }

// One workgroup: 128 tokens x 128 rows; wave w covers tokens 64 (w & 1) and
// rows 64 (w >> 1) as 2 x 2 MFMA tiles of 32 x 32.  Chunk c + 1 is loaded
// into registers while chunk c is consumed from LDS, then stored to the other
// stage (one barrier per chunk).
//   EPI 0: out[t * ld_out + row] = acc;  EPI 1: out = acc + resid (same index)
//   DOTS: also write every int32 block dot to dots[(t * rows + row) * blocks + b]
template <int EPI, bool DOTS>
__global__ __launch_bounds__(kMmqThreads, 2) void q8_mmq_kernel(Q8Matrix w, const int8_t *__restrict__ xq,
    const float *__restrict__ xs, int tokens, int ld, float *__restrict__ out, int ld_out,
    const float *__restrict__ resid, int32_t *__restrict__ dots) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    MmqStage *stage = reinterpret_cast<MmqStage *>(lds_raw);
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63, wave = tid >> 6;
    const int i = lane & 31, h = lane >> 5;
    const int t0 = static_cast<int>(blockIdx.y) * kTokTile;
    const int r0 = static_cast<int>(blockIdx.x) * kRowTile;
    const int twl = (wave & 1) * 64;   // wave's first token within the tile
    const int rwl = (wave >> 1) * 64;  // wave's first row within the tile
    const int chunks = w.chunks;
    const size_t bstride = static_cast<size_t>(ld) * 32;  // bytes per block of X8

    // global sources of this thread's share of a chunk:
    //  tokens: 4 blocks x 128 tokens x 2 halves = 1024 pieces, 4 per thread
    //  rows:   16 row groups x 64 lanes          = 1024 pieces, 4 per thread
    //  token scales: 512 floats, 2 per thread;  row scales: 128 x uint2, threads < 128
    const int g_last = w.row_groups - 1;
    u32x4_t ra[4], rb[4];  // plain vectors (arrays of the uint4 class stay in scratch)
    float rs[2];
    uint2 rws = make_uint2(0u, 0u);
    auto fetch = [&](int c) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int p = tid + k * kMmqThreads;          // 0..1023
            const int j = p >> 8, t = (p >> 1) & 127, hh = p & 1;
            ra[k] = *reinterpret_cast<const u32x4_t *>(xq + static_cast<size_t>(4 * c + j) * bstride +
                static_cast<size_t>(t0 + t) * 32 + hh * 16);
            const int g = min((r0 >> 3) + (p >> 6), g_last);  // clamped; rows past the end are not stored
            // cached loads: every token tile of the launch re-reads these rows
            rb[k] = reinterpret_cast<const u32x4_t *>(w.quants)[(static_cast<size_t>(g) * chunks + c) * 64 + (p & 63)];
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int p = tid + k * kMmqThreads;  // 0..511
            rs[k] = xs[static_cast<size_t>(4 * c + (p >> 7)) * ld + t0 + (p & 127)];
        }
        if (tid < kRowTile) {
            const int g = min((r0 >> 3) + (tid >> 3), g_last);
            rws = w.scales[(static_cast<size_t>(g) * chunks + c) * 8 + (tid & 7)];
        }
    };
    auto stash = [&](MmqStage &st) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int p = tid + k * kMmqThreads;
            const int j = p >> 8, t = (p >> 1) & 127, hh = p & 1;
            *reinterpret_cast<u32x4_t *>(&st.a[j][t][half_slot(t, hh)]) = ra[k];
        }
        // row piece: row (p >> 6) * 8 + r, bytes 4l..4l+3 of the four blocks
        uint32_t *dst = reinterpret_cast<uint32_t *>(&st.b[0][0][0]);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int p = tid + k * kMmqThreads;
            const int q = p & 63, r = q >> 3, l = q & 7;
            const int row = (p >> 6) * 8 + r;
            const int base = (row * 2 + half_slot(row, l >> 2)) * 4 + (l & 3);
            dst[base] = rb[k].x;
            dst[base + kRowTile * 8] = rb[k].y;
            dst[base + 2 * kRowTile * 8] = rb[k].z;
            dst[base + 3 * kRowTile * 8] = rb[k].w;
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int p = tid + k * kMmqThreads;
            st.as[p >> 7][p & 127] = rs[k];
        }
        if (tid < kRowTile) {
            st.bs[0][tid] = half_bits_to_float(static_cast<uint16_t>(rws.x & 0xffffu));
            st.bs[1][tid] = half_bits_to_float(static_cast<uint16_t>(rws.x >> 16));
            st.bs[2][tid] = half_bits_to_float(static_cast<uint16_t>(rws.y & 0xffffu));
            st.bs[3][tid] = half_bits_to_float(static_cast<uint16_t>(rws.y >> 16));
        }
    };

    float acc[2][2][16];
#pragma unroll
    for (int ta = 0; ta < 2; ++ta)
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[ta][f][v] = 0.0f;

    fetch(0);
    stash(stage[0]);
    __syncthreads();
    for (int c = 0; c < chunks; ++c) {
        const MmqStage &st = stage[c & 1];
        if (c + 1 < chunks) fetch(c + 1);
        // one block at a time (unrolled, the compiler hoists all 16 MFMAs of
        // the chunk and spills)
#pragma unroll 1
        for (int j = 0; j < 4; ++j) {
            uint4 af[2], bf[2];
            float wsc[2];
#pragma unroll
            for (int ta = 0; ta < 2; ++ta) {
                const int t = twl + 32 * ta + i;
                af[ta] = st.a[j][t][half_slot(t, h)];
            }
#pragma unroll
            for (int f = 0; f < 2; ++f) {
                const int row = rwl + 32 * f + i;
                bf[f] = st.b[j][row][half_slot(row, h)];
                wsc[f] = st.bs[j][row];
            }
#pragma unroll
            for (int ta = 0; ta < 2; ++ta) {
                // this lane's 16 tokens: twl + 32 ta + 8 (v / 4) + 4 h + v % 4
                float tsc[16];
                const float4 *s4 = reinterpret_cast<const float4 *>(&st.as[j][twl + 32 * ta + 4 * h]);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 s = s4[2 * q];
                    tsc[4 * q] = s.x; tsc[4 * q + 1] = s.y; tsc[4 * q + 2] = s.z; tsc[4 * q + 3] = s.w;
                }
#pragma unroll
                for (int f = 0; f < 2; ++f) {
                    const v16i zero = {};
                    const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(as_v4i(af[ta]), as_v4i(bf[f]), zero, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 16; ++v)
                        acc[ta][f][v] = __builtin_fmaf(wsc[f] * tsc[v], static_cast<float>(d[v]), acc[ta][f][v]);
                    // keep one MFMA result live at a time (the other wave of
                    // the SIMD covers the MFMA latency)
                    __builtin_amdgcn_sched_barrier(0);
                    if constexpr (DOTS) {
                        const int row = r0 + rwl + 32 * f + i, blk = 4 * c + j;
                        if (row < w.rows && blk < w.blocks) {
#pragma unroll
                            for (int v = 0; v < 16; ++v) {
                                const int t = t0 + twl + 32 * ta + 8 * (v >> 2) + 4 * h + (v & 3);
                                if (t < tokens) dots[(static_cast<size_t>(t) * w.rows + row) * w.blocks + blk] = d[v];
                            }
                        }
                    }
                }
            }
        }
        if (c + 1 < chunks) stash(stage[(c + 1) & 1]);
        __syncthreads();
    }
#pragma unroll
    for (int ta = 0; ta < 2; ++ta) {
#pragma unroll
        for (int f = 0; f < 2; ++f) {
            const int row = r0 + rwl + 32 * f + i;
            if (row >= w.rows) continue;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int t = t0 + twl + 32 * ta + 8 * (v >> 2) + 4 * h + (v & 3);
                if (t >= tokens) continue;
                const size_t o = static_cast<size_t>(t) * ld_out + row;
                if constexpr (EPI == 1) out[o] = acc[ta][f][v] + resid[o];
                else out[o] = acc[ta][f][v];
            }
        }
    }
}

// ------------------------------------------------------------- lane order
// The same product with the reference's AVX2 accumulation kept exactly
// (fortai_q8_dot.c:287-331): per (token, row) eight fp32 lane chains, lane L
// adding fma(f32(w_scale) * x_scale, f32(dot of bytes 4L..4L+3), acc_L) block
// by block, then the horizontal sum ((a0+a4)+(a2+a6))+((a1+a5)+(a3+a7)).  So
// every output is bit-identical to the decode matvec of that token.
//
// The 4-byte lane dots come from v_mfma_f32_16x16x4f16: four independent
// 16x16x4 products per instruction, one per lane part (lane l feeds block
// l / 16 with row or column l % 16; output register r of lane l is block
// r / 4, row 4 (l / 16) + r % 4, column l % 16), so two instructions give the
// eight lane dots of a 16 x 16 quadrant and block.  int8 values are exact in
// fp16, and the products and their 4-term sums (|sum| <= 4 * 128 * 127) are
// exact in the fp32 accumulator, so the dots arrive as exact floats and need
// no conversion.  Per lane dot the 16x16 shape costs the matrix cores what
// the 32x32x4 one does, with half the result registers, which leaves room
// for the next instruction's result while the vector ALUs run the fmas of
// the current one.  The int8 operands are widened to fp16 once, when a chunk
// (four blocks) is staged in LDS: the biased byte b + 128 under the fp16
// exponent of 1024 is 1024 + b + 128 exactly, and one packed fp16
// subtraction of 1152 leaves b.
//
// Staging: per block and token (or row) the eight 4-value lane parts in the
// order 0 4 1 5 2 6 3 7, so that the lane feeding block s reads parts s and
// s + 4 (one per instruction group) as 16 contiguous bytes.
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kXTile = 64;    // tokens and rows per workgroup (4 waves of 32 x 32)
constexpr int kXPitch = 36;   // halves per staged (block, token or row): 32 + 4 pad
constexpr int kXThreads = 256;

struct MmqExactStage {
    _Float16 a[4][kXTile][kXPitch];
    _Float16 b[4][kXTile][kXPitch];
    float as[4][kXTile];
    float bs[4][kXTile];
};

// the staged position of lane part L (order 0 4 1 5 2 6 3 7), in halves
__device__ __forceinline__ int part_slot(int L) { return ((L & 3) * 2 + (L >> 2)) * 4; }

// four signed bytes -> four fp16 values (exact)
__device__ __forceinline__ h4 i8x4_to_h4(uint32_t w) {
    const uint32_t u = w ^ 0x80808080u;  // b + 128
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const h2 bias = {static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
    const h2 a = __builtin_bit_cast(h2, lo) - bias;
    const h2 b = __builtin_bit_cast(h2, hi) - bias;
    return h4{a.x, a.y, b.x, b.y};
}

template <int EPI>
__global__ __launch_bounds__(kXThreads, 2) void q8_mmq_exact_kernel(Q8Matrix w, const int8_t *__restrict__ xq,
    const float *__restrict__ xs, int tokens, int ld, float *__restrict__ out, int ld_out,
    const float *__restrict__ resid) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    MmqExactStage *stage = reinterpret_cast<MmqExactStage *>(lds_raw);
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63, wave = tid >> 6;
    const int i = lane & 15, s4 = lane >> 4;  // quadrant row / column, and lane part (block) s4
    const int t0 = static_cast<int>(blockIdx.y) * kXTile;
    const int r0 = static_cast<int>(blockIdx.x) * kXTile;
    const int twl = (wave & 1) * 32;   // wave's first token within the tile
    const int rwl = (wave >> 1) * 32;  // wave's first row within the tile
    const int chunks = w.chunks;
    const size_t bstride = static_cast<size_t>(ld) * 32;  // bytes per block of X8
    const int g_last = w.row_groups - 1;

    // this thread's share of a chunk:
    //   tokens: 4 blocks x 64 tokens x 2 halves = 512 pieces of 16 bytes, 2 per thread
    //   rows:   8 row groups x 64 lanes         = 512 pieces of 16 bytes, 2 per thread
    //   token scales: 256 floats, 1 per thread; row scales: 64 x uint2, threads < 64
    u32x4_t ra[2], rb[2];
    float rs = 0.0f;
    uint2 rws = make_uint2(0u, 0u);
    auto fetch = [&](int c) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int p = tid + k * kXThreads;  // 0..511
            // a wave takes one (block, half) and 64 tokens, lane = token, so
            // that its LDS stores (rows 18 dwords apart) meet no bank twice
            const int j = p >> 7, hh = (p >> 6) & 1, t = p & 63;
            ra[k] = *reinterpret_cast<const u32x4_t *>(xq + static_cast<size_t>(4 * c + j) * bstride +
                static_cast<size_t>(t0 + t) * 32 + hh * 16);
            const int g = min((r0 >> 3) + (p >> 6), g_last);  // clamped; rows past the end are not stored
            rb[k] = reinterpret_cast<const u32x4_t *>(w.quants)[(static_cast<size_t>(g) * chunks + c) * 64 + (p & 63)];
        }
        rs = xs[static_cast<size_t>(4 * c + (tid >> 6)) * ld + t0 + (tid & 63)];
        if (tid < kXTile) {
            const int g = min((r0 >> 3) + (tid >> 3), g_last);
            rws = w.scales[(static_cast<size_t>(g) * chunks + c) * 8 + (tid & 7)];
        }
    };
    auto stash = [&](MmqExactStage &st) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int p = tid + k * kXThreads;
            const int j = p >> 7, hh = (p >> 6) & 1, t = p & 63;
            const uint32_t wd[4] = {ra[k].x, ra[k].y, ra[k].z, ra[k].w};
#pragma unroll
            for (int m = 0; m < 4; ++m)
                *reinterpret_cast<h4 *>(&st.a[j][t][part_slot(4 * hh + m)]) = i8x4_to_h4(wd[m]);
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            // row piece: row (p >> 6) * 8 + r, lane part l of the four blocks
            const int p = tid + k * kXThreads;
            const int q = p & 63, r = q >> 3, l = q & 7;
            const int row = (p >> 6) * 8 + r;
            const uint32_t wd[4] = {rb[k].x, rb[k].y, rb[k].z, rb[k].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) *reinterpret_cast<h4 *>(&st.b[j][row][part_slot(l)]) = i8x4_to_h4(wd[j]);
        }
        st.as[tid >> 6][tid & 63] = rs;
        if (tid < kXTile) {
            st.bs[0][tid] = half_bits_to_float(static_cast<uint16_t>(rws.x & 0xffffu));
            st.bs[1][tid] = half_bits_to_float(static_cast<uint16_t>(rws.x >> 16));
            st.bs[2][tid] = half_bits_to_float(static_cast<uint16_t>(rws.y & 0xffffu));
            st.bs[3][tid] = half_bits_to_float(static_cast<uint16_t>(rws.y >> 16));
        }
    };

    float acc[8][16];
#pragma unroll
    for (int L = 0; L < 8; ++L)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[L][v] = 0.0f;

    fetch(0);
    stash(stage[0]);
    __syncthreads();
    for (int c = 0; c < chunks; ++c) {
        const MmqExactStage &st = stage[c & 1];
        if (c + 1 < chunks) fetch(c + 1);
#pragma unroll 1
        for (int j = 0; j < 4; ++j) {
            // parts s4 and s4 + 4 of tokens twl + 16 th + i and rows rwl + 16 rh + i
            h4 av[2][2], bv[2][2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const h4 *ap = reinterpret_cast<const h4 *>(&st.a[j][twl + 16 * q + i][8 * s4]);
                const h4 *bp = reinterpret_cast<const h4 *>(&st.b[j][rwl + 16 * q + i][8 * s4]);
                av[q][0] = ap[0];
                av[q][1] = ap[1];
                bv[q][0] = bp[0];
                bv[q][1] = bp[1];
            }
            // scale products of this lane's outputs: tokens twl + 16 th + 4 s4 + u, rows rwl + 16 rh + i
            float sc[2][2][4];
#pragma unroll
            for (int rh = 0; rh < 2; ++rh) {
                const float wsc = st.bs[j][rwl + 16 * rh + i];
#pragma unroll
                for (int th = 0; th < 2; ++th) {
                    const float4 a4 = *reinterpret_cast<const float4 *>(&st.as[j][twl + 16 * th + 4 * s4]);
                    sc[th][rh][0] = wsc * a4.x;
                    sc[th][rh][1] = wsc * a4.y;
                    sc[th][rh][2] = wsc * a4.z;
                    sc[th][rh][3] = wsc * a4.w;
                }
            }
            // eight instructions (part group g, token half th, row half rh),
            // each issued before the fmas of the previous one
            const f32x16 zero = {};
            f32x16 d = __builtin_amdgcn_mfma_f32_16x16x4f16(av[0][0], bv[0][0], zero, 0, 0, 0);
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                const int g = m >> 2, th = (m >> 1) & 1, rh = m & 1;
                f32x16 dn = zero;
                if (m < 7) {
                    const int g1 = (m + 1) >> 2, th1 = ((m + 1) >> 1) & 1, rh1 = (m + 1) & 1;
                    dn = __builtin_amdgcn_mfma_f32_16x16x4f16(av[th1][g1], bv[rh1][g1], zero, 0, 0, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float &a_ = acc[4 * g + (r >> 2)][8 * th + 4 * rh + (r & 3)];
                    a_ = __builtin_fmaf(sc[th][rh][r & 3], d[r], a_);
                }
                __builtin_amdgcn_sched_barrier(0);
                d = dn;
            }
        }
        if (c + 1 < chunks) stash(stage[(c + 1) & 1]);
        __syncthreads();
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        // position v: token half v / 8, row half (v / 4) % 2, token 4 s4 + v % 4 of the half
        const int row = r0 + rwl + 16 * ((v >> 2) & 1) + i;
        const int t = t0 + twl + 16 * (v >> 3) + 4 * s4 + (v & 3);
        if (row >= w.rows || t >= tokens) continue;
        // the horizontal sum of fortai_q8_dot.c:323-330
        const float sum = ((acc[0][v] + acc[4][v]) + (acc[2][v] + acc[6][v])) +
            ((acc[1][v] + acc[5][v]) + (acc[3][v] + acc[7][v]));
        const size_t o = static_cast<size_t>(t) * ld_out + row;
        if constexpr (EPI == 1) out[o] = sum + resid[o];
        else out[o] = sum;
    }
}

// fortai_q8_quantize (fortai_q8_dot.c:153-198) of every token into X8: one
// thread per 4 values, 8 consecutive threads per block.
__global__ __launch_bounds__(256) void q8_quantize_tokens_kernel(const float *__restrict__ x, int tokens, int width,
    int ld_x, int ld, int blocks_pad, int8_t *__restrict__ xq, float *__restrict__ xs) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    const int groups_pad = blocks_pad * 8;
    const int t = static_cast<int>(idx / groups_pad), g = static_cast<int>(idx % groups_pad);
    if (t >= ld) return;  // whole 8-lane blocks exit together (groups_pad % 8 == 0)
    float4 y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (t < tokens && g < width / 4) y = reinterpret_cast<const float4 *>(x + static_cast<size_t>(t) * ld_x)[g];
    float scale;
    uint16_t bits;
    const uint32_t packed = quantize_group(y, scale, bits);
    const int b = g >> 3, l = g & 7;
    reinterpret_cast<uint32_t *>(xq + (static_cast<size_t>(b) * ld + t) * 32)[l] = packed;
    if (l == 0) xs[static_cast<size_t>(b) * ld + t] = scale;
}

}  // namespace

int q8_tokens_ld(int tokens) { return (tokens + kTokTile - 1) / kTokTile * kTokTile; }

size_t q8_tokens_bytes(int tokens, int width) {
    const size_t blocks_pad = static_cast<size_t>((width / kQ8Block + 3) / 4) * 4;
    return static_cast<size_t>(q8_tokens_ld(tokens)) * blocks_pad * (32 + 4);
}

hipError_t launch_q8_quantize_tokens(const float *x, int tokens, int width, int ld_x, void *x8, hipStream_t stream) {
    if (tokens <= 0 || width <= 0 || width % kQ8Block || ld_x < width || ld_x % 4) return hipErrorInvalidValue;
    const int ld = q8_tokens_ld(tokens);
    const int blocks_pad = (width / kQ8Block + 3) / 4 * 4;
    int8_t *xq = static_cast<int8_t *>(x8);
    float *xs = reinterpret_cast<float *>(xq + static_cast<size_t>(ld) * blocks_pad * 32);
    const size_t threads = static_cast<size_t>(ld) * blocks_pad * 8;
    hipLaunchKernelGGL(q8_quantize_tokens_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0,
        stream, x, tokens, width, ld_x, ld, blocks_pad, xq, xs);
    return hipGetLastError();
}

hipError_t launch_q8_mmq_exact(const Q8Matrix &w, const void *x8, int tokens, float *out, int ld_out,
    const float *resid, hipStream_t stream) {
    if (tokens <= 0 || ld_out < w.rows || w.rows <= 0) return hipErrorInvalidValue;
    const int ld = q8_tokens_ld(tokens);  // a multiple of the 64-token tile
    const int8_t *xq = static_cast<const int8_t *>(x8);
    const float *xs = reinterpret_cast<const float *>(xq + static_cast<size_t>(ld) * w.chunks * 4 * 32);
    const dim3 grid((w.rows + kXTile - 1) / kXTile, (tokens + kXTile - 1) / kXTile);
    const size_t lds = 2 * sizeof(MmqExactStage);
    if (resid)
        hipLaunchKernelGGL((q8_mmq_exact_kernel<1>), grid, dim3(kXThreads), lds, stream, w, xq, xs, tokens, ld, out,
            ld_out, resid);
    else
        hipLaunchKernelGGL((q8_mmq_exact_kernel<0>), grid, dim3(kXThreads), lds, stream, w, xq, xs, tokens, ld, out,
            ld_out, resid);
    note_launch("q8_mmq_exact_kernel<%s> grid %dx%d", resid ? "add" : "store", grid.x, grid.y);
    return hipGetLastError();
}

hipError_t launch_q8_mmq(const Q8Matrix &w, const void *x8, int tokens, float *out, int ld_out, const float *resid,
    int32_t *dots, hipStream_t stream) {
    if (tokens <= 0 || ld_out < w.rows || w.rows <= 0) return hipErrorInvalidValue;
    const int ld = q8_tokens_ld(tokens);
    const int8_t *xq = static_cast<const int8_t *>(x8);
    const float *xs = reinterpret_cast<const float *>(xq + static_cast<size_t>(ld) * w.chunks * 4 * 32);
    const dim3 grid((w.rows + kRowTile - 1) / kRowTile, ld / kTokTile);
    const size_t lds = 2 * sizeof(MmqStage);
    if (dots)
        hipLaunchKernelGGL((q8_mmq_kernel<0, true>), grid, dim3(kMmqThreads), lds, stream, w, xq, xs, tokens, ld, out,
            ld_out, resid, dots);
    else if (resid)
        hipLaunchKernelGGL((q8_mmq_kernel<1, false>), grid, dim3(kMmqThreads), lds, stream, w, xq, xs, tokens, ld, out,
            ld_out, resid, dots);
    else
        hipLaunchKernelGGL((q8_mmq_kernel<0, false>), grid, dim3(kMmqThreads), lds, stream, w, xq, xs, tokens, ld, out,
            ld_out, resid, dots);
    note_launch("q8_mmq_kernel<%s> grid %dx%d", resid ? "add" : "store", grid.x, grid.y);
    return hipGetLastError();
}

}  // namespace fortai_hip
