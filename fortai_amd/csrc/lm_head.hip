// fp16 LM head (tied token embedding) with a fused greedy argmax.
//
// The reference evaluates an F16 matrix row by row with a sequential fp32 dot,
// value(i) * x(i) accumulated left to right (fortai_gguf_runtime.f90:382-386,
// :390-422), and no activation quantisation.  Each thread here owns one row
// and runs exactly that chain, so the logits are bit-identical to the CPU
// path.  To keep the HBM stream coalesced, a 128-row x 128-column fp16 tile
// (full 128-byte lines) is staged through LDS, with the next two tiles in
// registers while one is consumed (measured: 6.3 TB/s, against 5.9 with
// 256 x 64 tiles and one tile ahead).
//
// The greedy step (maxloc, first maximum; app/fortai_cpu_run.f90:58) is
// fused: every workgroup reduces its 128 rows to (value, first index) and a
// one-workgroup follow-up kernel reduces the partials, writes the token,
// appends it to the trace and advances the device position, so a captured
// graph can replay decode steps back to back.  Tables without exponent-31
// halves (checked once at upload) use the plain hardware conversion.
#include "fortai_hip_internal.h"
#include "fortai_hip_kernels.h"

namespace fortai_hip {

namespace {

constexpr int kRows = 128;      // rows per workgroup (one per thread)

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

template <int M>
__device__ __forceinline__ void argmax_step(float &v, int &i) {
    const float ov = xor_lane<M>(v);
    const int oi = xor_lane<M>(i);
    if (better(ov, oi, v, i)) { v = ov; i = oi; }
}

// (value, index) first-maximum reduction over the workgroup; result valid in
// thread 0.
__device__ __forceinline__ void block_argmax(float &v, int &i, float *sv, int *si) {
    argmax_step<32>(v, i);
    argmax_step<16>(v, i);
    argmax_step<8>(v, i);
    argmax_step<4>(v, i);
    argmax_step<2>(v, i);
    argmax_step<1>(v, i);
    const int tid = static_cast<int>(threadIdx.x);
    const int waves = static_cast<int>(blockDim.x) >> 6;
    if ((tid & 63) == 0) { sv[tid >> 6] = v; si[tid >> 6] = i; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < waves; ++w)
            if (better(sv[w], si[w], v, i)) { v = sv[w]; i = si[w]; }
    }
}

// Reduce the per-workgroup (value, first index) partials and publish the
// greedy token; the trace append and the position advance let a captured
// graph replay decode steps back to back.
__global__ __launch_bounds__(256) void argmax_finish_kernel(int partials, ArgmaxState st) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int tid = static_cast<int>(threadIdx.x);
    const int seq = static_cast<int>(blockIdx.y);  // batch: sequence seq's partials, token, trace, position
    st.partial_value += static_cast<size_t>(seq) * partials;
    st.partial_index += static_cast<size_t>(seq) * partials;
    st.token += seq;
    if (st.trace) st.trace += static_cast<size_t>(seq) * st.trace_capacity;
    if (st.position) st.position += seq;
    if (st.embed && *st.embed >= 0) return;  // already finished (uniform)
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
    for (int w = tid; w < partials; w += 256)
        if (better(st.partial_value[w], st.partial_index[w], bv, bi)) { bv = st.partial_value[w]; bi = st.partial_index[w]; }
    block_argmax(bv, bi, sv, si);
    if (tid == 0) {
        // no candidate (every logit NaN): the first index, as maxloc over
        // comparisons that all fail; never an id outside the vocabulary
        const int64_t token = bi == 0x7fffffff ? 0 : bi;
        *st.token = token;
        if (st.position) {
            const int p = *st.position;
            if (st.trace && p >= 0 && p < st.trace_capacity) st.trace[p] = token;
            *st.position = p + 1;
        }
        if (st.embed) *st.embed = token;
    }
}

// The decode step's token embedding with the previous step's argmax finish
// folded in (launch_step_embedding).  Every workgroup that finds *embed < 0
// reduces all partials itself (the same first-maximum rule and all-NaN
// fallback as argmax_finish_kernel), so no workgroup depends on another's
// writes; only workgroup 0 writes token, trace[position] and position + 1,
// which no other workgroup of this launch reads.  *embed is left as it is:
// the next LM head writes -1 again, a finish writes the token.
__global__ __launch_bounds__(256) void step_embedding_kernel(const uint16_t *table16, Q8Matrix table8, int rows,
    int width, ArgmaxState st, int partials, float *out) {
    FORTAI_TRACE_SCOPE(6);
    __shared__ float sv[4];
    __shared__ int si[4];
    __shared__ int64_t chosen;
    const int tid = static_cast<int>(threadIdx.x);
    int64_t t = *st.embed;  // uniform
    if (t < 0) {
        float bv = -__builtin_inff();
        int bi = 0x7fffffff;
        // the first 8 * 256 partials in one round trip (clamped; duplicates
        // of the last partial change no first maximum), in the loop's order
        constexpr int kHeldParts = 8;
        float pv[kHeldParts];
        int pi[kHeldParts];
#pragma unroll
        for (int k = 0; k < kHeldParts; ++k) {
            const int w = min(tid + k * 256, partials - 1);
            pv[k] = st.partial_value[w];
            pi[k] = st.partial_index[w];
        }
#pragma unroll
        for (int k = 0; k < kHeldParts; ++k)
            if (better(pv[k], pi[k], bv, bi)) { bv = pv[k]; bi = pi[k]; }
        for (int w = tid + kHeldParts * 256; w < partials; w += 256)
            if (better(st.partial_value[w], st.partial_index[w], bv, bi)) { bv = st.partial_value[w]; bi = st.partial_index[w]; }
        block_argmax(bv, bi, sv, si);
        if (tid == 0) {
            const int64_t token = bi == 0x7fffffff ? 0 : bi;
            chosen = token;
            if (blockIdx.x == 0) {
                *st.token = token;
                const int p = *st.position;
                if (st.trace && p >= 0 && p < st.trace_capacity) st.trace[p] = token;
                *st.position = p + 1;
            }
        }
        __syncthreads();
        t = chosen;
    }
    if (t < 0 || t >= rows) t = 0;  // a device-fed id is never trusted as an address
    const int i = static_cast<int>(blockIdx.x) * 256 + tid;
    if (i >= width) return;
    if (table16) {
        out[i] = gguf_half_to_real(table16[t * width + i]);
        return;
    }
    // Q8_0 row t in the repacked layout: value i is byte i % 4 of lane part
    // (i % 32) / 4 of block i / 32
    const int g = static_cast<int>(t >> 3), r = static_cast<int>(t & 7);
    const int b = i / kQ8Block, within = i % kQ8Block, l = within >> 2, byte = within & 3;
    const int c = b >> 2, j = b & 3;
    const uint32_t *q32 = reinterpret_cast<const uint32_t *>(table8.quants);
    const uint32_t word = q32[((static_cast<size_t>(g) * table8.chunks + c) * 64 + r * 8 + l) * 4 + j];
    const int8_t q = static_cast<int8_t>((word >> (8 * byte)) & 0xffu);
    const uint16_t *s16 = reinterpret_cast<const uint16_t *>(table8.scales);
    const uint16_t sb = s16[((static_cast<size_t>(g) * table8.chunks + c) * 8 + r) * 4 + j];
    out[i] = half_bits_to_float(sb) * static_cast<float>(q);
}

// TILE fp16 columns per LDS tile (row pitch TILE + 8 halves: eight 16-byte
// reads of consecutive rows start on distinct 4-bank groups); two tiles are in
// flight in registers while one is consumed.
template <bool RMS, bool ARGMAX, bool FINITE, int TILE>
__global__ __launch_bounds__(kRows) void f16_matvec_kernel(const uint16_t *__restrict__ w, int rows, int width,
    const float *__restrict__ x, const float *__restrict__ norm, float eps, float *__restrict__ out,
    ArgmaxState st) {
    FORTAI_TRACE_SCOPE(7);
    constexpr int kPitch = TILE + 8;
    extern __shared__ __align__(16) unsigned char lds[];
    uint16_t *tile = reinterpret_cast<uint16_t *>(lds);
    float *xs = reinterpret_cast<float *>(lds + kRows * kPitch * 2);
    __shared__ double red[kRows / 64];
    __shared__ float sv[kRows / 64];
    __shared__ int si[kRows / 64];
    const int tid = static_cast<int>(threadIdx.x);
    const int row0 = static_cast<int>(blockIdx.x) * kRows;

    // tile loads: load j of thread t covers row (t + kRows j) / (TILE/8),
    // 16-byte segment (t + kRows j) % (TILE/8) of the row's TILE-column slice
    constexpr int kSegs = TILE / 8;
    constexpr int kLoads = TILE * 2 / 16;  // per thread and tile
    uint4 ra[kLoads], rb[kLoads];
    auto fetch = [&](int k0, uint4 (&regs)[kLoads]) {
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int li = tid + kRows * j;
            const int r = li / kSegs, seg = li % kSegs;
            const int grow = min(row0 + r, rows - 1);  // rows past the end re-read the last row
            regs[j] = load_stream(reinterpret_cast<const uint4 *>(w + static_cast<size_t>(grow) * width + k0 + seg * 8));
        }
    };
    auto stash = [&](const uint4 (&regs)[kLoads]) {
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int li = tid + kRows * j;
            const int r = li / kSegs, seg = li % kSegs;
            *reinterpret_cast<uint4 *>(tile + r * kPitch + seg * 8) = regs[j];
        }
    };
    const int tiles = width / TILE;
    // x and the norm weights of the first kXRegs * kRows columns first, into
    // registers (clamped, unconditional), then the first two tiles: the
    // RMSNorm then waits for x only, not for the tiles behind it
    constexpr int kXRegs = 8;
    float xr[kXRegs], nr[kXRegs];
#pragma unroll
    for (int k = 0; k < kXRegs; ++k) {
        const int i = min(tid + k * kRows, width - 1);
        xr[k] = x[i];
        nr[k] = RMS ? norm[i] : 0.0f;
    }
    fetch(0, ra);
    fetch(min(TILE, width - TILE), rb);  // (one tile: a harmless second copy)

    // x (optionally RMS-normalised, fortai_qwen35_cpu.f90:707) into LDS; each
    // thread sums its columns tid, tid + kRows, ... in order
    float inv = 1.0f;
    if constexpr (RMS) {
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < kXRegs; ++k)
            if (tid + k * kRows < width) ss += static_cast<double>(xr[k]) * static_cast<double>(xr[k]);
        for (int i = tid + kXRegs * kRows; i < width; i += kRows) ss += static_cast<double>(x[i]) * static_cast<double>(x[i]);
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        double total = 0.0;
        for (int i = 0; i < kRows / 64; ++i) total += red[i];
        inv = 1.0f / sqrtf(static_cast<float>(div_count(total, width)) + eps);
    }
#pragma unroll
    for (int k = 0; k < kXRegs; ++k) {
        const int i = tid + k * kRows;
        if (i < width) xs[i] = RMS ? (xr[k] * inv) * nr[k] : xr[k];
    }
    for (int i = tid + kXRegs * kRows; i < width; i += kRows) xs[i] = RMS ? (x[i] * inv) * norm[i] : x[i];

    // each thread's row: the reference's sequential chain value(i) * x(i)
    float acc = 0.0f;
    auto consume = [&](int k0) {
        const uint16_t *mine = tile + tid * kPitch;
#pragma unroll
        for (int s = 0; s < TILE / 8; ++s) {
            const uint4 h8 = *reinterpret_cast<const uint4 *>(mine + s * 8);
            const uint32_t hw[4] = {h8.x, h8.y, h8.z, h8.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float a = FINITE ? half_bits_to_float(static_cast<uint16_t>(hw[q] & 0xffffu))
                                       : gguf_half_to_real(static_cast<uint16_t>(hw[q] & 0xffffu));
                const float b = FINITE ? half_bits_to_float(static_cast<uint16_t>(hw[q] >> 16))
                                       : gguf_half_to_real(static_cast<uint16_t>(hw[q] >> 16));
                const int k = k0 + s * 8 + q * 2;
                acc = acc + a * xs[k];
                acc = acc + b * xs[k + 1];
            }
        }
    };
    for (int t = 0; t < tiles; t += 2) {
        __syncthreads();  // previous tile consumed (and xs written on the first pass)
        stash(ra);
        __syncthreads();
        if (t + 2 < tiles) fetch((t + 2) * TILE, ra);
        consume(t * TILE);
        if (t + 1 >= tiles) break;
        __syncthreads();
        stash(rb);
        __syncthreads();
        if (t + 3 < tiles) fetch((t + 3) * TILE, rb);
        consume((t + 1) * TILE);
    }
    const int row = row0 + tid;
    if (row < rows) out[row] = acc;
    if constexpr (ARGMAX) {
        float v = row < rows ? acc : -__builtin_inff();
        int i = row < rows ? row : 0x7fffffff;
        block_argmax(v, i, sv, si);
        if (tid == 0) {
            st.partial_value[blockIdx.x] = v;
            st.partial_index[blockIdx.x] = i;
            if (st.embed && blockIdx.x == 0) *st.embed = -1;  // the next step's embedding finishes the argmax
        }
    }
}

// Batched LM head: the fp16 table is read once for `batch` sequences.  Each
// thread owns one row and runs, for every sequence, the same sequential chain
// as f16_matvec_kernel (same tile order, same mul-then-add), and the final
// RMSNorm of each sequence uses that kernel's reduction layout (128 strided
// partial sums, then the two wave sums in order), so each sequence's logits
// equal the single-sequence kernel's bit for bit.  256 rows x 64 columns per
// tile; x of every sequence through scalar loads; per-sequence argmax partials.
constexpr int kBatchRows = 256;
constexpr int kBatchTile = 64;
constexpr int kXCols = 8;  // columns of x per scalar-load batch in the batched LM head
constexpr int kMaxBatch = 8;

// Final RMSNorm of each sequence (fortai_qwen35_cpu.f90:707), one workgroup
// of 128 threads per sequence with the single-sequence LM head's partition of
// the sum (128 strided partial sums in double, the two wave sums in order), so
// xnorm equals the x that kernel multiplies, bit for bit.  xnorm is
// interleaved, [width][kMaxBatch]: workgroup s writes slot s with sequence
// min(s, batch - 1), so the slots past the batch repeat the last sequence.
__global__ __launch_bounds__(128) void batch_output_norm_kernel(const float *__restrict__ x,
    const float *__restrict__ norm, float eps, int width, int batch, float *__restrict__ xnorm) {
    FORTAI_TRACE_SCOPE(14);
    __shared__ double red[2];
    const int tid = static_cast<int>(threadIdx.x);
    const int slot = static_cast<int>(blockIdx.x);
    const size_t base = static_cast<size_t>(min(slot, batch - 1)) * width;
    double ss = 0.0;
#pragma unroll 8
    for (int i = tid; i < width; i += 128) ss += static_cast<double>(x[base + i]) * static_cast<double>(x[base + i]);
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    double total = 0.0;
    total += red[0];
    total += red[1];
    const float inv = 1.0f / sqrtf(static_cast<float>(div_count(total, width)) + eps);
#pragma unroll 8
    for (int i = tid; i < width; i += 128) xnorm[static_cast<size_t>(i) * kMaxBatch + slot] = (x[base + i] * inv) * norm[i];
}

// xn: the normalized x of every sequence slot, interleaved [width][kMaxBatch].
// Its addresses are uniform across the workgroup, so the 32 values of four
// columns arrive by scalar loads into SGPRs and feed the VALU as operands: no
// LDS traffic and no VGPRs for x (which would otherwise hold 64 floats per
// column group and cap the occupancy at one wave per SIMD).
template <bool FINITE>
__global__ __launch_bounds__(kBatchRows) void f16_batch_lm_head_kernel(const uint16_t *__restrict__ w, int rows,
    int width, int batch, const float *__restrict__ xn, float *__restrict__ out, ArgmaxState st) {
    constexpr int kPitch = kBatchTile + 8;
    extern __shared__ __align__(16) unsigned char lds[];
    uint16_t *tile = reinterpret_cast<uint16_t *>(lds);
    __shared__ float sv[kBatchRows / 64];
    __shared__ int si[kBatchRows / 64];
    const int tid = static_cast<int>(threadIdx.x);
    const int row0 = static_cast<int>(blockIdx.x) * kBatchRows;

    constexpr int kSegs = kBatchTile / 8;
    constexpr int kLoads = kBatchTile * 2 / 16;  // 16-byte loads per thread and tile (one row's worth)
    uint4 ra[kLoads], rb[kLoads];
    auto fetch = [&](int k0, uint4 (&regs)[kLoads]) {
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int li = tid + kBatchRows * j;
            const int r = li / kSegs, seg = li % kSegs;
            const int grow = min(row0 + r, rows - 1);
            regs[j] = load_stream(reinterpret_cast<const uint4 *>(w + static_cast<size_t>(grow) * width + k0 + seg * 8));
        }
    };
    auto stash = [&](const uint4 (&regs)[kLoads]) {
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int li = tid + kBatchRows * j;
            const int r = li / kSegs, seg = li % kSegs;
            *reinterpret_cast<uint4 *>(tile + r * kPitch + seg * 8) = regs[j];
        }
    };
    const int tiles = width / kBatchTile;
    fetch(0, ra);
    if (tiles > 1) fetch(kBatchTile, rb);

    // every sequence slot is computed (slots past the batch repeat the last
    // sequence and are not written): no per-sequence branch in the inner loop
    float acc[kMaxBatch];
#pragma unroll
    for (int s = 0; s < kMaxBatch; ++s) acc[s] = 0.0f;
    // kXCols columns per scalar-load round trip (8 x kXCols SGPRs of x; the
    // wait for them is a full lgkmcnt(0), so more columns per load means
    // fewer exposed waits; the other waves of the SIMD cover the rest)
    auto xload = [&](int k, float (&xv)[kXCols][kMaxBatch]) {
        const float4 *src = reinterpret_cast<const float4 *>(xn + static_cast<size_t>(k) * kMaxBatch);
#pragma unroll
        for (int i = 0; i < kXCols * kMaxBatch / 4; ++i) {
            const float4 v = src[i];
            xv[i / 2][(i % 2) * 4 + 0] = v.x;
            xv[i / 2][(i % 2) * 4 + 1] = v.y;
            xv[i / 2][(i % 2) * 4 + 2] = v.z;
            xv[i / 2][(i % 2) * 4 + 3] = v.w;
        }
    };
    auto step = [&](const uint16_t *mine, int c, const float (&xv)[kXCols][kMaxBatch], int x0) {
        const uint2 h4 = *reinterpret_cast<const uint2 *>(mine + c * 4);
        float a[4];
        a[0] = FINITE ? half_bits_to_float(static_cast<uint16_t>(h4.x & 0xffffu))
                      : gguf_half_to_real(static_cast<uint16_t>(h4.x & 0xffffu));
        a[1] = FINITE ? half_bits_to_float(static_cast<uint16_t>(h4.x >> 16))
                      : gguf_half_to_real(static_cast<uint16_t>(h4.x >> 16));
        a[2] = FINITE ? half_bits_to_float(static_cast<uint16_t>(h4.y & 0xffffu))
                      : gguf_half_to_real(static_cast<uint16_t>(h4.y & 0xffffu));
        a[3] = FINITE ? half_bits_to_float(static_cast<uint16_t>(h4.y >> 16))
                      : gguf_half_to_real(static_cast<uint16_t>(h4.y >> 16));
#pragma unroll
        for (int s = 0; s < kMaxBatch; ++s) {
            float v = acc[s];
            v = v + a[0] * xv[x0][s]; v = v + a[1] * xv[x0 + 1][s]; v = v + a[2] * xv[x0 + 2][s];
            v = v + a[3] * xv[x0 + 3][s];
            acc[s] = v;
        }
    };
    auto consume = [&](int k0) {
        const uint16_t *mine = tile + tid * kPitch;
#pragma unroll 1
        for (int c = 0; c < kBatchTile / 4; c += kXCols / 4) {
            float xv[kXCols][kMaxBatch];
            xload(k0 + c * 4, xv);
#pragma unroll
            for (int u = 0; u < kXCols / 4; ++u) step(mine, c + u, xv, 4 * u);
        }
    };
    for (int t = 0; t < tiles; t += 2) {
        __syncthreads();
        stash(ra);
        __syncthreads();
        if (t + 2 < tiles) fetch((t + 2) * kBatchTile, ra);
        consume(t * kBatchTile);
        if (t + 1 >= tiles) break;
        __syncthreads();
        stash(rb);
        __syncthreads();
        if (t + 3 < tiles) fetch((t + 3) * kBatchTile, rb);
        consume((t + 1) * kBatchTile);
    }
    const int row = row0 + tid;
    const int parts = static_cast<int>(gridDim.x);
#pragma unroll
    for (int s = 0; s < kMaxBatch; ++s) {
        if (s < batch) {
            if (row < rows) out[static_cast<size_t>(s) * rows + row] = acc[s];
            float v = row < rows ? acc[s] : -__builtin_inff();
            int i = row < rows ? row : 0x7fffffff;
            block_argmax(v, i, sv, si);
            if (tid == 0) {
                st.partial_value[static_cast<size_t>(s) * parts + blockIdx.x] = v;
                st.partial_index[static_cast<size_t>(s) * parts + blockIdx.x] = i;
            }
            __syncthreads();  // sv / si are reused by the next sequence
        }
    }
}

__global__ __launch_bounds__(256) void argmax_kernel(const float *values, int n, ArgmaxState st) {
    __shared__ float sv[4];
    __shared__ int si[4];
    float v = -__builtin_inff();
    int i = 0x7fffffff;
    for (int k = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x); k < n;
         k += static_cast<int>(gridDim.x * blockDim.x))
        if (better(values[k], k, v, i)) { v = values[k]; i = k; }
    block_argmax(v, i, sv, si);
    if (threadIdx.x == 0) {
        st.partial_value[blockIdx.x] = v;
        st.partial_index[blockIdx.x] = i;
        if (st.embed && blockIdx.x == 0) *st.embed = -1;
    }
}

__global__ void count_nonfinite_halves_kernel(const uint16_t *w, size_t n, unsigned int *count) {
    unsigned int local = 0;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        local += (w[i] & 0x7c00u) == 0x7c00u;
    if (local) atomicAdd(count, local);
}

}  // namespace

int f16_matvec_workgroups(int rows) { return (rows + kRows - 1) / kRows; }

hipError_t launch_f16_matvec(const uint16_t *w, int rows, int width, bool finite, const float *x, const float *norm,
    float eps, float *out, const ArgmaxState *argmax, hipStream_t stream) {
    if (rows <= 0 || width <= 0 || width % 64) return hipErrorInvalidValue;
    const int grid = f16_matvec_workgroups(rows);
    const bool wide = width % 128 == 0;  // 128-column tiles where the width allows, else 64
    const size_t lds = static_cast<size_t>(kRows) * ((wide ? 128 : 64) + 8) * 2 + static_cast<size_t>(width) * 4;
    ArgmaxState st = argmax ? *argmax : ArgmaxState{};
#define FORTAI_LM(R, A, F)                                                                                         \
    do {                                                                                                          \
        if (wide)                                                                                                 \
            hipLaunchKernelGGL((f16_matvec_kernel<R, A, F, 128>), dim3(grid), dim3(kRows), lds, stream, w, rows,  \
                width, x, norm, eps, out, st);                                                                    \
        else                                                                                                      \
            hipLaunchKernelGGL((f16_matvec_kernel<R, A, F, 64>), dim3(grid), dim3(kRows), lds, stream, w, rows,   \
                width, x, norm, eps, out, st);                                                                    \
    } while (0)
    const bool rms = norm != nullptr, am = argmax != nullptr;
    if (rms && am && finite) FORTAI_LM(true, true, true);
    else if (rms && am) FORTAI_LM(true, true, false);
    else if (rms && finite) FORTAI_LM(true, false, true);
    else if (rms) FORTAI_LM(true, false, false);
    else if (am && finite) FORTAI_LM(false, true, true);
    else if (am) FORTAI_LM(false, true, false);
    else if (finite) FORTAI_LM(false, false, true);
    else FORTAI_LM(false, false, false);
#undef FORTAI_LM
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !argmax || st.embed) {  // with embed the next step's embedding finishes
        note_launch("f16_matvec_kernel<rms=%d,argmax=0,finite=%d,tile=%d> grid %d", norm != nullptr, finite, wide ? 128 : 64,
            grid);
        return e;
    }
    e = launch_argmax_finish(grid, st, stream);
    note_launch("f16_matvec_kernel<rms=%d,argmax=1,finite=%d,tile=%d> grid %d + argmax_finish_kernel", norm != nullptr,
        finite, wide ? 128 : 64, grid);
    return e;
}

int f16_batch_lm_head_workgroups(int rows) { return (rows + kBatchRows - 1) / kBatchRows; }

hipError_t launch_f16_batch_lm_head(const uint16_t *w, int rows, int width, bool finite, int batch, const float *x,
    const float *norm, float eps, float *xnorm, float *out, const ArgmaxState &argmax, hipStream_t stream) {
    if (rows <= 0 || width <= 0 || width % kBatchTile || batch < 1 || batch > kMaxBatch || !norm || !xnorm)
        return hipErrorInvalidValue;
    const int grid = f16_batch_lm_head_workgroups(rows);
    hipLaunchKernelGGL(batch_output_norm_kernel, dim3(kMaxBatch), dim3(128), 0, stream, x, norm, eps, width, batch,
        xnorm);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const size_t lds = static_cast<size_t>(kBatchRows) * (kBatchTile + 8) * 2;
    if (finite)
        hipLaunchKernelGGL(f16_batch_lm_head_kernel<true>, dim3(grid), dim3(kBatchRows), lds, stream, w, rows, width,
            batch, xnorm, out, argmax);
    else
        hipLaunchKernelGGL(f16_batch_lm_head_kernel<false>, dim3(grid), dim3(kBatchRows), lds, stream, w, rows, width,
            batch, xnorm, out, argmax);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    e = launch_argmax_finish(grid, argmax, stream, batch);
    note_launch("batch_output_norm_kernel grid %d + f16_batch_lm_head_kernel<finite=%d> grid %d + argmax_finish_kernel "
        "grid 1x%d", kMaxBatch, finite, grid, batch);
    return e;
}

hipError_t launch_argmax(const float *values, int n, const ArgmaxState &state, hipStream_t stream) {
    int grid = (n + 255) / 256;
    if (grid > 1024) grid = 1024;
    hipLaunchKernelGGL(argmax_kernel, dim3(grid), dim3(256), 0, stream, values, n, state);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    e = launch_argmax_finish(grid, state, stream);
    note_launch("argmax_kernel grid %d + argmax_finish_kernel", grid);
    return e;
}

hipError_t launch_argmax_finish(int partials, const ArgmaxState &state, hipStream_t stream, int batch) {
    if (batch < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(1, batch), dim3(256), 0, stream, partials, state);
    return hipGetLastError();
}

hipError_t launch_step_embedding(const uint16_t *table16, const Q8Matrix *table8, int rows, int width,
    const ArgmaxState &state, int partials, float *out, hipStream_t stream) {
    if (!table16 == !table8 || rows <= 0 || width <= 0 || partials <= 0 || !state.embed || !state.token ||
        !state.position || !state.partial_value || !state.partial_index || (table8 && table8->blocks * kQ8Block != width))
        return hipErrorInvalidValue;
    const Q8Matrix t8 = table8 ? *table8 : Q8Matrix{};
    hipLaunchKernelGGL(step_embedding_kernel, dim3((width + 255) / 256), dim3(256), 0, stream, table16, t8, rows,
        width, state, partials, out);
    note_launch("step_embedding_kernel<%s> grid %d (argmax finish of %d partials folded in)", table16 ? "f16" : "q8",
        (width + 255) / 256, partials);
    return hipGetLastError();
}

hipError_t launch_count_nonfinite_halves(const uint16_t *w, size_t n, unsigned int *count, hipStream_t stream) {
    hipLaunchKernelGGL(count_nonfinite_halves_kernel, dim3(1024), dim3(256), 0, stream, w, n, count);
    return hipGetLastError();
}

}  // namespace fortai_hip
