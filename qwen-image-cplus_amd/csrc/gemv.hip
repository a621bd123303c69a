// W4A16 GEMV for 1 <= m <= 16 rows: the adaLN / timestep modulation linears,
// whose cost is reading the int4 weights once from HBM.  The reference runs
// these linears in BF16 through cuBLAS SGEMM
// (qwen_image_cuda/src/transformer.cplus:716-730); there is no INT4 GEMV there
// to follow, so the arithmetic is the W4A16 GEMM's weights
// (qwen_image_cuda/cuda/gemm.cu:222-230) within the W4A16 tolerance.
//
// Layout (matrix-core forms): one workgroup owns one 16-row weight tile; in the tiled layout the
// tile's groups are consecutive 512-byte blocks, and each of the four
// wavefronts streams a contiguous quarter of them, with batches of groups of
// loads (one 8-byte code load and one scale pair per lane each) in flight.
// The activations are staged in LDS, and the wavefronts' partial sums are
// added through LDS.  Three kernels:
//   * w4a16_gemv_dot2_kernel (m = 1, 2): vector unit, dot2 on the codes
//     as exact fp16 integers with the factored per-group scale step, two weight
//     rows per lane and a wave-local x slice (its own layout, described at
//     the kernel);
//   * w4a16_gemv_factored_kernel (m <= 16, x fits in LDS): the same
//     factored form on the matrix core (16 rows per MFMA);
//   * w4a16_gemv_kernel: dequantised fp16 weights (the GEMM's exact weights)
//     on the matrix core, for x too large for LDS.

#include "qi_common.h"

namespace qi {

typedef unsigned v2u __attribute__((ext_vector_type(2)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
constexpr int GEMV_WAVES = 4;
constexpr int GEMV_BATCH = 4;  // groups per batch; two batches are in flight per wave
constexpr int GEMV_LDS_X = 48 * 1024;  // bytes of activations staged in LDS

// Output index of row r, column col: the parts layout [part][m][n_part]
// (n_part = n: the row-major [m][n]).  n_part is a multiple of 16, so a
// workgroup's 16 columns lie in one part.
__device__ __forceinline__ size_t gemv_out_index(int r, int col, int m, int n_part) {
    const int part = col / n_part;
    return (static_cast<size_t>(part) * m + r) * n_part + (col - part * n_part);
}

// XLDS: the workgroup first copies x (m rows x k fp16) into LDS, so the
// weight stream never waits on activation loads; used when m * k * 2 fits.
template <bool XLDS>
__global__ __launch_bounds__(GEMV_WAVES *WAVE) void w4a16_gemv_kernel(
    const uint16_t *__restrict__ x, const uint8_t *__restrict__ codes, const uint16_t *__restrict__ scales,
    const float *__restrict__ bias, void *__restrict__ y, int out_type, int epi, int m, int n, int k, int n_part) {
    __shared__ float partial[GEMV_WAVES][16][17];
    extern __shared__ __attribute__((aligned(16))) uint16_t xs_lds[];  // m * k fp16 when XLDS
    const int groups = k >> 6;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const int q = lane >> 4, r16 = lane & 15;
    const int tile = blockIdx.x;

    // Wave w streams groups [g_begin, g_end) of the tile: contiguous
    // 512-byte code blocks and 64-byte scale blocks.
    const int per_wave = (groups + GEMV_WAVES - 1) / GEMV_WAVES;
    const int g_begin = wave * per_wave;
    const int g_end = min(groups, g_begin + per_wave);
    const uint8_t *cp = codes + static_cast<size_t>(tile) * groups * 512 + lane * 8;
    const uint32_t *sp = reinterpret_cast<const uint32_t *>(scales) + static_cast<size_t>(tile) * groups * 16 + r16;

    // Batches of GEMV_BATCH groups, double-buffered: the loads of batch b + 1
    // are issued before batch b is consumed, so every wave overlaps its
    // dequantisation with its next loads.  The first two batches are
    // requested before the activations are staged.
    uint2 c[2][GEMV_BATCH];
    uint32_t sm[2][GEMV_BATCH];
    auto load_batch = [&](int b, int g) {
#pragma unroll
        for (int u = 0; u < GEMV_BATCH; ++u) {
            if (g + u < g_end) {
                const v2u t =
                    __builtin_nontemporal_load(reinterpret_cast<const v2u *>(cp + static_cast<size_t>(g + u) * 512));
                c[b][u] = uint2{t[0], t[1]};
                sm[b][u] = __builtin_nontemporal_load(sp + static_cast<size_t>(g + u) * 16);
            }
        }
    };
    load_batch(0, g_begin);
    load_batch(1, g_begin + GEMV_BATCH);

    if (XLDS) {
        const int chunks = m * k / 8;  // 16-byte chunks
        for (int i = threadIdx.x; i < chunks; i += GEMV_WAVES * WAVE)
            reinterpret_cast<uint4 *>(xs_lds)[i] = reinterpret_cast<const uint4 *>(x)[i];
    }
    // The matrix-core B operand: lane l supplies row m = l % 16 of x, inputs
    // 8q .. 8q + 7 of each 32-wide half group.  Lanes past the last row read
    // row 0: they only feed output columns that are never stored.
    const uint16_t *xrow = (XLDS ? xs_lds : x) + static_cast<size_t>(r16 < m ? r16 : 0) * k + 8 * q;
    if (XLDS) __syncthreads();

    // acc[r] = y[m = l % 16][n = 16 tile + 4 (l / 16) + r] over this wave's
    // groups (16x16 accumulator layout, A = weights, B = x).
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    auto consume = [&](int g, uint2 cc, uint32_t smm) {
        const uint32_t sb = smm & 0xFFFFu, mb = smm >> 16;
        // Wave-uniform, so a wave runs one dequantisation form, not both.
        const bool fast = __all(w4a16_single_rounding_exact(sb, mb));
        const uint4 w0 = w4a16_dequant8(cc.x, sb, mb, fast);   // elements [8q, 8q+8)
        const uint4 w1 = w4a16_dequant8(cc.y, sb, mb, fast);   // elements [32+8q, 32+8q+8)
        const uint4 x0 = *reinterpret_cast<const uint4 *>(xrow + g * 64);
        const uint4 x1 = *reinterpret_cast<const uint4 *>(xrow + g * 64 + 32);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, w0), __builtin_bit_cast(v8h, x0), acc, 0,
                                                     0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, w1), __builtin_bit_cast(v8h, x1), acc, 0,
                                                     0, 0);
    };
    for (int g = g_begin; g < g_end; g += 2 * GEMV_BATCH) {
#pragma unroll
        for (int u = 0; u < GEMV_BATCH; ++u)
            if (g + u < g_end) consume(g + u, c[0][u], sm[0][u]);
        load_batch(0, g + 2 * GEMV_BATCH);
#pragma unroll
        for (int u = 0; u < GEMV_BATCH; ++u)
            if (g + GEMV_BATCH + u < g_end) consume(g + GEMV_BATCH + u, c[1][u], sm[1][u]);
        load_batch(1, g + 3 * GEMV_BATCH);
    }

#pragma unroll
    for (int r = 0; r < 4; ++r) partial[wave][4 * q + r][r16] = acc[r];
    __syncthreads();
    // Thread t (of the first 256) finishes output n = t / 16 of row m = t % 16.
    {
        const int t = threadIdx.x, nn = t >> 4, mm = t & 15;
        if (mm < m) {
            float v = partial[0][nn][mm];
#pragma unroll
            for (int w = 1; w < GEMV_WAVES; ++w) v += partial[w][nn][mm];
            const int col = tile * 16 + nn;
            store_out(y, gemv_out_index(mm, col, m, n_part), epilogue(v, bias, col, epi), out_type);
        }
    }
}

// Factored form, used when x fits in LDS.  Per group g and output n:
//   y += s P + min X,  P = sum_k x_k c_k,  X = sum_k x_k
// The codes become exact fp16 integers without a multiply: a bit-field
// insert into 0x6400 gives 1024 + c and a packed fp16 add of -1024 gives c
// (both exact), so P is exact per product and summed in fp32 with no
// cancelled 1024 X term.  X comes from the matrix core too: two MFMAs with an
// all-ones weight operand, so no separate pass over x is needed.
// This is the group's dot product with the weights c s + min kept in fp32,
// instead of first rounding every weight to fp16 as the reference's
// dequantiser does (gemm.cu:229-230): the outputs differ from that form by
// the fp16 weight rounding only, well inside the W4A16 output tolerance.
__global__ __launch_bounds__(GEMV_WAVES *WAVE) void w4a16_gemv_factored_kernel(
    const uint16_t *__restrict__ x, const uint8_t *__restrict__ codes, const uint16_t *__restrict__ scales,
    const float *__restrict__ bias, void *__restrict__ y, int out_type, int epi, int m, int n, int k, int n_part) {
    __shared__ float partial[GEMV_WAVES][16][17];
    extern __shared__ __attribute__((aligned(16))) uint16_t xs_lds[];  // m * k fp16
    const int groups = k >> 6;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const int q = lane >> 4, r16 = lane & 15;
    const int tile = blockIdx.x;

    const int per_wave = (groups + GEMV_WAVES - 1) / GEMV_WAVES;
    const int g_begin = wave * per_wave;
    const int g_end = min(groups, g_begin + per_wave);
    const uint8_t *cp = codes + static_cast<size_t>(tile) * groups * 512 + lane * 8;
    // Lane l loads the (scale, minimum) pair of output 4q + l % 4; the pairs
    // of the lane's four outputs 4q .. 4q+3 are then its quad's four loads.
    const uint32_t *sp =
        reinterpret_cast<const uint32_t *>(scales) + static_cast<size_t>(tile) * groups * 16 + 4 * q + (lane & 3);

    // Two batches in flight cover a 3072-wide row's 12 groups per wave, so
    // each wave's whole weight stream is requested at once.
    constexpr int FB = 6;
    uint2 c[2][FB];
    uint32_t sc[2][FB];
    // When every wave's share is whole batches (groups % 48 == 0, e.g. k =
    // 3072), batches need no per-group bounds tests: one uniform test per
    // batch decides whether it exists.
    const bool whole = groups % (GEMV_WAVES * 2 * FB) == 0;
    auto load_batch = [&](int b, int g) {
        if (whole && g >= g_end) return;
#pragma unroll
        for (int u = 0; u < FB; ++u) {
            if (whole || g + u < g_end) {
                const v2u t =
                    __builtin_nontemporal_load(reinterpret_cast<const v2u *>(cp + static_cast<size_t>(g + u) * 512));
                c[b][u] = uint2{t[0], t[1]};
                sc[b][u] = __builtin_nontemporal_load(sp + static_cast<size_t>(g + u) * 16);
            }
        }
    };
    load_batch(0, g_begin);
    load_batch(1, g_begin + FB);

    const int chunks = m * k / 8;  // 16-byte chunks of x
    for (int i = threadIdx.x; i < chunks; i += GEMV_WAVES * WAVE)
        reinterpret_cast<uint4 *>(xs_lds)[i] = reinterpret_cast<const uint4 *>(x)[i];
    __syncthreads();

    // B operand: lane l supplies row m = l % 16 of x, inputs 8q .. 8q + 7 of
    // each 32-wide half group.  Lanes past the last row read row 0: they only
    // feed output columns that are never stored.
    const int xr = r16 < m ? r16 : 0;
    const uint16_t *xrow = xs_lds + static_cast<size_t>(xr) * k + 8 * q;
    uint32_t magic = 0x64006400u;
    asm volatile("" : "+v"(magic));  // kept in a VGPR: lets the insert be one v_bfi_b32

    // yacc[r] = y[m = l % 16][n = 16 tile + 4q + r] over this wave's groups.
    float yacc[4] = {0.f, 0.f, 0.f, 0.f};
    auto consume = [&](int g, uint2 cc, uint32_t scq) {
        // Bit-field insert of each nibble pair into 0x6400 (written in C, not
        // inline asm: these values feed the matrix core directly, and only
        // compiler-visible instructions get the VALU-to-MFMA wait states).
        // A packed fp16 add of -1024 then makes them the codes c exactly.
        const v2h m1024 = {static_cast<_Float16>(-1024.0f), static_cast<_Float16>(-1024.0f)};
        uint32_t a[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[i] = __builtin_bit_cast(
                uint32_t, __builtin_bit_cast(v2h, ((cc.x >> (4 * i)) & 0x000F000Fu) | (magic & ~0x000F000Fu)) + m1024);
            a[4 + i] = __builtin_bit_cast(
                uint32_t, __builtin_bit_cast(v2h, ((cc.y >> (4 * i)) & 0x000F000Fu) | (magic & ~0x000F000Fu)) + m1024);
        }
        const uint4 x0 = *reinterpret_cast<const uint4 *>(xrow + g * 64);
        const uint4 x1 = *reinterpret_cast<const uint4 *>(xrow + g * 64 + 32);
        // The nibble slot order of the tiled codes puts element 2i in nibble
        // i and 2i+1 in nibble 4+i, so a[i] holds elements (2i, 2i+1).
        // X = sum x (every output row of the all-ones operand is alike),
        // then P = sum x c.
        const uint4 ones = {0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u};
        const v4f zero = {0.f, 0.f, 0.f, 0.f};
        v4f xs = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, ones), __builtin_bit_cast(v8h, x0),
                                                         zero, 0, 0, 0);
        xs = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, ones), __builtin_bit_cast(v8h, x1), xs, 0,
                                                    0, 0);
        const float X = xs[0];
        v4f p = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, uint4{a[0], a[1], a[2], a[3]}),
                                                       __builtin_bit_cast(v8h, x0), zero, 0, 0, 0);
        p = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, uint4{a[4], a[5], a[6], a[7]}),
                                                   __builtin_bit_cast(v8h, x1), p, 0, 0, 0);
        // Quad broadcasts (DPP quad_perm r,r,r,r) gather the four pairs.
        const uint32_t sm4[4] = {
            static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(scq), 0x00, 0xF, 0xF, false)),
            static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(scq), 0x55, 0xF, 0xF, false)),
            static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(scq), 0xAA, 0xF, 0xF, false)),
            static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(scq), 0xFF, 0xF, 0xF, false))};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            yacc[r] = __builtin_fmaf(h2f(static_cast<uint16_t>(sm4[r] & 0xFFFFu)), p[r], yacc[r]);
            yacc[r] = __builtin_fmaf(h2f(static_cast<uint16_t>(sm4[r] >> 16)), X, yacc[r]);
        }
    };
    for (int g = g_begin; g < g_end; g += 2 * FB) {
#pragma unroll
        for (int u = 0; u < FB; ++u)
            if (whole || g + u < g_end) consume(g + u, c[0][u], sc[0][u]);
        load_batch(0, g + 2 * FB);
#pragma unroll
        for (int u = 0; u < FB; ++u)
            if (whole || g + FB + u < g_end) consume(g + FB + u, c[1][u], sc[1][u]);
        load_batch(1, g + 3 * FB);
    }

#pragma unroll
    for (int r = 0; r < 4; ++r) partial[wave][4 * q + r][r16] = yacc[r];
    __syncthreads();
    {
        const int t = threadIdx.x, nn = t >> 4, mm = t & 15;
        if (mm < m) {
            float v = partial[0][nn][mm];
#pragma unroll
            for (int w = 1; w < GEMV_WAVES; ++w) v += partial[w][nn][mm];
            const int col = tile * 16 + nn;
            store_out(y, gemv_out_index(mm, col, m, n_part), epilogue(v, bias, col, epi), out_type);
        }
    }
}

// Vector-unit form for m <= 2 (the modulation linears' one or two rows),
// where a 16-row MFMA would waste most of its work.  The kernel is bound by
// the weight stream at first and then by what follows the last arrival, so it
// keeps every latency chain off that path:
//   * lane l loads 16 bytes of a 1 KB pair of group blocks: slots 2j and
//     2j + 1 (j = l % 32) of group gc + 2u + l / 32, i.e. rows 2j % 16 and
//     2j % 16 + 1 with the same input chunk q = j / 8, so one read of x from
//     LDS serves two weight rows;
//   * each wave stages only its own slice of x (its groups, requested before
//     the weights, stored once it lands), so no workgroup barrier precedes
//     the arithmetic;
//   * the codes become the fp16 integers 1024 + c (a bit-field insert into
//     0x6400) and then c exactly (a packed fp16 add of -1024), and the
//     lane's share of a group is s P + min X with P = sum x c and X = sum x
//     over the lane's 16 inputs (v_dot2_f32_f16; X once per chunk of x as
//     it is staged, against ones, and read back from LDS);
//   * the lanes of a row differ in lane bits 3..5: bit 3 is folded by a DPP
//     row rotate, bits 4..5 and the waves through one LDS pass.
// This is the group's dot product with the weights c s + min in fp32, like
// the matrix-core factored form: the products are exact and only their fp32
// sums round, so the outputs differ from the reference's (whose weights are
// first rounded to fp16) by that weight rounding, inside the W4A16
// tolerance, and are bit-exact fp32(c s + min) on one-hot rows.  (Using the
// reference's fp16 weights here, exact double rounding included, measured
// 1.35x slower on the all-blocks launch.)
// W waves per workgroup (one 16-row tile), FB groups per wave and chunk
// (FB / 2 16-byte loads per lane; FB even).  Measured on MI355X (us, W 8
// FB 6 -> W 4 FB 4): every block's modulation linears as one fused record
// (120 matrices, 138240 tiles) at m = 1 693 -> 641, at m = 2 901 -> 770;
// one 3072 -> 18432 matrix 8.5 -> 8.6 (m = 1), 10.3 -> 10.1 (m = 2).  (W 4
// FB 6 was as fast fused and W 2 FB 6 slower on one matrix; one shape for
// every launch keeps a fused record's outputs bit-identical to per-matrix
// calls.)
constexpr int DOT2_WAVES = 4, DOT2_FB = 4;
template <int M, int W, int FB>
__global__ __launch_bounds__(W *WAVE) void w4a16_gemv_dot2_kernel(
    const uint16_t *__restrict__ x, const uint8_t *__restrict__ codes, const uint16_t *__restrict__ scales,
    const float *__restrict__ bias, void *__restrict__ y, int out_type, int epi, int n, int k, int n_part) {
    static_assert(FB % 2 == 0, "two groups per 16-byte load");
    constexpr int NI = FB / 2;
    constexpr int XC = M * FB * 8;  // 16-byte chunks of a wave's x slice
    constexpr int XR = (XC + WAVE - 1) / WAVE;
    __shared__ float partial[W][4][M][16];
    __shared__ __attribute__((aligned(16))) uint16_t xs[W][M * FB * 64];
    __shared__ float xsum[W][XC];  // [row][group][chunk pair q]: sum x over chunks q and q + 4
    const int groups = k >> 6;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const int h = lane >> 5, j = lane & 31, q = j >> 3, r0 = (2 * j) & 15;
    const int tile = blockIdx.x;
    const int per_wave = (groups + W - 1) / W;
    const int g_begin = min(groups, wave * per_wave), g_end = min(groups, g_begin + per_wave);
    const uint8_t *cp = codes + static_cast<size_t>(tile) * groups * 512 + h * 512 + j * 16;
    const uint32_t *sp = reinterpret_cast<const uint32_t *>(scales) + static_cast<size_t>(tile) * groups * 16 + h * 16 + r0;
    uint16_t *xw = xs[wave];
    float *xsw = xsum[wave];

    uint32_t magic = 0x64006400u;
    asm volatile("" : "+v"(magic));  // kept in a VGPR: lets the insert be one v_bfi_b32
    const v2h one2 = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
    const v2h m1024 = {static_cast<_Float16>(-1024.0f), static_cast<_Float16>(-1024.0f)};
    float ya[M], yb[M];
#pragma unroll
    for (int r = 0; r < M; ++r) ya[r] = yb[r] = 0.f;

    for (int gc = g_begin; gc < g_end; gc += FB) {
        // x slice: row r, groups gc .. gc + FB - 1 (clamped to the last group;
        // clamped groups are never used).  Indices past the slice repeat its
        // last chunk, so the loads and stores need no branch.
        uint4 xv[XR];
#pragma unroll
        for (int e = 0; e < XR; ++e) {
            const int i = min(lane + e * WAVE, XC - 1), r = i / (FB * 8), cc = i % (FB * 8);
            const int g = min(gc + (cc >> 3), groups - 1);
            xv[e] = *reinterpret_cast<const uint4 *>(x + static_cast<size_t>(r) * k + g * 64 + (cc & 7) * 8);
        }
        v4u c[NI];
        v2u sc[NI];
#pragma unroll
        for (int u = 0; u < NI; ++u) {
            const int g = min(gc + 2 * u, g_end - 1 - h);  // lane group gc + 2u + h, clamped into the wave's range
            c[u] = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(cp + static_cast<size_t>(g) * 512));
            sc[u] = __builtin_nontemporal_load(reinterpret_cast<const v2u *>(sp + static_cast<size_t>(g) * 16));
        }
        // X per (row, group, lane chunk pair): the slice's chunk sums (dot2
        // against ones), chunk q + 4's taken from lane ^ 4 (the same row and
        // group), so the lanes of the products read it instead of summing
        // their 16 inputs again.  Slots 4..7 and the clamped lanes' values
        // are never read.
#pragma unroll
        for (int e = 0; e < XR; ++e) {
            const int i = min(lane + e * WAVE, XC - 1);
            reinterpret_cast<uint4 *>(xw)[i] = xv[e];
            float t = __builtin_amdgcn_fdot2(one2, __builtin_bit_cast(v2h, xv[e].x), 0.f, false);
            t = __builtin_amdgcn_fdot2(one2, __builtin_bit_cast(v2h, xv[e].y), t, false);
            t = __builtin_amdgcn_fdot2(one2, __builtin_bit_cast(v2h, xv[e].z), t, false);
            t = __builtin_amdgcn_fdot2(one2, __builtin_bit_cast(v2h, xv[e].w), t, false);
            xsw[i] = t + __shfl_xor(t, 4);
        }
        // The slice is the wave's own: its LDS stores are complete once
        // lgkmcnt drains, and the wave barrier keeps the reads after them.
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int u = 0; u < NI; ++u) {
            // (1024 + c) - 1024 = c exactly in fp16 (one packed fp16 add per
            // two codes), so no 1024 X term is cancelled in fp32 later.
            v2h a[8], b[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a[i] = __builtin_bit_cast(v2h, ((c[u][0] >> (4 * i)) & 0x000F000Fu) | (magic & ~0x000F000Fu)) + m1024;
                a[4 + i] =
                    __builtin_bit_cast(v2h, ((c[u][1] >> (4 * i)) & 0x000F000Fu) | (magic & ~0x000F000Fu)) + m1024;
                b[i] = __builtin_bit_cast(v2h, ((c[u][2] >> (4 * i)) & 0x000F000Fu) | (magic & ~0x000F000Fu)) + m1024;
                b[4 + i] =
                    __builtin_bit_cast(v2h, ((c[u][3] >> (4 * i)) & 0x000F000Fu) | (magic & ~0x000F000Fu)) + m1024;
            }
            // A group past the wave's range contributes nothing: its scale
            // and minimum are taken as zero (selected here, where the loads
            // are awaited anyway).
            const v2u su = gc + 2 * u + h < g_end ? sc[u] : v2u{0u, 0u};
            const float sa = h2f(static_cast<uint16_t>(su[0] & 0xFFFFu)), ma = h2f(static_cast<uint16_t>(su[0] >> 16));
            const float sb = h2f(static_cast<uint16_t>(su[1] & 0xFFFFu)), mb = h2f(static_cast<uint16_t>(su[1] >> 16));
#pragma unroll
            for (int r = 0; r < M; ++r) {
                const uint16_t *xr = xw + (r * FB + 2 * u + h) * 64 + 8 * q;
                const uint4 x0 = *reinterpret_cast<const uint4 *>(xr);
                const uint4 x1 = *reinterpret_cast<const uint4 *>(xr + 32);
                const uint32_t xwd[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                const float xl = xsw[(r * FB + 2 * u + h) * 8 + q];
                float pa = 0.f, pb = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const v2h xq = __builtin_bit_cast(v2h, xwd[i]);
                    pa = __builtin_amdgcn_fdot2(a[i], xq, pa, false);
                    pb = __builtin_amdgcn_fdot2(b[i], xq, pb, false);
                }
                ya[r] = __builtin_fmaf(ma, xl, __builtin_fmaf(sa, pa, ya[r]));
                yb[r] = __builtin_fmaf(mb, xl, __builtin_fmaf(sb, pb, yb[r]));
            }
        }
    }

    // Lane bit 3 by a DPP row rotate of 8; bits 4..5 and the waves via LDS.
#pragma unroll
    for (int r = 0; r < M; ++r) {
        const float va =
            ya[r] + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, ya[r]), 0x128, 0xF,
                                                                          0xF, false));
        const float vb =
            yb[r] + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, yb[r]), 0x128, 0xF,
                                                                          0xF, false));
        if ((lane & 8) == 0) {
            partial[wave][lane >> 4][r][r0] = va;
            partial[wave][lane >> 4][r][r0 + 1] = vb;
        }
    }
    __syncthreads();
    if (threadIdx.x < M * 16) {
        const int r = threadIdx.x >> 4, nn = threadIdx.x & 15;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w)
#pragma unroll
            for (int s = 0; s < 4; ++s) v += partial[w][s][r][nn];
        const int col = tile * 16 + nn;
        store_out(y, gemv_out_index(r, col, M, n_part), epilogue(v, bias, col, epi), out_type);
    }
}

static void launch_gemv(const uint16_t *x, const uint8_t *c, const uint16_t *s, const float *bias, void *y,
                        int out_type, int epi, int m, int n, int k, int n_part, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(n / 16)), block(GEMV_WAVES * WAVE);
    const long long lds = static_cast<long long>(m) * k * 2;
    // One or two rows: the vector-unit form (its LDS does not grow with k).
    constexpr int W = DOT2_WAVES, FB = DOT2_FB;
    if (m == 1)
        w4a16_gemv_dot2_kernel<1, W, FB><<<grid, dim3(W * WAVE), 0, stream>>>(x, c, s, bias, y, out_type, epi, n, k, n_part);
    else if (m == 2)
        w4a16_gemv_dot2_kernel<2, W, FB><<<grid, dim3(W * WAVE), 0, stream>>>(x, c, s, bias, y, out_type, epi, n, k, n_part);
    else if (lds <= GEMV_LDS_X)
        w4a16_gemv_factored_kernel<<<grid, block, static_cast<size_t>(lds), stream>>>(x, c, s, bias, y, out_type, epi,
                                                                                      m, n, k, n_part);
    else
        w4a16_gemv_kernel<false><<<grid, block, 0, stream>>>(x, c, s, bias, y, out_type, epi, m, n, k, n_part);
}

}  // namespace qi

using namespace qi;

int qi_hip_w4a16_gemv_impl(const void *x_half, const void *w_tiled_codes, const void *w_tiled_scales,
                           const float *bias, void *y, int out_type, int epilogue, int m, int n, int k, int n_part,
                           hipStream_t stream) {
    const uint16_t *x = static_cast<const uint16_t *>(x_half);
    const uint8_t *c = static_cast<const uint8_t *>(w_tiled_codes);
    const uint16_t *s = static_cast<const uint16_t *>(w_tiled_scales);
    launch_gemv(x, c, s, bias, y, out_type, epilogue, m, n, k, n_part, stream);
    return launch_status();
}

QI_API int qi_hip_w4a16_gemv(const void *x_half, const void *w_tiled_codes, const void *w_tiled_scales,
                             const float *bias, void *y, int out_type, int epilogue, int m, int n, int k,
                             void *stream) {
    if (m <= 0 || m > 16 || n <= 0 || k <= 0 || n % 16 || k % 64) return kInvalid;
    if (!x_half || !w_tiled_codes || !w_tiled_scales || !y) return kInvalid;
    if (out_type != QI_HIP_OUT_F32 && out_type != QI_HIP_OUT_F16) return kInvalid;
    if (epilogue != QI_HIP_EPILOGUE_NONE && epilogue != QI_HIP_EPILOGUE_GELU_TANH) return kInvalid;
    if (reinterpret_cast<uintptr_t>(x_half) % 16 || reinterpret_cast<uintptr_t>(w_tiled_codes) % 8 ||
        reinterpret_cast<uintptr_t>(w_tiled_scales) % 4)
        return kInvalid;
    return qi_hip_w4a16_gemv_impl(x_half, w_tiled_codes, w_tiled_scales, bias, y, out_type, epilogue, m, n, k, n,
                                  stream_of(stream));
}
