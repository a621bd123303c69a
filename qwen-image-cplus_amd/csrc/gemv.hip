// W4A16 GEMV for 1 <= m <= 16 rows: the adaLN / timestep modulation linears,
// whose cost is reading the int4 weights once from HBM.
//
// Arithmetic: W = fp16(fmaf(code, scale, minimum)) exactly as the W4A16 GEMM
// (qwen_image_cuda/cuda/gemm.cu:222-230), computed two weights per packed
// fp16 instruction where that is provably the same value; weight x activation
// pairs accumulate in fp32 with v_dot2 (exact fp16 products).  The reference runs these linears in BF16 through
// cuBLAS SGEMM (qwen_image_cuda/src/transformer.cplus:716-730); there is no
// INT4 GEMV there to follow.
//
// Design.  One workgroup owns one 16-row weight tile; in the tiled layout the
// tile's groups are consecutive 512-byte blocks, so the four wavefronts take
// groups g = w, w+4, ... and the workgroup streams the tile front to back,
// each lane issuing one 8-byte load per group.  Each lane dequantises its 16
// weights, multiplies them with the matching activations of every row, and
// the partial sums are reduced over the four 16-lane k-slices with shuffles
// and over the wavefronts through LDS.

#include "qi_common.h"

namespace qi {

constexpr int GEMV_WAVES = 4;
constexpr int GEMV_UNROLL = 4;

template <int MR>
__global__ __launch_bounds__(GEMV_WAVES *WAVE) void w4a16_gemv_kernel(
    const uint16_t *__restrict__ x, const uint8_t *__restrict__ codes, const uint16_t *__restrict__ scales,
    const float *__restrict__ bias, void *__restrict__ y, int out_type, int epi, int m, int n, int k) {
    __shared__ float partial[GEMV_WAVES][MR][16];
    const int groups = k >> 6;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const int q = lane >> 4, r16 = lane & 15;
    const int tile = blockIdx.x;
    const uint8_t *cp = codes + static_cast<size_t>(tile) * groups * 512 + lane * 8;
    const uint32_t *sp = reinterpret_cast<const uint32_t *>(scales) + static_cast<size_t>(tile) * groups * 16 + r16;

    float acc[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[r] = 0.0f;

    auto consume = [&](int g, uint2 c, uint32_t sm) {
        const uint32_t sb = sm & 0xFFFFu, mb = sm >> 16;
        const bool fast = w4a16_single_rounding_exact(sb, mb);
        const uint4 w0 = w4a16_dequant8(c.x, sb, mb, fast);   // elements [8q, 8q+8)
        const uint4 w1 = w4a16_dequant8(c.y, sb, mb, fast);   // elements [32+8q, 32+8q+8)
        const uint32_t ws[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            if (r < m) {
                const uint16_t *xr = x + static_cast<size_t>(r) * k + g * 64 + 8 * q;
                const uint4 x0 = *reinterpret_cast<const uint4 *>(xr);
                const uint4 x1 = *reinterpret_cast<const uint4 *>(xr + 32);
                const uint32_t xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    acc[r] = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, ws[e]), __builtin_bit_cast(v2h, xs[e]),
                                                    acc[r], false);
            }
        }
    };

    int g = wave;
    for (; g + (GEMV_UNROLL - 1) * GEMV_WAVES < groups; g += GEMV_UNROLL * GEMV_WAVES) {
        uint2 c[GEMV_UNROLL];
        uint32_t sm[GEMV_UNROLL];
#pragma unroll
        for (int u = 0; u < GEMV_UNROLL; ++u) {
            const int gg = g + u * GEMV_WAVES;
            c[u] = *reinterpret_cast<const uint2 *>(cp + static_cast<size_t>(gg) * 512);
            sm[u] = sp[static_cast<size_t>(gg) * 16];
        }
#pragma unroll
        for (int u = 0; u < GEMV_UNROLL; ++u) consume(g + u * GEMV_WAVES, c[u], sm[u]);
    }
    for (; g < groups; g += GEMV_WAVES) {
        const uint2 c = *reinterpret_cast<const uint2 *>(cp + static_cast<size_t>(g) * 512);
        consume(g, c, sp[static_cast<size_t>(g) * 16]);
    }

#pragma unroll
    for (int r = 0; r < MR; ++r) {
        const float v = wave_sum16(acc[r]);
        if (q == 0) partial[wave][r][r16] = v;
    }
    __syncthreads();
    if (wave == 0 && lane < 16) {
        const int col = tile * 16 + lane;
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            if (r < m) {
                float v = partial[0][r][lane];
#pragma unroll
                for (int w = 1; w < GEMV_WAVES; ++w) v += partial[w][r][lane];
                store_out(y, static_cast<size_t>(r) * n + col, epilogue(v, bias, col, epi), out_type);
            }
        }
    }
}

}  // namespace qi

using namespace qi;

int qi_hip_w4a16_gemv_impl(const void *x_half, const void *w_tiled_codes, const void *w_tiled_scales,
                           const float *bias, void *y, int out_type, int epilogue, int m, int n, int k,
                           hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(n / 16)), block(GEMV_WAVES * WAVE);
    const uint16_t *x = static_cast<const uint16_t *>(x_half);
    const uint8_t *c = static_cast<const uint8_t *>(w_tiled_codes);
    const uint16_t *s = static_cast<const uint16_t *>(w_tiled_scales);
    if (m <= 1)
        w4a16_gemv_kernel<1><<<grid, block, 0, stream>>>(x, c, s, bias, y, out_type, epilogue, m, n, k);
    else if (m <= 2)
        w4a16_gemv_kernel<2><<<grid, block, 0, stream>>>(x, c, s, bias, y, out_type, epilogue, m, n, k);
    else if (m <= 4)
        w4a16_gemv_kernel<4><<<grid, block, 0, stream>>>(x, c, s, bias, y, out_type, epilogue, m, n, k);
    else if (m <= 8)
        w4a16_gemv_kernel<8><<<grid, block, 0, stream>>>(x, c, s, bias, y, out_type, epilogue, m, n, k);
    else
        w4a16_gemv_kernel<16><<<grid, block, 0, stream>>>(x, c, s, bias, y, out_type, epilogue, m, n, k);
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
    return qi_hip_w4a16_gemv_impl(x_half, w_tiled_codes, w_tiled_scales, bias, y, out_type, epilogue, m, n, k,
                                  stream_of(stream));
}
