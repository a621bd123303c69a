// W4A4 GEMM on gfx950 int8 MFMA: y[m, n] = sum_g float(P_g[m, n]) *
// (sa[m, g] * sw[n, g]), P_g the exact int32 dot product of the signed int4
// codes of group g (64 inputs).
//
// Reference arithmetic: qwen_image_cuda/cuda/gemm.cu:59-189 (w4a4_gemm_kernel,
// qi_w4a4_gemm): per group a fresh int32 partial, then, in ascending group
// order, acc = fmaf(float(P_g), sa * sw, acc) (nvcc contracts the accumulate).
//
// Design.  One v_mfma_i32_16x16x64_i8 is exactly one 16x16 output tile times
// one 64-group, so the int32 result *is* the reference's per-group partial and
// the fp32 scale step follows every MFMA.  Each lane unpacks its 16 nibbles
// (8 bytes) into int8 lanes holding 16*q (mask / shift, no sign fix-up); with
// both operands scaled by 16 the MFMA returns 256*P exactly, and the final
// multiply by 2^-8 is exact, so the fp32 result is bit-identical to the
// reference's accumulate order.  Operands are read straight from global
// memory into registers: weights in the tiled order are one coalesced 512-byte
// block per (16-row tile, group) and per wave; the next group is prefetched
// into registers while the current one computes.
//
// Work per output and group: 1/64 of an MFMA (16x16x64) plus three VALU
// operations (int->float, scale product, fma), so the kernel is bound by the
// VALU epilogue rather than by the matrix core when the operand traffic is
// hidden.

#include "qi_common.h"

namespace qi {

template <int TM, int TN, int WM, int WN, bool TILED>
__global__ __launch_bounds__(WM *WN *WAVE) void w4a4_gemm_kernel(
    const uint8_t *__restrict__ a_codes, const uint16_t *__restrict__ a_scales, const uint8_t *__restrict__ w_codes,
    const uint16_t *__restrict__ w_scales, const float *__restrict__ bias, void *__restrict__ y, int out_type,
    int epi, int m, int n, int k) {
    constexpr int BM = WM * TM * 16, BN = WN * TN * 16;
    const int groups = k >> 6;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int q = lane >> 4, r16 = lane & 15;
    const int tiles_n = (n + BN - 1) / BN;
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
    const int row_base = tm * BM + wm * TM * 16;
    const int col_base = tn * BN + wn * TN * 16;

    // Operand pointers at group 0; rows past the end are clamped (their
    // results are never stored).
    const uint8_t *ap[TM];
    const uint16_t *sap[TM][4];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int r = min(row_base + i * 16 + r16, m - 1);
        ap[i] = a_codes + static_cast<size_t>(r) * (k / 2) + 8 * q;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int rs = min(row_base + i * 16 + 4 * q + rr, m - 1);
            sap[i][rr] = a_scales + static_cast<size_t>(rs) * groups;
        }
    }
    const uint8_t *bp[TN];
    const uint16_t *swp[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int tile = min((col_base + j * 16) / 16, n / 16 - 1);
        if (TILED) {
            bp[j] = w_codes + static_cast<size_t>(tile) * groups * 512 + lane * 8;
            swp[j] = w_scales + static_cast<size_t>(tile) * groups * 16 + r16;
        } else {
            const int row = tile * 16 + r16;
            bp[j] = w_codes + static_cast<size_t>(row) * (k / 2) + 8 * q;
            swp[j] = w_scales + static_cast<size_t>(row) * groups;
        }
    }
    constexpr int kBStep = TILED ? 512 : 32;  // code bytes between groups
    constexpr int kSStep = TILED ? 16 : 1;    // scales between groups

    float acc[TM][TN][4];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) acc[i][j][rr] = 0.0f;

    uint2 a_next[TM], b_next[TN];
    uint16_t sa_next[TM][4], sw_next[TN];
    auto fetch = [&](int g) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            a_next[i] = *reinterpret_cast<const uint2 *>(ap[i] + g * 32);
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) sa_next[i][rr] = sap[i][rr][g];
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            b_next[j] = *reinterpret_cast<const uint2 *>(bp[j] + static_cast<size_t>(g) * kBStep);
            sw_next[j] = swp[j][static_cast<size_t>(g) * kSStep];
        }
    };

    fetch(0);
    for (int g = 0; g < groups; ++g) {
        v4i a_frag[TM], b_frag[TN];
        float sa[TM][4], sw[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            a_frag[i] = v4i{nib_lo16(a_next[i].x), nib_hi16(a_next[i].x), nib_lo16(a_next[i].y),
                            nib_hi16(a_next[i].y)};
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) sa[i][rr] = h2f(sa_next[i][rr]);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            b_frag[j] = v4i{nib_lo16(b_next[j].x), nib_hi16(b_next[j].x), nib_lo16(b_next[j].y),
                            nib_hi16(b_next[j].y)};
            sw[j] = h2f(sw_next[j]);
        }
        if (g + 1 < groups) fetch(g + 1);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const v4i p = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_frag[i], b_frag[j], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    acc[i][j][rr] = __builtin_fmaf(static_cast<float>(p[rr]), sa[i][rr] * sw[j], acc[i][j][rr]);
            }
    }

    // Epilogue: undo the 16 x 16 operand scaling (exact), bias, GELU, store.
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = col_base + j * 16 + r16;
            if (col >= n) continue;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int row = row_base + i * 16 + 4 * q + rr;
                if (row >= m) continue;
                const float v = epilogue(acc[i][j][rr] * 0.00390625f, bias, col, epi);
                store_out(y, static_cast<size_t>(row) * n + col, v, out_type);
            }
        }
}

template <int TM, int TN, int WM, int WN, bool TILED>
static int launch(const void *a_codes, const void *a_scales, const void *w_codes, const void *w_scales,
                  const float *bias, void *y, int out_type, int epi, int m, int n, int k, hipStream_t stream) {
    constexpr int BM = WM * TM * 16, BN = WN * TN * 16;
    const long long blocks = static_cast<long long>((m + BM - 1) / BM) * ((n + BN - 1) / BN);
    if (blocks > 0x7FFFFFFFLL) return kInvalid;
    w4a4_gemm_kernel<TM, TN, WM, WN, TILED><<<dim3(static_cast<unsigned>(blocks)), dim3(WM * WN * WAVE), 0, stream>>>(
        static_cast<const uint8_t *>(a_codes), static_cast<const uint16_t *>(a_scales),
        static_cast<const uint8_t *>(w_codes), static_cast<const uint16_t *>(w_scales), bias, y, out_type, epi, m,
        n, k);
    return launch_status();
}

template <bool TILED>
static int dispatch(const void *a_codes, const void *a_scales, const void *w_codes, const void *w_scales,
                    const float *bias, void *y, int out_type, int epi, int m, int n, int k, hipStream_t stream) {
    const long long big_tiles = static_cast<long long>((m + 127) / 128) * ((n + 127) / 128);
    if (big_tiles >= 512) return launch<4, 4, 2, 2, TILED>(a_codes, a_scales, w_codes, w_scales, bias, y, out_type, epi, m, n, k, stream);
    return launch<2, 2, 2, 2, TILED>(a_codes, a_scales, w_codes, w_scales, bias, y, out_type, epi, m, n, k, stream);
}

static bool check_common(const void *a_codes, const void *a_scales, const void *w_codes, const void *w_scales,
                         const void *y, int m, int n, int k) {
    if (m <= 0 || n <= 0 || k <= 0 || k % 256 || n % 16) return false;
    if (!a_codes || !a_scales || !w_codes || !w_scales || !y) return false;
    if (reinterpret_cast<uintptr_t>(a_codes) % 8 || reinterpret_cast<uintptr_t>(w_codes) % 8 ||
        reinterpret_cast<uintptr_t>(a_scales) % 2 || reinterpret_cast<uintptr_t>(w_scales) % 2)
        return false;
    return true;
}

}  // namespace qi

using namespace qi;

QI_API int qi_w4a4_gemm(const void *a_codes, const void *a_scales, const void *w_codes, const void *w_scales, float *y,
                        int m, int n, int k) {
    // gemm.cu:185: the reference accepts only m % 128, n % 128, k % 256.
    if (m % 128 || n % 128 || k % 256) return kInvalid;
    if (m == 0 || n == 0) return 0;
    if (!check_common(a_codes, a_scales, w_codes, w_scales, y, m, n, k)) return kInvalid;
    return dispatch<false>(a_codes, a_scales, w_codes, w_scales, nullptr, y, QI_HIP_OUT_F32, QI_HIP_EPILOGUE_NONE, m, n,
                           k, nullptr);
}

QI_API int qi_hip_w4a4_gemm_tiled(const void *a_codes, const void *a_scales, const void *w_tiled_codes,
                                  const void *w_tiled_scales, const float *bias, void *y, int out_type, int epilogue,
                                  int m, int n, int k, void *stream) {
    if (!check_common(a_codes, a_scales, w_tiled_codes, w_tiled_scales, y, m, n, k)) return kInvalid;
    if (out_type != QI_HIP_OUT_F32 && out_type != QI_HIP_OUT_F16) return kInvalid;
    if (epilogue != QI_HIP_EPILOGUE_NONE && epilogue != QI_HIP_EPILOGUE_GELU_TANH) return kInvalid;
    return dispatch<true>(a_codes, a_scales, w_tiled_codes, w_tiled_scales, bias, y, out_type, epilogue, m, n, k,
                          stream_of(stream));
}
