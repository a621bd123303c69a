// W4A16 GEMM on gfx950 fp16 MFMA: y[m, n] = sum_k x[m, k] * W[n, k], with
// W = fp16(fmaf(code, scale, minimum)) dequantised per 64-group.
//
// Reference arithmetic: qwen_image_cuda/cuda/gemm.cu:191-268
// (w4a16_gemm_kernel, qi_w4a16_gemm): the weight tile is expanded with
// __float2half(fmaf(code, scale, min)) and multiplied in fp16 with fp32
// accumulation.
//
// Design.  A workgroup is WM wavefronts stacked along M that share one BN-wide
// column strip.  Per 64-group, every thread dequantises exactly the 16
// weights one lane of one 16-column tile needs (two 8-element halves, one per
// v_mfma_f32_16x16x32_f16 K-step) and writes them to LDS in fragment order,
// so each weight is dequantised once per workgroup and each MFMA B operand is
// one conflict-free 16-byte LDS read.  Activations go straight from global
// memory to registers (16 contiguous bytes per lane and K-step).  LDS is
// double-buffered so one barrier per group suffices, and the next group's
// codes, scales and activations are loaded while the current group computes.

#include "qi_common.h"

namespace qi {

// 8 codes (one dword, element 2j in the low nibble of byte j) -> 8 fp16
// weights in element order, exactly fp16(fmaf(code, scale, minimum)).
__device__ __forceinline__ uint4 dequant8(uint32_t x, float scale, float minimum) {
    const uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
    uint32_t out[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float e0 = static_cast<float>((lo >> (8 * j)) & 0xFFu);
        const float e1 = static_cast<float>((hi >> (8 * j)) & 0xFFu);
        out[j] = static_cast<uint32_t>(dequant_w4a16(e0, scale, minimum)) |
                 (static_cast<uint32_t>(dequant_w4a16(e1, scale, minimum)) << 16);
    }
    return uint4{out[0], out[1], out[2], out[3]};
}

template <int TM, int TN, int WM, bool TILED>
__global__ __launch_bounds__(WM *WAVE) void w4a16_gemm_kernel(
    const uint16_t *__restrict__ x, const uint8_t *__restrict__ codes, const uint16_t *__restrict__ scales,
    const uint16_t *__restrict__ minimums, const float *__restrict__ bias, void *__restrict__ y, int out_type,
    int epi, int m, int n, int k) {
    constexpr int BM = WM * TM * 16, BN = TN * 16;
    // [buffer][tile][step][lane] 16-byte fragments.
    __shared__ uint4 lds[2][TN][2][WAVE];
    const int groups = k >> 6;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const int q = lane >> 4, r16 = lane & 15;
    const int tiles_n = (n + BN - 1) / BN;
    const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
    const int row_base = tm * BM + wave * TM * 16;
    const int col_base = tn * BN;

    // Activation fragment pointers: row (clamped), first k of this lane.
    const uint16_t *xp[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int r = min(row_base + i * 16 + r16, m - 1);
        xp[i] = x + static_cast<size_t>(r) * k + 8 * q;
    }

    // Dequantisation assignment: wave w handles tiles w, w + WM, ...
    constexpr int DQ = (TN + WM - 1) / WM;
    const uint8_t *cp[DQ];
    const uint16_t *sp[DQ];
    const uint16_t *mp[DQ];
#pragma unroll
    for (int d = 0; d < DQ; ++d) {
        const int jt = min(wave + d * WM, TN - 1);
        const int tile = min((col_base + jt * 16) / 16, n / 16 - 1);
        if (TILED) {
            cp[d] = codes + static_cast<size_t>(tile) * groups * 512 + lane * 8;
            sp[d] = scales + (static_cast<size_t>(tile) * groups * 16 + r16) * 2;
            mp[d] = sp[d] + 1;
        } else {
            const int row = tile * 16 + r16;
            cp[d] = codes + static_cast<size_t>(row) * (k / 2) + 4 * q;
            sp[d] = scales + static_cast<size_t>(row) * groups;
            mp[d] = minimums + static_cast<size_t>(row) * groups;
        }
    }
    constexpr int kCStep = TILED ? 512 : 32;
    constexpr int kSStep = TILED ? 32 : 1;

    v4f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    uint4 a_next[TM][2];
    uint2 c_next[DQ];
    uint16_t s_next[DQ], m_next[DQ];
    auto fetch = [&](int g) {
#pragma unroll
        for (int d = 0; d < DQ; ++d) {
            const uint8_t *c = cp[d] + static_cast<size_t>(g) * kCStep;
            if (TILED) {
                c_next[d] = *reinterpret_cast<const uint2 *>(c);
            } else {
                c_next[d].x = *reinterpret_cast<const uint32_t *>(c);
                c_next[d].y = *reinterpret_cast<const uint32_t *>(c + 16);
            }
            s_next[d] = sp[d][static_cast<size_t>(g) * kSStep];
            m_next[d] = mp[d][static_cast<size_t>(g) * kSStep];
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            a_next[i][0] = *reinterpret_cast<const uint4 *>(xp[i] + g * 64);
            a_next[i][1] = *reinterpret_cast<const uint4 *>(xp[i] + g * 64 + 32);
        }
    };
    auto dequant_to_lds = [&](int buf) {
#pragma unroll
        for (int d = 0; d < DQ; ++d) {
            const int jt = wave + d * WM;
            if (jt >= TN) continue;
            const float s = h2f(s_next[d]), mn = h2f(m_next[d]);
            lds[buf][jt][0][lane] = dequant8(c_next[d].x, s, mn);
            lds[buf][jt][1][lane] = dequant8(c_next[d].y, s, mn);
        }
    };

    fetch(0);
    dequant_to_lds(0);
    __syncthreads();
    for (int g = 0; g < groups; ++g) {
        const int buf = g & 1;
        uint4 a_cur[TM][2];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            a_cur[i][0] = a_next[i][0];
            a_cur[i][1] = a_next[i][1];
        }
        if (g + 1 < groups) fetch(g + 1);
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            v8h b_frag[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j) b_frag[j] = __builtin_bit_cast(v8h, lds[buf][j][s][lane]);
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const v8h a_frag = __builtin_bit_cast(v8h, a_cur[i][s]);
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_frag, b_frag[j], acc[i][j], 0, 0, 0);
            }
        }
        if (g + 1 < groups) dequant_to_lds(buf ^ 1);
        __syncthreads();
    }

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
                store_out(y, static_cast<size_t>(row) * n + col, epilogue(acc[i][j][rr], bias, col, epi), out_type);
            }
        }
}

template <int TM, int TN, int WM, bool TILED>
static int launch(const void *x, const void *codes, const void *scales, const void *minimums, const float *bias,
                  void *y, int out_type, int epi, int m, int n, int k, hipStream_t stream) {
    constexpr int BM = WM * TM * 16, BN = TN * 16;
    const long long blocks = static_cast<long long>((m + BM - 1) / BM) * ((n + BN - 1) / BN);
    if (blocks > 0x7FFFFFFFLL) return kInvalid;
    w4a16_gemm_kernel<TM, TN, WM, TILED><<<dim3(static_cast<unsigned>(blocks)), dim3(WM * WAVE), 0, stream>>>(
        static_cast<const uint16_t *>(x), static_cast<const uint8_t *>(codes), static_cast<const uint16_t *>(scales),
        static_cast<const uint16_t *>(minimums), bias, y, out_type, epi, m, n, k);
    return launch_status();
}

template <bool TILED>
static int dispatch(const void *x, const void *codes, const void *scales, const void *minimums, const float *bias,
                    void *y, int out_type, int epi, int m, int n, int k, hipStream_t stream) {
    const long long big = static_cast<long long>((m + 255) / 256) * ((n + 63) / 64);
    if (big >= 512) return launch<4, 4, 4, TILED>(x, codes, scales, minimums, bias, y, out_type, epi, m, n, k, stream);
    return launch<1, 4, 4, TILED>(x, codes, scales, minimums, bias, y, out_type, epi, m, n, k, stream);
}

}  // namespace qi

using namespace qi;

int qi_hip_w4a16_gemv_impl(const void *x_half, const void *w_tiled_codes, const void *w_tiled_scales,
                           const float *bias, void *y, int out_type, int epilogue, int m, int n, int k,
                           hipStream_t stream);

QI_API int qi_w4a16_gemm(const void *x_half, const void *codes, const void *scales, const void *minimums, float *y,
                         int m, int n, int k) {
    // gemm.cu:264: the reference accepts only m % 128, n % 128, k % 64.
    if (m % 128 || n % 128 || k % 64) return kInvalid;
    if (m == 0 || n == 0) return 0;
    if (m < 0 || n < 0 || k <= 0 || !x_half || !codes || !scales || !minimums || !y) return kInvalid;
    if (reinterpret_cast<uintptr_t>(x_half) % 16 || reinterpret_cast<uintptr_t>(codes) % 4) return kInvalid;
    return dispatch<false>(x_half, codes, scales, minimums, nullptr, y, QI_HIP_OUT_F32, QI_HIP_EPILOGUE_NONE, m, n, k,
                           nullptr);
}

QI_API int qi_hip_w4a16_gemm_tiled(const void *x_half, const void *w_tiled_codes, const void *w_tiled_scales,
                                   const float *bias, void *y, int out_type, int epilogue, int m, int n, int k,
                                   void *stream) {
    if (m <= 0 || n <= 0 || k <= 0 || n % 16 || k % 64) return kInvalid;
    if (!x_half || !w_tiled_codes || !w_tiled_scales || !y) return kInvalid;
    if (out_type != QI_HIP_OUT_F32 && out_type != QI_HIP_OUT_F16) return kInvalid;
    if (epilogue != QI_HIP_EPILOGUE_NONE && epilogue != QI_HIP_EPILOGUE_GELU_TANH) return kInvalid;
    if (reinterpret_cast<uintptr_t>(x_half) % 16 || reinterpret_cast<uintptr_t>(w_tiled_codes) % 8 ||
        reinterpret_cast<uintptr_t>(w_tiled_scales) % 4 || k % 8)
        return kInvalid;
    if (m <= 16)
        return qi_hip_w4a16_gemv_impl(x_half, w_tiled_codes, w_tiled_scales, bias, y, out_type, epilogue, m, n, k,
                                      stream_of(stream));
    const uint16_t *ts = static_cast<const uint16_t *>(w_tiled_scales);
    return dispatch<true>(x_half, w_tiled_codes, ts, ts + 1, bias, y, out_type, epilogue, m, n, k, stream_of(stream));
}
