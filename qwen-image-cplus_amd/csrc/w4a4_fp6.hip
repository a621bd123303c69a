// W4A4 GEMM on gfx950 f8f6f4 MFMA with fp6 (E2M3) operands.
//
// Arithmetic: the reference's (qwen_image_cuda/cuda/gemm.cu:137-168)
//   y[m, n] = sum over ascending groups g of fmaf(P_g[m, n], sa[m, g] * sw[n, g], y)
// with P_g the exact integer dot product of the int4 codes of group g.
//
// Why fp6.  Every int4 code -7..7 is exact in E2M3, products of two codes are
// exact, and a K-slice of 64 codes sums to at most 64 * 49 = 3136, so the
// f8f6f4 MFMA returns P_g exactly, already as fp32 (checked against the int8
// MFMA on the same codes).  One v_mfma_scale_f32_16x16x128_f8f6f4 covers one
// 64-group in half of its 128 K-slots (the weight operand's upper slots are
// zero) at the same cost as one v_mfma_i32_16x16x64_i8, but it saves the
// int -> float conversion in the per-group fp32 step, which is the bottleneck
// of W4A4 on this chip: a wave64 fp32 VALU instruction costs 4 cycles and
// overlaps little with the matrix core.  The scale products sa * sw (exact in
// fp32: two 11-bit significands) come from a v_mfma_f32_4x4x1_16b_f32 outer
// product, so the VALU does only the fma per output.  Results are
// bit-identical to the reference formula, like the int8 kernel's.
//
// Layouts (produced by qi_hip_w4a4_quantize_activations_fp6 and
// qi_hip_relayout_w4a4_fp6): per 16-row tile t and group g, 768 bytes =
// 64 lanes x 12 bytes of MFMA operand, lane q*16 + r holding the 16 E2M3 codes
// of inputs 16q..16q+15 of row 16t + r; scales per (t, g) as 16 fp16.
//
// Roles.  The MFMA A operand is the weight tile (16 outputs n) and B the
// activation tile (16 rows m), so a lane accumulates four consecutive outputs
// n of one row m and stores them with one wide write.
//
// Pipeline.  A ring of NSTAGE LDS slots holds the operand blocks of upcoming
// groups, filled with 12-byte-per-lane buffer_load ... lds (one instruction =
// one 768-byte tile block, which lands in LDS at a 16-byte lane pitch),
// NSTAGE-1 groups ahead; the scales ride in a
// register ring.  One barrier per group.

#include "qi_common.h"

namespace qi {

typedef int v8i __attribute__((ext_vector_type(8)));

__device__ __forceinline__ void buffer_load_lds12(__amdgpu_buffer_rsrc_t rsrc, void *lds, uint32_t voffset,
                                                  uint32_t soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)lds, 12, voffset,
                                             soffset, 0, 0);
}

template <int TM, int TN, int WM, int WN>
__global__ __launch_bounds__(WM *WN *WAVE, 2) void w4a4_fp6_kernel(
    const uint8_t *__restrict__ a6, const uint16_t *__restrict__ sa_t, const uint8_t *__restrict__ w6,
    const uint16_t *__restrict__ sw_t, const float *__restrict__ bias, void *__restrict__ y, int out_type, int epi,
    int m, int n, int k) {
    constexpr int NSTAGE = 4;
    constexpr int NW = WM * WN;
    constexpr int MT = WM * TM, NTL = WN * TN;  // 16-row tiles of the block
    constexpr int BM = MT * 16, BN = NTL * 16;
    static_assert((MT + NTL) % NW == 0, "loader mapping");
    constexpr int L_PER_W = (MT + NTL) / NW;
    constexpr int LOADS_PER_GROUP = L_PER_W + TM + TN;  // per wave
    // A 12-byte direct-to-LDS load writes lane i's bytes at offset 16 * i.
    __shared__ __attribute__((aligned(16))) uint8_t lds_x[NSTAGE][MT][1024];
    __shared__ __attribute__((aligned(16))) uint8_t lds_w[NSTAGE][NTL][1024];

    const int groups = k >> 6;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int r16 = lane & 15;
    const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN;
    int tm, tn;
    tile_of_block(blockIdx.x, tiles_m, tiles_n, 8, tm, tn);
    const int mt0 = tm * MT, nt0 = tn * NTL;  // first 16-row tiles
    const int m_tiles = (m + 15) / 16, n_tiles = n / 16;

    const uint32_t a_bytes = static_cast<uint32_t>(m_tiles) * groups * 768u;
    const uint32_t w_bytes = static_cast<uint32_t>(n_tiles) * groups * 768u;
    const uint32_t sa_bytes = static_cast<uint32_t>(m_tiles) * groups * 32u;
    const uint32_t sw_bytes = static_cast<uint32_t>(n_tiles) * groups * 32u;
    const auto ra = buffer_rsrc(a6, a_bytes);
    const auto rw = buffer_rsrc(w6, w_bytes);
    const auto rsa = buffer_rsrc(sa_t, sa_bytes);
    const auto rsw = buffer_rsrc(sw_t, sw_bytes);

    // Operand block loads: instruction I < MT is m-tile I, else n-tile I - MT.
    uint32_t vo[L_PER_W];
#pragma unroll
    for (int u = 0; u < L_PER_W; ++u) {
        const int I = wave * L_PER_W + u;
        if (I < MT) {
            const int t = mt0 + I;
            vo[u] = t < m_tiles ? static_cast<uint32_t>(t) * groups * 768u + lane * 12u : a_bytes;
        } else {
            const int t = nt0 + I - MT;
            vo[u] = t < n_tiles ? static_cast<uint32_t>(t) * groups * 768u + lane * 12u : w_bytes;
        }
    }
    // Scale operands of the 4x4x1 outer product: the weight lane value is
    // sw[4 * (lane / 16) + lane % 4], the activation lane value sa[lane % 16].
    uint32_t sa_vo[TM], sw_vo[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int t = mt0 + wm * TM + i;
        sa_vo[i] = t < m_tiles ? (static_cast<uint32_t>(t) * groups * 16u + r16) * 2u : sa_bytes;
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int t = nt0 + wn * TN + j;
        sw_vo[j] = t < n_tiles ? (static_cast<uint32_t>(t) * groups * 16u + 4 * (lane >> 4) + (lane & 3)) * 2u
                               : sw_bytes;
    }

    uint32_t sa_ring[NSTAGE][TM], sw_ring[NSTAGE][TN];
    auto issue = [&](int g, int slot) {
#pragma unroll
        for (int u = 0; u < L_PER_W; ++u) {
            const int I = wave * L_PER_W + u;
            if (I < MT)
                buffer_load_lds12(ra, &lds_x[slot][I][0], vo[u], g * 768);
            else
                buffer_load_lds12(rw, &lds_w[slot][I - MT][0], vo[u], g * 768);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
            sa_ring[slot][i] = __builtin_amdgcn_raw_buffer_load_b16(rsa, sa_vo[i], g * 32, 0);
#pragma unroll
        for (int j = 0; j < TN; ++j)
            sw_ring[slot][j] = __builtin_amdgcn_raw_buffer_load_b16(rsw, sw_vo[j], g * 32, 0);
    };

    v4f acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[j][i] = v4f{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int slot) {
        v8i wf[TN], xf[TM];
        float swl[TN], sal[TM];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint32_t *p = reinterpret_cast<const uint32_t *>(&lds_w[slot][wn * TN + j][lane * 16]);
            wf[j] = v8i{static_cast<int>(p[0]), static_cast<int>(p[1]), static_cast<int>(p[2]), 0, 0, 0, 0, 0};
            swl[j] = h2f(static_cast<uint16_t>(sw_ring[slot][j]));
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const uint32_t *p = reinterpret_cast<const uint32_t *>(&lds_x[slot][wm * TM + i][lane * 16]);
            xf[i] = v8i{static_cast<int>(p[0]), static_cast<int>(p[1]), static_cast<int>(p[2]), 0, 0, 0, 0, 0};
            sal[i] = h2f(static_cast<uint16_t>(sa_ring[slot][i]));
        }
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                // fmt 2 = FP6 E2M3 for both operands; block scales 2^0.
                const v4f p = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf[j], xf[i], v4f{0.f, 0.f, 0.f, 0.f},
                                                                             2, 2, 0, 127, 0, 127);
                const v4f s = __builtin_amdgcn_mfma_f32_4x4x1f32(swl[j], sal[i], v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[j][i][r] = __builtin_fmaf(p[r], s[r], acc[j][i][r]);
            }
    };

    // Prologue; loads past the last group read harmless bytes into slots
    // that are never consumed and keep the loads per group constant.
#pragma unroll
    for (int p = 0; p < NSTAGE - 1; ++p) issue(p, p);
    for (int g0 = 0; g0 < groups; g0 += NSTAGE) {
#pragma unroll
        for (int u = 0; u < NSTAGE; ++u) {
            const int g = g0 + u;
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NSTAGE - 2) * LOADS_PER_GROUP) : "memory");
            __syncthreads();
            issue(g + NSTAGE - 1, (u + NSTAGE - 1) % NSTAGE);
            if (g < groups) compute(u);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // acc[j][i][r] = y[row, col]: row = m-tile i, lane % 16; col = n-tile j,
    // 4 * (lane / 16) + r.
    const int q = lane >> 4;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = (nt0 + wn * TN + j) * 16 + 4 * q;
        if (col >= n) continue;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int row = (mt0 + wm * TM + i) * 16 + r16;
            if (row >= m) continue;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = epilogue(acc[j][i][r], bias, col + r, epi);
            const size_t idx = static_cast<size_t>(row) * n + col;
            if (out_type == QI_HIP_OUT_F16) {
                uint2 h;
                h.x = static_cast<uint32_t>(f2h(v[0])) | (static_cast<uint32_t>(f2h(v[1])) << 16);
                h.y = static_cast<uint32_t>(f2h(v[2])) | (static_cast<uint32_t>(f2h(v[3])) << 16);
                *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(y) + idx) = h;
            } else {
                *reinterpret_cast<float4 *>(reinterpret_cast<float *>(y) + idx) = float4{v[0], v[1], v[2], v[3]};
            }
        }
    }
}

template <int TM, int TN, int WM, int WN>
static int launch_fp6(const void *a6, const void *sa, const void *w6, const void *sw, const float *bias, void *y,
                      int out_type, int epi, int m, int n, int k, hipStream_t stream) {
    constexpr int BM = WM * TM * 16, BN = WN * TN * 16;
    const long long blocks = static_cast<long long>((m + BM - 1) / BM) * ((n + BN - 1) / BN);
    if (blocks > 0x7FFFFFFFLL) return kInvalid;
    w4a4_fp6_kernel<TM, TN, WM, WN><<<dim3(static_cast<unsigned>(blocks)), dim3(WM * WN * WAVE), 0, stream>>>(
        static_cast<const uint8_t *>(a6), static_cast<const uint16_t *>(sa), static_cast<const uint8_t *>(w6),
        static_cast<const uint16_t *>(sw), bias, y, out_type, epi, m, n, k);
    return launch_status();
}

}  // namespace qi

using namespace qi;

QI_API int qi_hip_w4a4_gemm_fp6(const void *a_codes6, const void *a_scales_tiled, const void *w_codes6,
                                const void *w_scales_tiled, const float *bias, void *y, int out_type, int epilogue,
                                int m, int n, int k, void *stream) {
    if (m <= 0 || n <= 0 || k <= 0 || n % 16 || k % 256) return kInvalid;
    if (!a_codes6 || !a_scales_tiled || !w_codes6 || !w_scales_tiled || !y) return kInvalid;
    if (out_type != QI_HIP_OUT_F32 && out_type != QI_HIP_OUT_F16) return kInvalid;
    if (epilogue != QI_HIP_EPILOGUE_NONE && epilogue != QI_HIP_EPILOGUE_GELU_TANH) return kInvalid;
    if (reinterpret_cast<uintptr_t>(a_codes6) % 4 || reinterpret_cast<uintptr_t>(w_codes6) % 4 ||
        reinterpret_cast<uintptr_t>(a_scales_tiled) % 2 || reinterpret_cast<uintptr_t>(w_scales_tiled) % 2)
        return kInvalid;
    const long long g = k / 64;
    if (static_cast<long long>((m + 15) / 16) * g * 768 >= (1LL << 32) || static_cast<long long>(n / 16) * g * 768 >= (1LL << 32))
        return kInvalid;
    hipStream_t s = stream_of(stream);
    if (m <= 512)
        return launch_fp6<2, 2, 2, 2>(a_codes6, a_scales_tiled, w_codes6, w_scales_tiled, bias, y, out_type, epilogue, m,
                                      n, k, s);
    return launch_fp6<4, 4, 2, 2>(a_codes6, a_scales_tiled, w_codes6, w_scales_tiled, bias, y, out_type, epilogue, m, n,
                                  k, s);
}
