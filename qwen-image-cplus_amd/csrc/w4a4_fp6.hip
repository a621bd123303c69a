// W4A4 GEMM on gfx950 f8f6f4 MFMA with fp6 (E2M3) operands.
//
// Arithmetic: the reference's (qwen_image_cuda/cuda/gemm.cu:137-168)
//   y[m, n] = sum over ascending groups g of fmaf(P_g[m, n], sa[m, g] * sw[n, g], y)
// with P_g the exact integer dot product of the int4 codes of group g.
//
// Why fp6 and 32x32x64.  Every int4 code -7..7 is exact in E2M3, products of
// two codes are exact, and a group of 64 products sums to at most
// 64 * 49 = 3136 < 2^24, so v_mfma_scale_f32_32x32x64_f8f6f4 (block scales
// 2^0) returns P_g exactly, already as fp32.  Its K = 64 is exactly one g64
// group with no padding, and at the fp6 rate it does the work of two int8
// 16x16x64 MFMAs per 16 cycles, so the matrix core is no longer the limit:
// the exact per-group fp32 step (one fma per output per group, with
// sa * sw formed exactly by v_mfma_f32_32x32x1_2b_f32 outer products) is.
// Results are bit-identical to the reference formula.
//
// Layouts (written by qi_hip_w4a4_quantize_activations_fp6 and
// qi_hip_relayout_w4a4_fp6): per 32-row tile T and group g, 1536 bytes = two
// halves of 64 lanes x 12 bytes; lane l of half h holds the E2M3 codes of
// inputs 32 * (l / 32) + 16h .. + 15 of row 32T + l % 32, which is the lane's
// MFMA operand (6 dwords) split in two.  Scales [rows/32][G][32] fp16 for
// both operands.
//
// Roles.  The MFMA A operand is the weight tile (32 outputs n), B the
// activation tile (32 rows m).  Lane l's accumulator register 4a + r then
// holds y[m = l % 32][n = 8a + 4 * (l / 32) + r]: four consecutive outputs,
// stored with one wide write.
//
// Pipeline.  A ring of NSTAGE LDS slots holds the operand and scale blocks
// of upcoming groups, filled NSTAGE-1 groups ahead by buffer_load ... lds
// (12 bytes per lane for operands: one instruction per 768-byte half block,
// landing at a 16-byte lane pitch; 4 bytes per lane for scales).  One barrier
// per group; each group's matrix-core work is issued before the barrier and
// the next group's LDS reads overlap its fp32 step.

#include <cstdlib>
#include <utility>

#include "qi_common.h"

namespace qi {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v3i __attribute__((ext_vector_type(3)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));

// f(std::integral_constant<int, I>) for I = 0 .. N-1, in order.
template <int N, typename F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

// The MFMA reads six dwords of an fp6 operand; the last two are don't-care.
// Each half is read as a full 16-byte slot (ds_read_b128 runs at twice the
// rate of ds_read_b96 on gfx950); its fourth dword is padding.
__device__ __forceinline__ v8i fp6_operand(v4i lo, v4i hi) {
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 4, 5, 6, -1, -1);
}

template <int TM, int TN, int WM, int WN, int NSTAGE>
__global__ __launch_bounds__(WM *WN *WAVE) __attribute__((amdgpu_waves_per_eu(2))) void w4a4_fp6_kernel(
    const uint8_t *__restrict__ a6, const uint16_t *__restrict__ sa_t, const uint8_t *__restrict__ w6,
    const uint16_t *__restrict__ sw_t, const float *__restrict__ bias, void *__restrict__ y, int out_type, int epi,
    int m, int n, int k) {
    constexpr int NW = WM * WN;
    constexpr int MT = WM * TM, NTL = WN * TN;  // 32-row tiles of the block
    constexpr int BM = MT * 32, BN = NTL * 32;
    constexpr int HALVES = 2 * (MT + NTL);      // 768-byte loads per group
    static_assert(HALVES % NW == 0, "loader mapping");
    constexpr int L_PER_W = HALVES / NW;
    static_assert(TM <= 4 && TN <= 2, "one scale load per operand per wave; scale products pair the n-tiles");
    constexpr int LOADS_PER_GROUP = L_PER_W + 2;  // per wave: operands + sa + sw
    constexpr int TILE = 2048, SLOT = (MT + NTL) * TILE;
    constexpr int SC_WAVE = 512, SC_SLOT = NW * SC_WAVE;  // scale bytes per wave / per slot
    static_assert(NSTAGE * (SLOT + SC_SLOT) <= 160 * 1024, "LDS size");
    __shared__ __attribute__((aligned(16))) uint8_t lds[NSTAGE * SLOT];
    __shared__ __attribute__((aligned(16))) uint8_t lds_sc[NSTAGE * SC_SLOT];

    const int groups = k >> 6;
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int r32 = lane & 31;
    const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN;
    int tm, tn;
    tile_of_block(blockIdx.x, tiles_m, tiles_n, 8, tm, tn);
    const int mt0 = tm * MT, nt0 = tn * NTL;  // first 32-row tiles
    const int m_tiles = (m + 31) / 32, n_tiles = n / 32;

    const uint32_t a_bytes = static_cast<uint32_t>(m_tiles) * groups * 1536u;
    const uint32_t w_bytes = static_cast<uint32_t>(n_tiles) * groups * 1536u;
    const v4i_rsrc ra = raw_rsrc(a6, a_bytes);
    const v4i_rsrc rw = raw_rsrc(w6, w_bytes);
    const v4i_rsrc rsa = raw_rsrc(sa_t, static_cast<uint32_t>(m_tiles) * groups * 64u);
    const v4i_rsrc rsw = raw_rsrc(sw_t, static_cast<uint32_t>(n_tiles) * groups * 64u);

    // This wave's operand loads: half blocks H0 .. H0 + L_PER_W - 1 of the
    // block's (MT + NTL) tiles, activation tiles first.  Missing tiles read
    // past the buffer end, which returns zeros.
    const int H0 = wave * L_PER_W;
    uint32_t vo[L_PER_W];
#pragma unroll
    for (int u = 0; u < L_PER_W; ++u) {
        const int H = H0 + u, X = H >> 1, half = H & 1;
        const bool from_a = H < 2 * MT;
        const int t = from_a ? mt0 + X : nt0 + X - MT;
        const bool ok = from_a ? t < m_tiles : t < n_tiles;
        vo[u] = ok ? static_cast<uint32_t>(t) * groups * 1536u + half * 768u + lane * 12u
                   : (from_a ? a_bytes : w_bytes);
    }
    // Scales, also loaded straight into LDS (so that every vector-memory load
    // of the loop is a direct-to-LDS load whose completion this code counts
    // itself): per wave and group, one 4-byte-per-lane load gathers the 64
    // bytes of each of its TM activation tiles (lanes 16i .. 16i+15) and one
    // those of its TN weight tiles.  Lanes past TM / TN read zeros.
    uint32_t sa_vo, sw_vo;
    {
        const int i = lane >> 4, t = mt0 + wm * TM + i;
        sa_vo = i < TM && t < m_tiles ? static_cast<uint32_t>(t) * groups * 64u + (lane & 15) * 4u : 0x7FFFFFF0u;
        const int tw = nt0 + wn * TN + i;
        sw_vo = i < TN && tw < n_tiles ? static_cast<uint32_t>(tw) * groups * 64u + (lane & 15) * 4u : 0x7FFFFFF0u;
    }

    const uint32_t lds0 = lds_address(lds), sc0 = lds_address(lds_sc);
    auto issue = [&](int g, int slot) {
#pragma unroll
        for (int u = 0; u < L_PER_W; ++u) {
            const int H = H0 + u;
            dma_dwordx3(H < 2 * MT ? ra : rw, lds0 + slot * SLOT + (H >> 1) * TILE + (H & 1) * 1024, vo[u], g * 1536);
        }
        dma_dword(rsa, sc0 + slot * SC_SLOT + wave * SC_WAVE, sa_vo, g * 64);
        dma_dword(rsw, sc0 + slot * SC_SLOT + wave * SC_WAVE + 256, sw_vo, g * 64);
    };

    v16f acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.f;

    // This lane's fragments: weight tile j half h at
    // lds[slot][MT + wn * TN + j][h][16 lane], activation tile i likewise.
    // Scales inside the wave's scale block: sa of row l % 32 of tile i at
    // 64i + 2 (l % 32); the weight scale at 256 + 64 (l / 32) + 2 (l % 32),
    // i.e. output l % 32 of n-tile l / 32.
    const uint8_t *w_frag = lds + (MT + wn * TN) * TILE + lane * 16;
    const uint8_t *x_frag = lds + wm * TM * TILE + lane * 16;
    const uint8_t *sa_lds = lds_sc + wave * SC_WAVE + r32 * 2;
    const uint8_t *sw_lds = lds_sc + wave * SC_WAVE + 256 + lane * 2;

    struct Frags {  // raw LDS reads; converted where consumed
        v8i wf[TN], xf[TM];
        uint32_t sal[TM], swl;
    };
    auto read_frags = [&](auto slot_c, Frags &F) {
        constexpr int slot = decltype(slot_c)::value;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const v4i lo = *reinterpret_cast<const v4i *>(w_frag + slot * SLOT + j * TILE);
            const v4i hi = *reinterpret_cast<const v4i *>(w_frag + slot * SLOT + j * TILE + 1024);
            F.wf[j] = fp6_operand(lo, hi);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const v4i lo = *reinterpret_cast<const v4i *>(x_frag + slot * SLOT + i * TILE);
            const v4i hi = *reinterpret_cast<const v4i *>(x_frag + slot * SLOT + i * TILE + 1024);
            F.xf[i] = fp6_operand(lo, hi);
            F.sal[i] = *reinterpret_cast<const uint16_t *>(sa_lds + slot * SC_SLOT + 64 * i);
        }
        F.swl = *reinterpret_cast<const uint16_t *>(sw_lds + slot * SC_SLOT);
    };
    // Matrix-core work of one group: the scale outer products and the
    // partial tiles.  Block b of the 32x32x1 outer product has rows = outputs
    // of n-tile b (lanes 32b .. 32b+31 supply them) and columns = rows m of
    // tile i; its result registers 16b .. 16b+15 line up with the
    // accumulator registers.
    v32f sp[TM];
    v16f p[TN][TM];
    auto mfma = [&](const Frags &F) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            v32f z32;
#pragma unroll
            for (int r = 0; r < 32; ++r) z32[r] = 0.f;
            sp[i] = __builtin_amdgcn_mfma_f32_32x32x1f32(h2f(static_cast<uint16_t>(F.swl)),
                                                         h2f(static_cast<uint16_t>(F.sal[i])), z32, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                v16f z;
#pragma unroll
                for (int r = 0; r < 16; ++r) z[r] = 0.f;
                // fmt 2 = FP6 E2M3 for both operands; block scales 2^0.
                p[j][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(F.wf[j], F.xf[i], z, 2, 2, 0, 127, 0, 127);
            }
    };
    // The exact fp32 step of one group, in ascending group order.
    auto fmas = [&]() {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[j][i][r] = __builtin_fmaf(p[j][i][r], sp[i][16 * j + r], acc[j][i][r]);
    };

    // Software pipeline, per group g (slots are g mod NSTAGE):
    //   matrix-core work of g (fragments read during g - 1);
    //   wait until this wave's loads of g + 1 are done, barrier (then every
    //   wave's are, and every wave has consumed its reads of slot g - 1);
    //   issue the loads of g + NSTAGE - 1 into slot g - 1;
    //   read the fragments of g + 1, which land during
    //   the fp32 step of g.
    // Loads past the last group read harmless bytes into slots that are
    // never consumed and keep the loads per group constant.
    static_assert(NSTAGE % 4 == 0, "whole quarters of the ring per group count (groups % 4 == 0)");
    Frags F[2];
#pragma unroll
    for (int q = 0; q < NSTAGE - 1; ++q) issue(q, q);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NSTAGE - 2) * LOADS_PER_GROUP) : "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read_frags(std::integral_constant<int, 0>{}, F[0]);
    for (int g0 = 0; g0 < groups; g0 += NSTAGE) {
        static_for<NSTAGE>([&](auto uc) {
            constexpr int u = decltype(uc)::value;
            const int g = g0 + u;
            // groups is a multiple of 4, so only whole quarters of a
            // NSTAGE = 8 ring can be missing at the end; the test is uniform
            // and covers a whole iteration, so no partial tile stays live
            // across iterations.  After the last group the reads of group
            // `groups` fetch harmless slot contents that are never used.
            if (u < 4 || g < groups) {
                // Scheduling fences pin the phase order: the compiler would
                // otherwise sink the matrix-core work below the barrier and
                // the next group's reads, and wait for those reads.
                __builtin_amdgcn_sched_barrier(0);
                mfma(F[u & 1]);
                __builtin_amdgcn_sched_barrier(0);
                // A bare s_barrier: __syncthreads' release fence would also
                // wait for the loads of the groups still in flight.
                asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((NSTAGE - 3) * LOADS_PER_GROUP) : "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                issue(g + NSTAGE - 1, (u + NSTAGE - 1) % NSTAGE);
                read_frags(std::integral_constant<int, (u + 1) % NSTAGE>{}, F[(u + 1) & 1]);
                __builtin_amdgcn_sched_barrier(0);
                fmas();
                __builtin_amdgcn_sched_barrier(0);
            }
        });
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // acc[j][i][4a + r] = y[row, col]: row = m-tile i, lane % 32; col = n-tile
    // j, 8a + 4 * (lane / 32) + r.
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int row = (mt0 + wm * TM + i) * 32 + r32;
        if (row >= m) continue;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int tile_col = (nt0 + wn * TN + j) * 32;
            if (tile_col >= n) continue;
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const int col = tile_col + 8 * a + 4 * (lane >> 5);
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = epilogue(acc[j][i][4 * a + r], bias, col + r, epi);
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
}

template <int TM, int TN, int WM, int WN, int NSTAGE>
static int launch_fp6(const void *a6, const void *sa, const void *w6, const void *sw, const float *bias, void *y,
                      int out_type, int epi, int m, int n, int k, hipStream_t stream) {
    constexpr int BM = WM * TM * 32, BN = WN * TN * 32;
    const long long blocks = static_cast<long long>((m + BM - 1) / BM) * ((n + BN - 1) / BN);
    if (blocks > 0x7FFFFFFFLL) return kInvalid;
    w4a4_fp6_kernel<TM, TN, WM, WN, NSTAGE><<<dim3(static_cast<unsigned>(blocks)), dim3(WM * WN * WAVE), 0, stream>>>(
        static_cast<const uint8_t *>(a6), static_cast<const uint16_t *>(sa), static_cast<const uint8_t *>(w6),
        static_cast<const uint16_t *>(sw), bias, y, out_type, epi, m, n, k);
    return launch_status();
}

}  // namespace qi

using namespace qi;

QI_API int qi_hip_w4a4_gemm_fp6(const void *a_codes6, const void *a_scales_tiled, const void *w_codes6,
                                const void *w_scales_tiled, const float *bias, void *y, int out_type, int epilogue,
                                int m, int n, int k, void *stream) {
    if (m <= 0 || n <= 0 || k <= 0 || n % 32 || k % 256) return kInvalid;
    if (!a_codes6 || !a_scales_tiled || !w_codes6 || !w_scales_tiled || !y) return kInvalid;
    if (out_type != QI_HIP_OUT_F32 && out_type != QI_HIP_OUT_F16) return kInvalid;
    if (epilogue != QI_HIP_EPILOGUE_NONE && epilogue != QI_HIP_EPILOGUE_GELU_TANH) return kInvalid;
    if (reinterpret_cast<uintptr_t>(a_codes6) % 4 || reinterpret_cast<uintptr_t>(w_codes6) % 4 ||
        reinterpret_cast<uintptr_t>(a_scales_tiled) % 2 || reinterpret_cast<uintptr_t>(w_scales_tiled) % 2 ||
        reinterpret_cast<uintptr_t>(y) % (out_type == QI_HIP_OUT_F16 ? 8 : 16))
        return kInvalid;
    const long long g = k / 64;
    if (static_cast<long long>((m + 31) / 32) * g * 1536 >= (1LL << 31) ||
        static_cast<long long>(n / 32) * g * 1536 >= (1LL << 31))
        return kInvalid;
    hipStream_t s = stream_of(stream);
    // Tile shapes (measured on MI355X): 128 x 128 with four waves when that
    // already gives two workgroups per CU; otherwise, for short M, single-
    // wave 32 x 32 tiles with an 8-deep ring, or 64 x 128 four-wave tiles
    // when N is wide.  QI_HIP_FP6_TILES (0..4) overrides the choice, for
    // tuning.
    static const int forced = [] {
        const char *e = getenv("QI_HIP_FP6_TILES");
        return e ? atoi(e) : -1;
    }();
    int cfg;
    if (static_cast<long long>((m + 127) / 128) * ((n + 127) / 128) >= 512)
        cfg = 0;
    else
        cfg = n >= 8192 ? 3 : 4;
    if (forced >= 0) cfg = forced;
    switch (cfg) {
    case 0:
        return launch_fp6<2, 2, 2, 2, 4>(a_codes6, a_scales_tiled, w_codes6, w_scales_tiled, bias, y, out_type,
                                         epilogue, m, n, k, s);
    case 1:
        return launch_fp6<1, 2, 1, 1, 8>(a_codes6, a_scales_tiled, w_codes6, w_scales_tiled, bias, y, out_type,
                                         epilogue, m, n, k, s);
    case 2:
        return launch_fp6<2, 2, 1, 1, 8>(a_codes6, a_scales_tiled, w_codes6, w_scales_tiled, bias, y, out_type,
                                         epilogue, m, n, k, s);
    case 3:
        return launch_fp6<1, 2, 2, 2, 4>(a_codes6, a_scales_tiled, w_codes6, w_scales_tiled, bias, y, out_type,
                                         epilogue, m, n, k, s);
    case 4:
        return launch_fp6<1, 1, 1, 1, 8>(a_codes6, a_scales_tiled, w_codes6, w_scales_tiled, bias, y, out_type,
                                         epilogue, m, n, k, s);
    default:
        return launch_fp6<2, 2, 2, 2, 4>(a_codes6, a_scales_tiled, w_codes6, w_scales_tiled, bias, y, out_type,
                                         epilogue, m, n, k, s);
    }
}
