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

// ---------------------------------------------------------------------------
// Tiled-weight kernel.
//
// Stages.  A stage is four 64-groups (256 inputs).  The codes of the next
// stage go from memory straight into LDS with buffer_load ... lds, issued at
// the start of the current stage into the other half of a double buffer, so
// one barrier per stage suffices.  One such wave instruction fills 1 KiB of
// LDS contiguously (64 lanes x 16 bytes), so both LDS images are laid out
// group-major:
//   lds_a [buf][group][row][32 bytes]      a row's 64 codes of one group
//   lds_b [buf][tile][group][lane][8 bytes] the tiled weight layout itself
// and every fragment read is one 8-byte LDS read per lane, a contiguous
// 512-byte block per wave (conflict-free).  The small scale vectors are
// staged through registers.
//
// Group pipeline.  Per group a wave issues TM*TN MFMAs into one of two
// partial-sum register sets; the fp32 scale steps of the previous group
// (int->float, scale product, fma per output) run between those MFMAs, so no
// VALU instruction waits on an MFMA that was issued just before it.
template <int TM, int TN, int WM, int WN>
__global__ __launch_bounds__(WM *WN *WAVE, 3) void w4a4_tiled_kernel(
    const uint8_t *__restrict__ a_codes, const uint16_t *__restrict__ a_scales, const uint8_t *__restrict__ w_codes,
    const uint16_t *__restrict__ w_scales, const float *__restrict__ bias, void *__restrict__ y, int out_type,
    int epi, int m, int n, int k) {
    constexpr int BM = WM * TM * 16, BN = WN * TN * 16, NW = WM * WN, NT = NW * WAVE;
    constexpr int BT = BN / 16;              // weight tiles per block
    constexpr int A_INSTR = BM / 8;          // 1 KiB direct loads per stage
    constexpr int B_INSTR = BT * 2;
    static_assert(A_INSTR % NW == 0 && B_INSTR % NW == 0, "loader mapping");
    static_assert(BM <= NT && BT * 8 <= NT, "scale loader mapping");
    constexpr int A_PER_W = A_INSTR / NW, B_PER_W = B_INSTR / NW;
    __shared__ __attribute__((aligned(1024))) uint8_t lds_a[2][4][BM][32];
    __shared__ __attribute__((aligned(1024))) uint8_t lds_b[2][BT][4][WAVE][8];
    __shared__ __attribute__((aligned(16))) uint16_t lds_sa[2][4][BM];
    __shared__ __attribute__((aligned(16))) uint16_t lds_sw[2][BT][4][16];

    const int groups = k >> 6, quads = groups >> 2;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int q = lane >> 4, r16 = lane & 15;
    const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN;
    int tm, tn;
    tile_of_block(blockIdx.x, tiles_m, tiles_n, 8, tm, tn);
    const int block_row = tm * BM, block_col = tn * BN;

    const uint32_t a_bytes = static_cast<uint32_t>(m) * static_cast<uint32_t>(k / 2);
    const uint32_t sa_bytes = static_cast<uint32_t>(m) * static_cast<uint32_t>(groups) * 2u;
    const uint32_t b_bytes = static_cast<uint32_t>(n) * static_cast<uint32_t>(k / 2);
    const uint32_t sw_bytes = static_cast<uint32_t>(n) * static_cast<uint32_t>(groups) * 2u;
    const auto ra = buffer_rsrc(a_codes, a_bytes);
    const auto rsa = buffer_rsrc(a_scales, sa_bytes);
    const auto rb = buffer_rsrc(w_codes, b_bytes);
    const auto rsw = buffer_rsrc(w_scales, sw_bytes);

    // Direct-load offsets.  A instruction I: group I % 4, rows 32 * (I / 4)
    // + lane / 2, half lane % 2 of the row's 32-byte group run.  B instruction
    // J: tile J / 2, bytes 1024 * (J % 2) + 16 * lane of the tile's 2 KiB
    // stage block (four consecutive 512-byte group blocks).
    uint32_t a_vo[A_PER_W], b_vo[B_PER_W];
#pragma unroll
    for (int u = 0; u < A_PER_W; ++u) {
        const int I = wave * A_PER_W + u;
        const int row = block_row + 32 * (I >> 2) + (lane >> 1);
        a_vo[u] = row < m ? static_cast<uint32_t>(row) * (k / 2) + ((I & 3) * 2 + (lane & 1)) * 16 : a_bytes;
    }
#pragma unroll
    for (int u = 0; u < B_PER_W; ++u) {
        const int J = wave * B_PER_W + u;
        const int tile = block_col / 16 + (J >> 1);
        b_vo[u] = tile < n / 16 ? static_cast<uint32_t>(tile) * groups * 512u + (J & 1) * 1024u + lane * 16u : b_bytes;
    }
    // Scales: thread t < BM loads its row's 4 activation scales (8 bytes);
    // thread t < 8 * BT loads 16 bytes (8 columns x 1 group... a tile's
    // 4 x 16 weight scales are one 128-byte run).
    const int sa_row = block_row + tid;
    const uint32_t sa_vo = (tid < BM && sa_row < m) ? static_cast<uint32_t>(sa_row) * groups * 2u : sa_bytes;
    const int sw_tile = block_col / 16 + (tid >> 3);
    const uint32_t sw_vo = (tid < 8 * BT && sw_tile < n / 16)
                               ? static_cast<uint32_t>(sw_tile) * groups * 32u + (tid & 7) * 16u
                               : sw_bytes;

    v2i sa_stage = v2i{0, 0};
    v4i sw_stage = v4i{0, 0, 0, 0};
    auto issue_stage = [&](int qd, int buf) {
#pragma unroll
        for (int u = 0; u < A_PER_W; ++u) {
            const int I = wave * A_PER_W + u;
            buffer_load_lds16(ra, &lds_a[buf][I & 3][32 * (I >> 2)][0], a_vo[u], qd * 128);
        }
#pragma unroll
        for (int u = 0; u < B_PER_W; ++u) {
            const int J = wave * B_PER_W + u;
            buffer_load_lds16(rb, &lds_b[buf][J >> 1][2 * (J & 1)][0][0], b_vo[u], qd * 2048);
        }
        if (tid < BM) sa_stage = __builtin_amdgcn_raw_buffer_load_b64(rsa, sa_vo, qd * 8, 0);
        if (tid < 8 * BT) sw_stage = __builtin_amdgcn_raw_buffer_load_b128(rsw, sw_vo, qd * 128, 0);
    };
    auto store_scales = [&](int buf) {
        if (tid < BM) {
            lds_sa[buf][0][tid] = static_cast<uint16_t>(sa_stage[0] & 0xFFFF);
            lds_sa[buf][1][tid] = static_cast<uint16_t>(static_cast<uint32_t>(sa_stage[0]) >> 16);
            lds_sa[buf][2][tid] = static_cast<uint16_t>(sa_stage[1] & 0xFFFF);
            lds_sa[buf][3][tid] = static_cast<uint16_t>(static_cast<uint32_t>(sa_stage[1]) >> 16);
        }
        if (tid < 8 * BT)
            *reinterpret_cast<v4i *>(&lds_sw[buf][tid >> 3][0][0] + (tid & 7) * 8) = sw_stage;
    };

    float acc[TM][TN][4];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;

    // Previous group's partials and scales (fp16 bits, used through mixed fma).
    v4i pp[TM][TN];
    v2i sap[TM];
    uint16_t swp[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        sap[i] = v2i{0, 0};
#pragma unroll
        for (int j = 0; j < TN; ++j) pp[i][j] = v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) swp[j] = 0;

    auto scale_step = [&](int i, int j) {
        const uint32_t s01 = static_cast<uint32_t>(sap[i][0]), s23 = static_cast<uint32_t>(sap[i][1]);
        const float sw = h2f(swp[j]);
        acc[i][j][0] = __builtin_fmaf(static_cast<float>(pp[i][j][0]), h2f(static_cast<uint16_t>(s01 & 0xFFFFu)) * sw,
                                      acc[i][j][0]);
        acc[i][j][1] = __builtin_fmaf(static_cast<float>(pp[i][j][1]), h2f(static_cast<uint16_t>(s01 >> 16)) * sw,
                                      acc[i][j][1]);
        acc[i][j][2] = __builtin_fmaf(static_cast<float>(pp[i][j][2]), h2f(static_cast<uint16_t>(s23 & 0xFFFFu)) * sw,
                                      acc[i][j][2]);
        acc[i][j][3] = __builtin_fmaf(static_cast<float>(pp[i][j][3]), h2f(static_cast<uint16_t>(s23 >> 16)) * sw,
                                      acc[i][j][3]);
    };

    issue_stage(0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    store_scales(0);
    __syncthreads();
    const int wrow = wm * TM * 16, wt = wn * TN;
    for (int qd = 0; qd < quads; ++qd) {
        const int buf = qd & 1;
        if (qd + 1 < quads) issue_stage(qd + 1, buf ^ 1);
#pragma unroll 1
        for (int g4 = 0; g4 < 4; ++g4) {
            v4i af[TM], bf[TN];
            v2i sac[TM];
            uint16_t swc[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const v2i x = *reinterpret_cast<const v2i *>(&lds_a[buf][g4][wrow + i * 16 + r16][q * 8]);
                af[i] = v4i{nib_lo16(x[0]), nib_hi16(x[0]), nib_lo16(x[1]), nib_hi16(x[1])};
                sac[i] = *reinterpret_cast<const v2i *>(&lds_sa[buf][g4][wrow + i * 16 + 4 * q]);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const v2i x = *reinterpret_cast<const v2i *>(&lds_b[buf][wt + j][g4][lane][0]);
                bf[j] = v4i{nib_lo16(x[0]), nib_hi16(x[0]), nib_lo16(x[1]), nib_hi16(x[1])};
                swc[j] = lds_sw[buf][wt + j][g4][r16];
            }
            v4i pc[TM][TN];
#pragma unroll
            for (int t = 0; t < TM * TN; ++t) {
                const int i = t / TN, j = t % TN;
                pc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], v4i{0, 0, 0, 0}, 0, 0, 0);
                scale_step(i, j);
            }
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                sap[i] = sac[i];
#pragma unroll
                for (int j = 0; j < TN; ++j) pp[i][j] = pc[i][j];
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) swp[j] = swc[j];
            // Fragment reads, unpacking, then one MFMA per 12 scale-step
            // instructions of the previous group.
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * TM + 2 * TN, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 6 * (TM + TN), 0);
#pragma unroll
            for (int t = 0; t < TM * TN; ++t) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 14, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (qd + 1 < quads) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            store_scales(buf ^ 1);
        }
        __syncthreads();
    }
    // Drain: the last group's scale steps.
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) scale_step(i, j);

    const int row0 = block_row + wrow, col0 = block_col + wt * 16;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = col0 + j * 16 + r16;
            if (col >= n) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = row0 + i * 16 + 4 * q + r;
                if (row >= m) continue;
                store_out(y, static_cast<size_t>(row) * n + col, epilogue(acc[i][j][r] * 0.00390625f, bias, col, epi),
                          out_type);
            }
        }
}

template <int TM, int TN, int WM, int WN>
static int launch_tiled(const void *a_codes, const void *a_scales, const void *w_codes, const void *w_scales,
                        const float *bias, void *y, int out_type, int epi, int m, int n, int k, hipStream_t stream) {
    constexpr int BM = WM * TM * 16, BN = WN * TN * 16;
    const long long blocks = static_cast<long long>((m + BM - 1) / BM) * ((n + BN - 1) / BN);
    if (blocks > 0x7FFFFFFFLL) return kInvalid;
    w4a4_tiled_kernel<TM, TN, WM, WN><<<dim3(static_cast<unsigned>(blocks)), dim3(WM * WN * WAVE), 0, stream>>>(
        static_cast<const uint8_t *>(a_codes), static_cast<const uint16_t *>(a_scales),
        static_cast<const uint8_t *>(w_codes), static_cast<const uint16_t *>(w_scales), bias, y, out_type, epi, m,
        n, k);
    return launch_status();
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
[[maybe_unused]] static int dispatch(const void *a_codes, const void *a_scales, const void *w_codes, const void *w_scales,
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
    // 32-bit buffer offsets: every operand must stay below 4 GiB.
    if (static_cast<long long>(m) * (k / 2) >= (1LL << 32) || static_cast<long long>(n) * (k / 2) >= (1LL << 32))
        return kInvalid;
    const long long big_tiles = static_cast<long long>((m + 127) / 128) * ((n + 127) / 128);
    if (big_tiles >= 384)
        return launch_tiled<4, 2, 2, 2>(a_codes, a_scales, w_tiled_codes, w_tiled_scales, bias, y, out_type, epilogue,
                                        m, n, k, stream_of(stream));
    return launch_tiled<2, 2, 2, 2>(a_codes, a_scales, w_tiled_codes, w_tiled_scales, bias, y, out_type, epilogue, m,
                                    n, k, stream_of(stream));
}
