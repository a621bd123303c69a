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

// One 64-group of a wave's W4A16 tile: dequantise its TN weight tiles (code
// dword pairs c[j], (scale, minimum) words sc[j]) and multiply them with the
// TM activation row tiles staged at xs ([TM * 16][128] bytes, the 16-byte
// chunks of row r XOR-swizzled by r & 7) into acc.
//
// Both steps' weights are dequantised before the MFMAs.  Words come
// from packed fp16 (and-or to 1024 + c, one packed fma) when that is provably
// the reference's value for every group of the wave; otherwise a rare
// uniform branch replaces them with the reference's fp32 fma + RNE before
// they are used.
// Activation fragment f = step * TM + i of a group: rows 16 i .. 16 i + 15
// of the LDS slot, inputs 32 step + 8q .. + 7 (chunks XOR-swizzled by row).
template <int TM>
__device__ __forceinline__ void w4a16_read_x(const uint8_t *xs, int f, int r16, int q, v8h (&xr)[2 * TM]) {
    const int st = f / TM, row = 16 * (f % TM) + r16;
    xr[f] = *reinterpret_cast<const v8h *>(xs + row * 128 + ((4 * st + q) ^ (row & 7)) * 16);
}

// The group's MFMAs: fragment f's read LA fragments ahead, the first LA
// already requested by the caller.
template <int TM, int TN>
__device__ __forceinline__ void w4a16_steps(const uint8_t *xs, const uint32_t (&w0)[TN][4],
                                            const uint32_t (&w1)[TN][4], int r16, int q, v8h (&xr)[2 * TM],
                                            v4f (&acc)[TN][TM]) {
    constexpr int NF = 2 * TM, LA = NF < 4 ? NF : 4;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        if (f + LA < NF) w4a16_read_x<TM>(xs, f + LA, r16, q, xr);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint32_t *w = f < TM ? w0[j] : w1[j];
            acc[j][f % TM] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                __builtin_bit_cast(v8h, uint4{w[0], w[1], w[2], w[3]}), xr[f], acc[j][f % TM], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <int TM, int TN>
__device__ __forceinline__ void w4a16_group_mfma(const uint8_t *xs, const v2i (&c)[TN], const uint32_t (&sc)[TN],
                                                 int r16, int q, v4f (&acc)[TN][TM]) {
    bool fast = true;
#pragma unroll
    for (int j = 0; j < TN; ++j) fast = fast && w4a16_single_rounding_exact(sc[j] & 0xFFFFu, sc[j] >> 16);
    fast = __all(fast);
    const v2h k1024 = v2h{static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
    uint32_t magic = 0x64006400u;
    asm volatile("" : "+v"(magic));
    v2h s2[TN], m2[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const uint32_t sb = sc[j] & 0xFFFFu, mb = sc[j] >> 16;
        s2[j] = __builtin_bit_cast(v2h, sb | (sb << 16));
        m2[j] = __builtin_bit_cast(v2h, mb | (mb << 16));
    }
    // Word i of code dword `half` of tile j: nibbles i and 4 + i.
    auto word = [&](int j, int half, int i) -> uint32_t {
        const uint32_t x = static_cast<uint32_t>(c[j][half]);
        const uint32_t biased = ((x >> (4 * i)) & 0x000F000Fu) | (magic & ~0x000F000Fu);
        const v2h cc = __builtin_bit_cast(v2h, biased) - k1024;
        return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(cc, s2[j], m2[j]));
    };
    auto exact_words = [&](int half, uint32_t(&w)[TN][4]) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const uint4 e = w4a16_dequant8(static_cast<uint32_t>(c[j][half]), sc[j] & 0xFFFFu, sc[j] >> 16, false);
            w[j][0] = e.x;
            w[j][1] = e.y;
            w[j][2] = e.z;
            w[j][3] = e.w;
        }
    };
    uint32_t w0[TN][4], w1[TN][4];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) w0[j][i] = word(j, 0, i);
    if (!fast) exact_words(0, w0);
    // The activation fragments of both steps as one sequence f = step * TM
    // + i, each requested LA fragments ahead of its MFMAs, so that only the
    // first LA reads of a group are waited for (measured on MI355X against
    // reading eight row tiles at a time: 4096 x 12288 x 3072 315 -> 284 us,
    // 4096 x 3072 x 12288 296 -> 277 us).
    constexpr int NF = 2 * TM, LA = NF < 4 ? NF : 4;
    v8h xr[NF];
#pragma unroll
    for (int f = 0; f < LA; ++f) w4a16_read_x<TM>(xs, f, r16, q, xr);
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) w1[j][i] = word(j, 1, i);
    if (!fast) exact_words(1, w1);
    __builtin_amdgcn_sched_barrier(0);
    w4a16_steps<TM, TN>(xs, w0, w1, r16, q, xr, acc);
}

// The same group step on weights dequantised beforehand (fp16 fragments,
// w[j][step] = the A operand of tile j's MFMA for K step `step`).
template <int TM, int TN>
__device__ __forceinline__ void w4a16_group_mfma_f16w(const uint8_t *xs, const v4i (&w)[TN][2], int r16, int q,
                                                      v4f (&acc)[TN][TM]) {
    constexpr int NF = 2 * TM, LA = NF < 4 ? NF : 4;
    v8h xr[NF];
#pragma unroll
    for (int f = 0; f < LA; ++f) w4a16_read_x<TM>(xs, f, r16, q, xr);
    uint32_t w0[TN][4], w1[TN][4];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w0[j][i] = static_cast<uint32_t>(w[j][0][i]);
            w1[j][i] = static_cast<uint32_t>(w[j][1][i]);
        }
    __builtin_amdgcn_sched_barrier(0);
    w4a16_steps<TM, TN>(xs, w0, w1, r16, q, xr, acc);
}

// ---------------------------------------------------------------------------
// Tiled-weight kernel.
//
// Roles.  The MFMA's A operand is the dequantised weight tile (16 outputs n)
// and its B operand the activation tile (16 rows m), so the accumulator holds
// y^T: each lane owns four consecutive outputs n of one row m and stores them
// with one 8-byte (fp16) or 16-byte (fp32) write.
//
// Work split.  The NW wavefronts of a workgroup share the same BM activation
// rows and own disjoint 16*TN-column slices of the weights, so every weight is
// dequantised exactly once per workgroup, in registers, by the wave that uses
// it, and only the activations need LDS.
//
// Latency.  Activation tiles (fp16 [BM][64] per 64-group) go memory -> LDS
// with buffer_load ... lds into a ring of NSTAGE slots, and weight codes and
// scales into a register ring, issued NSTAGE-1 groups ahead: at the MI355X's
// memory latency a single group of MFMA work is far too short to cover a
// load.  One barrier per group.  The eight 16-byte chunks of each activation
// row are XOR-swizzled by (row & 7) so fragment reads spread over the banks.
//
// Dequantisation uses packed fp16 (two weights per instruction) when that is
// provably the reference's value for the group's (scale, minimum), and the
// reference's fp32 fma + RNE otherwise.
template <int TM, int TN, int NW, int NSTAGE, bool F16W>
__global__ __launch_bounds__(NW *WAVE, (NW >= 8 ? 1 : 2)) void w4a16_tiled_kernel(
    const uint16_t *__restrict__ x, const uint8_t *__restrict__ codes, const uint16_t *__restrict__ scales,
    const float *__restrict__ bias, void *__restrict__ y, int out_type, int epi, int m, int n, int k, int n_part,
    OutMap out, TileGrid2 gd) {
    static_assert((NSTAGE - 2) * (TM * 2 / NW + 2 * TN) <= 63, "vmcnt range");
    constexpr int BM = TM * 16, BN = NW * TN * 16;
    constexpr int A_INSTR = BM / 8;  // 1 KiB = 8 rows x 128 bytes per direct load
    static_assert(A_INSTR % NW == 0, "loader mapping");
    constexpr int A_PER_W = A_INSTR / NW;
    constexpr int LOADS_PER_GROUP = A_PER_W + 2 * TN;  // per wave
    __shared__ __attribute__((aligned(1024))) uint8_t lds_a[NSTAGE][BM][128];

    const int groups = k >> 6;
    // K split over gridDim.y: this workgroup's groups [g_lo, g_lo + g_cnt).
    const int g_lo = static_cast<int>(blockIdx.y * groups / gridDim.y);
    const int g_cnt = static_cast<int>((blockIdx.y + 1) * groups / gridDim.y) - g_lo;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const int q = lane >> 4, r16 = lane & 15;
    int tm, tn;
    grid_tile(gd, blockIdx.x, tm, tn);
    const int block_row = tm * BM, block_col = tn * BN;

    const uint32_t x_bytes = static_cast<uint32_t>(m) * static_cast<uint32_t>(k) * 2u;
    // F16W: `codes` holds the weights dequantised beforehand, fp16 MFMA
    // fragments [n / 16][groups][64 lanes][2 steps][8], 2 KiB per tile and
    // group; `scales` is unused.
    const uint32_t c_bytes = static_cast<uint32_t>(n) * static_cast<uint32_t>(F16W ? 2 * k : k / 2);
    const uint32_t s_bytes = static_cast<uint32_t>(n) * static_cast<uint32_t>(groups) * 4u;
    const auto rx = buffer_rsrc(x, x_bytes);
    const auto rc = buffer_rsrc(codes, c_bytes);
    const auto rs = buffer_rsrc(scales, s_bytes);

    // Activation direct loads: instruction I covers rows 8I..8I+7; lane L
    // fills LDS chunk L % 8 of row 8I + L / 8 with global chunk
    // (L % 8) ^ (row & 7).
    uint32_t x_vo[A_PER_W];
#pragma unroll
    for (int u = 0; u < A_PER_W; ++u) {
        const int I = wave * A_PER_W + u;
        const int row = 8 * I + (lane >> 3), grow = block_row + row;
        const int chunk = (lane & 7) ^ (row & 7);
        x_vo[u] = grow < m ? static_cast<uint32_t>(grow) * k * 2u + chunk * 16u : x_bytes;
    }
    // This wave's weight tiles.
    uint32_t c_vo[TN], s_vo[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int tile = block_col / 16 + wave * TN + j;
        const bool ok = tile < n / 16;
        c_vo[j] = ok ? (F16W ? static_cast<uint32_t>(tile) * groups * 2048u + lane * 32u
                             : static_cast<uint32_t>(tile) * groups * 512u + lane * 8u)
                     : c_bytes;
        s_vo[j] = ok ? static_cast<uint32_t>(tile) * groups * 64u + r16 * 4u : s_bytes;
    }

    v2i c_ring[NSTAGE][TN];
    uint32_t s_ring[NSTAGE][TN];
    v4i w_ring[NSTAGE][TN][2];
    auto issue = [&](int g, int slot) {
#pragma unroll
        for (int u = 0; u < A_PER_W; ++u) {
            const int I = wave * A_PER_W + u;
            buffer_load_lds16(rx, &lds_a[slot][8 * I][0], x_vo[u], g * 128);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            if constexpr (F16W) {
                w_ring[slot][j][0] = __builtin_amdgcn_raw_buffer_load_b128(rc, c_vo[j], g * 2048, 0);
                w_ring[slot][j][1] = __builtin_amdgcn_raw_buffer_load_b128(rc, c_vo[j] + 16u, g * 2048, 0);
            } else {
                c_ring[slot][j] = __builtin_amdgcn_raw_buffer_load_b64(rc, c_vo[j], g * 512, 0);
                s_ring[slot][j] = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rs, s_vo[j], g * 64, 0));
            }
        }
    };

    v4f acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[j][i] = v4f{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int slot) {
        if constexpr (F16W)
            w4a16_group_mfma_f16w<TM, TN>(&lds_a[slot][0][0], w_ring[slot], r16, q, acc);
        else
            w4a16_group_mfma<TM, TN>(&lds_a[slot][0][0], c_ring[slot], s_ring[slot], r16, q, acc);
    };

    // Prologue: groups 0 .. NSTAGE-2 in flight.  Loads are issued
    // unconditionally, also past the last group: those read harmless bytes
    // (the next tile or row, or zeros past the end) into slots that are never
    // consumed, and keep the number of loads in flight per group constant.
#pragma unroll
    for (int p = 0; p < NSTAGE - 1; ++p) issue(g_lo + p, p);

    // Main loop, unrolled by the ring length so ring indices are constants.
    for (int g0 = 0; g0 < g_cnt; g0 += NSTAGE) {
#pragma unroll
        for (int u = 0; u < NSTAGE; ++u) {
            const int g = g0 + u;
            // Group g's loads are complete once at most the (NSTAGE - 2)
            // later groups' loads remain in flight.
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NSTAGE - 2) * LOADS_PER_GROUP) : "memory");
            __syncthreads();
            issue(g_lo + g + NSTAGE - 1, (u + NSTAGE - 1) % NSTAGE);
            if (g < g_cnt) compute(u);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // A K split writes its raw fp32 partial tile to slice blockIdx.y of the
    // workspace (the host passes y = workspace, fp32, no epilogue, plain
    // [m, n] map); w4a16_splitk_reduce adds the slices.
    if (gridDim.y > 1) y = reinterpret_cast<float *>(y) + static_cast<size_t>(blockIdx.y) * m * n;

    // acc[j][i][r] = y[row, col]: row = m-tile i, lane r16; col = this wave's
    // n-tile j, 4q + r.
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col0 = block_col + (wave * TN + j) * 16;  // wave-uniform
        const int col = col0 + 4 * q;
        if (col >= n) continue;
        const int fold = col0 >= out.n_out ? out.n_out : 0;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int row = block_row + 16 * i + r16;
            if (row >= m) continue;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = epilogue(acc[j][i][r], bias, col + r, epi);
            const size_t idx = out_index(out.row_base + row, col - fold, col0 - fold, out.m_out, out.n_out, n_part);
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

// The K-split reduction: y = epilogue(sum over s = 0 .. splits - 1, in that
// order, of ws[s][row][col]) written through the output map.  Four
// consecutive outputs per thread.
__global__ __launch_bounds__(256) void w4a16_splitk_reduce_kernel(const float *__restrict__ ws, int splits,
                                                                   const float *__restrict__ bias,
                                                                   void *__restrict__ y, int out_type, int epi, int m,
                                                                   int n, int n_part, OutMap out) {
    const long long t = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int n4 = n >> 2;
    if (t >= static_cast<long long>(m) * n4) return;
    const int row = static_cast<int>(t / n4), col = static_cast<int>(t % n4) * 4;
    const size_t plane = static_cast<size_t>(m) * n;
    const float4 *p = reinterpret_cast<const float4 *>(ws + static_cast<size_t>(row) * n + col);
    float4 a = p[0];
    for (int s = 1; s < splits; ++s) {
        const float4 b = p[s * (plane / 4)];
        a.x += b.x;
        a.y += b.y;
        a.z += b.z;
        a.w += b.w;
    }
    float v[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = epilogue(v[r], bias, col + r, epi);
    // The parts layout (n_part divides n and is a multiple of 16, so the
    // four outputs lie in one part).
    const int part = col / n_part;
    const size_t idx = static_cast<size_t>(part) * out.m_out * n_part +
                       static_cast<size_t>(out.row_base + row) * n_part + (col - part * n_part);
    if (out_type == QI_HIP_OUT_F16) {
        uint2 h;
        h.x = static_cast<uint32_t>(f2h(v[0])) | (static_cast<uint32_t>(f2h(v[1])) << 16);
        h.y = static_cast<uint32_t>(f2h(v[2])) | (static_cast<uint32_t>(f2h(v[3])) << 16);
        *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(y) + idx) = h;
    } else {
        *reinterpret_cast<float4 *>(reinterpret_cast<float *>(y) + idx) = float4{v[0], v[1], v[2], v[3]};
    }
}

static int launch_splitk_reduce(const float *ws, int splits, const float *bias, void *y, int out_type, int epi,
                                int m, int n, int n_part, OutMap out, hipStream_t stream) {
    const long long threads = static_cast<long long>(m) * (n / 4);
    const long long blocks = (threads + 255) / 256;
    if (blocks > 0x7FFFFFFFLL) return kInvalid;
    w4a16_splitk_reduce_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream>>>(
        ws, splits, bias, y, out_type, epi, m, n, n_part, out);
    return launch_status();
}

// Pre-pass of the fp16-weight path: the tiled codes of n rows dequantised
// once into the MFMA fragments the tiled kernel reads
// ([n / 16][groups][64 lanes][2 steps][8] fp16), with the reference's values
// (packed fp16 where the single rounding is provably the reference's double
// one, its fp32 fma + RNE otherwise).  One thread per 16-byte fragment half
// (lane, step) of a tile group, so both the 4-byte code reads and the
// 16-byte stores of consecutive threads are contiguous.
__global__ __launch_bounds__(256) void w4a16_expand_kernel(const uint8_t *__restrict__ codes,
                                                           const uint16_t *__restrict__ scales,
                                                           uint4 *__restrict__ out, long long halves) {
    const long long t = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= halves) return;
    const long long tg = t >> 7;  // tile * groups + group
    const int lane = static_cast<int>((t >> 1) & 63), step = static_cast<int>(t & 1);
    const uint32_t c = *reinterpret_cast<const uint32_t *>(codes + tg * 512 + lane * 8 + step * 4);
    const uint32_t sm = *reinterpret_cast<const uint32_t *>(scales + tg * 32 + (lane & 15) * 2);
    const uint32_t sb = sm & 0xFFFFu, mb = sm >> 16;
    out[t] = w4a16_dequant8(c, sb, mb, w4a16_single_rounding_exact(sb, mb));
}

static int launch_expand(const void *codes, const void *scales, void *out, int n, int k, hipStream_t stream) {
    const long long halves = static_cast<long long>(n / 16) * (k / 64) * 128;
    const long long blocks = (halves + 255) / 256;
    if (blocks > 0x7FFFFFFFLL) return kInvalid;
    w4a16_expand_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream>>>(
        static_cast<const uint8_t *>(codes), static_cast<const uint16_t *>(scales), static_cast<uint4 *>(out), halves);
    return launch_status();
}

template <int TM, int TN, int NW, int NSTAGE = 4, bool F16W = false>
static int launch_tiled(const void *x, const void *codes, const void *scales, const float *bias, void *y,
                        int out_type, int epi, int m, int n, int k, int n_part, OutMap out, int m_split,
                        hipStream_t stream, int splits = 1, float *ws = nullptr) {
    constexpr int BM = TM * 16, BN = NW * TN * 16;
    // One grid (m_split = 0), or the two streams' diagonal blocks (m_split
    // and out.n_out multiples of BM and BN, checked by the caller).
    TileGrid2 gd;
    if (m_split > 0)
        gd = TileGrid2{(m_split / BM) * (out.n_out / BN), m_split / BM, out.n_out / BN, (m - m_split + BM - 1) / BM,
                       (n - out.n_out + BN - 1) / BN};
    else
        gd = TileGrid2{((m + BM - 1) / BM) * ((n + BN - 1) / BN), (m + BM - 1) / BM, (n + BN - 1) / BN, 0, 0};
    const long long blocks = static_cast<long long>(gd.t0) + static_cast<long long>(gd.tm1) * gd.tn1;
    if (blocks > 0x7FFFFFFFLL) return kInvalid;
    if (splits > 1) {
        // Partials into the workspace, then one reduction with the epilogue.
        w4a16_tiled_kernel<TM, TN, NW, NSTAGE, F16W>
            <<<dim3(static_cast<unsigned>(blocks), static_cast<unsigned>(splits)), dim3(NW * WAVE), 0, stream>>>(
                static_cast<const uint16_t *>(x), static_cast<const uint8_t *>(codes),
                static_cast<const uint16_t *>(scales), nullptr, ws, QI_HIP_OUT_F32, QI_HIP_EPILOGUE_NONE, m, n, k, n,
                OutMap{0, m, n}, gd);
        if (const int st = launch_status()) return st;
        return launch_splitk_reduce(ws, splits, bias, y, out_type, epi, m, n, n_part, out, stream);
    }
    w4a16_tiled_kernel<TM, TN, NW, NSTAGE, F16W><<<dim3(static_cast<unsigned>(blocks)), dim3(NW * WAVE), 0, stream>>>(
        static_cast<const uint16_t *>(x), static_cast<const uint8_t *>(codes), static_cast<const uint16_t *>(scales),
        bias, y, out_type, epi, m, n, k, n_part, out, gd);
    return launch_status();
}

// ---------------------------------------------------------------------------
// K-split kernel for short M (the text stream's 256 rows).
//
// With few rows the grid is small and a tile's 64-groups run one after
// another, so the tiled kernel is latency-bound.  Here the four wavefronts of
// a workgroup share one BM x BN output tile and each streams a contiguous
// quarter of the groups through its own LDS ring (no barrier in the loop);
// the four partial tiles are then added in a fixed order (wave 0 + 1 + 2 + 3)
// through LDS, so results do not depend on timing.  Summation order differs
// from the tiled kernel's by the K split only, inside the W4A16 tolerance.
template <int TM, int TN>
__global__ __launch_bounds__(4 * WAVE) void w4a16_splitk_kernel(
    const uint16_t *__restrict__ x, const uint8_t *__restrict__ codes, const uint16_t *__restrict__ scales,
    const float *__restrict__ bias, void *__restrict__ y, int out_type, int epi, int m, int n, int k, int n_part,
    OutMap out) {
    constexpr int NW = 4, NSTAGE = 4;
    constexpr int BM = TM * 16, BN = TN * 16;
    constexpr int A_PER_W = BM / 8;  // 1 KiB direct loads: rows 8u .. 8u+7
    constexpr int LOADS_PER_GROUP = A_PER_W + 2 * TN;
    constexpr int RING = NSTAGE * BM * 128;  // bytes per wave
    static_assert(BM * BN * 4 <= RING, "a wave's partial tile fits in its ring");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[NW * RING];

    const int groups = k >> 6;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const int q = lane >> 4, r16 = lane & 15;
    const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN;
    int tm, tn;
    tile_of_block(blockIdx.x, tiles_m, tiles_n, 8, tm, tn);
    const int block_row = tm * BM, block_col = tn * BN;
    const int g_lo = wave * groups / NW, cnt = (wave + 1) * groups / NW - g_lo;
    uint8_t *ring = lds + wave * RING;

    const uint32_t x_bytes = static_cast<uint32_t>(m) * static_cast<uint32_t>(k) * 2u;
    const uint32_t c_bytes = static_cast<uint32_t>(n) * static_cast<uint32_t>(k / 2);
    const uint32_t s_bytes = static_cast<uint32_t>(n) * static_cast<uint32_t>(groups) * 4u;
    const auto rx = buffer_rsrc(x, x_bytes);
    const auto rc = buffer_rsrc(codes, c_bytes);
    const auto rs = buffer_rsrc(scales, s_bytes);
    uint32_t x_vo[A_PER_W];
#pragma unroll
    for (int u = 0; u < A_PER_W; ++u) {
        const int row = 8 * u + (lane >> 3), grow = block_row + row;
        const int chunk = (lane & 7) ^ (row & 7);
        x_vo[u] = grow < m ? static_cast<uint32_t>(grow) * k * 2u + (g_lo * 128u) + chunk * 16u : x_bytes;
    }
    uint32_t c_vo[TN], s_vo[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int tile = block_col / 16 + j;
        const bool ok = tile < n / 16;
        c_vo[j] = ok ? (static_cast<uint32_t>(tile) * groups + g_lo) * 512u + lane * 8u : c_bytes;
        s_vo[j] = ok ? (static_cast<uint32_t>(tile) * groups + g_lo) * 64u + r16 * 4u : s_bytes;
    }

    v2i c_ring[NSTAGE][TN];
    uint32_t s_ring[NSTAGE][TN];
    // Group g_lo + gi into ring slot `slot`.  Past this wave's range the loads
    // read harmless bytes (the next groups, tile or row, or zeros past the
    // end) into slots that are never consumed.
    auto issue = [&](int gi, int slot) {
#pragma unroll
        for (int u = 0; u < A_PER_W; ++u) buffer_load_lds16(rx, ring + (slot * BM + 8 * u) * 128, x_vo[u], gi * 128);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            c_ring[slot][j] = __builtin_amdgcn_raw_buffer_load_b64(rc, c_vo[j], gi * 512, 0);
            s_ring[slot][j] = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rs, s_vo[j], gi * 64, 0));
        }
    };

    v4f acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[j][i] = v4f{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int p = 0; p < NSTAGE - 1; ++p) issue(p, p);
    for (int g0 = 0; g0 < cnt; g0 += NSTAGE) {
#pragma unroll
        for (int u = 0; u < NSTAGE; ++u) {
            const int gi = g0 + u;
            // Only this wave reads its ring, so completing its own loads is
            // enough: no workgroup barrier.  The slot refilled next was last
            // read by this wave's previous group, whose reads have completed
            // (their values fed that group's MFMAs).
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NSTAGE - 2) * LOADS_PER_GROUP) : "memory");
            issue(gi + NSTAGE - 1, (u + NSTAGE - 1) % NSTAGE);
            if (gi < cnt) w4a16_group_mfma<TM, TN>(ring + u * BM * 128, c_ring[u], s_ring[u], r16, q, acc);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // Partial tiles through LDS, each wave into its own ring, then summed in
    // wave order: position ((j * TM + i) * 64 + lane) holds acc[j][i].
    __syncthreads();
    float4 *part = reinterpret_cast<float4 *>(ring);
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i)
            part[(j * TM + i) * WAVE + lane] = float4{acc[j][i][0], acc[j][i][1], acc[j][i][2], acc[j][i][3]};
    __syncthreads();
    for (int pos = threadIdx.x; pos < TN * TM * WAVE; pos += NW * WAVE) {
        float4 v = reinterpret_cast<const float4 *>(lds)[pos];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            const float4 t = reinterpret_cast<const float4 *>(lds + w * RING)[pos];
            v.x += t.x;
            v.y += t.y;
            v.z += t.z;
            v.w += t.w;
        }
        // acc[j][i][r] = y[row, col]: row = m-tile i, lane % 16; col = n-tile
        // j, 4 (lane / 16) + r.
        const int ln = pos % WAVE, ji = pos / WAVE, i = ji % TM, j = ji / TM;
        const int col0 = block_col + 16 * j;  // wave-uniform: pos / WAVE is
        const int row = block_row + 16 * i + (ln & 15), col = col0 + 4 * (ln >> 4);
        if (row >= m || col >= n) continue;
        const float vv[4] = {epilogue(v.x, bias, col, epi), epilogue(v.y, bias, col + 1, epi),
                             epilogue(v.z, bias, col + 2, epi), epilogue(v.w, bias, col + 3, epi)};
        const size_t idx = out_index(out.row_base + row, col, col0, out.m_out, out.n_out, n_part);
        if (out_type == QI_HIP_OUT_F16) {
            uint2 h;
            h.x = static_cast<uint32_t>(f2h(vv[0])) | (static_cast<uint32_t>(f2h(vv[1])) << 16);
            h.y = static_cast<uint32_t>(f2h(vv[2])) | (static_cast<uint32_t>(f2h(vv[3])) << 16);
            *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(y) + idx) = h;
        } else {
            *reinterpret_cast<float4 *>(reinterpret_cast<float *>(y) + idx) = float4{vv[0], vv[1], vv[2], vv[3]};
        }
    }
}

template <int TM, int TN>
static int launch_splitk(const void *x, const void *codes, const void *scales, const float *bias, void *y,
                         int out_type, int epi, int m, int n, int k, int n_part, OutMap out, hipStream_t stream) {
    constexpr int BM = TM * 16, BN = TN * 16;
    const long long blocks = static_cast<long long>((m + BM - 1) / BM) * ((n + BN - 1) / BN);
    if (blocks > 0x7FFFFFFFLL) return kInvalid;
    w4a16_splitk_kernel<TM, TN><<<dim3(static_cast<unsigned>(blocks)), dim3(4 * WAVE), 0, stream>>>(
        static_cast<const uint16_t *>(x), static_cast<const uint8_t *>(codes), static_cast<const uint16_t *>(scales),
        bias, y, out_type, epi, m, n, k, n_part, out);
    return launch_status();
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
                           const float *bias, void *y, int out_type, int epilogue, int m, int n, int k, int n_part,
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

namespace qi {

// Rows from which a call with a workspace runs on fp16 weights.
constexpr int W4A16_F16W_MIN_M = 2048;

// Kernel shape for m > 16 rows and n_out outputs per stream (measured on
// MI355X): 1 K-split 64 x 64, 3 tiled 64 x 64, 4 tiled 128 x 192, 5 tiled
// 256 x 256, 6 tiled 128 x 128 (2, tiled 32 x 64, is no longer chosen).
static int select_w4a16_tiles(int m, int n_out) {
    // Short M with few 64 x 64 tiles (the text stream's 256 x 3072 outputs):
    // the tiled grid is too small to fill the chip, so split K across the
    // workgroup's waves instead; with more tiles the 64 x 64 tiled kernel
    // (measured on MI355X, us, K-split / 32 x 64 / 64 x 64 tiles:
    // 256 x 3072 x 3072 16.0 / 18.7 / 19.3, 256 x 3072 x 12288 47.0 / 62.7 /
    // 68.4, 64 x 12288 x 3072 16.9 / 20.2 / 20.3, 128 x 9216 x 3072 30.7 /
    // 24.2 / 22.0, 256 x 9216 x 3072 47.0 / 35.8 / 30.6, 256 x 12288 x 3072
    // 45.6 / 40.0 / 31.9).
    const long long tiles64 = static_cast<long long>((m + 63) / 64) * ((n_out + 63) / 64);
    // Short M with very many 64 x 64 tiles (an encoder's 300 prompt rows
    // through a 37888-wide gate + up): 64 x 128 tiles, each activation
    // fragment read for two weight tiles (300 x 37888 x 3584: 126 -> 114 us;
    // at 768 - 1536 tiles 64 x 64 stays faster, e.g. 256 x 9216 x 3072 30.4
    // against 37.3).
    if (m <= 512 && tiles64 >= 2048 && n_out % 128 == 0) return 7;
    if (m <= 256) return tiles64 < 256 ? 1 : 3;
    // 128 x 192 tiles once they make three quarters of a round of
    // workgroups (two per CU) or more, else 64 x 64 tiles (measured:
    // 1024 x 12288 x 3072 123.5 -> 94.8 us with 512 large tiles; 1536 x 3072
    // x 3072 with 192 large tiles 74.7 us against 54.5 for small ones).
    if (!(n_out % 192 == 0 && static_cast<long long>((m + 127) / 128) * (n_out / 192) >= 384) &&
        (m <= 1024 || n_out % 192 == 0))
        return 3;
    // 256 x 256 tiles (eight waves, one workgroup per CU: each weight is
    // dequantised for twice the rows) when they still give three or more
    // workgroups per CU; measured 11 % faster at 4096 x 12288 x 3072.
    if (n_out % 256 == 0 && static_cast<long long>((m + 255) / 256) * (n_out / 256) >= 768) return 5;
    if (n_out % 192 == 0) return 4;
    return 6;
}

// K split over workgroups for a single-stream launch of m rows and n_out
// outputs (1 = none).  Few 64 x 64 tiles leave most CUs with one wave per
// SIMD walking all of K, which is latency-bound; splitting K into s slices
// (their fp32 partials added by a second, small kernel in slice order)
// multiplies the workgroups.  s brings the workgroups to about three per CU
// with at least 16 groups per slice; where the in-workgroup K split (tile
// choice 1) runs, only for long K (>= 96 groups), where it measured slower.
// Measured on MI355X (us, unsplit -> split): 300 x 1024 x 3584 23.5 ->
// 14.8 (s = 3), 300 x 3584 x 3584 28.7 -> 26.3 (3), 300 x 3584 x 18944
// 109 -> 78 (3), 512 x 3072 x 12288 75.5 -> 64.6 (2), 512 x 1024 x 3072
// 20.9 -> 15.7 (3), 256 x 3072 x 12288 51.9 -> 37.5 (4), 64 x 3072 x 12288
// 48.6 -> 20.7 (12); 256 x 3072 x 3072 stays on choice 1 (18.5 against 21.0
// split).
static int select_w4a16_splits(int m, int n_out, int k) {
    const int cfg = select_w4a16_tiles(m, n_out);
    if (cfg != 1 && cfg != 3) return 1;
    const long long tiles = static_cast<long long>((m + 63) / 64) * ((n_out + 63) / 64);
    const int groups = k / 64;
    if (tiles >= 512 || (cfg == 1 && groups < 96)) return 1;
    const long long want = (3LL * device_cus() + tiles - 1) / tiles;
    const int s = static_cast<int>(want < groups / 16 ? want : groups / 16);
    return s > 1 ? s : 1;
}

// Short M with a long K (an encoder's MLP down, 300 x 3584 x 18944; the text
// stream's MLP down, 256 x 3072 x 12288): tall tiles -- 128 rows for 161 to
// 256 rows, 160 for 257 to 320, 64 columns -- so each weight is dequantised
// for more rows, with K split into as many slices as keep the launch within
// two workgroups per CU.  Measured on MI355X (us, 64 x 64 split -> tall):
// 300 x 3584 x 18944 74.7 -> 58.9 (4 slices; 5 slices, one workgroup past a
// round, 80.7), 320 x 3072 x 12288 43.5 -> 39.2, 256 x 3072 x 12288 34.4 ->
// 32.6, 200 x 3072 x 12288 32.8 -> 30.5; slower below 128 groups (256 x 3072
// x 3072 16.0 -> 19.6) and at 160 rows or fewer (no gain).  From 257 rows
// (where 64-row tiles leave a partial fifth tile) down to 48 groups while
// the launch keeps 1.5 workgroups per CU: 300 x 4608 x 3584 (an encoder's
// fused q, k, v) 29.4 -> 25.5 (432 workgroups); 300 x 3584 x 3584 (336)
// 24.1 either way, 320 x 3072 x 3072 (288) 20.6 -> 22.6 and 300 x 1024 x
// 3584 (96) 14.5 -> 17.9, so those keep the 64 x 64 split.  Returns the
// slices (0: not used) and the tile's 16-row blocks in tm.
static int select_w4a16_tall(int m, int n_out, int k, int &tm) {
    const int groups = k / 64;
    tm = m > 256 ? 10 : 8;
    if (m <= 160 || m > 320 || groups < 48) return 0;
    const long long tiles = static_cast<long long>((m + 16 * tm - 1) / (16 * tm)) * ((n_out + 63) / 64);
    const long long s = 2LL * device_cus() / tiles;
    if (s < 2) return 0;
    const int st = static_cast<int>(s < groups / 16 ? s : groups / 16);
    if (groups < 128 && (m <= 256 || tiles * st * 2 < 3LL * device_cus())) return 0;
    return st;
}

static size_t splitk_bytes(int m, int n_out, int k) {
    int tm;
    if (const int st = select_w4a16_tall(m, n_out, k, tm)) return static_cast<size_t>(st) * m * n_out * 4;
    const int s = select_w4a16_splits(m, n_out, k);
    return s > 1 ? static_cast<size_t>(s) * m * n_out * 4 : 0;
}

static const int kTileRows[] = {0, 64, 32, 64, 128, 256, 128, 64}, kTileCols[] = {0, 64, 64, 64, 192, 256, 128, 128};

// One launch over both streams (m_split > 0) only when its tiles fit both
// blocks and it takes no more rounds of workgroups than stream 0 alone
// (these kernels are not persistent: stream 1's tiles would otherwise run
// as an extra, mostly idle round).
static bool w4a16_one_launch(int cfg, int m, int m_split, int n_out) {
    const int bm = kTileRows[cfg], bn = kTileCols[cfg];
    if (m_split <= 0 || cfg == 1 || m_split % bm || n_out % bn) return false;
    const long long slots = static_cast<long long>(device_cus()) * (cfg == 5 ? 1 : 2);
    const long long t0 = static_cast<long long>(m_split / bm) * (n_out / bn);
    const long long t1 = static_cast<long long>((m - m_split + bm - 1) / bm) * (n_out / bn);
    return (t0 + t1 + slots - 1) / slots == (t0 + slots - 1) / slots;
}

// The fp16-weight path: with many rows every weight would be dequantised
// once per row tile (m / 128 or m / 256 times), so the weights are
// dequantised once into the workspace (n k fp16) and the tiled kernel reads
// fp16 fragments instead of codes.
static bool w4a16_use_f16w(int cfg, int m, int rows, int k) {
    return (cfg == 4 || cfg == 5 || cfg == 6) && m >= W4A16_F16W_MIN_M &&
           static_cast<long long>(rows) * k * 2 < (1LL << 32);
}

// Workspace a call needs for its K splits or its fp16 weights (0: none).  A
// dual call split into two launches runs them in stream order, so they
// share it.
static size_t w4a16_workspace(int m, int m_split, int n_out, int k) {
    const int cfg = select_w4a16_tiles(m, n_out);
    if (m_split <= 0)
        return w4a16_use_f16w(cfg, m, n_out, k) ? static_cast<size_t>(n_out) * k * 2 : splitk_bytes(m, n_out, k);
    if (w4a16_one_launch(cfg, m, m_split, n_out))
        return w4a16_use_f16w(cfg, m, 2 * n_out, k) ? static_cast<size_t>(2 * n_out) * k * 2 : 0;
    const size_t a = w4a16_workspace(m_split, 0, n_out, k), b = w4a16_workspace(m - m_split, 0, n_out, k);
    return a > b ? a : b;
}

// Kernel shape for m rows and n_out outputs per stream (measured on
// MI355X), and its launch.  m_split = 0: one stream (n = n_out).  m_split >
// 0: the two streams' diagonal blocks over the stacked rows (n = 2 n_out
// weight rows) in one launch when the chosen tiles fit both blocks, else
// one launch per stream.  ws (ws_bytes) is the caller's workspace for K
// splits, or null: without it no launch splits K.  Arguments are checked by
// the callers; m > 16 per stream.
static int dispatch_w4a16(const void *x, const void *codes, const void *scales, const float *bias, void *y,
                          int out_type, int epi, int m, int n, int k, int n_part, OutMap out, int m_split,
                          hipStream_t s, float *ws, size_t ws_bytes) {
    const int n_out = out.n_out;
    const int cfg = select_w4a16_tiles(m, n_out);
    if (m_split > 0 && !w4a16_one_launch(cfg, m, m_split, n_out)) {
        // One launch per stream, each writing its rows of the stacked y.
        const size_t g = static_cast<size_t>(k / 64);
        int st = dispatch_w4a16(x, codes, scales, bias, y, out_type, epi, m_split, n_out, k, n_part,
                                OutMap{out.row_base, out.m_out, n_out}, 0, s, ws, ws_bytes);
        if (st) return st;
        return dispatch_w4a16(static_cast<const uint16_t *>(x) + static_cast<size_t>(m_split) * k,
                              static_cast<const uint8_t *>(codes) + static_cast<size_t>(n_out / 16) * g * 512,
                              static_cast<const uint8_t *>(scales) + static_cast<size_t>(n_out / 16) * g * 64,
                              bias ? bias + n_out : nullptr, y, out_type, epi, m - m_split, n_out, k, n_part,
                              OutMap{out.row_base + m_split, out.m_out, n_out}, 0, s, ws, ws_bytes);
    }
    if (m_split == 0 && ws) {
        int tm;
        const int st = select_w4a16_tall(m, n_out, k, tm);
        if (st > 1 && static_cast<size_t>(st) * m * n * 4 <= ws_bytes) {
            if (tm == 8)
                return launch_tiled<8, 1, 4>(x, codes, scales, bias, y, out_type, epi, m, n, k, n_part, out, 0, s, st,
                                             ws);
            return launch_tiled<10, 1, 4>(x, codes, scales, bias, y, out_type, epi, m, n, k, n_part, out, 0, s, st,
                                          ws);
        }
        const int splits = select_w4a16_splits(m, n_out, k);
        if (splits > 1 && static_cast<size_t>(splits) * m * n * 4 <= ws_bytes)
            return launch_tiled<4, 1, 4>(x, codes, scales, bias, y, out_type, epi, m, n, k, n_part, out, 0, s,
                                         splits, ws);
    }
    if (ws && w4a16_use_f16w(cfg, m, n, k) && static_cast<size_t>(n) * k * 2 <= ws_bytes) {
        if (const int st = launch_expand(codes, scales, ws, n, k, s)) return st;
        switch (cfg) {
        case 4:
            return launch_tiled<8, 3, 4, 4, true>(x, ws, nullptr, bias, y, out_type, epi, m, n, k, n_part, out,
                                                  m_split, s);
        case 5:
            return launch_tiled<16, 2, 8, 4, true>(x, ws, nullptr, bias, y, out_type, epi, m, n, k, n_part, out,
                                                   m_split, s);
        default:
            return launch_tiled<8, 2, 4, 4, true>(x, ws, nullptr, bias, y, out_type, epi, m, n, k, n_part, out,
                                                  m_split, s);
        }
    }
    switch (cfg) {
    case 1:
        return launch_splitk<4, 4>(x, codes, scales, bias, y, out_type, epi, m, n, k, n_part, out, s);
    case 3:
        return launch_tiled<4, 1, 4>(x, codes, scales, bias, y, out_type, epi, m, n, k, n_part, out, m_split, s);
    case 4:
        return launch_tiled<8, 3, 4>(x, codes, scales, bias, y, out_type, epi, m, n, k, n_part, out, m_split, s);
    case 5:
        return launch_tiled<16, 2, 8>(x, codes, scales, bias, y, out_type, epi, m, n, k, n_part, out, m_split, s);
    case 7:
        return launch_tiled<4, 2, 4>(x, codes, scales, bias, y, out_type, epi, m, n, k, n_part, out, m_split, s);
    default:
        return launch_tiled<8, 2, 4>(x, codes, scales, bias, y, out_type, epi, m, n, k, n_part, out, m_split, s);
    }
}

static int check_w4a16_args(const void *x_half, const void *w_tiled_codes, const void *w_tiled_scales, const void *y,
                            int out_type, int epilogue, int m, int n, int k, int n_part) {
    if (m <= 0 || n <= 0 || k <= 0 || n % 16 || k % 64) return kInvalid;
    if (n_part <= 0 || n_part % 16 || n % n_part) return kInvalid;
    if (!x_half || !w_tiled_codes || !w_tiled_scales || !y) return kInvalid;
    if (out_type != QI_HIP_OUT_F32 && out_type != QI_HIP_OUT_F16) return kInvalid;
    if (epilogue != QI_HIP_EPILOGUE_NONE && epilogue != QI_HIP_EPILOGUE_GELU_TANH) return kInvalid;
    if (reinterpret_cast<uintptr_t>(x_half) % 16 || reinterpret_cast<uintptr_t>(w_tiled_codes) % 8 ||
        reinterpret_cast<uintptr_t>(w_tiled_scales) % 4 || k % 8)
        return kInvalid;
    return 0;
}

}  // namespace qi

namespace qi {

// Every tiled W4A16 entry: m_split = 0 one stream of n outputs, else the two
// streams of a dual call (n outputs each, 2n weight rows).
static int w4a16_entry(const void *x_half, const void *w_tiled_codes, const void *w_tiled_scales, const float *bias,
                       void *y, int out_type, int epilogue, int m, int m_split, int n, int k, int n_part,
                       void *workspace, long long workspace_bytes, void *stream) {
    if (const int st = check_w4a16_args(x_half, w_tiled_codes, w_tiled_scales, y, out_type, epilogue, m, n, k, n_part))
        return st;
    if (workspace_bytes < 0 || (workspace_bytes > 0 && (!workspace || reinterpret_cast<uintptr_t>(workspace) % 16)))
        return kInvalid;
    const int rows = m_split > 0 ? 2 * n : n;
    if (static_cast<long long>(m) * k * 2 >= (1LL << 32) || static_cast<long long>(rows) * (k / 2) >= (1LL << 32))
        return kInvalid;
    if (m_split > 0) {
        if (m_split <= 16 || m - m_split <= 16) return kInvalid;
    } else if (m <= 16) {
        // The GEMV writes the parts layout itself: one launch over all parts
        // (e.g. every block's modulation linears, which share their input).
        return qi_hip_w4a16_gemv_impl(x_half, w_tiled_codes, w_tiled_scales, bias, y, out_type, epilogue, m, n, k,
                                      n_part, stream_of(stream));
    }
    return dispatch_w4a16(x_half, w_tiled_codes, w_tiled_scales, bias, y, out_type, epilogue, m, rows, k, n_part,
                          OutMap{0, m, n}, m_split, stream_of(stream), static_cast<float *>(workspace),
                          static_cast<size_t>(workspace_bytes));
}

}  // namespace qi

QI_API int qi_hip_w4a16_gemm_tiled_parts(const void *x_half, const void *w_tiled_codes, const void *w_tiled_scales,
                                         const float *bias, void *y, int out_type, int epilogue, int m, int n, int k,
                                         int n_part, void *stream) {
    return w4a16_entry(x_half, w_tiled_codes, w_tiled_scales, bias, y, out_type, epilogue, m, 0, n, k, n_part,
                       nullptr, 0, stream);
}

QI_API int qi_hip_w4a16_gemm_tiled_dual(const void *x_half, const void *w_tiled_codes, const void *w_tiled_scales,
                                        const float *bias, void *y, int out_type, int epilogue, int m, int m_split,
                                        int n, int k, int n_part, void *stream) {
    if (m_split <= 0) return kInvalid;
    return w4a16_entry(x_half, w_tiled_codes, w_tiled_scales, bias, y, out_type, epilogue, m, m_split, n, k, n_part,
                       nullptr, 0, stream);
}

QI_API int qi_hip_w4a16_gemm_tiled(const void *x_half, const void *w_tiled_codes, const void *w_tiled_scales,
                                   const float *bias, void *y, int out_type, int epilogue, int m, int n, int k,
                                   void *stream) {
    return qi_hip_w4a16_gemm_tiled_parts(x_half, w_tiled_codes, w_tiled_scales, bias, y, out_type, epilogue, m, n, k,
                                         n, stream);
}

QI_API long long qi_hip_w4a16_workspace_bytes(int m, int m_split, int n, int k) {
    if (m <= 16 || n <= 0 || k <= 0 || n % 16 || k % 64 || m_split < 0 || m_split >= m) return 0;
    if (m_split > 0 && (m_split <= 16 || m - m_split <= 16)) return 0;
    return static_cast<long long>(w4a16_workspace(m, m_split, n, k));
}

QI_API int qi_hip_w4a16_gemm_tiled_ws(const void *x_half, const void *w_tiled_codes, const void *w_tiled_scales,
                                      const float *bias, void *y, int out_type, int epilogue, int m, int m_split,
                                      int n, int k, int n_part, void *workspace, long long workspace_bytes,
                                      void *stream) {
    if (m_split < 0) return kInvalid;
    return w4a16_entry(x_half, w_tiled_codes, w_tiled_scales, bias, y, out_type, epilogue, m, m_split, n, k, n_part,
                       workspace, workspace_bytes, stream);
}

QI_API int qi_hip_w4a16_tiles(int m, int n_out) {
    if (m <= 0 || n_out <= 0) return -1;
    return m <= 16 ? 0 : select_w4a16_tiles(m, n_out);
}
