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
// qi_hip_relayout_w4a4_fp6): per 32-row tile T and group g, 1792 bytes = half
// 0 (64 lanes x 16 bytes) then half 1 (64 lanes x 12 bytes); lane l of half h
// holds the E2M3 codes of inputs 32 * (l / 32) + 16h .. + 15 of row
// 32T + l % 32, which is the lane's MFMA operand (6 dwords) split in two.
// Bytes 12..13 of a half-0 lane slot hold the fp16 group scale of row
// 32T + l % 32 (bytes 14..15 are zero), so the scales arrive with the codes.
//
// Roles.  The MFMA A operand is the weight tile (32 outputs n), B the
// activation tile (32 rows m).  Lane l's accumulator register 4a + r then
// holds y[m = l % 32][n = 8a + 4 * (l / 32) + r]: four consecutive outputs,
// stored with one wide write.
//
// Pipeline.  A ring of NSTAGE LDS slots holds the operand blocks of
// upcoming groups, filled NSTAGE groups ahead by buffer_load ... lds (16
// bytes per lane, landing at a 16-byte lane pitch).  One barrier per group.
// The matrix-core work of group g + 1 is interleaved, tile by tile, with the
// fp32 step of group g, so the two units work side by side within a wave.

#include <utility>

#include "qi_common.h"

// Measurement builds only (build.py builds them beside the probe, bench.py
// --ablate-w4a4 times them; their outputs are wrong by design): each
// QI_ABLATE_* macro removes one part of the GEMM's work so that its cost
// shows as the time saved -- QI_ABLATE_DMA the direct-to-LDS operand loads,
// QI_ABLATE_LDS the fragment reads after the first group, QI_ABLATE_BARRIER
// the per-group workgroup barrier, QI_ABLATE_VMWAIT the per-group wait for
// the next group's operand loads, QI_ABLATE_FMA the exact fp32 group steps,
// QI_ABLATE_MFMA the matrix-core work (partials and scale products).  The
// product library defines none of them.

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

using Fp6Out = OutMap;
using Fp6Grid = TileGrid2;

template <int TM, int TN, int WM, int WN, int NSTAGE>
struct Fp6Shape {
    static constexpr int MT = WM * TM, NTL = WN * TN;  // 32-row tiles of the block
    static constexpr int BM = MT * 32, BN = NTL * 32;
    static constexpr int TILE = 2048, SLOT = (MT + NTL) * TILE;
    static constexpr int LDS_BYTES = NSTAGE * SLOT;
};

// The GEMM work of one workgroup: `count` output tiles of BM x BN, the j-th
// starting at 32-row tile coordinates map(j, mt0, nt0).  The LDS ring and
// the software pipeline run on across tile boundaries: the loads of the next
// tile's first groups are in flight while the current tile finishes, and its
// first partial tiles are formed during the current tile's last fp32 step,
// so only the epilogue stores sit between two tiles.
template <int TM, int TN, int WM, int WN, int NSTAGE, bool WHOLE, typename Map>
__device__ __forceinline__ void fp6_tiles(uint8_t *lds, const uint8_t *__restrict__ a6,
                                          const uint8_t *__restrict__ w6, const float *__restrict__ bias,
                                          void *__restrict__ y, int out_type, int epi, int m, int n, int k, int n_part,
                                          Fp6Out out, int count, Map map) {
    using S = Fp6Shape<TM, TN, WM, WN, NSTAGE>;
    constexpr int NW = WM * WN;
    constexpr int MT = S::MT, NTL = S::NTL;
    constexpr int HALVES = 2 * (MT + NTL);  // 1 KiB loads per group
    static_assert(HALVES % NW == 0, "loader mapping");
    constexpr int L_PER_W = HALVES / NW;
    static_assert(TN <= 2, "scale products pair the n-tiles");
    constexpr int LOADS_PER_GROUP = L_PER_W;  // per wave
    constexpr int TILE = S::TILE, SLOT = S::SLOT;
    constexpr uint32_t BLOCK = FP6_BLOCK;  // global bytes per (tile, group)
    static_assert(S::LDS_BYTES <= 160 * 1024, "LDS size");

    const int groups = k >> 6;
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int r32 = lane & 31;
    const int m_tiles = (m + 31) / 32, n_tiles = n / 32;

    const uint32_t a_bytes = static_cast<uint32_t>(m_tiles) * groups * BLOCK;
    const uint32_t w_bytes = static_cast<uint32_t>(n_tiles) * groups * BLOCK;
    const v4i_rsrc ra = raw_rsrc(a6, a_bytes);
    const v4i_rsrc rw = raw_rsrc(w6, w_bytes);

    // This wave's operand loads: half blocks H0 .. H0 + L_PER_W - 1 of the
    // block's (MT + NTL) tiles, activation tiles first, for output tile j.
    // With WHOLE (every tile of every output tile exists: count > 1 is only
    // used so) the lane part of each address is fixed and the tile part is
    // a scalar offset, so a tile switch only changes scalar registers; tiles
    // j >= count repeat the last tile's loads, which are never consumed.
    // Otherwise (one output tile) missing tiles read past the buffer end,
    // which returns zeros.
    const int H0 = wave * L_PER_W;
    uint32_t vo[L_PER_W];
    uint32_t sbase[L_PER_W];
    auto set_tile_loads = [&](int j) {
        if (WHOLE && j >= count) return;
        int mt0 = m_tiles, nt0 = n_tiles;
        if (j < count) map(j, mt0, nt0);
#pragma unroll
        for (int u = 0; u < L_PER_W; ++u) {
            const int H = H0 + u, X = H >> 1, half = H & 1;
            const bool from_a = H < 2 * MT;
            const int t = from_a ? mt0 + X : nt0 + X - MT;
            if constexpr (WHOLE) {
                sbase[u] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(t) * groups * BLOCK);
            } else {
                const bool ok = from_a ? t < m_tiles : t < n_tiles;
                vo[u] = ok ? static_cast<uint32_t>(t) * groups * BLOCK + (half ? 1024u + lane * 12u : lane * 16u)
                           : (from_a ? a_bytes : w_bytes);
                sbase[u] = 0;
            }
        }
    };
    if constexpr (WHOLE) {
#pragma unroll
        for (int u = 0; u < L_PER_W; ++u) vo[u] = ((H0 + u) & 1) ? 1024u + lane * 12u : lane * 16u;
    }

    // Every vector-memory load of the loop is a direct-to-LDS load whose
    // completion this code counts itself, and every one moves 16 bytes per
    // lane.  In half 1 (12-byte lane stride) a lane's last 4 bytes are the
    // next lane's codes, or bytes past the buffer, which read as zero; they
    // land in the slot's unused fourth dword.
    const uint32_t lds0 = lds_address(lds);
    auto issue_one = [&](int g, int slot, int u) {
#ifdef QI_ABLATE_DMA
        return;
#endif
        const int H = H0 + u;
        dma_dwordx4(H < 2 * MT ? ra : rw, lds0 + slot * SLOT + (H >> 1) * TILE + (H & 1) * 1024, vo[u],
                    sbase[u] + g * BLOCK);
    };
    auto issue = [&](int g, int slot) {
#pragma unroll
        for (int u = 0; u < L_PER_W; ++u) issue_one(g, slot, u);
    };

    v16f acc[TN][TM];
    auto zero_acc = [&]() {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.f;
    };

    // This lane's fragments: weight tile j half h at
    // lds[slot][MT + wn * TN + j][h][16 lane], activation tile i likewise.
    // The fourth dword of a half-0 slot is the scale of row l % 32: sa of
    // activation tile i, and for the weight, output l % 32 of n-tile l / 32
    // (the outer product's block l / 32).
    const uint8_t *w_frag = lds + (MT + wn * TN) * TILE + lane * 16;
    const uint8_t *x_frag = lds + wm * TM * TILE + lane * 16;

#ifdef QI_ABLATE_LDS
    bool first_read = true;
#endif
    struct Frags {  // raw LDS reads; converted where consumed
        v8i wf[TN], xf[TM];
        uint32_t sal[TM], swl;
    };
    auto read_frags = [&](auto slot_c, Frags &F) {
        constexpr int slot = decltype(slot_c)::value;
#ifdef QI_ABLATE_LDS
        if (!first_read) {
#pragma unroll
            for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(F.wf[j]));
#pragma unroll
            for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(F.xf[i]), "+v"(F.sal[i]));
            asm volatile("" : "+v"(F.swl));
            return;
        }
        first_read = false;
#endif
        uint32_t sw[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const v4i lo = *reinterpret_cast<const v4i *>(w_frag + slot * SLOT + j * TILE);
            const v4i hi = *reinterpret_cast<const v4i *>(w_frag + slot * SLOT + j * TILE + 1024);
            F.wf[j] = fp6_operand(lo, hi);
            sw[j] = static_cast<uint32_t>(lo[3]);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const v4i lo = *reinterpret_cast<const v4i *>(x_frag + slot * SLOT + i * TILE);
            const v4i hi = *reinterpret_cast<const v4i *>(x_frag + slot * SLOT + i * TILE + 1024);
            F.xf[i] = fp6_operand(lo, hi);
            F.sal[i] = static_cast<uint32_t>(lo[3]);
        }
        // Lanes 32..63 supply block 1 of the outer product (n-tile 1); with
        // one n-tile that block is unused.
        F.swl = TN == 1 ? sw[0] : (lane < 32 ? sw[0] : sw[TN - 1]);
    };
    // Matrix-core work: the scale outer products and the partial tiles.
    // Block b of the 32x32x1 outer product has rows = outputs of n-tile b
    // (lanes 32b .. 32b+31 supply them) and columns = rows m of tile i; its
    // result registers 16b .. 16b+15 line up with the accumulator registers.
    v32f sp[TM];
    v16f p[TN][TM];
    auto scale_mfma = [&](const Frags &F, int i) {
        v32f z32;
#pragma unroll
        for (int r = 0; r < 32; ++r) z32[r] = 0.f;
        // Issued at raised wave priority, so the matrix core's next
        // instruction wins issue over the other wave's vector work:
        // measured 2-3 % faster on MI355X.  The partial tiles below run at
        // normal priority: with the loads spread over the tile steps,
        // raising it for them too measured 2-3 % slower.
#ifdef QI_ABLATE_MFMA
        asm volatile("" : "+v"(sp[i]));
        return;
#endif
        __builtin_amdgcn_s_setprio(1);
        sp[i] = __builtin_amdgcn_mfma_f32_32x32x1f32(h2f(static_cast<uint16_t>(F.swl)),
                                                     h2f(static_cast<uint16_t>(F.sal[i])), z32, 0, 0, 0);
        __builtin_amdgcn_s_setprio(0);
    };
    auto tile_mfma = [&](const Frags &F, int j, int i) {
        v16f z;
#pragma unroll
        for (int r = 0; r < 16; ++r) z[r] = 0.f;
        // fmt 2 = FP6 E2M3 for both operands; block scales 2^0.
#ifdef QI_ABLATE_MFMA
        asm volatile("" : "+v"(p[j][i]));
        return;
#endif
        p[j][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(F.wf[j], F.xf[i], z, 2, 2, 0, 127, 0, 127);
    };
    // The exact fp32 step of one tile and group, in ascending group order.
    auto tile_fma = [&](int j, int i) {
#ifdef QI_ABLATE_FMA
        asm volatile("" ::"v"(p[j][i]), "v"(sp[i]));
        return;
#endif
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][i][r] = __builtin_fmaf(p[j][i][r], sp[i][16 * j + r], acc[j][i][r]);
    };

    // acc[j][i][4a + r] = y[row, col]: row = m-tile i, lane % 32; col = n-tile
    // j, 8a + 4 * (lane / 32) + r.
    auto store_tile = [&](int jt) {
        int mt0, nt0;
        map(jt, mt0, nt0);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int row = (mt0 + wm * TM + i) * 32 + r32;
            if (row >= m) continue;
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int tile_col = (nt0 + wn * TN + j) * 32;
                if (tile_col >= n) continue;
                const int fold = tile_col >= out.n_out ? out.n_out : 0;  // uniform
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    const int col = tile_col + 8 * a + 4 * (lane >> 5);
                    float v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) v[r] = epilogue(acc[j][i][4 * a + r], bias, col + r, epi);
                    const size_t idx =
                        out_index(out.row_base + row, col - fold, tile_col - fold, out.m_out, out.n_out, n_part);
                    if (out_type == QI_HIP_OUT_F16) {
                        uint2 h;
                        h.x = static_cast<uint32_t>(f2h(v[0])) | (static_cast<uint32_t>(f2h(v[1])) << 16);
                        h.y = static_cast<uint32_t>(f2h(v[2])) | (static_cast<uint32_t>(f2h(v[3])) << 16);
                        *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(y) + idx) = h;
                    } else {
                        *reinterpret_cast<float4 *>(reinterpret_cast<float *>(y) + idx) =
                            float4{v[0], v[1], v[2], v[3]};
                    }
                }
            }
        }
    };

    // Software pipeline.  The matrix-core work of group g + 1 runs during
    // the fp32 step of group g, interleaved tile by tile: the fp32 step of
    // tile (j, i) frees p[j][i], whose next partial tile is issued at once and
    // computes while the vector unit steps the next tile; sp[i] is refilled
    // once both n-tiles of row tile i have used it.  So the fragments are
    // needed one group ahead only.  Groups are numbered along the whole
    // sequence (tile j's group g is j * groups + g).  Per group (slots are
    // the group's number mod NSTAGE):
    //   wait until this wave's loads of the next group are done, barrier
    //   (then every wave's are, and every wave has consumed its reads of
    //   this group's slot);
    //   issue the loads of the group NSTAGE ahead into this slot;
    //   read the fragments of the next group;
    //   fp32 step of this group interleaved with the next one's matrix-core
    //   work.
    // Loads past the last group read zeros into slots that are never
    // consumed, keeping the loads per group constant; the last step's
    // matrix-core work is likewise discarded.
    static_assert(NSTAGE % 4 == 0, "whole quarters of the ring per group count (groups % 4 == 0)");
    static_assert(NSTAGE >= 2 && (NSTAGE - 1) * LOADS_PER_GROUP <= 63, "vmcnt range");
    // Several tiles (WHOLE) use a 4-deep ring, so that tiles end on ring
    // boundaries; otherwise count == 1.
    Frags F;
    // One step of the ring: the fp32 step of the group in slot u, the loads
    // of group `gload` (of the tile set_tile_loads chose) into slot u, and
    // the next group's matrix-core work -- except in the last step of a tile
    // (LAST), which leaves that work until the tile is stored, so that the
    // partials are not live across the epilogue.
    auto group_step = [&](auto uc, int gload, auto last_c) {
        constexpr int u = decltype(uc)::value;
        constexpr bool LAST = decltype(last_c)::value;
        // Scheduling fences pin the order; without them the compiler
        // gathers the matrix-core work into one block.  A bare s_barrier:
        // __syncthreads' release fence would also wait for the loads of the
        // groups still in flight.
        __builtin_amdgcn_sched_barrier(0);
#ifdef QI_ABLATE_VMWAIT
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#else
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((NSTAGE - 2) * LOADS_PER_GROUP) : "memory");
#endif
#ifndef QI_ABLATE_BARRIER
        __builtin_amdgcn_s_barrier();
#endif
        asm volatile("" ::: "memory");
        if constexpr (!LAST) read_frags(std::integral_constant<int, (u + 1) % NSTAGE>{}, F);
        __builtin_amdgcn_sched_barrier(0);
        // Tile q = i * TN + j.  Its next partial tile is issued LAG tiles
        // later, so the fragment reads above have the fp32 steps of LAG
        // tiles to land.
        constexpr int T = TM * TN, LAG = T > 2 ? 2 : 0;
        static_for<T + LAG>([&](auto qc) {
            constexpr int q = decltype(qc)::value;
            if constexpr (q < T) {
                constexpr int i = q / TN, j = q % TN;
                // The next group's DMA loads go out one per tile step, ahead
                // of the step's fp32 work, so their issue cost overlaps the
                // MFMA chain instead of stalling it at the group's start;
                // the vmcnt wait per group is unchanged.
                if constexpr (q < L_PER_W) issue_one(gload, u, q);
                if constexpr (q == T - 1) {
#pragma unroll
                    for (int uu = T; uu < L_PER_W; ++uu) issue_one(gload, u, uu);
                }
                __builtin_amdgcn_sched_barrier(0);
                tile_fma(j, i);
                __builtin_amdgcn_sched_barrier(0);
                // sp[i] is free once the last tile of row tile i has
                // stepped.
                if constexpr (j == TN - 1 && !LAST) {
                    scale_mfma(F, i);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            if constexpr (q >= LAG && !LAST) {
                constexpr int d = q - LAG;
                tile_mfma(F, d % TN, d / TN);
                __builtin_amdgcn_sched_barrier(0);
            }
        });
    };

    // The matrix-core work of the group whose fragments F holds.
    auto start_group = [&]() {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            scale_mfma(F, i);
#pragma unroll
            for (int j = 0; j < TN; ++j) tile_mfma(F, j, i);
        }
    };
    using Mid = std::false_type;

    zero_acc();
    set_tile_loads(0);
#pragma unroll
    for (int q = 0; q < NSTAGE; ++q) issue(q, q);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NSTAGE - 1) * LOADS_PER_GROUP) : "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read_frags(std::integral_constant<int, 0>{}, F);
    start_group();
    if constexpr (WHOLE) {
        static_assert(NSTAGE == 4, "tiles end on ring boundaries");
        // Tiles end on ring boundaries (groups % 4 == 0).  One loop over the
        // rings of all the tiles; at a tile's end (a uniform branch) the
        // load offsets move to the next tile and the tile is stored.
        const int total = count * groups;
        int gl = NSTAGE, jl = 0, gc = 0, jc = 0;  // next loads: tile jl group gl; step: tile jc group gc
        if (gl >= groups) {
            gl -= groups;
            jl = 1;
            set_tile_loads(1);
        }
        for (int g0 = 0; g0 < total; g0 += NSTAGE) {
            static_for<NSTAGE>([&](auto uc) { group_step(uc, gl + decltype(uc)::value, Mid{}); });
            // Branch-free: the load tile is re-derived every ring.
            gl += NSTAGE;
            const bool wrap = gl >= groups;
            gl = wrap ? gl - groups : gl;
            jl += wrap ? 1 : 0;
            set_tile_loads(min(jl, count - 1));
            gc += NSTAGE;
            if (gc >= groups) {
                gc = 0;
                store_tile(jc);
                zero_acc();
                ++jc;
            }
        }
    } else {
        // One tile (count == 1).  groups is a multiple of 4, so only whole
        // quarters of a NSTAGE = 8 ring can be missing at the end; the test
        // is uniform and covers a whole ring, so no partial tile stays live
        // across rings.  Loads past the last group read bytes that are never
        // consumed.
        for (int g0 = 0; g0 < groups; g0 += NSTAGE)
            static_for<NSTAGE>([&](auto uc) {
                constexpr int u = decltype(uc)::value;
                if (u < 4 || g0 + u < groups) group_step(uc, g0 + NSTAGE + u, Mid{});
            });
        store_tile(0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// One output tile per workgroup, in XCD-aware order.
template <int TM, int TN, int WM, int WN, int NSTAGE>
__global__ __launch_bounds__(WM *WN *WAVE) __attribute__((amdgpu_waves_per_eu(2))) void w4a4_fp6_kernel(
    const uint8_t *__restrict__ a6, const uint8_t *__restrict__ w6, const float *__restrict__ bias,
    void *__restrict__ y, int out_type, int epi, int m, int n, int k, int n_part, Fp6Out out) {
    using S = Fp6Shape<TM, TN, WM, WN, NSTAGE>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[S::LDS_BYTES];
    const int tiles_m = (m + S::BM - 1) / S::BM, tiles_n = (n + S::BN - 1) / S::BN;
    int tm, tn;
    tile_of_block(blockIdx.x, tiles_m, tiles_n, 8, tm, tn);
    fp6_tiles<TM, TN, WM, WN, NSTAGE, false>(lds, a6, w6, bias, y, out_type, epi, m, n, k, n_part, out, 1,
                                      [&](int, int &mt0, int &nt0) {
                                          mt0 = tm * S::MT;
                                          nt0 = tn * S::NTL;
                                      });
}

// Persistent form for large problems: gridDim.x workgroups (two per CU)
// walk the 128 x 128 tiles t = blockIdx.x + j * gridDim.x, t < full_tiles,
// in XCD-aware order, with one pipeline across their tiles.  When the
// tiles left after the full rounds would keep at most half of the
// workgroups busy, the host passes them as half_units = 2 x that many
// 64 x 128 halves instead (one per workgroup), so that the last round is as
// long as half a full one with every workgroup busy.  Halves of one tile go
// to workgroups on the same XCD (ids 8 apart) when the count allows.  A
// workgroup's tile list (at most FP6_MAX_TILES tiles, checked by the host)
// is computed once into LDS, outside the pipelined loop.
constexpr int FP6_MAX_TILES = 128;

template <int TN, int WM, int WN, int NSTAGE>
__global__ __launch_bounds__(WM *WN *WAVE) __attribute__((amdgpu_waves_per_eu(2))) void w4a4_fp6_persistent_kernel(
    const uint8_t *__restrict__ a6, const uint8_t *__restrict__ w6, const float *__restrict__ bias,
    void *__restrict__ y, int out_type, int epi, int m, int n, int k, int n_part, Fp6Out out, Fp6Grid gd,
    int full_tiles, int half_units) {
    static_assert(NSTAGE == 4, "tiles end on ring boundaries");
    using S2 = Fp6Shape<2, TN, WM, WN, NSTAGE>;
    using S1 = Fp6Shape<1, TN, WM, WN, NSTAGE>;
    static_assert(S2::LDS_BYTES >= S1::LDS_BYTES, "one LDS ring for both phases");
    __shared__ __attribute__((aligned(16))) uint8_t lds[S2::LDS_BYTES];
    __shared__ uint32_t tile_list[FP6_MAX_TILES];  // mt0 | nt0 << 16
    const int b = blockIdx.x, stride = gridDim.x;
    const int count = b < full_tiles ? (full_tiles - 1 - b) / stride + 1 : 0;
    for (int j = threadIdx.x; j < count; j += blockDim.x) {
        int tm, tn;
        grid_tile(gd, b + j * stride, tm, tn);
        tile_list[j] = static_cast<uint32_t>(tm * S2::MT) | (static_cast<uint32_t>(tn * S2::NTL) << 16);
    }
    __syncthreads();
    if (count > 0)
        fp6_tiles<2, TN, WM, WN, NSTAGE, true>(lds, a6, w6, bias, y, out_type, epi, m, n, k, n_part, out, count,
                                               [&](int j, int &mt0, int &nt0) {
                                                   const uint32_t e = __builtin_amdgcn_readfirstlane(tile_list[j]);
                                                   mt0 = static_cast<int>(e & 0xFFFFu);
                                                   nt0 = static_cast<int>(e >> 16);
                                               });
    if (b < half_units) {
        // The ring is reused: every wave has finished with it (each wave's
        // own loads were drained at the end of the first phase).
        __syncthreads();
        int t, half;
        if (half_units % 16 == 0) {
            t = full_tiles + (b >> 4) * 8 + (b & 7);
            half = (b >> 3) & 1;
        } else {
            t = full_tiles + (b >> 1);
            half = b & 1;
        }
        int tm, tn;
        grid_tile(gd, t, tm, tn);
        fp6_tiles<1, TN, WM, WN, NSTAGE, false>(lds, a6, w6, bias, y, out_type, epi, m, n, k, n_part, out, 1,
                                                [&](int, int &mt0, int &nt0) {
                                                    mt0 = tm * S2::MT + half * S1::MT;
                                                    nt0 = tn * S1::NTL;
                                                });
    }
}

template <int TM, int TN, int WM, int WN, int NSTAGE>
static int launch_fp6(const void *a6, const void *w6, const float *bias, void *y,
                      int out_type, int epi, int m, int n, int k, int n_part, Fp6Out out, hipStream_t stream) {
    constexpr int BM = WM * TM * 32, BN = WN * TN * 32;
    const long long blocks = static_cast<long long>((m + BM - 1) / BM) * ((n + BN - 1) / BN);
    if (blocks > 0x7FFFFFFFLL) return kInvalid;
    w4a4_fp6_kernel<TM, TN, WM, WN, NSTAGE><<<dim3(static_cast<unsigned>(blocks)), dim3(WM * WN * WAVE), 0, stream>>>(
        static_cast<const uint8_t *>(a6), static_cast<const uint8_t *>(w6), bias, y, out_type, epi, m, n, k, n_part,
        out);
    return launch_status();
}

// 128 x 128 tiles, two workgroups per CU, persistent (see the kernel); m,
// n multiples of 128 (and for a dual call m_split and n_out too).  m_split
// = 0: one stream.
static int launch_fp6_persistent(const void *a6, const void *w6, const float *bias, void *y, int out_type, int epi,
                                 int m, int n, int k, int n_part, Fp6Out out, int m_split, hipStream_t stream) {
    Fp6Grid gd;
    if (m_split > 0) {
        gd = Fp6Grid{(m_split / 128) * (out.n_out / 128), m_split / 128, out.n_out / 128, (m - m_split) / 128,
                     (n - out.n_out) / 128};
    } else {
        gd = Fp6Grid{(m / 128) * (n / 128), m / 128, n / 128, 0, 0};
    }
    const long long tiles = static_cast<long long>(gd.t0) + static_cast<long long>(gd.tm1) * gd.tn1;
    const long long slots = 2LL * device_cus();
    long long full = tiles, halves = 0, grid;
    if (tiles >= slots) {
        const long long rem = tiles % slots;
        if (rem > 0 && 2 * rem <= slots) {
            full = tiles - rem;
            halves = 2 * rem;
        }
        grid = slots;
    } else if (2 * tiles <= slots) {
        full = 0;
        halves = 2 * tiles;
        grid = halves;
    } else {
        grid = tiles;
    }
    if (tiles <= 0) return 0;
    if (tiles > 0x7FFFFFFFLL || (full + grid - 1) / grid > FP6_MAX_TILES) return kInvalid;
    w4a4_fp6_persistent_kernel<2, 2, 2, 4><<<dim3(static_cast<unsigned>(grid)), dim3(4 * WAVE), 0, stream>>>(
        static_cast<const uint8_t *>(a6), static_cast<const uint8_t *>(w6), bias, y, out_type, epi, m, n, k, n_part,
        out, gd, static_cast<int>(full), static_cast<int>(halves));
    return launch_status();
}

}  // namespace qi

using namespace qi;

namespace qi {

// Tile shapes for one stream of m rows and n outputs (measured on
// MI355X): 0 = 128 x 128 tiles with four waves when that already gives two
// workgroups per CU (persistent when m and n are multiples of 128);
// otherwise, for short M, 3 = 64 x 128 four-wave tiles when N is wide, or
// 4 = single-wave 32 x 32 tiles with an 8-deep ring.
static int select_fp6_tiles(int m, int n) {
    if (static_cast<long long>((m + 127) / 128) * ((n + 127) / 128) >= 512) return 0;
    return n >= 8192 ? 3 : 4;
}

// Tile-shape choice for one stream (see qi_hip_w4a4_gemm_fp6_parts); the
// arguments are checked by the callers.
static int dispatch_fp6(const void *a_codes6, const void *w_codes6, const float *bias, void *y, int out_type,
                        int epilogue, int m, int n, int k, int n_part, Fp6Out out, hipStream_t s) {
    const int cfg = select_fp6_tiles(m, n);
    switch (cfg) {
    case 0:
        // The persistent kernel takes whole 128 x 128 tiles only.
        if (m % 128 == 0 && n % 128 == 0)
            return launch_fp6_persistent(a_codes6, w_codes6, bias, y, out_type, epilogue, m, n, k, n_part, out, 0, s);
        return launch_fp6<2, 2, 2, 2, 4>(a_codes6, w_codes6, bias, y, out_type, epilogue, m, n, k, n_part, out, s);
    case 3:
        return launch_fp6<1, 2, 2, 2, 4>(a_codes6, w_codes6, bias, y, out_type, epilogue, m, n, k, n_part, out, s);
    case 4:
        return launch_fp6<1, 1, 1, 1, 8>(a_codes6, w_codes6, bias, y, out_type, epilogue, m, n, k, n_part, out, s);
    default:
        return launch_fp6<2, 2, 2, 2, 4>(a_codes6, w_codes6, bias, y, out_type, epilogue, m, n, k, n_part, out, s);
    }
}

}  // namespace qi

QI_API int qi_hip_w4a4_gemm_fp6_parts(const void *a_codes6, const void *w_codes6, const float *bias, void *y,
                                      int out_type, int epilogue, int m, int n, int k, int n_part, void *stream) {
    if (m <= 0 || n <= 0 || k <= 0 || n % 32 || k % 256) return kInvalid;
    if (n_part <= 0 || n_part % 32 || n % n_part) return kInvalid;
    if (!a_codes6 || !w_codes6 || !y) return kInvalid;
    if (out_type != QI_HIP_OUT_F32 && out_type != QI_HIP_OUT_F16) return kInvalid;
    if (epilogue != QI_HIP_EPILOGUE_NONE && epilogue != QI_HIP_EPILOGUE_GELU_TANH) return kInvalid;
    if (reinterpret_cast<uintptr_t>(a_codes6) % 16 || reinterpret_cast<uintptr_t>(w_codes6) % 16 ||
        reinterpret_cast<uintptr_t>(y) % (out_type == QI_HIP_OUT_F16 ? 8 : 16))
        return kInvalid;
    const long long g = k / 64;
    if (static_cast<long long>((m + 31) / 32) * g * FP6_BLOCK >= (1LL << 31) ||
        static_cast<long long>(n / 32) * g * FP6_BLOCK >= (1LL << 31))
        return kInvalid;
    return dispatch_fp6(a_codes6, w_codes6, bias, y, out_type, epilogue, m, n, k, n_part, Fp6Out{0, m, n},
                        stream_of(stream));
}

QI_API int qi_hip_w4a4_gemm_fp6_dual(const void *a_codes6, const void *w_codes6, const float *bias, void *y,
                                     int out_type, int epilogue, int m, int m_split, int n, int k, int n_part,
                                     void *stream) {
    if (m_split <= 0 || m_split >= m || m_split % 32) return kInvalid;
    if (m <= 0 || n <= 0 || k <= 0 || n % 32 || k % 256) return kInvalid;
    if (n_part <= 0 || n_part % 32 || n % n_part) return kInvalid;
    if (!a_codes6 || !w_codes6 || !y) return kInvalid;
    if (out_type != QI_HIP_OUT_F32 && out_type != QI_HIP_OUT_F16) return kInvalid;
    if (epilogue != QI_HIP_EPILOGUE_NONE && epilogue != QI_HIP_EPILOGUE_GELU_TANH) return kInvalid;
    if (reinterpret_cast<uintptr_t>(a_codes6) % 16 || reinterpret_cast<uintptr_t>(w_codes6) % 16 ||
        reinterpret_cast<uintptr_t>(y) % (out_type == QI_HIP_OUT_F16 ? 8 : 16))
        return kInvalid;
    const long long g = k / 64;
    if (static_cast<long long>((m + 31) / 32) * g * FP6_BLOCK >= (1LL << 31) ||
        static_cast<long long>(2 * (n / 32)) * g * FP6_BLOCK >= (1LL << 31))
        return kInvalid;
    hipStream_t s = stream_of(stream);
    // Both streams in one persistent launch when every tile is whole.
    if (m % 128 == 0 && m_split % 128 == 0 && n % 128 == 0)
        return launch_fp6_persistent(a_codes6, w_codes6, bias, y, out_type, epilogue, m, 2 * n, k, n_part,
                                     Fp6Out{0, m, n}, m_split, s);
    // Otherwise one launch per stream, each writing its rows of y.
    const size_t gs = static_cast<size_t>(k / 64);
    int st = dispatch_fp6(a_codes6, w_codes6, bias, y, out_type, epilogue, m_split, n, k, n_part, Fp6Out{0, m, n}, s);
    if (st) return st;
    return dispatch_fp6(static_cast<const uint8_t *>(a_codes6) + static_cast<size_t>(m_split / 32) * gs * FP6_BLOCK,
                        static_cast<const uint8_t *>(w_codes6) + static_cast<size_t>(n / 32) * gs * FP6_BLOCK,
                        bias ? bias + n : nullptr, y, out_type, epilogue, m - m_split, n, k, n_part,
                        Fp6Out{m_split, m, n}, s);
}

QI_API int qi_hip_w4a4_gemm_fp6(const void *a_codes6, const void *w_codes6, const float *bias, void *y,
                                int out_type, int epilogue, int m, int n, int k, void *stream) {
    return qi_hip_w4a4_gemm_fp6_parts(a_codes6, w_codes6, bias, y, out_type, epilogue, m, n, k, n, stream);
}

QI_API int qi_hip_w4a4_fp6_tiles(int m, int n) {
    if (m <= 0 || n <= 0) return -1;
    const int cfg = select_fp6_tiles(m, n);
    // 1: the persistent form of the 128 x 128 tiles.
    return cfg == 0 && m % 128 == 0 && n % 128 == 0 ? 1 : cfg;
}
