// Fused attention for the MMDiT blocks (the reference's qi_flash_attention,
// qwen_image_cuda/cuda/flash.cu:1-244) on gfx950 fp16 MFMA.
//
// out[q, h, :] = softmax(Q[q, h] . K[:, h]^T / sqrt(128), mask) . V[:, h] for
// head dim 128, without materialising the scores.  Arithmetic as the
// reference: Q is scaled by log2(e) / sqrt(128) in fp32 and rounded to fp16
// (flash.cu:86-97), scores accumulate in fp32, the softmax is the online
// (running max / sum) form in the log2 domain with exp2 (flash.cu:160-186),
// probabilities are rounded to fp16 for the P V product while the row sums
// add the fp32 values, and out = O / sum (0 for a row with nothing visible,
// flash.cu:212-226).  Summation orders are this kernel's own, so results
// agree with the reference within fp16-input tolerance, not bit for bit.
//
// Mask (flash.cu:11-13, 46-49): global query row r = q + query_offset sees
// keys [0, visible_keys[r]) when visible_keys is given, else [0, r + 1) when
// r < causal_rows, else every key.
//
// Design.  One wave owns 32 queries of one head; a workgroup of eight waves
// shares 64-key tiles of K (row-major) and V (transposed) staged in two LDS
// slots, every thread staging part of each tile, one barrier per tile.
// Scores are formed transposed, S^T = K Q^T on v_mfma_f32_32x32x16_f16
// (A = K from LDS, B = Q^T held in registers), so lane l holds 32 scores of
// ONE query (l % 32): the row max and sum are lane-local plus one exchange
// with lane l ^ 32.  The output is likewise formed transposed, O^T += V^T
// P^T: the probabilities feed the second MFMA straight from the score
// registers (B operand), the K slots of each 16-key step being the keys the
// lane holds, in the MFMA output order, and the V^T fragments (A operand)
// are read with the same key order from the transposed tile.  O^T lanes also
// hold one query each, so the online rescaling is lane-local.
//
// Balanced split (flash_attention_stream_kernel, mask-free calls with a
// workspace).  One workgroup fills a CU, so the grid of (head, query block)
// units runs in whole rounds of CUs, and a mostly empty last round (4352
// tokens x 16 heads: 272 units on 256 CUs) costs nearly a full one.  The
// split runs the whole rounds in lockstep, one workgroup per CU, then cuts
// each remaining unit into aligned key segments, its parts dealt out one
// per CU; each part leaves its O^T, offset and sum in the workspace, and
// the unit's part that arrives last (an arrival counter per unit) merges
// them in segment order, so the result does not depend on timing.

#include "qi_common.h"

namespace qi {

typedef _Float16 v8h_t __attribute__((ext_vector_type(8)));
typedef float v16f_t __attribute__((ext_vector_type(16)));

constexpr int ATT_HD = 128;           // head dim
constexpr int ATT_KT = 64;            // keys per tile
constexpr int ATT_WAVES = 8;          // waves per workgroup, 32 queries each (8: measured 6-10 % faster than 4 at two workgroups per CU)
constexpr int ATT_KCH = ATT_KT * ATT_HD / 8 / (ATT_WAVES * 64);  // K chunks per thread
constexpr int ATT_QB = ATT_WAVES * 32;
constexpr int ATT_KROW = ATT_HD + 8;  // K tile row pitch, halves (keeps the 32 rows a fragment read touches apart)
constexpr int ATT_VROW = ATT_KT + 4;  // V^T tile row pitch, halves (34 dwords: 16 rows, 8-byte reads, distinct banks)

__device__ __forceinline__ int att_visible(int global_row, int keys, int causal_rows, const int *visible_keys) {
    if (visible_keys != nullptr) return visible_keys[global_row];
    return global_row < causal_rows ? global_row + 1 : keys;
}

struct AttLds {
    __attribute__((aligned(16))) uint16_t k[2][ATT_KT * ATT_KROW];
    __attribute__((aligned(16))) uint16_t vt[2][ATT_HD * ATT_VROW];
    int visible;
    int last;
};

// Keys [kbegin, kend) of one unit (head, query block `qblk`) for this
// thread's wave: O^T (o), running offset and sum, from zero.  `visible` is
// the lane's visible key count, `wmin` the wave's smallest; every thread of
// the workgroup calls it with the same unit and range (tile staging and
// barriers are shared), and it returns after a barrier, so the LDS tiles are
// free again.
__device__ __forceinline__ void att_keys(const float *__restrict__ q, const uint16_t *__restrict__ k,
                                         const uint16_t *__restrict__ v, int queries, int keys, int heads, int head,
                                         int qblk, int kbegin, int kend, int visible, int wmin, AttLds &lds,
                                         v16f_t (&o)[4], float &m_run, float &l_run) {
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    const int h = lane >> 5, l32 = lane & 31;
    const int width = heads * ATT_HD;
    const int qi = qblk * ATT_QB + wave * 32 + l32;  // this lane's query
    const bool q_ok = qi < queries;
    // Q^T fragments (B operand): K-step s holds dims 16s + 8h .. + 7 of the
    // lane's query, scaled into the log2 domain and rounded to fp16.
    const float scale = 1.4426950408889634f / __builtin_sqrtf(static_cast<float>(ATT_HD));
    v8h_t qf[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        float4 a = float4{0.f, 0.f, 0.f, 0.f}, b = a;
        if (q_ok) {
            const float *src = q + static_cast<size_t>(qi) * width + head * ATT_HD + 16 * s + 8 * h;
            a = *reinterpret_cast<const float4 *>(src);
            b = *reinterpret_cast<const float4 *>(src + 4);
        }
        qf[s] = v8h_t{static_cast<_Float16>(a.x * scale), static_cast<_Float16>(a.y * scale),
                      static_cast<_Float16>(a.z * scale), static_cast<_Float16>(a.w * scale),
                      static_cast<_Float16>(b.x * scale), static_cast<_Float16>(b.y * scale),
                      static_cast<_Float16>(b.z * scale), static_cast<_Float16>(b.w * scale)};
    }

#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[j][r] = 0.f;
    m_run = -__builtin_inff();
    l_run = 0.f;

    // Tile staging through registers into the LDS slot not being read: K as
    // 16-byte chunks per thread (row-major), V as a 2-key x 8-dim block per
    // thread (every thread takes part; the two rows' halves are paired into
    // the transposed tile with byte permutes, one dword per dim, keys fastest
    // across lanes so the 32 lanes of a row write distinct banks).
    uint4 kn[ATT_KCH];
    // V: 32 key pairs x 16 dim blocks of 8 over the workgroup's threads.
    constexpr int ATT_VDB = 16 / (ATT_WAVES * WAVE / 32);  // dim blocks per thread
    uint32_t vn[ATT_VDB][2][4];
    // Buffer loads: a lane's 16-byte chunks sit at fixed byte offsets from
    // the tile's first row of this head (voffset), the tile's base and
    // range are scalar, and rows at or past `keys` lie beyond the range, so
    // they read as zeros with no per-key test or branch.
    uint32_t k_vo[ATT_KCH], v_vo[ATT_VDB][2];
#pragma unroll
    for (int i = 0; i < ATT_KCH; ++i) {
        const int idx = tid + i * ATT_WAVES * WAVE, key = idx >> 4, chunk = idx & 15;
        k_vo[i] = static_cast<uint32_t>(key * width * 2 + chunk * 16);
    }
#pragma unroll
    for (int b = 0; b < ATT_VDB; ++b)
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int kp = tid & 31, db = (tid >> 5) + b * (ATT_WAVES * WAVE / 32);
            v_vo[b][r] = static_cast<uint32_t>((2 * kp + r) * width * 2 + 16 * db);
        }
    auto load_tile = [&](int start) {
        // Bytes of this head's rows from `start` on; a tile reads at most
        // 64 rows (< 2^31 bytes), so clamping the range keeps it exact.
        const long long left = static_cast<long long>(keys - start) * width * 2 - head * ATT_HD * 2;
        const uint32_t bytes = static_cast<uint32_t>(left < 0x7FFFFFF0LL ? left : 0x7FFFFFF0LL);
        const size_t base = static_cast<size_t>(start) * width + head * ATT_HD;
        const auto rk = buffer_rsrc(k + base, bytes), rv = buffer_rsrc(v + base, bytes);
#pragma unroll
        for (int i = 0; i < ATT_KCH; ++i)
            kn[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, k_vo[i], 0, 0));
#pragma unroll
        for (int b = 0; b < ATT_VDB; ++b)
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const uint4 t = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, v_vo[b][r], 0, 0));
                vn[b][r][0] = t.x;
                vn[b][r][1] = t.y;
                vn[b][r][2] = t.z;
                vn[b][r][3] = t.w;
            }
    };
    auto store_tile = [&](int buf) {
        uint16_t *k_lds = lds.k[buf];
        uint16_t *vt_lds = lds.vt[buf];
#pragma unroll
        for (int i = 0; i < ATT_KCH; ++i) {
            const int idx = tid + i * ATT_WAVES * WAVE, key = idx >> 4, chunk = idx & 15;
            *reinterpret_cast<uint4 *>(k_lds + key * ATT_KROW + chunk * 8) = kn[i];
        }
#pragma unroll
        for (int b = 0; b < ATT_VDB; ++b) {
            const int kp = tid & 31, db = (tid >> 5) + b * (ATT_WAVES * WAVE / 32);
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
                *reinterpret_cast<uint32_t *>(vt_lds + (8 * db + c) * ATT_VROW + 2 * kp) =
                    __builtin_amdgcn_perm(vn[b][1][c >> 1], vn[b][0][c >> 1], sel);
            }
        }
    };

    // Two LDS slots: tile i is read from slot i % 2 while tile i + 1 (loaded
    // into registers during tile i - 1) is stored into the other after the
    // tile's products; one barrier per tile then orders both.
    if (kbegin < kend) {
        load_tile(kbegin);
        store_tile(0);
        __syncthreads();
        if (kbegin + ATT_KT < kend) load_tile(kbegin + ATT_KT);
    }
    int buf = 0;
    for (int start = kbegin; start < kend; start += ATT_KT, buf ^= 1) {
        const uint16_t *k_lds = lds.k[buf];
        const uint16_t *vt_lds = lds.vt[buf];

        // S^T for the tile's two 32-key halves t: register 4a + b of s[t]
        // holds key start + 32t + 8a + 4h + b of the lane's query.  The two
        // halves' MFMA chains alternate (step f: dims 16 (f / 2), half f % 2)
        // and each K fragment is read KLA steps ahead of its MFMA.
        v16f_t s[2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) s[t][r] = 0.f;
        {
            constexpr int KLA = 4;
            v8h_t kf[16];
            auto read_k = [&](int f) {
                kf[f] = *reinterpret_cast<const v8h_t *>(k_lds + (32 * (f & 1) + l32) * ATT_KROW + 8 * h +
                                                         16 * (f >> 1));
            };
#pragma unroll
            for (int f = 0; f < KLA; ++f) read_k(f);
#pragma unroll
            for (int f = 0; f < 16; ++f) {
                if (f + KLA < 16) read_k(f + KLA);
                __builtin_amdgcn_sched_barrier(0);
                s[f & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[f], qf[f >> 1], s[f & 1], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // Mask, row max (this lane's 32 keys, then the other half's).
        if (start + ATT_KT > wmin) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = start + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (key >= visible) s[t][r] = -__builtin_inff();
                }
        }
        constexpr int VLA = 4;
        v8h_t vf[16];
        auto read_v = [&](int f) {
            const uint16_t *vrow = vt_lds + (32 * (f >> 2) + l32) * ATT_VROW + 4 * h + 32 * ((f >> 1) & 1) + 16 * (f & 1);
            const uint2 lo = *reinterpret_cast<const uint2 *>(vrow);
            const uint2 hi = *reinterpret_cast<const uint2 *>(vrow + 8);
            vf[f] = __builtin_bit_cast(v8h_t, uint4{lo.x, lo.y, hi.x, hi.y});
        };
        // Issue order g: the d-tile j = g % 4 changes fastest, so that
        // consecutive MFMAs accumulate into different tiles of O (four
        // apart) instead of waiting on each other's results.
        auto pv_f = [](int g) { return 4 * (g & 3) + (g >> 2); };
#pragma unroll
        for (int g = 0; g < VLA; ++g) read_v(pv_f(g));
        __builtin_amdgcn_sched_barrier(0);
        // p = exp2(s - offset) with the running offset first (a row with
        // nothing visible yet takes 0: all its p are 0).  The hardware exp2
        // (v_exp_f32): results below 2^-126 flush to zero, which changes p
        // only where it is already below fp16's range and the row sum by
        // less than 2^-120.
        float lsum = 0.f;
        v8h_t pb[2][2];  // P^T B operands: tile t, 16-key step e
        auto probabilities = [&](float base) {
            lsum = 0.f;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float p = __builtin_amdgcn_exp2f(s[t][r] - base);
                    lsum += p;
                    pb[t][r >> 3][r & 7] = static_cast<_Float16>(p);
                }
        };
        const float base0 = m_run == -__builtin_inff() ? 0.f : m_run;
        probabilities(base0);
        // The offset moves only when some lane's 32 probabilities sum past
        // 2^8 (so every p stays <= 256: exact in fp16's normal range as
        // relative values, and O / sum is unchanged in exact arithmetic), or
        // while a row has no offset yet: then to the rows' exact maximum,
        // with O and the sum rescaled and the probabilities formed again.
        // No maximum is taken otherwise.
        if (__any(!(lsum <= 256.f) || m_run == -__builtin_inff())) {
            float mx = -__builtin_inff();
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[t][r]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float new_m = mx > m_run ? mx : m_run;
            const float base = new_m == -__builtin_inff() ? 0.f : new_m;
            probabilities(base);
            // alpha is exactly 1 for rows whose offset stayed; O and the sum
            // so far were formed at offset base0.
            const float alpha = __builtin_amdgcn_exp2f(base0 - base);
            l_run *= alpha;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[j][r] *= alpha;
            m_run = new_m;
        }
        l_run += lsum;
        // O^T += V^T P^T.  Step (t, e) covers keys 32t + 16e + 8(i / 4) +
        // 4h + i % 4 in K slot 8h + i: from the V^T row of dim d, the runs
        // of 4 keys at 32t + 16e + 4h and 32t + 16e + 8 + 4h.  MFMA f = 4j
        // + 2t + e; its V fragment is read VLA MFMAs ahead (the first ones
        // before the softmax, above).
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            if (g + VLA < 16) read_v(pv_f(g + VLA));
            __builtin_amdgcn_sched_barrier(0);
            const int f = pv_f(g), j = f >> 2, t = (f >> 1) & 1, e = f & 1;
            o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[f], pb[t][e], o[j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (start + ATT_KT < kend) store_tile(buf ^ 1);
        __syncthreads();
        if (start + 2 * ATT_KT < kend) load_tile(start + 2 * ATT_KT);
    }

}

// O / sum for this lane's query (0 when nothing was visible): both key
// halves' sums, then the lane's 64 dims.  o as att_keys leaves it (O^T
// register 4a + b of d-tile j = dim 32j + 8a + 4h + b).
__device__ __forceinline__ void att_store(float *__restrict__ out, const v16f_t (&o)[4], float l_run, int queries,
                                          int heads, int head, int qblk) {
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    const int h = lane >> 5, l32 = lane & 31;
    const int width = heads * ATT_HD;
    const int qi = qblk * ATT_QB + wave * 32 + l32;
    const float total = l_run + __shfl_xor(l_run, 32, 64);
    const float inverse = total > 0.f ? 1.0f / total : 0.f;
    if (qi < queries) {
        float *dst = out + static_cast<size_t>(qi) * width + head * ATT_HD + 4 * h;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int a = 0; a < 4; ++a)
                *reinterpret_cast<float4 *>(dst + 32 * j + 8 * a) =
                    float4{o[j][4 * a] * inverse, o[j][4 * a + 1] * inverse, o[j][4 * a + 2] * inverse,
                           o[j][4 * a + 3] * inverse};
    }
}

__global__ __launch_bounds__(ATT_WAVES *WAVE, 1) void flash_attention_kernel(
    const float *__restrict__ q, const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    float *__restrict__ out, int queries, int keys, int heads, int query_offset, int causal_rows,
    const int *__restrict__ visible_keys) {
    __shared__ AttLds lds;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    const int l32 = lane & 31;
    int head, qblk;
    {
        const int nqb = gridDim.x, nh = gridDim.y;
        const int id = blockIdx.x + nqb * blockIdx.y, total = nqb * nh;
        const int xcd = id % 8, slot = id / 8;
        // The hardware hands workgroup `id` to XCD id % 8; XCD x takes the
        // linear work items [x * per, (x + 1) * per) of head-major order, so
        // one head's query blocks share an XCD's L2 (measured 2 % faster).
        const int per = (total + 7) / 8;
        int w = xcd * per + slot;
        if (total % 8 != 0 || w >= total) w = id;  // uneven split: keep the plain order
        head = w / nqb;
        qblk = w % nqb;
    }
    const int qi = qblk * ATT_QB + wave * 32 + l32;  // this lane's query
    const bool q_ok = qi < queries;
    const int visible = q_ok ? min(att_visible(qi + query_offset, keys, causal_rows, visible_keys), keys) : 0;

    // How far this workgroup reads: the largest visible count of its rows.
    if (tid == 0) lds.visible = 0;
    __syncthreads();
    int wv = visible;
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) wv = max(wv, __shfl_xor(wv, s, 64));
    if (lane == 0) atomicMax(&lds.visible, wv);
    __syncthreads();
    const int limit = lds.visible;

    // The smallest visible count of this wave's queries: tiles below it need
    // no mask.
    int wmin = q_ok ? visible : keys;
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) wmin = min(wmin, __shfl_xor(wmin, s, 64));

    v16f_t o[4];
    float m_run, l_run;
    att_keys(q, k, v, queries, keys, heads, head, qblk, 0, limit, visible, wmin, lds, o, m_run, l_run);
    att_store(out, o, l_run, queries, heads, head, qblk);
}

// Workspace of the balanced split for `tail` split units of `segs` parts:
// the arrival counters (one per split unit), then per part its offsets and
// sums (two floats per thread) and O^T (64 floats per thread,
// register-major so that each access of a wave is 256 contiguous bytes).
constexpr int ATT_THREADS = ATT_WAVES * WAVE;
inline size_t att_counter_bytes(long long tail) { return (static_cast<size_t>(tail) * 4 + 255) / 256 * 256; }
inline size_t att_split_bytes(long long tail, int segs) {
    return att_counter_bytes(tail) + static_cast<size_t>(tail) * segs * ATT_THREADS * (8 + 64 * 4);
}

__global__ void att_clear_kernel(unsigned *__restrict__ counters, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) counters[i] = 0u;
}

// Parts cross workgroups (and XCDs, whose L2s are not coherent with each
// other) through device-scope atomic stores and loads, which the compiler
// issues as coherent (sc1) dword accesses: a device-scope fence would write
// back and invalidate the whole L2 of the XCD instead, evicting the K/V
// tiles its other workgroups are reading (measured: 24 heads 280 -> 401 us).
__device__ __forceinline__ void att_put(float *p, float x) {
    __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float att_get(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One workgroup per CU.  First `rounds` rounds of whole units in lockstep
// (unit i * gridDim.x + r in round i: the workgroups of an XCD then read
// the same key tiles of the same heads at the same time, as the plain grid
// does), then the remaining `tail` units, each cut into `segs` aligned
// segments of `seg_len` key tiles, as parts dealt out in the same way.
__global__ __launch_bounds__(ATT_WAVES *WAVE, 1) void flash_attention_stream_kernel(
    const float *__restrict__ q, const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    float *__restrict__ out, int queries, int keys, int heads, unsigned *__restrict__ arrivals,
    float *__restrict__ part_ml, float *__restrict__ part_o, int rounds, int tail, int nt, int nqb, int segs,
    int seg_len) {
    __shared__ AttLds lds;
    const int tid = threadIdx.x;
    const int wgs = gridDim.x;
    // Ranges in XCD-major order (workgroup id goes to XCD id % 8), so that
    // neighbouring units and ranges -- the same head's -- share an XCD's L2.
    const int id = blockIdx.x;
    const int r = wgs % 8 == 0 ? (id % 8) * (wgs / 8) + id / 8 : id;
    for (int i = 0; i < rounds; ++i) {
        const int u = i * wgs + r;
        v16f_t o[4];
        float m_run, l_run;
        att_keys(q, k, v, queries, keys, heads, u / nqb, u % nqb, 0, keys, keys, keys, lds, o, m_run, l_run);
        att_store(out, o, l_run, queries, heads, u / nqb, u % nqb);
    }
    // The tail: each remaining unit cut into `segs` segments of `seg_len`
    // key tiles; part p = seg * tail + unit (segment-major, so that the
    // workgroups of an XCD take consecutive parts: the same segment of the
    // same heads' units, the same key tiles at the same time).
    const int ubase = rounds * wgs;
    const int nparts = tail * segs;
    for (int p = r; p < nparts; p += wgs) {
        const int seg = p / tail, ut = p - seg * tail, u = ubase + ut;
        const int head = u / nqb, qblk = u % nqb;
        const int tb = seg * seg_len, te = min(nt, tb + seg_len);
        v16f_t o[4];
        float m_run, l_run;
        att_keys(q, k, v, queries, keys, heads, head, qblk, tb * ATT_KT, min(te * ATT_KT, keys), keys, keys, lds, o,
                 m_run, l_run);
        // Part p in slot p; the unit's last part to arrive merges them.
        att_put(part_ml + (2 * p) * ATT_THREADS + tid, m_run);
        att_put(part_ml + (2 * p + 1) * ATT_THREADS + tid, l_run);
        float *po = part_o + static_cast<size_t>(p) * 64 * ATT_THREADS + tid;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) att_put(po + (16 * j + e) * ATT_THREADS, o[j][e]);
        // Every thread's stores complete (acknowledged at the coherent
        // level), then one arrival.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0)
            lds.last = __hip_atomic_fetch_add(&arrivals[ut], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                       static_cast<unsigned>(segs - 1);
        __syncthreads();
        if (!lds.last) continue;
        float mx = -__builtin_inff();
        for (int sg = 0; sg < segs; ++sg)
            mx = fmaxf(mx, att_get(part_ml + (2 * (sg * tail + ut)) * ATT_THREADS + tid));
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) o[j][e] = 0.f;
        float l_sum = 0.f;
        for (int sg = 0; sg < segs; ++sg) {
            const int sl = sg * tail + ut;
            const float m_s = att_get(part_ml + (2 * sl) * ATT_THREADS + tid);
            const float w = m_s == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(m_s - mx);
            l_sum += w * att_get(part_ml + (2 * sl + 1) * ATT_THREADS + tid);
            const float *pi = part_o + static_cast<size_t>(sl) * 64 * ATT_THREADS + tid;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) o[j][e] += w * att_get(pi + (16 * j + e) * ATT_THREADS);
        }
        att_store(out, o, l_sum, queries, heads, head, qblk);
    }
}

static int check_attention(const float *q, const void *k, const void *v, float *out, int queries, int keys,
                           int heads) {
    if (queries < 0 || keys < 0 || heads <= 0 || heads > 65535) return kInvalid;
    if (queries > 0 && (!q || !out || (keys > 0 && (!k || !v)))) return kInvalid;
    if (reinterpret_cast<uintptr_t>(q) % 16 || reinterpret_cast<uintptr_t>(out) % 16 ||
        reinterpret_cast<uintptr_t>(k) % 16 || reinterpret_cast<uintptr_t>(v) % 16)
        return kInvalid;
    return 0;
}

static int launch_attention(const float *q, const void *k, const void *v, float *out, int queries, int keys,
                            int heads, int query_offset, int causal_rows, const int *visible_keys,
                            hipStream_t stream) {
    if (const int e = check_attention(q, k, v, out, queries, keys, heads)) return e;
    if (queries == 0) return 0;
    const dim3 grid(static_cast<unsigned>((queries + ATT_QB - 1) / ATT_QB), static_cast<unsigned>(heads));
    flash_attention_kernel<<<grid, dim3(ATT_THREADS), 0, stream>>>(
        q, static_cast<const uint16_t *>(k), static_cast<const uint16_t *>(v), out, queries, keys, heads,
        query_offset, causal_rows, visible_keys);
    return launch_status();
}

// The balanced split's shape for a mask-free call on the current device:
// `wgs` workgroups (one per CU) run `rounds` lockstep rounds of whole units
// (of `nt` key tiles), then the remaining `tail` units as `segs` aligned
// segments of `seg_len` tiles each.  Returns false where that would not
// pay (see below).  The CU count is the current device's (256 when no
// device is visible).
struct AttSplit {
    long long units;
    int nt, nqb, wgs, rounds, tail, segs, seg_len;
};
static bool attention_split(int queries, int keys, int heads, AttSplit &sp) {
    if (queries <= 0 || keys <= 0) return false;
    const int cus = device_cus();
    sp.nqb = (queries + ATT_QB - 1) / ATT_QB;
    sp.nt = (keys + ATT_KT - 1) / ATT_KT;
    sp.units = static_cast<long long>(sp.nqb) * heads;
    if (sp.units >= (1ll << 31) || sp.nt < 4) return false;
    sp.rounds = static_cast<int>(sp.units / cus);
    sp.tail = static_cast<int>(sp.units - static_cast<long long>(sp.rounds) * cus);
    sp.wgs = cus;
    if (sp.tail == 0) return false;
    // The segment count with the fewest tile steps per CU for the tail, its
    // parts all in one round of CUs (a part has fixed costs -- its Q
    // fragments, the first tile's latency, its store and merge -- that made
    // several rounds of parts slower than the plain grid: 4352 tokens x 24
    // heads 251 -> 271 us in three rounds of 14-tile parts): the segment
    // length, plus one tile step per part beyond the first for the merge
    // that reads it; at most 16 segments.
    long long best = -1;
    for (int s = 2; s <= 16 && s <= sp.nt && static_cast<long long>(sp.tail) * s <= cus; ++s) {
        const int len = (sp.nt + s - 1) / s, segs = (sp.nt + len - 1) / len;
        const long long cost = len + (segs - 1);
        if (best < 0 || cost < best) {
            best = cost;
            sp.segs = segs;
            sp.seg_len = len;
        }
    }
    if (best < 0 || static_cast<long long>(sp.tail) * sp.segs * ATT_THREADS * 264 >= (1ll << 40)) return false;
    // Take it where the tail costs at most 85 % of the plain grid's extra
    // round of whole units.  Measured at 4352 tokens (us, plain -> split):
    // 16 heads 251 -> 187, 20 heads 250 -> 212, 32 heads 397 -> 343, 48
    // heads 541 -> 487; 24 heads (152 tail units) stay plain at 251.
    return best * 100 <= 85LL * sp.nt;
}

static long long attention_workspace(int queries, int keys, int heads) {
    AttSplit sp;
    if (!attention_split(queries, keys, heads, sp)) return 0;
    return static_cast<long long>(att_split_bytes(sp.tail, sp.segs));
}

static int launch_attention_ws(const float *q, const void *k, const void *v, float *out, int queries, int keys,
                               int heads, int query_offset, int causal_rows, const int *visible_keys,
                               void *workspace, long long workspace_bytes, hipStream_t stream) {
    if (const int e = check_attention(q, k, v, out, queries, keys, heads)) return e;
    if (workspace_bytes < 0 || reinterpret_cast<uintptr_t>(workspace) % 16) return kInvalid;
    AttSplit sp;
    // Only calls where every row sees every key split: no visible_keys and
    // no causal row among these rows.
    const bool mask_free = visible_keys == nullptr && causal_rows <= query_offset;
    if (!mask_free || !workspace || !attention_split(queries, keys, heads, sp) ||
        workspace_bytes < static_cast<long long>(att_split_bytes(sp.tail, sp.segs)))
        return launch_attention(q, k, v, out, queries, keys, heads, query_offset, causal_rows, visible_keys,
                                stream);
    auto *base = static_cast<unsigned char *>(workspace);
    auto *arrivals = reinterpret_cast<unsigned *>(base);
    auto *part_ml = reinterpret_cast<float *>(base + att_counter_bytes(sp.tail));
    auto *part_o = reinterpret_cast<float *>(base + att_counter_bytes(sp.tail) +
                                             static_cast<size_t>(sp.tail) * sp.segs * ATT_THREADS * 8);
    // The counters start at zero on every call (a fill kernel, not a memset,
    // so the pair can sit in a captured graph).
    att_clear_kernel<<<static_cast<unsigned>((sp.tail + 255) / 256), 256, 0, stream>>>(arrivals, sp.tail);
    if (const int e = launch_status()) return e;
    flash_attention_stream_kernel<<<sp.wgs, dim3(ATT_THREADS), 0, stream>>>(
        q, static_cast<const uint16_t *>(k), static_cast<const uint16_t *>(v), out, queries, keys, heads, arrivals,
        part_ml, part_o, sp.rounds, sp.tail, sp.nt, sp.nqb, sp.segs, sp.seg_len);
    return launch_status();
}

}  // namespace qi

QI_API int qi_flash_attention(const float *q, const void *k_half, const void *v_half, float *out, int queries,
                              int keys, int heads, int query_offset, int causal_rows, const int *visible_keys) {
    return qi::launch_attention(q, k_half, v_half, out, queries, keys, heads, query_offset, causal_rows,
                                visible_keys, nullptr);
}

QI_API int qi_hip_flash_attention(const float *q, const void *k_half, const void *v_half, float *out, int queries,
                                  int keys, int heads, int query_offset, int causal_rows, const int *visible_keys,
                                  void *stream) {
    return qi::launch_attention(q, k_half, v_half, out, queries, keys, heads, query_offset, causal_rows,
                                visible_keys, qi::stream_of(stream));
}

QI_API long long qi_hip_flash_attention_workspace_bytes(int queries, int keys, int heads) {
    if (queries < 0 || keys < 0 || heads <= 0 || heads > 65535) return 0;
    return qi::attention_workspace(queries, keys, heads);
}

QI_API int qi_hip_flash_attention_ws(const float *q, const void *k_half, const void *v_half, float *out, int queries,
                                     int keys, int heads, int query_offset, int causal_rows,
                                     const int *visible_keys, void *workspace, long long workspace_bytes,
                                     void *stream) {
    return qi::launch_attention_ws(q, k_half, v_half, out, queries, keys, heads, query_offset, causal_rows,
                                   visible_keys, workspace, workspace_bytes, qi::stream_of(stream));
}
