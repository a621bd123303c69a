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
constexpr int ATT_VROW = ATT_KT + 8;  // V^T tile row pitch, halves

__device__ __forceinline__ int att_visible(int global_row, int keys, int causal_rows, const int *visible_keys) {
    if (visible_keys != nullptr) return visible_keys[global_row];
    return global_row < causal_rows ? global_row + 1 : keys;
}

__global__ __launch_bounds__(ATT_WAVES *WAVE, 1) void flash_attention_kernel(
    const float *__restrict__ q, const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    float *__restrict__ out, int queries, int keys, int heads, int query_offset, int causal_rows,
    const int *__restrict__ visible_keys) {
    __shared__ __attribute__((aligned(16))) uint16_t k_lds2[2][ATT_KT * ATT_KROW];
    __shared__ __attribute__((aligned(16))) uint16_t vt_lds2[2][ATT_HD * ATT_VROW];
    __shared__ int wg_visible;

    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wave = tid >> 6;
    const int h = lane >> 5, l32 = lane & 31;
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
    const int width = heads * ATT_HD;
    const int qi = qblk * ATT_QB + wave * 32 + l32;  // this lane's query
    const bool q_ok = qi < queries;
    const int visible = q_ok ? min(att_visible(qi + query_offset, keys, causal_rows, visible_keys), keys) : 0;

    // How far this workgroup reads: the largest visible count of its rows.
    if (tid == 0) wg_visible = 0;
    __syncthreads();
    int wv = visible;
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) wv = max(wv, __shfl_xor(wv, s, 64));
    if (lane == 0) atomicMax(&wg_visible, wv);
    __syncthreads();
    const int limit = wg_visible;

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

    v16f_t o[4];  // O^T: d-tile j, register 4a + b = dim 32j + 8a + 4h + b
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[j][r] = 0.f;
    float m_run = -__builtin_inff(), l_run = 0.f;

    // The smallest visible count of this wave's queries: tiles below it need
    // no mask.
    int wmin = q_ok ? visible : keys;
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) wmin = min(wmin, __shfl_xor(wmin, s, 64));

    // Tile staging through registers into the LDS slot not being read: K as
    // 16-byte chunks per thread (row-major), V as a 2-key x 8-dim block per
    // thread (every thread takes part; the two rows' halves are paired into
    // the transposed tile with byte permutes, one dword per dim, keys fastest
    // across lanes so the 32 lanes of a row write distinct banks).
    uint4 kn[ATT_KCH];
    // V: 32 key pairs x 16 dim blocks of 8 over the workgroup's threads.
    constexpr int ATT_VDB = 16 / (ATT_WAVES * WAVE / 32);  // dim blocks per thread
    uint32_t vn[ATT_VDB][2][4];
    auto load_tile = [&](int start) {
#pragma unroll
        for (int i = 0; i < ATT_KCH; ++i) {
            const int idx = tid + i * ATT_WAVES * WAVE, key = idx >> 4, chunk = idx & 15;
            kn[i] = uint4{0u, 0u, 0u, 0u};
            if (start + key < keys)
                kn[i] = *reinterpret_cast<const uint4 *>(k + static_cast<size_t>(start + key) * width +
                                                         head * ATT_HD + chunk * 8);
        }
#pragma unroll
        for (int b = 0; b < ATT_VDB; ++b) {
            const int kp = tid & 31, db = (tid >> 5) + b * (ATT_WAVES * WAVE / 32);
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                uint4 t = uint4{0u, 0u, 0u, 0u};
                const int key = start + 2 * kp + r;
                if (key < keys)
                    t = *reinterpret_cast<const uint4 *>(v + static_cast<size_t>(key) * width + head * ATT_HD + 8 * db);
                vn[b][r][0] = t.x;
                vn[b][r][1] = t.y;
                vn[b][r][2] = t.z;
                vn[b][r][3] = t.w;
            }
        }
    };
    auto store_tile = [&](int buf) {
        uint16_t *k_lds = k_lds2[buf];
        uint16_t *vt_lds = vt_lds2[buf];
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
    if (limit > 0) {
        load_tile(0);
        store_tile(0);
        __syncthreads();
        if (ATT_KT < limit) load_tile(ATT_KT);
    }
    int buf = 0;
    for (int start = 0; start < limit; start += ATT_KT, buf ^= 1) {
        const uint16_t *k_lds = k_lds2[buf];
        const uint16_t *vt_lds = vt_lds2[buf];

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
#pragma unroll
        for (int f = 0; f < VLA; ++f) read_v(f);
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
        for (int f = 0; f < 16; ++f) {
            if (f + VLA < 16) read_v(f + VLA);
            __builtin_amdgcn_sched_barrier(0);
            const int j = f >> 2, t = (f >> 1) & 1, e = f & 1;
            o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[f], pb[t][e], o[j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (start + ATT_KT < limit) store_tile(buf ^ 1);
        __syncthreads();
        if (start + 2 * ATT_KT < limit) load_tile(start + 2 * ATT_KT);
    }

    // Both halves' sums, then O / sum (0 when nothing was visible).
    const float total = l_run + __shfl_xor(l_run, 32, 64);
    const float inverse = total > 0.f ? 1.0f / total : 0.f;
    if (q_ok) {
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

static int launch_attention(const float *q, const void *k, const void *v, float *out, int queries, int keys,
                            int heads, int query_offset, int causal_rows, const int *visible_keys,
                            hipStream_t stream) {
    if (queries < 0 || keys < 0 || heads <= 0 || heads > 65535) return kInvalid;
    if (queries == 0) return 0;
    if (!q || !out || (keys > 0 && (!k || !v))) return kInvalid;
    if (reinterpret_cast<uintptr_t>(q) % 16 || reinterpret_cast<uintptr_t>(out) % 16 ||
        reinterpret_cast<uintptr_t>(k) % 16 || reinterpret_cast<uintptr_t>(v) % 16)
        return kInvalid;
    const dim3 grid(static_cast<unsigned>((queries + ATT_QB - 1) / ATT_QB), static_cast<unsigned>(heads));
    flash_attention_kernel<<<grid, dim3(ATT_WAVES * WAVE), 0, stream>>>(
        q, static_cast<const uint16_t *>(k), static_cast<const uint16_t *>(v), out, queries, keys, heads,
        query_offset, causal_rows, visible_keys);
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
