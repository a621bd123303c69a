// Device-side QIPACK weight quantiser: fp16 [N, K] -> codes [N, K/2],
// fp16 scales [N, G] (+ fp16 minimums for W4A16), bit-exact with the
// reference packer's arithmetic (qwen_image_cuda/src/int4_pack.cplus:237-468).
//
// A workgroup takes 256 consecutive 64-groups of the flattened matrix (rows
// are contiguous, so group i is elements [64i, 64i + 64)).  It stages them in
// LDS with a 65-float pitch (conflict-free column reads), applies the H256
// butterfly per 256-chunk for W4A4 with one wavefront per chunk, and then each
// thread runs one group's quantiser sequentially, in the reference's fp32
// order, from registers.  The clip search's squared error is a sequential
// fp32 sum in the reference (:300-307, :343-350), so it stays per-thread.

#include "qi_common.h"

namespace qi {

constexpr int PACK_GROUPS = 256;  // groups per workgroup
constexpr int PITCH = 65;         // LDS floats per group

// int4_pack.cplus:237-245 candidates, as the f32 values the reference forms:
// (0.5 * c) as f32 for the affine search (:297), (c / 7) as f32 for the
// symmetric one (:341).  Constant-folded in double, rounded once to float.
__constant__ float kAffineHalf[7] = {static_cast<float>(0.5 * 1.0),  static_cast<float>(0.5 * 0.95),
                                     static_cast<float>(0.5 * 0.9),  static_cast<float>(0.5 * 0.85),
                                     static_cast<float>(0.5 * 0.8),  static_cast<float>(0.5 * 0.75),
                                     static_cast<float>(0.5 * 0.7)};
__constant__ float kSymmetricFactor[7] = {static_cast<float>(1.0 / 7.0),  static_cast<float>(0.95 / 7.0),
                                          static_cast<float>(0.9 / 7.0),  static_cast<float>(0.85 / 7.0),
                                          static_cast<float>(0.8 / 7.0),  static_cast<float>(0.75 / 7.0),
                                          static_cast<float>(0.7 / 7.0)};

constexpr float kScaleFloor = 0.000000059604645f;  // int4_pack.cplus:53

__device__ __forceinline__ float half_round(float v) { return h2f(f2h(v)); }
// Reference f32 min/max (a.min(b) / a.max(b)) for non-NaN inputs.
__device__ __forceinline__ float rmin(float a, float b) { return b < a ? b : a; }
__device__ __forceinline__ float rmax(float a, float b) { return b > a ? b : a; }

__device__ __forceinline__ float lds_at(const float *chunk, int e) { return chunk[(e >> 6) * PITCH + (e & 63)]; }
__device__ __forceinline__ void lds_set(float *chunk, int e, float v) { chunk[(e >> 6) * PITCH + (e & 63)] = v; }

// int4_pack.cplus:322-363, scheme 6.  Writes 32 code bytes and the scale.
__device__ void quantize_symmetric(const float *v, int clip, uint8_t *codes, uint16_t *scale_out) {
#pragma clang fp contract(off)
    float peak = 0.0f;
    for (int i = 0; i < 64; ++i) peak = rmax(peak, fabsf(v[i]));
    float best_error = 0.0f, best_scale = 0.0f;
    const int candidates = clip ? 7 : 1;
    for (int cand = 0; cand < candidates; ++cand) {
        const float scale = half_round(rmax(peak * kSymmetricFactor[cand], kScaleFloor));
        float error = 0.0f;
        for (int i = 0; i < 64; ++i) {
            const float code = rmin(rmax(rintf(v[i] / scale), -7.0f), 7.0f);
            const float difference = code * scale - v[i];
            error = error + difference * difference;
        }
        if (cand == 0 || error < best_error) {
            best_error = error;
            best_scale = scale;
        }
    }
    *scale_out = f2h(best_scale);
    for (int i = 0; i < 64; i += 8) {
        uint32_t word = 0;
        for (int j = 0; j < 8; ++j) {
            const float code = rmin(rmax(rintf(v[i + j] / best_scale), -7.0f), 7.0f);
            word |= (static_cast<uint32_t>(static_cast<int>(code)) & 15u) << (4 * j);
        }
        *reinterpret_cast<uint32_t *>(codes + i / 2) = word;
    }
}

// int4_pack.cplus:275-320, scheme 5.
__device__ void quantize_affine(const float *v, int clip, uint8_t *codes, uint16_t *scale_out,
                                uint16_t *minimum_out) {
#pragma clang fp contract(off)
    float low = v[0], high = v[0];
    for (int i = 1; i < 64; ++i) {
        low = rmin(low, v[i]);
        high = rmax(high, v[i]);
    }
    float best_error = 0.0f, best_scale = 0.0f, best_minimum = 0.0f;
    const int candidates = clip ? 7 : 1;
    for (int cand = 0; cand < candidates; ++cand) {
        const float center = (high + low) * 0.5f;
        const float half_range = (high - low) * kAffineHalf[cand];
        const float minimum = half_round(center - half_range);
        const float scale = half_round(rmax((center + half_range - minimum) / 15.0f, kScaleFloor));
        float error = 0.0f;
        for (int i = 0; i < 64; ++i) {
            const float code = rmin(rmax(rintf((v[i] - minimum) / scale), 0.0f), 15.0f);
            const float difference = code * scale + minimum - v[i];
            error = error + difference * difference;
        }
        if (cand == 0 || error < best_error) {
            best_error = error;
            best_scale = scale;
            best_minimum = minimum;
        }
    }
    *scale_out = f2h(best_scale);
    *minimum_out = f2h(best_minimum);
    for (int i = 0; i < 64; i += 8) {
        uint32_t word = 0;
        for (int j = 0; j < 8; ++j) {
            const float code = rmin(rmax(rintf((v[i + j] - best_minimum) / best_scale), 0.0f), 15.0f);
            word |= static_cast<uint32_t>(code) << (4 * j);
        }
        *reinterpret_cast<uint32_t *>(codes + i / 2) = word;
    }
}

__device__ __forceinline__ void butterfly4(float &a, float &b, float &c, float &d) {
    const float x0 = a, x1 = b, x2 = c, x3 = d;
    a = (x0 + x1 + x2 - x3) * 0.5f;
    b = (x0 + x1 - x2 + x3) * 0.5f;
    c = (x0 - x1 + x2 + x3) * 0.5f;
    d = (-x0 + x1 + x2 + x3) * 0.5f;
}

__global__ __launch_bounds__(256) void pack_kernel(const uint16_t *__restrict__ w, uint8_t *__restrict__ codes,
                                                   uint16_t *__restrict__ scales, uint16_t *__restrict__ minimums,
                                                   long long total_groups, int scheme, int clip) {
    __shared__ float lds[PACK_GROUPS * PITCH];
    const long long first = static_cast<long long>(blockIdx.x) * PACK_GROUPS;
    const int tid = threadIdx.x;

    // Stage 256 groups (16384 fp16, 4 per thread per step, coalesced).
    for (int e = tid * 4; e < PACK_GROUPS * 64; e += 256 * 4) {
        const int gl = e >> 6, off = e & 63;
        float f[4] = {0.f, 0.f, 0.f, 0.f};
        if (first + gl < total_groups) {
            const uint2 t = *reinterpret_cast<const uint2 *>(w + (first + gl) * 64 + off);
            f[0] = h2f(static_cast<uint16_t>(t.x & 0xFFFFu));
            f[1] = h2f(static_cast<uint16_t>(t.x >> 16));
            f[2] = h2f(static_cast<uint16_t>(t.y & 0xFFFFu));
            f[3] = h2f(static_cast<uint16_t>(t.y >> 16));
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) lds[gl * PITCH + off + j] = f[j];
    }
    __syncthreads();

    if (scheme == 6) {
        // 64 chunks of 256; wave w rotates chunks w, w+4, ... (16 each).  The
        // chunk boundaries are 4-group aligned because G % 4 == 0.
        const int lane = tid & 63, wave = tid >> 6;
        for (int c = wave; c < PACK_GROUPS / 4; c += 4) {
            float *chunk = lds + c * 4 * PITCH;
#pragma unroll
            for (int stride = 1; stride < 256; stride *= 4) {
                const int i0 = (lane / stride) * (stride * 4) + (lane % stride);
                float a = lds_at(chunk, i0), b = lds_at(chunk, i0 + stride), cc = lds_at(chunk, i0 + 2 * stride),
                      d = lds_at(chunk, i0 + 3 * stride);
                butterfly4(a, b, cc, d);
                lds_set(chunk, i0, a);
                lds_set(chunk, i0 + stride, b);
                lds_set(chunk, i0 + 2 * stride, cc);
                lds_set(chunk, i0 + 3 * stride, d);
                __syncthreads();
            }
        }
    }

    const long long group = first + tid;
    if (group >= total_groups) return;
    float v[64];
#pragma unroll
    for (int i = 0; i < 64; ++i) v[i] = lds[tid * PITCH + i];
    if (scheme == 6)
        quantize_symmetric(v, clip, codes + group * 32, scales + group);
    else
        quantize_affine(v, clip, codes + group * 32, scales + group, minimums + group);
}

}  // namespace qi

using namespace qi;

QI_API int qi_hip_pack_weights(const void *w_half, void *codes, void *scales, void *minimums, int n, int k, int scheme,
                               int clip, void *stream) {
    if (n <= 0 || k <= 0 || !w_half || !codes || !scales) return kInvalid;
    if (scheme != 5 && scheme != 6) return kInvalid;
    if (scheme == 5 && (!minimums || k % GROUP)) return kInvalid;
    if (scheme == 6 && k % 256) return kInvalid;
    if (reinterpret_cast<uintptr_t>(w_half) % 8 || reinterpret_cast<uintptr_t>(codes) % 4 ||
        reinterpret_cast<uintptr_t>(scales) % 2 || (minimums && reinterpret_cast<uintptr_t>(minimums) % 2))
        return kInvalid;
    const long long total = static_cast<long long>(n) * (k / GROUP);
    const long long blocks = (total + PACK_GROUPS - 1) / PACK_GROUPS;
    if (blocks > 0x7FFFFFFFLL) return kInvalid;
    pack_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream_of(stream)>>>(
        static_cast<const uint16_t *>(w_half), static_cast<uint8_t *>(codes), static_cast<uint16_t *>(scales),
        static_cast<uint16_t *>(minimums), total, scheme, clip ? 1 : 0);
    return launch_status();
}
