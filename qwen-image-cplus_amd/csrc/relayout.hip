// One-time re-layout of QIPACK INT4 weights into MFMA-tile order, and its
// inverse.  The QIPACK arrays (int4_pack.cplus:6-15, record layout
// :476-518) are row-major codes [N, K/2], scales [N, G], minimums [N, G].
//
// The tiled order groups, for every 16-row tile t and every 64-group g, the
// 512 code bytes that one wavefront feeds to one MFMA K-step: lane l's eight
// bytes are contiguous, so a wave reads a whole (t, g) tile with one
// coalesced 8-byte load per lane, and consecutive groups of a tile are
// consecutive 512-byte blocks.  Which eight bytes a lane owns depends on the
// MFMA it feeds (see qwen_image_hip.h).  Scales follow the same (t, g) order
// so a lane's scale sits next to its neighbours'.

#include "qi_common.h"

namespace qi {

__global__ void relayout_w4a4_codes(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int n, int k,
                                    int inverse) {
    const int groups = k / GROUP;
    const long long total = static_cast<long long>(n / 16) * groups * WAVE;
    for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int lane = static_cast<int>(i % WAVE);
        const long long tg = i / WAVE;
        const int g = static_cast<int>(tg % groups);
        const long long t = tg / groups;
        const long long row = t * 16 + (lane & 15);
        const long long q = lane >> 4;
        const long long s = row * (k / 2) + g * 32 + 8 * q;
        const long long d = i * 8;
        if (inverse)
            *reinterpret_cast<uint2 *>(dst + s) = *reinterpret_cast<const uint2 *>(src + d);
        else
            *reinterpret_cast<uint2 *>(dst + d) = *reinterpret_cast<const uint2 *>(src + s);
    }
}

__global__ void relayout_w4a16_codes(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int n, int k,
                                     int inverse) {
    const int groups = k / GROUP;
    const long long total = static_cast<long long>(n / 16) * groups * WAVE;
    for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int lane = static_cast<int>(i % WAVE);
        const long long tg = i / WAVE;
        const int g = static_cast<int>(tg % groups);
        const long long t = tg / groups;
        const long long row = t * 16 + (lane & 15);
        const long long q = lane >> 4;
        const long long s0 = row * (k / 2) + g * 32 + 4 * q;  // k in [8q, 8q+8)
        const long long s1 = s0 + 16;                         // k in [32+8q, 32+8q+8)
        const long long d = i * 8;
        // Within each dword the nibbles are also permuted (w4a16_permute_nibbles)
        // so the kernels unpack element pairs with one shift-and-mask.
        if (inverse) {
            *reinterpret_cast<uint32_t *>(dst + s0) =
                w4a16_unpermute_nibbles(*reinterpret_cast<const uint32_t *>(src + d));
            *reinterpret_cast<uint32_t *>(dst + s1) =
                w4a16_unpermute_nibbles(*reinterpret_cast<const uint32_t *>(src + d + 4));
        } else {
            *reinterpret_cast<uint32_t *>(dst + d) = w4a16_permute_nibbles(*reinterpret_cast<const uint32_t *>(src + s0));
            *reinterpret_cast<uint32_t *>(dst + d + 4) =
                w4a16_permute_nibbles(*reinterpret_cast<const uint32_t *>(src + s1));
        }
    }
}

// Scales (and for W4A16 the minimums, interleaved as (scale, minimum)).
__global__ void relayout_scales(const uint16_t *__restrict__ scales, const uint16_t *__restrict__ minimums,
                                uint16_t *__restrict__ tiled, int n, int k, int inverse,
                                uint16_t *__restrict__ out_scales, uint16_t *__restrict__ out_minimums) {
    const int groups = k / GROUP;
    const long long total = static_cast<long long>(n) * groups;
    const int pair = minimums || out_minimums ? 2 : 1;
    for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<long long>(gridDim.x) * blockDim.x) {
        // i enumerates the tiled order (t, g, c).
        const int c = static_cast<int>(i % 16);
        const long long tg = i / 16;
        const int g = static_cast<int>(tg % groups);
        const long long t = tg / groups;
        const long long s = (t * 16 + c) * groups + g;
        if (inverse) {
            out_scales[s] = tiled[i * pair];
            if (pair == 2) out_minimums[s] = tiled[i * pair + 1];
        } else {
            tiled[i * pair] = scales[s];
            if (pair == 2) tiled[i * pair + 1] = minimums[s];
        }
    }
}

// W4A4 weights as fp6 MFMA operands, the layout the activation quantiser
// writes: per 32-row tile T and group g, half 0 (64 lanes x 16 bytes) then
// half 1 (64 lanes x 12 bytes); lane l of half h holds the E2M3 codes of
// inputs 32 * (l / 32) + 16h .. + 15 of row 32T + l % 32, and bytes 12..15 of
// a half-0 slot hold that row's fp16 scale, zero-extended.  One thread per
// lane slot.
__global__ void relayout_w4a4_fp6_codes(const uint8_t *__restrict__ src, const uint16_t *__restrict__ scales,
                                        uint8_t *__restrict__ dst, int n, int k) {
    const int groups = k / GROUP;
    const long long total = static_cast<long long>(n / 32) * groups * 2 * WAVE;
    for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int lane = static_cast<int>(i % WAVE);
        const int half = static_cast<int>((i / WAVE) & 1);
        const long long tg = i / (2 * WAVE);
        const int g = static_cast<int>(tg % groups);
        const long long t = tg / groups;
        const long long row = t * 32 + (lane & 31);
        const int first = 32 * (lane >> 5) + 16 * half;  // input within the group
        const uint2 w = *reinterpret_cast<const uint2 *>(src + row * (k / 2) + g * 32 + first / 2);
        uint32_t out[3] = {0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const uint32_t word = e < 8 ? w.x : w.y;
            const int nib = static_cast<int>((word >> (4 * (e & 7))) & 15u);
            const uint32_t v = int4_to_e2m3(nib >= 8 ? nib - 16 : nib);
            const int bit = 6 * e;
            out[bit >> 5] |= v << (bit & 31);
            if ((bit & 31) > 26) out[(bit >> 5) + 1] |= v >> (32 - (bit & 31));
        }
        uint8_t *d = dst + tg * FP6_BLOCK + (half ? FP6_HALF0 + lane * 12 : lane * 16);
        *reinterpret_cast<uint32_t *>(d) = out[0];
        *reinterpret_cast<uint32_t *>(d + 4) = out[1];
        *reinterpret_cast<uint32_t *>(d + 8) = out[2];
        if (!half) *reinterpret_cast<uint32_t *>(d + 12) = scales[row * groups + g];
    }
}

// W4A4 fp6-path weight scales: [N/32][G][32] (tile, group, row).
__global__ void relayout_fp6_weight_scales(const uint16_t *__restrict__ scales, uint16_t *__restrict__ tiled, int n,
                                           int k) {
    const int groups = k / GROUP;
    const long long total = static_cast<long long>(n) * groups;
    for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int r = static_cast<int>(i % 32);
        const long long tg = i / 32;
        const int g = static_cast<int>(tg % groups);
        const long long t = tg / groups;
        tiled[i] = scales[(t * 32 + r) * groups + g];
    }
}

static unsigned grid_for(long long work, int block) {
    long long b = (work + block - 1) / block;
    if (b > 65536LL * 8) b = 65536LL * 8;
    if (b < 1) b = 1;
    return static_cast<unsigned>(b);
}

static bool aligned(const void *p, int bytes) { return reinterpret_cast<uintptr_t>(p) % bytes == 0; }

}  // namespace qi

using namespace qi;

QI_API int qi_hip_relayout_w4a4(const void *codes, const void *scales, void *tiled_codes, void *tiled_scales, int n,
                                int k, void *stream) {
    if (n <= 0 || k <= 0 || n % 16 || k % 256 || !codes || !scales || !tiled_codes || !tiled_scales) return kInvalid;
    if (!aligned(codes, 8) || !aligned(tiled_codes, 8) || !aligned(scales, 2) || !aligned(tiled_scales, 2))
        return kInvalid;
    hipStream_t s = stream_of(stream);
    const long long lanes = static_cast<long long>(n / 16) * (k / GROUP) * WAVE;
    relayout_w4a4_codes<<<grid_for(lanes, 256), 256, 0, s>>>(static_cast<const uint8_t *>(codes),
                                                              static_cast<uint8_t *>(tiled_codes), n, k, 0);
    relayout_scales<<<grid_for(static_cast<long long>(n) * (k / GROUP), 256), 256, 0, s>>>(
        static_cast<const uint16_t *>(scales), nullptr, static_cast<uint16_t *>(tiled_scales), n, k, 0, nullptr,
        nullptr);
    return launch_status();
}

QI_API int qi_hip_relayout_w4a4_inverse(const void *tiled_codes, const void *tiled_scales, void *codes, void *scales,
                                        int n, int k, void *stream) {
    if (n <= 0 || k <= 0 || n % 16 || k % 256 || !codes || !scales || !tiled_codes || !tiled_scales) return kInvalid;
    if (!aligned(codes, 8) || !aligned(tiled_codes, 8) || !aligned(scales, 2) || !aligned(tiled_scales, 2))
        return kInvalid;
    hipStream_t s = stream_of(stream);
    const long long lanes = static_cast<long long>(n / 16) * (k / GROUP) * WAVE;
    relayout_w4a4_codes<<<grid_for(lanes, 256), 256, 0, s>>>(static_cast<const uint8_t *>(tiled_codes),
                                                              static_cast<uint8_t *>(codes), n, k, 1);
    relayout_scales<<<grid_for(static_cast<long long>(n) * (k / GROUP), 256), 256, 0, s>>>(
        nullptr, nullptr, const_cast<uint16_t *>(static_cast<const uint16_t *>(tiled_scales)), n, k, 1,
        static_cast<uint16_t *>(scales), nullptr);
    return launch_status();
}

QI_API int qi_hip_relayout_w4a16(const void *codes, const void *scales, const void *minimums, void *tiled_codes,
                                 void *tiled_scales, int n, int k, void *stream) {
    if (n <= 0 || k <= 0 || n % 16 || k % 64 || !codes || !scales || !minimums || !tiled_codes || !tiled_scales)
        return kInvalid;
    if (!aligned(codes, 4) || !aligned(tiled_codes, 8) || !aligned(scales, 2) || !aligned(minimums, 2) ||
        !aligned(tiled_scales, 4))
        return kInvalid;
    hipStream_t s = stream_of(stream);
    const long long lanes = static_cast<long long>(n / 16) * (k / GROUP) * WAVE;
    relayout_w4a16_codes<<<grid_for(lanes, 256), 256, 0, s>>>(static_cast<const uint8_t *>(codes),
                                                               static_cast<uint8_t *>(tiled_codes), n, k, 0);
    relayout_scales<<<grid_for(static_cast<long long>(n) * (k / GROUP), 256), 256, 0, s>>>(
        static_cast<const uint16_t *>(scales), static_cast<const uint16_t *>(minimums),
        static_cast<uint16_t *>(tiled_scales), n, k, 0, nullptr, nullptr);
    return launch_status();
}

QI_API int qi_hip_relayout_w4a16_inverse(const void *tiled_codes, const void *tiled_scales, void *codes,
                                         void *scales, void *minimums, int n, int k, void *stream) {
    if (n <= 0 || k <= 0 || n % 16 || k % 64 || !codes || !scales || !minimums || !tiled_codes || !tiled_scales)
        return kInvalid;
    if (!aligned(codes, 4) || !aligned(tiled_codes, 8) || !aligned(scales, 2) || !aligned(minimums, 2) ||
        !aligned(tiled_scales, 4))
        return kInvalid;
    hipStream_t s = stream_of(stream);
    const long long lanes = static_cast<long long>(n / 16) * (k / GROUP) * WAVE;
    relayout_w4a16_codes<<<grid_for(lanes, 256), 256, 0, s>>>(static_cast<const uint8_t *>(tiled_codes),
                                                               static_cast<uint8_t *>(codes), n, k, 1);
    relayout_scales<<<grid_for(static_cast<long long>(n) * (k / GROUP), 256), 256, 0, s>>>(
        nullptr, nullptr, const_cast<uint16_t *>(static_cast<const uint16_t *>(tiled_scales)), n, k, 1,
        static_cast<uint16_t *>(scales), static_cast<uint16_t *>(minimums));
    return launch_status();
}

QI_API int qi_hip_relayout_w4a4_fp6(const void *codes, const void *scales, void *codes6, void *tiled_scales, int n,
                                    int k, void *stream) {
    if (n <= 0 || k <= 0 || n % 32 || k % 256 || !codes || !scales || !codes6) return kInvalid;
    if (!aligned(codes, 8) || !aligned(codes6, 4) || !aligned(scales, 2) || !aligned(tiled_scales, 2)) return kInvalid;
    hipStream_t s = stream_of(stream);
    const long long slots = static_cast<long long>(n / 32) * (k / GROUP) * 2 * WAVE;
    relayout_w4a4_fp6_codes<<<grid_for(slots, 256), 256, 0, s>>>(
        static_cast<const uint8_t *>(codes), static_cast<const uint16_t *>(scales), static_cast<uint8_t *>(codes6), n, k);
    if (tiled_scales)  // optional: the GEMM reads the scales from codes6
        relayout_fp6_weight_scales<<<grid_for(static_cast<long long>(n) * (k / GROUP), 256), 256, 0, s>>>(
        static_cast<const uint16_t *>(scales), static_cast<uint16_t *>(tiled_scales), n, k);
    return launch_status();
}
