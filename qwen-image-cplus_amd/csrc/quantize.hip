// W4A4 activation quantiser (H256 rotation + per-64 absmax int4) and the
// f32 -> f16 conversion used by the W4A16 path.
//
// Reference arithmetic: qwen_image_cuda/cuda/gemm.cu:22-52
// (quantize_activations_kernel); fp16-input twin
// qwen_image_cuda/cuda/bench/bench_w4a4.cu:30-66; conversion ops.cu:204-212.
//
// Design.  The H256 rotation and the 64-groups never cross a 256-element
// chunk, so a chunk is the unit of work: one wavefront owns one chunk, each
// lane four consecutive elements (one 16-byte load).  The first butterfly
// stage (stride 1) runs in registers; strides 4, 16 and 64 go through a
// 1 KiB wave-private LDS slice.  Lanes 16g..16g+15 then hold group g, reduce
// its absmax with 16-lane shuffles, and each lane writes two code bytes.  A
// row of any length is just more chunks, so there is no per-row LDS limit
// and the grid has m * k / 256 wavefronts to spread over the 256 CUs.

#include "qi_common.h"

namespace qi {

constexpr int QUANT_WAVES = 4;  // chunks per workgroup

// The butterfly of int4_pack.cplus:263-266 / gemm.cu:33-36 in its exact
// fp32 operation order (left-to-right sums, then * 0.5).
__device__ __forceinline__ void butterfly4(float &a, float &b, float &c, float &d) {
    const float x0 = a, x1 = b, x2 = c, x3 = d;
    a = (x0 + x1 + x2 - x3) * 0.5f;
    b = (x0 + x1 - x2 + x3) * 0.5f;
    c = (x0 - x1 + x2 + x3) * 0.5f;
    d = (-x0 + x1 + x2 + x3) * 0.5f;
}

template <typename In>
__device__ __forceinline__ void load4(const In *src, float v[4]);

template <>
__device__ __forceinline__ void load4<float>(const float *src, float v[4]) {
    const float4 t = *reinterpret_cast<const float4 *>(src);
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
}

template <>
__device__ __forceinline__ void load4<uint16_t>(const uint16_t *src, float v[4]) {
    const uint2 t = *reinterpret_cast<const uint2 *>(src);
    v[0] = h2f(static_cast<uint16_t>(t.x & 0xFFFFu));
    v[1] = h2f(static_cast<uint16_t>(t.x >> 16));
    v[2] = h2f(static_cast<uint16_t>(t.y & 0xFFFFu));
    v[3] = h2f(static_cast<uint16_t>(t.y >> 16));
}

// FMT 0: QIPACK activation layout (codes [m, k/2] nibbles, scales [m, k/64]).
// FMT 1: fp6 MFMA-operand layout: per 32-row tile T and group g, 1536 bytes
//        = 2 halves x 64 lanes x 12 bytes; lane l of half h holds the E2M3
//        codes (6 bits each, little-endian) of inputs 32 * (l / 32) + 16h ..
//        + 15 of the group, row 32T + l % 32.  Scales [m/32][G][32] fp16.
template <typename In, int FMT>
__global__ __launch_bounds__(QUANT_WAVES * WAVE) void quantize_chunks_kernel(
    const In *__restrict__ x, uint8_t *__restrict__ codes, uint16_t *__restrict__ scales, long long chunks,
    int chunks_per_row) {
    __shared__ float lds[QUANT_WAVES][256];
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = threadIdx.x >> 6;
    const long long chunk = static_cast<long long>(blockIdx.x) * QUANT_WAVES + wave;
    const bool active = chunk < chunks;
    float *row = lds[wave];

    // Chunk c covers elements [256c, 256c + 256) of the flattened [m, k]
    // array (k % 256 == 0, so chunks never straddle rows).
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (active) load4<In>(x + chunk * 256 + lane * 4, v);
    butterfly4(v[0], v[1], v[2], v[3]);  // stride 1: in registers
    row[lane * 4 + 0] = v[0];
    row[lane * 4 + 1] = v[1];
    row[lane * 4 + 2] = v[2];
    row[lane * 4 + 3] = v[3];
    __syncthreads();
#pragma unroll
    for (int stride = 4; stride < 256; stride *= 4) {
        // Lane b owns butterfly b of this stage.
        const int i0 = (lane / stride) * (stride * 4) + (lane % stride);
        float a = row[i0], b = row[i0 + stride], c = row[i0 + 2 * stride], d = row[i0 + 3 * stride];
        butterfly4(a, b, c, d);
        // A stage's butterflies partition the chunk, so a lane rewrites only
        // the four elements it just read; the barrier orders the stages.
        row[i0] = a;
        row[i0 + stride] = b;
        row[i0 + 2 * stride] = c;
        row[i0 + 3 * stride] = d;
        __syncthreads();
    }
    v[0] = row[lane * 4 + 0];
    v[1] = row[lane * 4 + 1];
    v[2] = row[lane * 4 + 2];
    v[3] = row[lane * 4 + 3];

    // Group g of the chunk = lanes 16g .. 16g+15.  absmax is order-free.
    float peak = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
    for (int s = 8; s > 0; s >>= 1) peak = fmaxf(peak, __shfl_xor(peak, s, 64));
    // gemm.cu:45-48: IEEE division by 7, fp16 RNE scale, IEEE v / scale,
    // rint (nearest even), clamp to [-7, 7].
    const uint16_t scale_bits = f2h(fmaxf(peak / 7.0f, 5.9604645e-08f));
    const float scale = h2f(scale_bits);
    int c[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) c[j] = static_cast<int>(fminf(fmaxf(rintf(v[j] / scale), -7.0f), 7.0f));
    if (active) {
        if (FMT == 0) {
            const uint16_t packed = static_cast<uint16_t>((c[0] & 0xF) | ((c[1] & 0xF) << 4) | ((c[2] & 0xF) << 8) |
                                                          ((c[3] & 0xF) << 12));
            reinterpret_cast<uint16_t *>(codes)[chunk * 64 + lane] = packed;
            if ((lane & 15) == 0) scales[chunk * 4 + (lane >> 4)] = scale_bits;
        } else {
            // This lane's four inputs are 4p..4p+3 of slice q of group g
            // (inputs 16q..16q+15).  Slice q goes to half q & 1 of the
            // (32-row tile, group) block, lane slot 32 * (q >> 1) + row % 32,
            // whose 12 bytes are the 24-bit runs of lanes p = 0..3: lane p
            // < 3 assembles and stores dword p.
            const long long row = chunk / chunks_per_row;
            const int groups = chunks_per_row * 4;
            const int g = static_cast<int>(chunk % chunks_per_row) * 4 + (lane >> 4);
            const int q = (lane & 15) >> 2, p = lane & 3;
            const uint32_t bits = int4_to_e2m3(c[0]) | (int4_to_e2m3(c[1]) << 6) | (int4_to_e2m3(c[2]) << 12) |
                                  (int4_to_e2m3(c[3]) << 18);
            const uint32_t next = static_cast<uint32_t>(__shfl_down(static_cast<int>(bits), 1, 64));
            const long long block = (row >> 5) * groups + g;
            const int r32 = static_cast<int>(row & 31);
            if (p < 3) {
                const uint32_t word = (bits >> (8 * p)) | (next << (24 - 8 * p));
                uint32_t *dst = reinterpret_cast<uint32_t *>(codes + block * 1536 + (q & 1) * 768 +
                                                             ((q >> 1) * 32 + r32) * 12);
                dst[p] = word;
            }
            if ((lane & 15) == 0) scales[block * 32 + r32] = scale_bits;
        }
    }
}

__global__ void f32_to_f16_kernel(const float *__restrict__ src, uint16_t *__restrict__ out,
                                  unsigned long long count) {
    const unsigned long long stride = static_cast<unsigned long long>(gridDim.x) * blockDim.x * 4;
    for (unsigned long long i = (static_cast<unsigned long long>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
         i < count; i += stride) {
        if (i + 4 <= count && ((reinterpret_cast<uintptr_t>(src + i) & 15) == 0) &&
            ((reinterpret_cast<uintptr_t>(out + i) & 7) == 0)) {
            const float4 t = *reinterpret_cast<const float4 *>(src + i);
            uint2 o;
            o.x = static_cast<uint32_t>(f2h(t.x)) | (static_cast<uint32_t>(f2h(t.y)) << 16);
            o.y = static_cast<uint32_t>(f2h(t.z)) | (static_cast<uint32_t>(f2h(t.w)) << 16);
            *reinterpret_cast<uint2 *>(out + i) = o;
        } else {
            for (unsigned long long j = i; j < i + 4 && j < count; ++j) out[j] = f2h(src[j]);
        }
    }
}

template <typename In, int FMT>
static int launch_quantize(const In *x, void *codes, void *scales, int m, int k, hipStream_t stream) {
    if (m < 0 || k <= 0 || k % 256 != 0 || (m > 0 && (!x || !codes || !scales))) return kInvalid;
    if (m == 0) return 0;
    // Vector loads: 4 elements per lane; 2-byte (QIPACK) or 4-byte (fp6) code stores.
    if (reinterpret_cast<uintptr_t>(x) % (4 * sizeof(In)) != 0 ||
        reinterpret_cast<uintptr_t>(codes) % (FMT == 0 ? 2 : 4) != 0 ||
        reinterpret_cast<uintptr_t>(scales) % 2 != 0)
        return kInvalid;
    const long long chunks = static_cast<long long>(m) * (k / 256);
    const long long blocks = (chunks + QUANT_WAVES - 1) / QUANT_WAVES;
    if (blocks > 0x7FFFFFFFLL) return kInvalid;
    quantize_chunks_kernel<In, FMT><<<dim3(static_cast<unsigned>(blocks)), dim3(QUANT_WAVES * WAVE), 0, stream>>>(
        x, static_cast<uint8_t *>(codes), static_cast<uint16_t *>(scales), chunks, k / 256);
    return launch_status();
}

static int launch_f32_to_f16(const float *src, void *out, unsigned long long count, hipStream_t stream) {
    if (count == 0) return 0;
    if (!src || !out) return kInvalid;
    unsigned long long threads = (count + 3) / 4;
    unsigned long long blocks = (threads + 255) / 256;
    if (blocks > 65536ull * 16) blocks = 65536ull * 16;
    f32_to_f16_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream>>>(
        src, static_cast<uint16_t *>(out), count);
    return launch_status();
}

}  // namespace qi

QI_API int qi_hip_abi_version(void) { return QI_HIP_ABI_VERSION; }

QI_API int qi_w4a4_quantize_activations(const float *x, void *codes, void *scales, int m, int k) {
    return qi::launch_quantize<float, 0>(x, codes, scales, m, k, nullptr);
}

QI_API int qi_hip_w4a4_quantize_activations(const float *x, void *codes, void *scales, int m, int k,
                                            void *stream) {
    return qi::launch_quantize<float, 0>(x, codes, scales, m, k, qi::stream_of(stream));
}

QI_API int qi_hip_w4a4_quantize_activations_f16(const void *x_half, void *codes, void *scales, int m, int k,
                                                void *stream) {
    return qi::launch_quantize<uint16_t, 0>(static_cast<const uint16_t *>(x_half), codes, scales, m, k,
                                            qi::stream_of(stream));
}

QI_API int qi_hip_w4a4_quantize_activations_fp6(const void *x, int x_is_half, void *codes6, void *scales_tiled, int m,
                                                int k, void *stream) {
    if (x_is_half)
        return qi::launch_quantize<uint16_t, 1>(static_cast<const uint16_t *>(x), codes6, scales_tiled, m, k,
                                                qi::stream_of(stream));
    return qi::launch_quantize<float, 1>(static_cast<const float *>(x), codes6, scales_tiled, m, k,
                                         qi::stream_of(stream));
}

QI_API int qi_f32_to_f16(const float *source, void *out, unsigned long long count) {
    return qi::launch_f32_to_f16(source, out, count, nullptr);
}

QI_API int qi_hip_f32_to_f16(const float *source, void *out, unsigned long long count, void *stream) {
    return qi::launch_f32_to_f16(source, out, count, qi::stream_of(stream));
}
