// W4A4 activation quantiser (H256 rotation + per-64 absmax int4) and the
// f32 -> f16 conversion used by the W4A16 path.
//
// Reference arithmetic: qwen_image_cuda/cuda/gemm.cu:22-52
// (quantize_activations_kernel); fp16-input twin
// qwen_image_cuda/cuda/bench/bench_w4a4.cu:30-66; conversion ops.cu:204-212.
//
// Design.  The H256 rotation and the 64-groups never cross a 256-element
// chunk, so a chunk is the unit of work: one wavefront owns one chunk, each
// lane four consecutive elements (one 8- or 16-byte load).  The first
// butterfly stage (stride 1) runs in registers; strides 4, 16 and 64 go
// through a 1 KiB wave-private, bank-swizzled LDS slice without barriers.
// Lanes 16g..16g+15 then hold group g and reduce its absmax with 16-lane
// shuffles.  A row of any length is just more chunks, so there is no per-row
// LDS limit, and the grid has m * k / 256 wavefronts to spread over the CUs.

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "qi_common.h"

namespace qi {

constexpr int QUANT_WAVES = 4;  // chunks per workgroup

// The butterfly of int4_pack.cplus:263-266 / gemm.cu:33-36 in its exact
// fp32 operation order (left-to-right sums, then * 0.5).  HALF = false
// leaves out the * 0.5: scaling by a power of two commutes with every
// rounding of the sums as long as no value overflows or turns subnormal, so
// the four stages' factors can be applied once, as 1/16, where the values are
// used.  That holds for fp16 inputs (every intermediate is a multiple of
// 2^-28 and below 2^25); fp32 inputs keep the factor per stage.
template <bool HALF>
__device__ __forceinline__ void butterfly4(float &a, float &b, float &c, float &d) {
    const float x0 = a, x1 = b, x2 = c, x3 = d;
    const float f = HALF ? 0.5f : 1.0f;
    a = (x0 + x1 + x2 - x3) * f;
    b = (x0 + x1 - x2 + x3) * f;
    c = (x0 - x1 + x2 + x3) * f;
    d = (-x0 + x1 + x2 + x3) * f;
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

// v from another lane of the same 16-lane row, by a DPP control word.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}

// LDS word of element i of a chunk: an XOR swizzle that makes every access
// pattern below (4 consecutive words per lane, and the strided butterfly
// quadruples of strides 4, 16, 64) conflict-free for 32 lanes at a time.
__device__ __forceinline__ int swz(int i) { return i ^ ((i >> 2) & 31); }

// E2M3 code of the int4 value q: |q| 0..7 -> 0, 8, 16, 20, 24, 26, 28, 30,
// i.e. twice the nibble |q| of 0xFEDCA840, plus the sign bit 32.
__device__ __forceinline__ uint32_t e2m3_of(int q) {
    const uint32_t a = static_cast<uint32_t>(q < 0 ? -q : q);
    return (__builtin_amdgcn_ubfe(0xFEDCA840u, 4 * a, 4) << 1) | (q < 0 ? 32u : 0u);
}

// One 256-element chunk held by a wave, lane l owning elements 4l .. 4l+3
// (v, in place): the H256 rotation in the reference's exact fp32 operation
// order, then the group absmax, fp16 scale and int4 codes.  Lanes 16g ..
// 16g+15 hold group g of the chunk; every lane of a group gets its scale.
// buf is the wave's private 256-float LDS slice.
template <typename In>
__device__ __forceinline__ void quantize_chunk(float (&v)[4], float *buf, int lane, int (&q)[4],
                                               uint16_t &scale_bits) {
    // In = uint16_t: the values are fp16 inputs (see butterfly4); any other
    // type: arbitrary fp32 values.
    constexpr bool HALF = !__is_same(In, uint16_t);  // see butterfly4
    butterfly4<HALF>(v[0], v[1], v[2], v[3]);  // stride 1: in registers
#pragma unroll
    for (int j = 0; j < 4; ++j) buf[swz(lane * 4 + j)] = v[j];
    // The chunk belongs to this wave alone, and a wave's LDS accesses execute
    // in order, so the stages need no barrier -- only a compiler fence.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int stride = 4; stride < 256; stride *= 4) {
        // Lane b owns butterfly b of this stage.
        const int i0 = (lane / stride) * (stride * 4) + (lane % stride);
        float a = buf[swz(i0)], b = buf[swz(i0 + stride)], cc = buf[swz(i0 + 2 * stride)],
              d = buf[swz(i0 + 3 * stride)];
        butterfly4<HALF>(a, b, cc, d);
        // A stage's butterflies partition the chunk, so a lane rewrites only
        // the four elements it just read.
        buf[swz(i0)] = a;
        buf[swz(i0 + stride)] = b;
        buf[swz(i0 + 2 * stride)] = cc;
        buf[swz(i0 + 3 * stride)] = d;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = buf[swz(lane * 4 + j)];
    // The next chunk's first writes must follow these reads.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();

    // The rotated values are v / unit (unit = 16 without the per-stage
    // halving, else 1; exact).  absmax is order-free.
    constexpr float unit = HALF ? 1.0f : 16.0f;
    float peak = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    // Max over the 16 lanes of the group with DPP moves (no LDS round
    // trips): lane ^ 1, lane ^ 2 within quads, then the 8-lane and 16-lane
    // mirrors pair the quads and the two halves.
    peak = fmaxf(peak, dpp_f32<0xB1>(peak));   // quad_perm [1,0,3,2]
    peak = fmaxf(peak, dpp_f32<0x4E>(peak));   // quad_perm [2,3,0,1]
    peak = fmaxf(peak, dpp_f32<0x141>(peak));  // row_half_mirror
    peak = fmaxf(peak, dpp_f32<0x140>(peak));  // row_mirror
    // gemm.cu:45-48: IEEE division by 7, fp16 RNE scale, IEEE v / scale,
    // rint (nearest even), clamp to [-7, 7].
    scale_bits = f2h(fmaxf((peak * (1.0f / unit)) / 7.0f, 5.9604645e-08f));
    // v / scale as one correctly rounded quotient per element, without a
    // division each: with y = RN(1 / d) (one IEEE division per lane), q0 =
    // RN(v y), r = v - q0 d (exact by fma) and q0 + r y rounded once give
    // RN(v / d) (Markstein's theorem) whenever the quotient is a normal
    // number; below 2^-126 both are 0 after rint, and a zero's sign does not
    // survive the conversion to int.  d = unit * scale: (v / unit) / scale
    // and v / (unit * scale) are the same real number.
    const float d = h2f(scale_bits) * unit;
    const float y = 1.0f / d;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float q0 = v[j] * y;
        const float quot = __builtin_fmaf(__builtin_fmaf(-q0, d, v[j]), y, q0);
        q[j] = static_cast<int>(fminf(fmaxf(rintf(quot), -7.0f), 7.0f));
    }
}

// QIPACK layout (FMT 0).  Grid: x = row, y = group of QUANT_WAVES * CPW
// chunks of the row.  Wave w of the workgroup owns chunks base + w +
// QUANT_WAVES * i, i < CPW (chunk c = elements [256c, 256c + 256) of the
// row); it issues all their loads first.  Each lane stores its four nibbles
// as one 2-byte word, so a wave writes 128 contiguous bytes.
template <typename In, int CPW>
__global__ __launch_bounds__(QUANT_WAVES * WAVE) void quantize_chunks_kernel(
    const In *__restrict__ x, uint8_t *__restrict__ codes, uint16_t *__restrict__ scales, int k) {
    __shared__ float lds[QUANT_WAVES][256];
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = threadIdx.x >> 6;
    const int chunks_per_row = k >> 8;
    const int c0 = blockIdx.y * QUANT_WAVES * CPW + wave;
    if (c0 >= chunks_per_row) return;  // whole wave; no workgroup barrier below
    const uint32_t row = blockIdx.x;
    float *buf = lds[wave];

    float in[CPW][4];
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
        const int c = c0 + QUANT_WAVES * i;
        if (c < chunks_per_row) load4<In>(x + static_cast<size_t>(row) * k + c * 256 + lane * 4, in[i]);
    }
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
        const int c = c0 + QUANT_WAVES * i;
        if (c >= chunks_per_row) break;
        float v[4] = {in[i][0], in[i][1], in[i][2], in[i][3]};
        int q[4];
        uint16_t scale_bits;
        quantize_chunk<In>(v, buf, lane, q, scale_bits);
        const int g = c * 4 + (lane >> 4);  // group within the row
        const uint16_t packed =
            static_cast<uint16_t>((q[0] & 0xF) | ((q[1] & 0xF) << 4) | ((q[2] & 0xF) << 8) | ((q[3] & 0xF) << 12));
        reinterpret_cast<uint16_t *>(codes)[static_cast<size_t>(row) * (k >> 2) + c * 64 + lane] = packed;
        if ((lane & 15) == 0) scales[static_cast<size_t>(row) * (k >> 6) + g] = scale_bits;
    }
}

// fp6 MFMA-operand layout (FMT 1): per 32-row tile T and group g, 1792 bytes
// = half 0 (64 lanes x 16 bytes) then half 1 (64 lanes x 12 bytes); lane l
// of half h holds the E2M3 codes (6 bits each, little-endian) of inputs
// 32 * (l / 32) + 16h .. + 15 of the group, row 32T + l % 32; bytes 12..15 of
// a half-0 slot hold that row's fp16 scale, zero-extended.  Scales also
// [m/32][G][32] fp16 when requested.
//
// Grid: x = 32-row tile, y = chunk.  A workgroup quantises the tile's 32 rows
// of one chunk -- the tile's blocks for the chunk's four groups, 7168
// contiguous bytes -- assembling them in LDS and writing them with 16-byte
// stores (one row per workgroup would scatter 4-byte stores of 32
// workgroups over every block).  Wave w takes rows w * RPW .. + RPW - 1 and
// issues all their loads first.  Rows past m quantise zeros; their codes are
// written but never used.
// No producer: the quantiser reads its input as is.
struct NoProducer {
    static constexpr bool active = false;
    __device__ void operator()(int, int, float (&)[4]) const {}
};

template <typename In, int RPW, typename Producer = NoProducer>
__global__ __launch_bounds__(32 / RPW * WAVE) void quantize_fp6_strip_kernel(
    const In *__restrict__ x, uint8_t *__restrict__ codes, uint16_t *__restrict__ scales, int m, int k,
    Producer produce = Producer{}) {
    // With a producer the values are arbitrary fp32, whatever the input type.
    using Vals = typename std::conditional<Producer::active, float, In>::type;
    constexpr int NWV = 32 / RPW;
    __shared__ float lds[NWV][256];
    __shared__ __attribute__((aligned(16))) uint32_t blocks[4 * FP6_BLOCK / 4];
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = threadIdx.x >> 6;
    const int groups = k >> 6;
    const int tile = blockIdx.x, c = blockIdx.y;
    float *buf = lds[wave];

    float in[RPW][4];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int row = tile * 32 + wave * RPW + i;
        if (row < m) {
            load4<In>(x + static_cast<size_t>(row) * k + c * 256 + lane * 4, in[i]);
            produce(row, c * 256 + lane * 4, in[i]);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) in[i][j] = 0.f;
        }
    }
    // This lane's four inputs are 4p..4p+3 of slice sl of its group (inputs
    // 16 sl .. 16 sl + 15).  Slice sl goes to half sl & 1 of the group's
    // block, lane slot 32 (sl >> 1) + row % 32, whose 12 code bytes are the
    // 24-bit runs of lanes p = 0..3: lane p < 3 assembles and stores dword
    // p.  In half 0 (16-byte slots) lane p = 3 stores the scale as dword 3.
    const int sl = (lane & 15) >> 2, p = lane & 3, gb = lane >> 4;
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        float v[4] = {in[i][0], in[i][1], in[i][2], in[i][3]};
        int q[4];
        uint16_t scale_bits;
        quantize_chunk<Vals>(v, buf, lane, q, scale_bits);
        const int r32 = wave * RPW + i;
        const uint32_t bits =
            e2m3_of(q[0]) | (e2m3_of(q[1]) << 6) | (e2m3_of(q[2]) << 12) | (e2m3_of(q[3]) << 18);
        const uint32_t next = dpp_u32<0x101>(bits);  // row_shl:1 -- lane + 1 (unused by p = 3)
        const int slot = (sl >> 1) * 32 + r32;
        uint32_t *dst = blocks + (gb * FP6_BLOCK + ((sl & 1) ? FP6_HALF0 + slot * 12 : slot * 16)) / 4;
        if (p < 3)
            dst[p] = (bits >> (8 * p)) | (next << (24 - 8 * p));
        else if ((sl & 1) == 0)
            dst[3] = scale_bits;
        if (scales && (lane & 15) == 0)
            scales[(static_cast<size_t>(tile) * groups + c * 4 + gb) * 32 + r32] = scale_bits;
    }
    __syncthreads();
    uint4 *out = reinterpret_cast<uint4 *>(codes + (static_cast<size_t>(tile) * groups + c * 4) * FP6_BLOCK);
    for (int idx = threadIdx.x; idx < 4 * FP6_BLOCK / 16; idx += NWV * WAVE)
        out[idx] = reinterpret_cast<const uint4 *>(blocks)[idx];
}

// The strip quantiser as a persistent, software-pipelined kernel (fp16
// inputs, no producer, rows >= 2048): the grid's workgroups walk the (32-row tile, chunk) items with
// stride gridDim.x, and the next item's inputs are loaded while the current
// item is quantised and stored, so the load latency hides behind the vector
// work instead of adding to it.  Same arithmetic, codes and layout as
// quantize_fp6_strip_kernel.  The LDS hand-offs use a bare barrier after an
// LDS-only wait: __syncthreads' release fence would also wait for the next
// item's loads.
template <typename In, int RPW, typename Producer = NoProducer>
__global__ __launch_bounds__(32 / RPW * WAVE) void quantize_fp6_stream_kernel(
    const In *__restrict__ x, uint8_t *__restrict__ codes, uint16_t *__restrict__ scales, int m, int k, int items,
    Producer produce = Producer{}) {
    using Vals = typename std::conditional<Producer::active, float, In>::type;
    constexpr int NWV = 32 / RPW;
    __shared__ float lds[NWV][256];
    __shared__ __attribute__((aligned(16))) uint32_t blocks[4 * FP6_BLOCK / 4];
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = threadIdx.x >> 6;
    const int groups = k >> 6, chunks = k >> 8;
    float *buf = lds[wave];
    const int sl = (lane & 15) >> 2, p = lane & 3, gb = lane >> 4;

    // Raw input words, converted where they are used: loads are
    // unconditional (rows past m read row m - 1 and are zeroed later), so
    // the compiler waits for them only at their first use.
    using Raw = typename std::conditional<__is_same(In, uint16_t), uint2, float4>::type;
    auto load = [&](int item, Raw (&dst)[RPW]) {
        const int tile = item / chunks, c = item - tile * chunks;
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const int row = min(tile * 32 + wave * RPW + i, m - 1);
            dst[i] = *reinterpret_cast<const Raw *>(x + static_cast<size_t>(row) * k + c * 256 + lane * 4);
        }
    };
    auto widen = [&](const Raw &r, float (&v)[4]) {
        if constexpr (__is_same(In, uint16_t)) {
            v[0] = h2f(static_cast<uint16_t>(r.x & 0xFFFFu));
            v[1] = h2f(static_cast<uint16_t>(r.x >> 16));
            v[2] = h2f(static_cast<uint16_t>(r.y & 0xFFFFu));
            v[3] = h2f(static_cast<uint16_t>(r.y >> 16));
        } else {
            v[0] = r.x;
            v[1] = r.y;
            v[2] = r.z;
            v[3] = r.w;
        }
    };
    // One item: quantise `cur` (item `item`) after issuing the loads of item
    // `next` into `nxt`.  Two named buffers alternate (the loop below is
    // unrolled by two), so no register copy waits for the next loads.
    auto step = [&](int item, Raw (&cur)[RPW], Raw (&nxt)[RPW]) {
        // Unconditional (the last items reload item items - 1, unused), so
        // that the waits for `cur` do not also wait for these loads.
        load(min(item + static_cast<int>(gridDim.x), items - 1), nxt);
        const int tile = item / chunks, c = item - tile * chunks;
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const int row = tile * 32 + wave * RPW + i;
            float v[4];
            widen(cur[i], v);
            if (row < m) {
                produce(row, c * 256 + lane * 4, v);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = 0.f;
            }
            int q[4];
            uint16_t scale_bits;
            quantize_chunk<Vals>(v, buf, lane, q, scale_bits);
            const int r32 = wave * RPW + i;
            const uint32_t bits =
                e2m3_of(q[0]) | (e2m3_of(q[1]) << 6) | (e2m3_of(q[2]) << 12) | (e2m3_of(q[3]) << 18);
            const uint32_t nb = dpp_u32<0x101>(bits);  // row_shl:1 -- lane + 1 (unused by p = 3)
            const int slot = (sl >> 1) * 32 + r32;
            uint32_t *dst = blocks + (gb * FP6_BLOCK + ((sl & 1) ? FP6_HALF0 + slot * 12 : slot * 16)) / 4;
            if (p < 3)
                dst[p] = (bits >> (8 * p)) | (nb << (24 - 8 * p));
            else if ((sl & 1) == 0)
                dst[3] = scale_bits;
            if (scales && (lane & 15) == 0)
                scales[(static_cast<size_t>(tile) * groups + c * 4 + gb) * 32 + r32] = scale_bits;
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        uint4 *out = reinterpret_cast<uint4 *>(codes + (static_cast<size_t>(tile) * groups + c * 4) * FP6_BLOCK);
        for (int idx = threadIdx.x; idx < 4 * FP6_BLOCK / 16; idx += NWV * WAVE)
            out[idx] = reinterpret_cast<const uint4 *>(blocks)[idx];
        // The block reads above complete before any wave rewrites blocks.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };
    int item = blockIdx.x;
    if (item >= items) return;  // whole workgroup
    Raw ra[RPW], rb[RPW];
    load(item, ra);
    for (;;) {
        step(item, ra, rb);
        item += gridDim.x;
        if (item >= items) break;
        step(item, rb, ra);
        item += gridDim.x;
        if (item >= items) break;
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

// Grid: x = 32-row tile, y = chunk.  Four rows per wave (8 waves per
// workgroup) when there are rows enough to fill the chip, else two (16
// waves).  Shapes and pointers are checked by the callers.
template <typename In, typename Producer>
static int launch_fp6_strip(const In *x, void *codes, void *scales, int m, int k, hipStream_t stream,
                            Producer produce) {
    const int chunks = k / 256;
    if (chunks > 65535) return kInvalid;
    const dim3 grid(static_cast<unsigned>((m + 31) / 32), static_cast<unsigned>(chunks));
    if (m >= 2048 && !Producer::active && __is_same(In, uint16_t)) {
        // Persistent and pipelined, for fp16 inputs without a producer
        // (measured 3-4 % faster from 4352 rows, slower at 1024; with a
        // producer, whose own loads are not pipelined, slower: LayerNorm
        // 4096 x 3072 18.8 -> 22.4 us, SwiGLU 4096 x 12288 110 -> 116).
        const long long items = static_cast<long long>((m + 31) / 32) * chunks;
        if (items > 0x7FFFFFFFLL) return kInvalid;
        const long long wgs = std::min<long long>(items, 4LL * device_cus());
        quantize_fp6_stream_kernel<In, 4, Producer><<<dim3(static_cast<unsigned>(wgs)), dim3(8 * WAVE), 0, stream>>>(
            x, static_cast<uint8_t *>(codes), static_cast<uint16_t *>(scales), m, k, static_cast<int>(items),
            produce);
    } else if (m >= 1024)
        quantize_fp6_strip_kernel<In, 4, Producer><<<grid, dim3(8 * WAVE), 0, stream>>>(
            x, static_cast<uint8_t *>(codes), static_cast<uint16_t *>(scales), m, k, produce);
    else
        quantize_fp6_strip_kernel<In, 2, Producer><<<grid, dim3(16 * WAVE), 0, stream>>>(
            x, static_cast<uint8_t *>(codes), static_cast<uint16_t *>(scales), m, k, produce);
    return launch_status();
}

template <typename In, int FMT>
static int launch_quantize(const In *x, void *codes, void *scales, int m, int k, hipStream_t stream) {
    // The fp6 layout carries the scales inside the code blocks; its separate
    // scale array is optional (null: not written).
    if (m < 0 || k <= 0 || k % 256 != 0 || (m > 0 && (!x || !codes || (FMT == 0 && !scales)))) return kInvalid;
    if (m == 0) return 0;
    // Vector loads: 4 elements per lane; 2-byte (QIPACK) or 16-byte (fp6)
    // code stores.
    if (reinterpret_cast<uintptr_t>(x) % (4 * sizeof(In)) != 0 ||
        reinterpret_cast<uintptr_t>(codes) % (FMT == 0 ? 2 : 16) != 0 ||
        reinterpret_cast<uintptr_t>(scales) % 2 != 0)
        return kInvalid;
    const int chunks = k / 256;
    if (FMT == 1) return launch_fp6_strip<In>(x, codes, scales, m, k, stream, NoProducer{});
    // Several chunks per wave when there are rows enough to fill the chip.
    if (m >= 1024) {
        constexpr int CPW = 4;
        const int chunk_groups = (chunks + QUANT_WAVES * CPW - 1) / (QUANT_WAVES * CPW);
        if (chunk_groups > 65535) return kInvalid;
        quantize_chunks_kernel<In, CPW><<<dim3(static_cast<unsigned>(m), chunk_groups), dim3(QUANT_WAVES * WAVE), 0,
                                          stream>>>(x, static_cast<uint8_t *>(codes), static_cast<uint16_t *>(scales),
                                                    k);
    } else {
        const int chunk_groups = (chunks + QUANT_WAVES - 1) / QUANT_WAVES;
        if (chunk_groups > 65535) return kInvalid;
        quantize_chunks_kernel<In, 1><<<dim3(static_cast<unsigned>(m), chunk_groups), dim3(QUANT_WAVES * WAVE), 0,
                                        stream>>>(x, static_cast<uint8_t *>(codes), static_cast<uint16_t *>(scales),
                                                  k);
    }
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


// ---------------------------------------------------------------------------
// Producers fused with the quantiser.  The reference runs each as its own
// kernel writing fp32 activations that the quantiser then reads back
// (transformer.cplus:759-760, 808-813): the affine-free LayerNorm with
// modulation scale (ops.cu:37-58) before q/k/v and the MLP, and SwiGLU
// (ops.cu:134-143) before the MLP's down projection.  Here the quantiser
// applies them to the values it loads, so the fp32 intermediate never goes
// through HBM.  The plain producer kernels below use the same device
// arithmetic, so quantising their output gives the fused codes bit for bit.
// Neither reproduces the reference's own reduction order or its CUDA
// rsqrtf / expf: their outputs agree with the formulas within a few fp32
// ulps.

constexpr float LN_EPSILON = 1e-6f;  // ops.cu:12

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) v += __shfl_xor(v, s, 64);
    return v;  // the same value in every lane (each pairwise sum is symmetric)
}

// Row statistics of ops.cu:40-50: mean, then the mean of squared deviations
// (two passes), inverse = 1 / sqrt(variance + 1e-6), correctly rounded sqrt
// and division.  One wave per row; lane l sums elements 4l + 256 i, i = 0,
// 1, ... in order, then the wave adds the lanes.  k % 4 == 0.
__device__ __forceinline__ float2 ln_row_stats(const float *__restrict__ row, int k, int lane) {
    float s = 0.f;
    for (int i = lane * 4; i < k; i += 256) {
        const float4 t = *reinterpret_cast<const float4 *>(row + i);
        s = ((s + t.x) + t.y + t.z) + t.w;
    }
    const float mean = wave_sum64(s) / static_cast<float>(k);
    float sq = 0.f;
    for (int i = lane * 4; i < k; i += 256) {
        const float4 t = *reinterpret_cast<const float4 *>(row + i);
        float d = t.x - mean;
        sq = __builtin_fmaf(d, d, sq);
        d = t.y - mean;
        sq = __builtin_fmaf(d, d, sq);
        d = t.z - mean;
        sq = __builtin_fmaf(d, d, sq);
        d = t.w - mean;
        sq = __builtin_fmaf(d, d, sq);
    }
    const float var = wave_sum64(sq) / static_cast<float>(k);
    return float2{mean, 1.0f / __builtin_sqrtf(var + LN_EPSILON)};
}

// ops.cu:52-53: (x - mean) * inverse * (1 + scale[i]), the scale row chosen
// by row < split (row 1 of the modulation, the prefix) or not (row 0).
__device__ __forceinline__ void ln_scale_apply(float2 st, const float *__restrict__ s, float (&v)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = ((v[e] - st.x) * st.y) * (1.0f + s[e]);
}

struct LnScaleProducer {
    static constexpr bool active = true;
    const float2 *stats;
    const float *scale;
    int scale_stride, split;
    __device__ void operator()(int row, int col, float (&v)[4]) const {
        ln_scale_apply(stats[row], scale + (row < split ? scale_stride : 0) + col, v);
    }
};

// ops.cu:134-139: silu(gate) * up = gate / (1 + exp(-gate)) * up.
__device__ __forceinline__ float swiglu1(float g, float u) { return g / (1.0f + expf(-g)) * u; }

struct SwigluProducer {  // the quantiser's input is the gate
    static constexpr bool active = true;
    const float *up;
    int k;
    __device__ void operator()(int row, int col, float (&v)[4]) const {
        const float4 u = *reinterpret_cast<const float4 *>(up + static_cast<size_t>(row) * k + col);
        v[0] = swiglu1(v[0], u.x);
        v[1] = swiglu1(v[1], u.y);
        v[2] = swiglu1(v[2], u.z);
        v[3] = swiglu1(v[3], u.w);
    }
};

// One wave per row: the row statistics into stats[row].
__global__ __launch_bounds__(4 * WAVE) void ln_stats_kernel(const float *__restrict__ x, float2 *__restrict__ stats,
                                                             int m, int k) {
    const int lane = threadIdx.x & (WAVE - 1), row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= m) return;
    const float2 st = ln_row_stats(x + static_cast<size_t>(row) * k, k, lane);
    if (lane == 0) stats[row] = st;
}

// The plain LayerNorm-scale (qi_layer_norm_scale), one wave per row, fp32 or
// fp16 (RNE) output.
__global__ __launch_bounds__(4 * WAVE) void layer_norm_scale_kernel(const float *__restrict__ x,
                                                                     const float *__restrict__ scale, int scale_stride,
                                                                     int split, void *__restrict__ out, int out_type,
                                                                     int m, int k) {
    const int lane = threadIdx.x & (WAVE - 1), row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= m) return;
    const float *src = x + static_cast<size_t>(row) * k;
    const float2 st = ln_row_stats(src, k, lane);
    const float *s = scale + (row < split ? scale_stride : 0);
    for (int i = lane * 4; i < k; i += 256) {
        const float4 t = *reinterpret_cast<const float4 *>(src + i);
        float v[4] = {t.x, t.y, t.z, t.w};
        ln_scale_apply(st, s + i, v);
        const size_t o = static_cast<size_t>(row) * k + i;
        if (out_type == QI_HIP_OUT_F16) {
            uint2 h;
            h.x = static_cast<uint32_t>(f2h(v[0])) | (static_cast<uint32_t>(f2h(v[1])) << 16);
            h.y = static_cast<uint32_t>(f2h(v[2])) | (static_cast<uint32_t>(f2h(v[3])) << 16);
            *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(out) + o) = h;
        } else {
            *reinterpret_cast<float4 *>(static_cast<float *>(out) + o) = float4{v[0], v[1], v[2], v[3]};
        }
    }
}

// The plain SwiGLU (qi_swiglu), four elements per thread, fp32 or fp16 out.
__global__ void swiglu_kernel(const float *__restrict__ gate, const float *__restrict__ up, void *__restrict__ out,
                              int out_type, unsigned long long count) {
    const unsigned long long stride = static_cast<unsigned long long>(gridDim.x) * blockDim.x * 4;
    for (unsigned long long i = (static_cast<unsigned long long>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
         i < count; i += stride) {
        const float4 g = *reinterpret_cast<const float4 *>(gate + i);
        const float4 u = *reinterpret_cast<const float4 *>(up + i);
        const float v[4] = {swiglu1(g.x, u.x), swiglu1(g.y, u.y), swiglu1(g.z, u.z), swiglu1(g.w, u.w)};
        if (out_type == QI_HIP_OUT_F16) {
            uint2 h;
            h.x = static_cast<uint32_t>(f2h(v[0])) | (static_cast<uint32_t>(f2h(v[1])) << 16);
            h.y = static_cast<uint32_t>(f2h(v[2])) | (static_cast<uint32_t>(f2h(v[3])) << 16);
            *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(out) + i) = h;
        } else {
            *reinterpret_cast<float4 *>(static_cast<float *>(out) + i) = float4{v[0], v[1], v[2], v[3]};
        }
    }
}

static bool aligned16(const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

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

QI_API int qi_hip_layer_norm_scale(const float *x, const float *scale, int scale_stride, void *out, int out_type,
                                   int rows, int width, int split, void *stream) {
    using namespace qi;
    if (rows < 0 || width <= 0 || width % 4 || scale_stride < 0) return kInvalid;
    if (out_type != QI_HIP_OUT_F32 && out_type != QI_HIP_OUT_F16) return kInvalid;
    if (rows == 0) return 0;
    if (!x || !scale || !out || !aligned16(x) || !aligned16(out) || !aligned16(scale) || scale_stride % 4)
        return kInvalid;
    layer_norm_scale_kernel<<<dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(4 * WAVE), 0, stream_of(stream)>>>(
        x, scale, scale_stride, split, out, out_type, rows, width);
    return launch_status();
}

QI_API int qi_hip_layer_norm_scale_quantize_fp6(const float *x, const float *scale, int scale_stride, int split,
                                                void *row_stats, void *codes6, int m, int k, void *stream) {
    using namespace qi;
    if (m < 0 || k <= 0 || k % 256 || scale_stride < 0) return kInvalid;
    if (m == 0) return 0;
    if (!x || !scale || !row_stats || !codes6 || !aligned16(x) || !aligned16(scale) || scale_stride % 4 ||
        !aligned16(codes6) || reinterpret_cast<uintptr_t>(row_stats) % 8)
        return kInvalid;
    hipStream_t s = stream_of(stream);
    ln_stats_kernel<<<dim3(static_cast<unsigned>((m + 3) / 4)), dim3(4 * WAVE), 0, s>>>(
        x, static_cast<float2 *>(row_stats), m, k);
    const int st = launch_status();
    if (st) return st;
    return launch_fp6_strip<float>(x, codes6, nullptr, m, k, s,
                                   LnScaleProducer{static_cast<const float2 *>(row_stats), scale, scale_stride, split});
}

// ---------------------------------------------------------------------------
// The same fused LayerNorm -> quantise without a caller workspace and
// without allocating: the row statistics go to `scratch`, a fixed device
// array that each GPU the library runs on holds until the process ends.
// Every call on a GPU uses that GPU's array (calls that overlap on one GPU
// race); ln_stats_kernel writes every row it covers before the quantiser
// reads it, so nothing needs clearing between calls.
namespace {

static __device__ __align__(256) float2 scratch[QI_HIP_NOALLOC_MAX_ROWS];

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
float2 *scratch_address[kMaxDevices] = {};

// The current device's copy of `scratch` (its device address, looked up once
// per device with that device current); null with *status set on failure.
float2 *scratch_for_current_device(int *status) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        *status = static_cast<int>(e);
        return nullptr;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        *status = static_cast<int>(hipErrorInvalidDevice);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (!scratch_address[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            *status = static_cast<int>(e != hipSuccess ? e : hipErrorInvalidSymbol);
            return nullptr;
        }
        scratch_address[dev] = static_cast<float2 *>(p);
    }
    return scratch_address[dev];
}

}  // namespace

QI_API int qi_hip_layer_norm_scale_quantize_fp6_noalloc(const float *x, const float *scale, int scale_stride,
                                                        int split, void *codes6, int m, int k, void *stream) {
    using namespace qi;
    if (m > QI_HIP_NOALLOC_MAX_ROWS) return kInvalid;
    if (m < 0 || k <= 0 || k % 256 || scale_stride < 0) return kInvalid;
    if (m == 0) return 0;
    if (!x || !scale || !codes6 || !aligned16(x) || !aligned16(scale) || scale_stride % 4 || !aligned16(codes6))
        return kInvalid;
    int status = 0;
    float2 *stats = scratch_for_current_device(&status);
    if (!stats) return status;
    hipStream_t s = stream_of(stream);
    ln_stats_kernel<<<dim3(static_cast<unsigned>((m + 3) / 4)), dim3(4 * WAVE), 0, s>>>(x, stats, m, k);
    const int st = launch_status();
    if (st) return st;
    return launch_fp6_strip<float>(x, codes6, nullptr, m, k, s, LnScaleProducer{stats, scale, scale_stride, split});
}

QI_API int qi_hip_swiglu(const float *gate, const float *up, void *out, int out_type, unsigned long long count,
                         void *stream) {
    using namespace qi;
    if (count == 0) return 0;
    if (count % 4 || out_type < 0 || out_type > 1 || !gate || !up || !out || !aligned16(gate) || !aligned16(up) ||
        !aligned16(out))
        return kInvalid;
    unsigned long long blocks = (count / 4 + 255) / 256;
    if (blocks > 65536ull * 16) blocks = 65536ull * 16;
    swiglu_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream_of(stream)>>>(gate, up, out, out_type,
                                                                                            count);
    return launch_status();
}

QI_API int qi_hip_swiglu_quantize_fp6(const float *gate, const float *up, void *codes6, int m, int k, void *stream) {
    using namespace qi;
    if (m < 0 || k <= 0 || k % 256) return kInvalid;
    if (m == 0) return 0;
    if (!gate || !up || !codes6 || !aligned16(gate) || !aligned16(up) || !aligned16(codes6)) return kInvalid;
    return launch_fp6_strip<float>(gate, codes6, nullptr, m, k, stream_of(stream), SwigluProducer{up, k});
}
