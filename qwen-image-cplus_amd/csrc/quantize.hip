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
// That form serves the QIPACK layout; the fp6 layout (the fast path) uses
// sixteen inputs per lane (quantize_lane16_kernel), which leaves two of
// the four stages in registers and one LDS round trip for the other two.

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
    // The shared first sums: -x0 + x1 rounds to exactly -(x0 - x1), and
    // (-(x0 - x1)) + x2 is x2 - (x0 - x1), so each output keeps the
    // reference's three roundings in its order.
    const float sum = x0 + x1, dif = x0 - x1;
    a = ((sum + x2) - x3) * f;
    b = ((sum - x2) + x3) * f;
    c = ((dif + x2) + x3) * f;
    d = ((x2 - dif) + x3) * f;
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

// LDS word of element i of a chunk: an XOR swizzle that makes every access
// pattern below (4 consecutive words per lane, and the strided butterfly
// quadruples of strides 4, 16, 64) conflict-free for 32 lanes at a time.
__device__ __forceinline__ int swz(int i) { return i ^ ((i >> 2) & 31); }


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
// workgroups over every block).  Rows past m quantise zeros; their codes
// are written but never used.
// No producer: the quantiser reads its input as is.
struct NoProducer {
    static constexpr bool active = false;
    __device__ void operator()(int, int, float (&)[4]) const {}
};

// The fp6 quantiser, sixteen inputs per lane: lane (r, s) of the
// 512-lane workgroup holds inputs 16s .. 16s + 15 of row r of the 32-row
// tile's chunk (r = 4 * wave + lane / 16, s = lane % 16).  The H256 stages
// of strides 1 and 4 run in registers; for strides 16 and 64 the values go
// through a wave-private LDS row and each lane takes the 16 elements
// s + 16x + 64y, whose two stages again run in registers, and back (16-byte
// accesses on the home side).  A 64-group is then one quad of lanes: the
// absmax is in-lane plus two DPP steps, and the lane's 16 codes are one
// half-slot of the fp6 layout, converted by v_cvt_scalef32_2xpk16_fp6_f32
// from the exact integers q (scale 1; a zero's sign is cleared).  Same
// arithmetic, operation order and codes as quantize_chunk.
typedef float v16f_q __attribute__((ext_vector_type(16)));

typedef unsigned v6u_q __attribute__((ext_vector_type(6)));

// FMT 1 writes the fp6 layout (the code blocks assembled in LDS, 16-byte
// stores); FMT 0 the QIPACK layout (each lane's 16 nibbles as one 8-byte
// store, scales [m, k/64]).
template <typename In, typename Producer = NoProducer, int FMT = 1>
__global__ __launch_bounds__(8 * WAVE) void quantize_lane16_kernel(
    const In *__restrict__ x, uint8_t *__restrict__ codes, uint16_t *__restrict__ scales, int m, int k,
    Producer produce = Producer{}) {
    using Vals = typename std::conditional<Producer::active, float, In>::type;
    constexpr bool HALF = !__is_same(Vals, uint16_t);  // see butterfly4
    constexpr float unit = HALF ? 1.0f : 16.0f;
    constexpr int ROW = 256 + 16;  // floats per LDS row: 16 bytes of padding after every 64 values
    // The tile's rows (34 KiB) and code blocks (7 KiB): three workgroups
    // per CU.  Putting the blocks in the rows' bytes after a barrier (four
    // per CU) measured no faster.
    __shared__ __attribute__((aligned(16))) float rows[32 * ROW];
    __shared__ __attribute__((aligned(16))) uint32_t blocks[4 * FP6_BLOCK / 4];
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x >> 6;
    const int r = wave * 4 + (lane >> 4), s = lane & 15, j = s & 3;
    const int groups = k >> 6;
    const int tile = blockIdx.x, c = blockIdx.y;
    const int row = tile * 32 + r;
    auto addr = [](int e) { return e + 4 * (e >> 6); };  // padded LDS word of element e of a row
    float *lrow = rows + r * ROW;

    float v[16];
    {
        const int rr = min(row, m - 1);
        const In *src = x + static_cast<size_t>(rr) * k + c * 256 + 16 * s;
        if constexpr (__is_same(In, uint16_t) && !Producer::active) {
            // Rows past m quantise zeros: the raw words are cleared.
            uint4 h[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                h[t] = *reinterpret_cast<const uint4 *>(src + 8 * t);
                if (row >= m) h[t] = uint4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const uint32_t w4[4] = {h[t].x, h[t].y, h[t].z, h[t].w};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    v[8 * t + 2 * u] = h2f(static_cast<uint16_t>(w4[u] & 0xFFFFu));
                    v[8 * t + 2 * u + 1] = h2f(static_cast<uint16_t>(w4[u] >> 16));
                }
            }
        } else {
            // All loads first, the producer's included (it runs on the
            // clamped row, branch-free), so that none waits for another
            // chunk's arithmetic; rows past m are zeroed after.
            float w[4][4];
#pragma unroll
            for (int t = 0; t < 4; ++t) load4<In>(src + 4 * t, w[t]);
#pragma unroll
            for (int t = 0; t < 4; ++t) produce(rr, c * 256 + 16 * s + 4 * t, w[t]);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int u = 0; u < 4; ++u) v[4 * t + u] = row < m ? w[t][u] : 0.f;
        }
    }
    // Strides 1 and 4.
#pragma unroll
    for (int t = 0; t < 4; ++t) butterfly4<HALF>(v[4 * t], v[4 * t + 1], v[4 * t + 2], v[4 * t + 3]);
#pragma unroll
    for (int t = 0; t < 4; ++t) butterfly4<HALF>(v[t], v[t + 4], v[t + 8], v[t + 12]);
    // Strides 16 and 64 through the wave's LDS rows (no other wave touches
    // them): the lane takes the 16 elements s + 16x + 64y (x, y = 0..3),
    // whose stride-16 butterflies run over x and stride-64 ones over y, then
    // the values go back to their home lanes.
#pragma unroll
    for (int t = 0; t < 4; ++t)
        *reinterpret_cast<float4 *>(lrow + addr(16 * s + 4 * t)) = float4{v[4 * t], v[4 * t + 1], v[4 * t + 2], v[4 * t + 3]};
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    {
        float w[4][4];  // [x][y]
#pragma unroll
        for (int xx = 0; xx < 4; ++xx)
#pragma unroll
            for (int yy = 0; yy < 4; ++yy) w[xx][yy] = lrow[addr(s + 16 * xx + 64 * yy)];
#pragma unroll
        for (int yy = 0; yy < 4; ++yy) butterfly4<HALF>(w[0][yy], w[1][yy], w[2][yy], w[3][yy]);
#pragma unroll
        for (int xx = 0; xx < 4; ++xx) butterfly4<HALF>(w[xx][0], w[xx][1], w[xx][2], w[xx][3]);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int xx = 0; xx < 4; ++xx)
#pragma unroll
            for (int yy = 0; yy < 4; ++yy) lrow[addr(s + 16 * xx + 64 * yy)] = w[xx][yy];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const float4 w = *reinterpret_cast<const float4 *>(lrow + addr(16 * s + 4 * t));
        v[4 * t] = w.x;
        v[4 * t + 1] = w.y;
        v[4 * t + 2] = w.z;
        v[4 * t + 3] = w.w;
    }

    // Group (quad) absmax, fp16 scale, quotients (gemm.cu:45-48), as
    // quantize_chunk.
    float peak = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) peak = fmaxf(peak, fabsf(v[i]));
    peak = fmaxf(peak, dpp_f32<0xB1>(peak));  // quad_perm [1,0,3,2]
    peak = fmaxf(peak, dpp_f32<0x4E>(peak));  // quad_perm [2,3,0,1]
    const uint16_t scale_bits = f2h(fmaxf((peak * (1.0f / unit)) / 7.0f, 5.9604645e-08f));
    const float dd = h2f(scale_bits) * unit;
    const float y = 1.0f / dd;
    // rint by the shift M = 1.5 * 2^23 (|quot| < 11 here): quot + M rounds to
    // M + rint(quot), ties to even like rintf, and is clamped there; its low
    // mantissa bits are the two's-complement code (the QIPACK nibble), and
    // subtracting M gives the integer as a float, +0 for a quotient in
    // [-0.5, 0) (the reference's integer code 0, where rintf would give -0,
    // code 32 after the fp6 conversion).
    constexpr float M = 12582912.0f;
    float qs[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float q0 = v[i] * y;
        const float quot = __builtin_fmaf(__builtin_fmaf(-q0, dd, v[i]), y, q0);
        qs[i] = __builtin_amdgcn_fmed3f(quot + M, M - 7.0f, M + 7.0f);
    }
    const int gb = s >> 2;
    if constexpr (FMT == 0) {
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            w0 |= (__builtin_bit_cast(uint32_t, qs[i]) & 15u) << (4 * i);
            w1 |= (__builtin_bit_cast(uint32_t, qs[8 + i]) & 15u) << (4 * i);
        }
        if (row < m) {
            *reinterpret_cast<uint2 *>(codes + static_cast<size_t>(row) * (k >> 1) + c * 128 + s * 8) = uint2{w0, w1};
            if (j == 0) scales[static_cast<size_t>(row) * groups + c * 4 + gb] = scale_bits;
        }
        return;
    }
    v16f_q qa, qb;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float q = qs[i] - M;
        if (i & 1) qb[i >> 1] = q; else qa[i >> 1] = q;
    }
#pragma unroll
    for (int i = 8; i < 16; ++i) qa[i] = qb[i] = 0.f;
    const v6u_q cw = __builtin_amdgcn_cvt_scalef32_2xpk16_fp6_f32(qa, qb, 1.0f);
    // Half-slot of group gb = s / 4: half j & 1, slot (j >> 1) * 32 + r.
    const int slot = (j >> 1) * 32 + r;
    if ((j & 1) == 0) {
        *reinterpret_cast<uint4 *>(blocks + (gb * FP6_BLOCK + slot * 16) / 4) = uint4{cw[0], cw[1], cw[2], scale_bits};
    } else {
        uint32_t *dst = blocks + (gb * FP6_BLOCK + FP6_HALF0 + slot * 12) / 4;
        dst[0] = cw[0];
        dst[1] = cw[1];
        dst[2] = cw[2];
    }
    if (scales && j == 0) scales[(static_cast<size_t>(tile) * groups + c * 4 + gb) * 32 + r] = scale_bits;
    __syncthreads();
    uint4 *out = reinterpret_cast<uint4 *>(codes + (static_cast<size_t>(tile) * groups + c * 4) * FP6_BLOCK);
    for (int idx = threadIdx.x; idx < 4 * FP6_BLOCK / 16; idx += 8 * WAVE)
        out[idx] = reinterpret_cast<const uint4 *>(blocks)[idx];
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
    quantize_lane16_kernel<In, Producer><<<grid, dim3(8 * WAVE), 0, stream>>>(
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
    if (reinterpret_cast<uintptr_t>(codes) % 8 == 0 && chunks <= 65535) {
        // Sixteen inputs per lane, 8-byte code stores (see the kernel).
        const dim3 grid(static_cast<unsigned>((m + 31) / 32), static_cast<unsigned>(chunks));
        quantize_lane16_kernel<In, NoProducer, 0><<<grid, dim3(8 * WAVE), 0, stream>>>(
            x, static_cast<uint8_t *>(codes), static_cast<uint16_t *>(scales), m, k, NoProducer{});
        return launch_status();
    }
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
