// Shared device helpers for the gfx950 QIPACK linear kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/qwen_image_hip.h"

#define QI_API extern "C" __attribute__((visibility("default")))

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// The direct-to-LDS loads below set M0 inside inline asm; nothing else in
// these kernels uses it, so the clobber warning does not apply.
#pragma clang diagnostic ignored "-Winline-asm"

namespace qi {

constexpr int GROUP = 64;      // QIPACK v6 group size along K
constexpr int WAVE = 64;       // CDNA wavefront
// fp6 operand blocks (one 32-row tile, one group): half 0 = 64 lanes x 16
// bytes (12 code bytes + the row's fp16 scale + 2 zero bytes), then half 1 =
// 64 lanes x 12 code bytes.
constexpr unsigned FP6_HALF0 = 1024, FP6_BLOCK = 1792;

inline hipStream_t stream_of(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline int launch_status() { return static_cast<int>(hipGetLastError()); }

constexpr int kInvalid = static_cast<int>(hipErrorInvalidValue);

// Compute units of the current device, read once per device.
inline int device_cus() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
        cus[dev] = c;
    }
    return cus[dev];
}



// fp16 bits <-> float on the device.  __builtin bit casts keep this exact.
__device__ __forceinline__ float h2f(uint16_t bits) {
    _Float16 h = __builtin_bit_cast(_Float16, bits);
    return static_cast<float>(h);
}
// Round-to-nearest-even float -> fp16 bits (v_cvt_f16_f32 under the default
// RNE mode register).
__device__ __forceinline__ uint16_t f2h(float v) {
    _Float16 h = static_cast<_Float16>(v);
    return __builtin_bit_cast(uint16_t, h);
}

// Pins a value to an fp32 register.  The backend otherwise folds
// fp16(fmaf(a, b, c)) into one mixed-precision fma with a single rounding,
// while the reference rounds to fp32 first and then to fp16.
__device__ __forceinline__ float f32_round_point(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

// fp16(fmaf(code, scale, minimum)) with the reference's two roundings
// (qwen_image_cuda/cuda/gemm.cu:229-230).
__device__ __forceinline__ uint16_t dequant_w4a16(float code, float scale, float minimum) {
    return f2h(f32_round_point(__builtin_fmaf(code, scale, minimum)));
}

// W4A16 tiled codes hold a lane's 8 elements per dword with element 2i in
// nibble slot i and element 2i+1 in slot 4+i, so (x >> 4i) & 0x000F000F is
// the fp16-lane pair (e[2i], e[2i+1]) of small integers.
__device__ __forceinline__ uint32_t w4a16_permute_nibbles(uint32_t x) {
    uint32_t out = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) out |= ((x >> (4 * e)) & 15u) << (4 * ((e & 1) ? 4 + (e >> 1) : (e >> 1)));
    return out;
}
__device__ __forceinline__ uint32_t w4a16_unpermute_nibbles(uint32_t x) {
    uint32_t out = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) out |= ((x >> (4 * ((e & 1) ? 4 + (e >> 1) : (e >> 1)))) & 15u) << (4 * e);
    return out;
}

// True when every c * scale + minimum (c = 0..15) is exactly representable in
// fp32, so that one fp16 rounding of it equals the reference's two roundings.
// c * scale has at most 15 significant bits and minimum 11; their exact sum
// fits 24 bits when the exponent fields satisfy -12 <= es - em <= 8
// (subnormals count as exponent field 1), or when minimum is zero.
__device__ __forceinline__ bool w4a16_single_rounding_exact(uint32_t scale_bits, uint32_t minimum_bits) {
    if ((minimum_bits & 0x7FFFu) == 0) return true;
    const int es = max(static_cast<int>((scale_bits >> 10) & 31u), 1);
    const int em = max(static_cast<int>((minimum_bits >> 10) & 31u), 1);
    const int d = es - em;
    return d <= 8 && d >= -12;
}

// 8 tiled (slot-permuted) codes -> 8 fp16 weights in element order.  Fast
// path: packed fp16 integer trick and one fused fp16 fma per pair; exact
// path: fp32 fma then RNE to fp16, per element (the reference's rounding).
__device__ __forceinline__ uint4 w4a16_dequant8(uint32_t x, uint32_t scale_bits, uint32_t minimum_bits, bool fast) {
    uint32_t out[4];
    if (fast) {
        const v2h s2 = __builtin_bit_cast(v2h, scale_bits | (scale_bits << 16));
        const v2h m2 = __builtin_bit_cast(v2h, minimum_bits | (minimum_bits << 16));
        const v2h k1024 = v2h{static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
        uint32_t magic = 0x64006400u;
        asm volatile("" : "+v"(magic));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // Nibble pair -> fp16 1024 + c: one and-or with the 0x6400
            // pattern held in a VGPR.
            const uint32_t biased = ((x >> (4 * i)) & 0x000F000Fu) | (magic & ~0x000F000Fu);
            const v2h c = __builtin_bit_cast(v2h, biased) - k1024;
            out[i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c, s2, m2));
        }
    } else {
        const float s = h2f(static_cast<uint16_t>(scale_bits)), mn = h2f(static_cast<uint16_t>(minimum_bits));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float e0 = static_cast<float>((x >> (4 * i)) & 15u);
            const float e1 = static_cast<float>((x >> (4 * i + 16)) & 15u);
            out[i] = static_cast<uint32_t>(dequant_w4a16(e0, s, mn)) |
                     (static_cast<uint32_t>(dequant_w4a16(e1, s, mn)) << 16);
        }
    }
    return uint4{out[0], out[1], out[2], out[3]};
}

// The tanh-form GELU of ops.cu:156-160 (gelu_tanh_kernel),
//   0.5 v (1 + tanh(u)),  u = sqrt(2 / pi) (v + 0.044715 v^3),
// through the logistic identity 0.5 (1 + tanh(u)) = 1 / (1 + exp(-2u)):
// v / (1 + 2^(c t)) with t = v (1 + 0.044715 v^2) and c = -2 sqrt(2 / pi)
// log2(e), on the hardware exp2 and reciprocal (a few ulp in fp32; the
// outputs are compared within the fp16 output tolerance).  Large |v| are
// safe: 2^(c t) goes to +inf (v -> -0) or to 0 (v -> v).
__device__ __forceinline__ float gelu_tanh(float v) {
    const float t = v * __builtin_fmaf(0.044715f * v, v, 1.0f);
    return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-2.3022082f * t));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) v = fmaxf(v, __shfl_xor(v, s, 64));
    return v;
}

__device__ __forceinline__ float wave_sum16(float v) {
    // Sum over the four 16-lane groups (lanes l, l+16, l+32, l+48).
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// Signed int4 nibbles -> int8 lanes scaled by 16 (value 16*q in each byte).
// lo: the low nibble of every byte moved up; hi: the high nibble kept in
// place.  A 16*q operand on both MFMA sides yields 256*P exactly.
__device__ __forceinline__ int nib_lo16(uint32_t x) { return static_cast<int>((x << 4) & 0xF0F0F0F0u); }
__device__ __forceinline__ int nib_hi16(uint32_t x) { return static_cast<int>(x & 0xF0F0F0F0u); }

// Signed int4 code (-7..7) -> fp6 E2M3 bits (sign, 2 exponent bits with bias
// 1, 3 mantissa bits).  Every integer in [-7, 7] is exact in E2M3, so MFMAs
// on these operands accumulate the exact integer dot product.
__device__ __forceinline__ uint32_t int4_to_e2m3(int q) {
    // |q| 0..7 -> magnitude codes 0, 8 (1.0), 16 (2.0), 20 (3.0), 24 (4.0),
    // 26 (5.0), 28 (6.0), 30 (7.0).
    const uint32_t a = static_cast<uint32_t>(q < 0 ? -q : q);
    const uint32_t code = a == 0 ? 0u : (a == 1 ? 8u : (a < 4 ? 16u + 4u * (a - 2) : 24u + 2u * (a - 4)));
    return (q < 0 ? 32u : 0u) | code;
}

typedef int v4i_rsrc __attribute__((ext_vector_type(4)));

// Raw buffer resource (base, size in bytes; loads past the end return zero)
// as four scalar dwords for the inline loads below.
__device__ __forceinline__ v4i_rsrc raw_rsrc(const void *p, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    return v4i_rsrc{static_cast<int>(a), static_cast<int>((a >> 32) & 0xFFFF), static_cast<int>(bytes), 0x00020000};
}

// Direct-to-LDS buffer loads, written as inline asm so the compiler does not
// track them: it would otherwise make every LDS read and every barrier wait
// for all of them, including the loads of later groups into other slots.
// Their completion is counted explicitly with s_waitcnt vmcnt.  Lane i's
// data lands at lds_addr + 16 i (12- and 16-byte forms) or + 4 i (4-byte
// form).
// Nothing else in these kernels uses M0.
__device__ __forceinline__ void dma_dwordx3(v4i_rsrc rsrc, uint32_t lds_addr, uint32_t voffset, uint32_t soffset) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx3 %1, %2, %3 offen lds" ::"s"(lds_addr),
                 "v"(voffset), "s"(rsrc), "s"(soffset)
                 : "memory", "m0");
}

__device__ __forceinline__ void dma_dwordx4(v4i_rsrc rsrc, uint32_t lds_addr, uint32_t voffset, uint32_t soffset) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds_addr),
                 "v"(voffset), "s"(rsrc), "s"(soffset)
                 : "memory", "m0");
}

__device__ __forceinline__ void dma_dword(v4i_rsrc rsrc, uint32_t lds_addr, uint32_t voffset, uint32_t soffset) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, %3 offen lds" ::"s"(lds_addr),
                 "v"(voffset), "s"(rsrc), "s"(soffset)
                 : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_address(const void *p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) uint8_t *)p));
}

// Buffer resource over [p, p + bytes): loads past the end return zeros, which
// is how partial tiles read their missing rows.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), static_cast<short>(0), static_cast<int>(bytes),
                                             0x00020000);
}

// 16 bytes per lane from a buffer straight into LDS (buffer_load ... lds):
// lane i's bytes land at lds + 16 * i, so one wave instruction fills 1 KiB of
// LDS contiguously starting at the wave-uniform `lds`.
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rsrc, void *lds, uint32_t voffset,
                                                  uint32_t soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)lds, 16, voffset,
                                             soffset, 0, 0);
}

// Workgroup order that keeps the tiles resident on one XCD close together:
// the hardware deals workgroups round-robin over the 8 XCDs, so consecutive
// ids are remapped to one XCD's contiguous range, and tiles are walked in
// bands of `band` tile-rows so an XCD's tiles share A rows and B columns in
// its own L2.
__device__ __forceinline__ void tile_of_block(int block, int tiles_m, int tiles_n, int band, int &tm, int &tn) {
    const int total = tiles_m * tiles_n;
    int b = block;
    if (total % 8 == 0) b = (block % 8) * (total / 8) + block / 8;
    const int per_band = band * tiles_n;
    const int first_m = (b / per_band) * band;
    const int rows = min(tiles_m - first_m, band);
    const int in_band = b % per_band;
    tm = first_m + in_band % rows;
    tn = in_band / rows;
}

// Where a GEMM's outputs go.  Output (row, col) is element
// (row_base + row, col - fold) of a y made of n_out / n_part parts of
// [m_out, n_part] (out_index), where fold = n_out for the second stream's
// columns (col >= n_out) of a dual-stream call and 0 otherwise.  A plain
// call has row_base 0, m_out = m, n_out = n.
struct OutMap {
    int row_base, m_out, n_out;
};

// The output-tile grid of a launch: t0 = tm0 * tn0 tiles of stream 0 (tile
// rows and columns from 0), then tm1 * tn1 tiles of stream 1 (tile rows
// from tm0, columns from tn0) -- the two diagonal blocks of a dual-stream
// call.  A plain call has tm1 = tn1 = 0.
struct TileGrid2 {
    int t0, tm0, tn0, tm1, tn1;
};

// Tile t of the grid, in XCD-aware order within each stream.
__device__ __forceinline__ void grid_tile(const TileGrid2 &gd, int t, int &tm, int &tn) {
    if (t < gd.t0) {
        tile_of_block(t, gd.tm0, gd.tn0, 8, tm, tn);
    } else {
        tile_of_block(t - gd.t0, gd.tm1, gd.tn1, 8, tm, tn);
        tm += gd.tm0;
        tn += gd.tn0;
    }
}

// Epilogue store of one fp32 value.
__device__ __forceinline__ void store_out(void *y, size_t index, float v, int out_type) {
    if (out_type == QI_HIP_OUT_F16)
        reinterpret_cast<uint16_t *>(y)[index] = f2h(v);
    else
        reinterpret_cast<float *>(y)[index] = v;
}

// Index of output (row, col) when y holds n / n_part consecutive [m, n_part]
// arrays (a fused record's parts, e.g. q, k, v); n_part == n is the plain
// [m, n] layout.  col0 is a wave-uniform column in the same part as col.
__device__ __forceinline__ size_t out_index(int row, int col, int col0, int m, int n, int n_part) {
    if (n_part == n) return static_cast<size_t>(row) * n + col;
    const int part = static_cast<int>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(col0))) / n_part;
    return static_cast<size_t>(part) * m * n_part + static_cast<size_t>(row) * n_part + (col - part * n_part);
}

__device__ __forceinline__ float epilogue(float v, const float *bias, int col, int epi) {
    if (bias) v += bias[col];
    if (epi == QI_HIP_EPILOGUE_GELU_TANH) v = gelu_tanh(v);
    return v;
}

}  // namespace qi
