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

namespace qi {

constexpr int GROUP = 64;      // QIPACK v6 group size along K
constexpr int WAVE = 64;       // CDNA wavefront

inline hipStream_t stream_of(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline int launch_status() { return static_cast<int>(hipGetLastError()); }

constexpr int kInvalid = static_cast<int>(hipErrorInvalidValue);

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

// ops.cu:156-160 (gelu_tanh_kernel) formula, evaluated in fp32.
__device__ __forceinline__ float gelu_tanh(float v) {
    return 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
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

// Epilogue store of one fp32 value.
__device__ __forceinline__ void store_out(void *y, size_t index, float v, int out_type) {
    if (out_type == QI_HIP_OUT_F16)
        reinterpret_cast<uint16_t *>(y)[index] = f2h(v);
    else
        reinterpret_cast<float *>(y)[index] = v;
}

__device__ __forceinline__ float epilogue(float v, const float *bias, int col, int epi) {
    if (bias) v += bias[col];
    if (epi == QI_HIP_EPILOGUE_GELU_TANH) v = gelu_tanh(v);
    return v;
}

}  // namespace qi
