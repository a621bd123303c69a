// Micro-benchmark of matrix-core / vector-unit co-execution on gfx950, the
// measurement behind the W4A4 kernel's instruction mix (not part of the
// product library; built twice by build.py: MFMA results in ordinary VGPRs,
// as the product is compiled, and in accumulator registers, the compiler's
// default).
//
// Each wave runs `iters` iterations of one of these bodies on values held in
// registers (no memory traffic inside the timed loop):
//   0  four independent fp6 32x32x64 MFMAs (v_mfma_scale_f32_32x32x64_f8f6f4),
//      each accumulating into its own tile (four dependence chains)
//   1  64 independent fp32 FMAs (v_fmac_f32, 64 accumulators)
//   2  bodies 0 and 1 interleaved (one MFMA, then 16 FMAs), no dependences
//   3  the W4A4 kernel's per-group mix for a 64 x 64 wave tile: four fp6
//      MFMAs (the integer partials P), two f32 32x32x1 outer-product MFMAs
//      (sa * sw), and 64 FMAs y = fma(P, sa * sw, y) that consume the
//      previous iteration's MFMA results, each partial tile re-issued right
//      after its FMAs (the kernel's software pipeline)
//   4  body 0 with the MFMAs issued in pairs after every 32 FMAs of body 1
//   5  body 3 in the product kernel's order (partial tiles issued two tiles
//      after the FMAs that free them)
//   6  eight ds_read_b128 (1 KiB per wave each) per iteration: LDS read
//      throughput
//   7  64 FMAs on 16 accumulators (few registers), for issue rate against
//      waves per SIMD
//   8  direct-to-LDS loads, 4 KiB per wave per iteration from an
//      L2-resident window: L2 -> LDS throughput
//   9  four independent v_mfma_f32_32x32x1_2b_f32 (the W4A4 kernel's exact
//      scale outer product: 2048 products each)
//  10  four independent v_mfma_f32_32x32x4_2b_f16 (2048 outputs each; with
//      one non-zero K slot, an exact product of two fp16 values)
//  11  four independent v_mfma_f32_32x32x8_f16 (1024 outputs each)
//  12  four independent v_mfma_f32_16x16x4_4b_f16 (1024 outputs each)
//  13  four independent v_mfma_f32_4x4x4_16b_f16 (256 outputs each)
//  14  body 2 in a kernel held to two waves per SIMD (overlap_kernel)
//  15  body 0 in the same kernel
//  16  body 14 with the MFMA results forced into AGPRs (inline asm)
//  17  body 15 likewise
//  18  four independent v_mfma_f32_32x32x16_f16 (the attention's)
//  19  four independent v_mfma_f32_16x16x32_f16 (the W4A16 GEMM's)
// and records s_memtime (shader clock) around the loop.
#include <hip/hip_runtime.h>
#include <stdint.h>

// The direct-to-LDS load below sets M0 inside inline asm; nothing else here
// uses it.
#pragma clang diagnostic ignored "-Winline-asm"

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ void opaque(T &v) {
    asm volatile("" : "+v"(v));
}


// One fp6 MFMA with C = 0 (the kernel's form).
__device__ __forceinline__ v16f mfma6(v8i a, v8i b) {
    v16f z = {};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, z, 2, 2, 0, 127, 0, 127);
}
// The same, accumulating into c (bodies whose results are otherwise dead).
__device__ __forceinline__ v16f mfma6_acc(v8i a, v8i b, v16f c) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 2, 2, 0, 127, 0, 127);
}

template <int BODY>
__global__ __launch_bounds__(256) void probe_kernel(int iters, const int *__restrict__ seed, float *__restrict__ out,
                                                    unsigned long long *__restrict__ cycles) {
    const int lane = threadIdx.x & 63;
    // Four distinct A operands, made opaque (in place) every iteration, so
    // no MFMA is merged with another or hoisted out of the loop.
    v8i a[4], b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int t = 0; t < 4; ++t) a[t][i] = seed[(lane + i + 8 * t) & 63];
        b[i] = seed[(lane + 3 * i + 1) & 63];
    }
    float acc[64], x[16];
#pragma unroll
    for (int r = 0; r < 64; ++r) acc[r] = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = static_cast<float>(seed[(lane + r) & 63] & 7) * 0.25f;
    const float y = 1.0009765625f;
    constexpr bool MATRIX = BODY <= 5;  // bodies that use the matrix core
    v16f p[4] = {};
    v32f sp[2] = {};
    v32f w32[4] = {};
    v4f w4[4] = {};
    if constexpr (MATRIX) {
#pragma unroll
        for (int t = 0; t < 4; ++t) p[t] = mfma6(a[t], b);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            v32f z = {};
            sp[t] = __builtin_amdgcn_mfma_f32_32x32x1f32(x[t], x[t + 2], z, 0, 0, 0);
        }
    }
    __shared__ __attribute__((aligned(16))) v4i lds[8][256];
    if constexpr (BODY == 6) {
#pragma unroll
        for (int r = 0; r < 8; ++r) lds[r][threadIdx.x] = v4i{r, lane, 1, 2};
    }
    typedef int v4i_rsrc __attribute__((ext_vector_type(4)));
    const uint64_t base = reinterpret_cast<uint64_t>(out);
    const v4i_rsrc rsrc = {static_cast<int>(base), static_cast<int>((base >> 32) & 0xFFFF), 256 * 1024, 0x00020000};
    v4i rd[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) rd[r] = v4i{0, 0, 0, 0};
    __syncthreads();
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int t = 0; t < 4; ++t) opaque(a[t]);
        opaque(b);
        if constexpr (BODY == 0) {
#pragma unroll
            for (int t = 0; t < 4; ++t) p[t] = mfma6_acc(a[t], b, p[t]);
        } else if constexpr (BODY == 1) {
#pragma unroll
            for (int r = 0; r < 64; ++r) acc[r] = __builtin_fmaf(x[r & 15], y, acc[r]);
        } else if constexpr (BODY == 2) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                p[t] = mfma6_acc(a[t], b, p[t]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[16 * t + r] = __builtin_fmaf(x[r], y, acc[16 * t + r]);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else if constexpr (BODY == 3) {
            // tile t = (i, j), i = t / 2 (row tile, scale product sp[i]),
            // j = t % 2 (n-tile, half j of sp[i]).
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int i = t / 2, j = t % 2;
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[16 * t + r] = __builtin_fmaf(p[t][r], sp[i][16 * j + r], acc[16 * t + r]);
                __builtin_amdgcn_sched_barrier(0);
                if (j == 1) {
                    v32f z = {};
                    float sa = x[i], sw = x[i + 2];
                    opaque(sa);
                    sp[i] = __builtin_amdgcn_mfma_f32_32x32x1f32(sa, sw, z, 0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                }
                p[t] = mfma6(a[t], b);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else if constexpr (BODY == 5) {
            // Body 3 in the order of the product kernel's group step: the
            // FMAs of tile q, the scale product of row tile i after its last
            // n-tile, and the partial tile of tile q - 2 (two tiles of
            // look-ahead for its operands).
#pragma unroll
            for (int q = 0; q < 6; ++q) {
                if (q < 4) {
                    const int i = q / 2, j = q % 2;
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        acc[16 * q + r] = __builtin_fmaf(p[q][r], sp[i][16 * j + r], acc[16 * q + r]);
                    __builtin_amdgcn_sched_barrier(0);
                    if (j == 1) {
                        v32f z = {};
                        float sa = x[i], sw = x[i + 2];
                        opaque(sa);
                        sp[i] = __builtin_amdgcn_mfma_f32_32x32x1f32(sa, sw, z, 0, 0, 0);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                if (q >= 2) {
                    p[q - 2] = mfma6(a[q - 2], b);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        } else if constexpr (BODY == 7) {
            // Body 1 on 16 accumulators (few registers: up to eight waves
            // per SIMD fit): vector-unit issue rate against waves per SIMD.
#pragma unroll
            for (int rep = 0; rep < 4; ++rep)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[r] = __builtin_fmaf(x[r], y, acc[r]);
        } else if constexpr (BODY == 8) {
            // Direct-to-LDS loads (buffer_load_dwordx4 ... lds), four 1 KiB
            // wave loads per iteration from an L2-resident 256 KiB window of
            // `out`, at most eight in flight: L2 -> LDS throughput.
            const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t off = __builtin_amdgcn_readfirstlane(
                    static_cast<uint32_t>(((blockIdx.x * 4 + wv) * 4 + t + 16 * it) & 255) * 1024u);
                const uint32_t dst = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
                    (const __attribute__((address_space(3))) uint8_t *)&lds[2 * wv + (t & 1)][0])));
                asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(dst),
                             "v"(static_cast<uint32_t>(lane * 16)), "s"(rsrc), "s"(off)
                             : "memory", "m0");
            }
            asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        } else if constexpr (BODY == 6) {
            // LDS read throughput: eight ds_read_b128 per iteration (1 KiB
            // each per wave), consumed by one integer add each.
            const int wv = threadIdx.x >> 6;
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                v4i v = lds[(r + it) & 7][64 * wv + lane];
                rd[r] += v;
            }
        } else if constexpr (BODY == 18 || BODY == 19) {
            // The fp16 MFMAs of the product kernels: 32x32x16 (attention)
            // and 16x16x32 (W4A16), four chains.
            typedef _Float16 v8h_p __attribute__((ext_vector_type(8)));
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const v8h_p ha8 = __builtin_bit_cast(v8h_p, __builtin_shufflevector(a[t], a[t], 0, 1, 2, 3));
                const v8h_p hb8 = __builtin_bit_cast(v8h_p, __builtin_shufflevector(b, b, 0, 1, 2, 3));
                if constexpr (BODY == 18)
                    p[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ha8, hb8, p[t], 0, 0, 0);
                else
                    w4[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ha8, hb8, w4[t], 0, 0, 0);
            }
        } else if constexpr (BODY >= 9 && BODY <= 13) {
            // Output-rate of the small-K MFMA shapes (four accumulation
            // chains; operands made opaque above through a and b).
            v4h ha[4], hb;
#pragma unroll
            for (int t = 0; t < 4; ++t) ha[t] = __builtin_bit_cast(v4h, __builtin_shufflevector(a[t], a[t], 0, 1));
            hb = __builtin_bit_cast(v4h, __builtin_shufflevector(b, b, 0, 1));
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                if constexpr (BODY == 9)
                    w32[t] = __builtin_amdgcn_mfma_f32_32x32x1f32(x[t], x[t + 4], w32[t], 0, 0, 0);
                else if constexpr (BODY == 10)
                    w32[t] = __builtin_amdgcn_mfma_f32_32x32x4f16(ha[t], hb, w32[t], 0, 0, 0);
                else if constexpr (BODY == 11)
                    p[t] = __builtin_amdgcn_mfma_f32_32x32x8f16(ha[t], hb, p[t], 0, 0, 0);
                else if constexpr (BODY == 12)
                    p[t] = __builtin_amdgcn_mfma_f32_16x16x4f16(ha[t], hb, p[t], 0, 0, 0);
                else
                    w4[t] = __builtin_amdgcn_mfma_f32_4x4x4f16(ha[t], hb, w4[t], 0, 0, 0);
            }
        } else if constexpr (BODY == 4) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int r = 0; r < 32; ++r) acc[32 * h + r] = __builtin_fmaf(x[r & 15], y, acc[32 * h + r]);
                __builtin_amdgcn_sched_barrier(0);
                p[2 * h] = mfma6_acc(a[2 * h], b, p[2 * h]);
                p[2 * h + 1] = mfma6_acc(a[2 * h + 1], b, p[2 * h + 1]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < 64; ++r) s += acc[r];
    if constexpr (MATRIX) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) s += p[t][r];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 32; ++r) s += sp[t][r];
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) s += static_cast<float>(rd[r][0] + rd[r][1] + rd[r][2] + rd[r][3]);
    if constexpr (BODY >= 9 && BODY <= 19) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int r = 0; r < 32; ++r) s += w32[t][r];
#pragma unroll
            for (int r = 0; r < 16; ++r) s += p[t][r];
#pragma unroll
            for (int r = 0; r < 4; ++r) s += w4[t][r];
        }
    }
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    out[gid] = s;
    if (lane == 0) cycles[gid >> 6] = t1 - t0;
}

// Bodies 14 and 15: body 2 (four fp6 MFMA chains interleaved with 64
// independent FMAs) and body 0 alone, in a kernel held to two waves per SIMD
// (at most 256 registers per lane, so in the accumulator-register build the
// MFMA results live in AGPRs while two waves share each SIMD).
// fp6 MFMA accumulating into accumulator registers (AGPRs), whatever the
// build's register form.
typedef int v6i __attribute__((ext_vector_type(6)));
__device__ __forceinline__ void mfma6_agpr(v8i a, v8i b, v16f &c) {
    const int one = 127;  // E8M0 2^0
    const v6i a6 = __builtin_shufflevector(a, a, 0, 1, 2, 3, 4, 5), b6 = __builtin_shufflevector(b, b, 0, 1, 2, 3, 4, 5);
    asm volatile("v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %3 op_sel_hi:[0,0,0] cbsz:2 blgp:2"
                 : "+a"(c)
                 : "v"(a6), "v"(b6), "v"(one));
}

template <bool FMA, bool AGPR = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void overlap_kernel(
    int iters, const int *__restrict__ seed, float *__restrict__ out, unsigned long long *__restrict__ cycles) {
    const int lane = threadIdx.x & 63;
    v8i a[4], b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int t = 0; t < 4; ++t) a[t][i] = seed[(lane + i + 8 * t) & 63];
        b[i] = seed[(lane + 3 * i + 1) & 63];
    }
    float acc[64], x[16];
#pragma unroll
    for (int r = 0; r < 64; ++r) acc[r] = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = static_cast<float>(seed[(lane + r) & 63] & 7) * 0.25f;
    const float y = 1.0009765625f;
    v16f p[4] = {};
    __syncthreads();
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int t = 0; t < 4; ++t) opaque(a[t]);
        opaque(b);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            if constexpr (AGPR)
                mfma6_agpr(a[t], b, p[t]);
            else
                p[t] = mfma6_acc(a[t], b, p[t]);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (FMA) {
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[16 * t + r] = __builtin_fmaf(x[r], y, acc[16 * t + r]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < 64; ++r) s += acc[r];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += p[t][r];
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    out[gid] = s;
    if (lane == 0) cycles[gid >> 6] = t1 - t0;
}

// Runs body `body` on `blocks` workgroups of four waves; cycles[w] receives
// wave w's loop time in shader clocks.  Returns a hipError_t.
extern "C" __attribute__((visibility("default"))) int qi_probe_run(int body, int blocks, int iters, const int *seed,
                                                                    float *out, unsigned long long *cycles,
                                                                    void *stream) {
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    dim3 g(blocks), t(256);
    switch (body) {
    case 0: probe_kernel<0><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 1: probe_kernel<1><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 2: probe_kernel<2><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 3: probe_kernel<3><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 4: probe_kernel<4><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 5: probe_kernel<5><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 6: probe_kernel<6><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 7: probe_kernel<7><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 8:
        if (blocks * 256 < 64 * 1024) return static_cast<int>(hipErrorInvalidValue);  // the 256 KiB window
        probe_kernel<8><<<g, t, 0, s>>>(iters, seed, out, cycles);
        break;
    case 9: probe_kernel<9><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 10: probe_kernel<10><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 11: probe_kernel<11><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 12: probe_kernel<12><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 13: probe_kernel<13><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 14: overlap_kernel<true><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 15: overlap_kernel<false><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 16: overlap_kernel<true, true><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 18: probe_kernel<18><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 19: probe_kernel<19><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    case 17: overlap_kernel<false, true><<<g, t, 0, s>>>(iters, seed, out, cycles); break;
    default: return static_cast<int>(hipErrorInvalidValue);
    }
    return static_cast<int>(hipGetLastError());
}
