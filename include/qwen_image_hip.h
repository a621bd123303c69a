/*
 * qwen_image_hip.h -- C ABI of the MI355X (gfx950) QIPACK INT4 linear backend.
 *
 * Conventions (shared with the reference's libqwen_image_cuda, whose entry
 * points are cited as file:line in netdur/qwen-image-cplus 0.2.5):
 *   - every pointer argument is a DEVICE pointer owned by the caller; nothing
 *     on this path allocates or frees device memory;
 *   - every function returns a hipError_t as int, 0 = success; shape or
 *     argument violations return hipErrorInvalidValue (1) before any launch;
 *     otherwise the launch status (hipGetLastError) is returned and the work
 *     completes asynchronously;
 *   - the four reference-named entry points run on the null (legacy default)
 *     stream, as the reference does; every qi_hip_* entry point takes a
 *     hipStream_t passed as void * (NULL = null stream);
 *   - layouts are row-major, little-endian; fp16 is IEEE binary16 passed as
 *     void * (uint16_t storage); "G" is K / 64 groups.
 *
 * Weight layouts.  A QIPACK record stores codes [N, K/2] (even k in the low
 * nibble), fp16 scales [N, G] and, for W4A16, fp16 minimums [N, G]
 * (int4_pack.cplus:6-15).  The qi_hip_relayout_* functions permute those
 * arrays once, at upload, into the MFMA-tile order the *_tiled kernels read:
 *
 *   W4A4 tiled codes   [N/16][G][64 lanes][8 bytes]
 *                      lane l carries row 16*t + (l % 16), bytes
 *                      [8*(l/16), 8*(l/16) + 8) of that row's 32-byte group.
 *   W4A4 tiled scales  [N/16][G][16] fp16
 *   W4A16 tiled codes  [N/16][G][64 lanes][2 dwords]
 *                      lane l carries row 16*t + (l % 16), elements
 *                      [8q, 8q+8) and [32+8q, 32+8q+8) of the group,
 *                      q = l / 16, one dword each; within a dword element
 *                      2i sits in nibble i and element 2i+1 in nibble 4+i.
 *   W4A16 tiled scales [N/16][G][16][2] fp16 pairs (scale, minimum)
 *
 * The re-layout is a permutation of nibbles and scales; the *_inverse functions
 * restore the QIPACK arrays exactly.  A tiled buffer has the same byte size
 * as the source arrays (scales and minimums are interleaved into one array of
 * twice the size for W4A16).
 */
#ifndef QWEN_IMAGE_HIP_H
#define QWEN_IMAGE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version of this header; bumped on any signature change. */
#define QI_HIP_ABI_VERSION 5
int qi_hip_abi_version(void);

/* ---------------------------------------------------------------------------
 * Reference-named entry points (drop-in for libqwen_image_cuda).
 * ------------------------------------------------------------------------- */

/* Replaces qwen_image_cuda/cuda/gemm.cu:54 (qi_w4a4_quantize_activations),
 * bound at qwen_image_cuda/src/cuda.cplus:53-54.  x f32 [m, k] -> codes
 * [m, k/2] (H256-rotated, signed int4, even k low nibble), scales fp16
 * [m, k/64] = fp16(max(absmax / 7, 2^-24)).  Requires k % 256 == 0 (the
 * reference leaves k unchecked; this build rejects it) and m >= 0. */
int qi_w4a4_quantize_activations(const float *x, void *codes, void *scales, int m, int k);

/* Replaces gemm.cu:183 (qi_w4a4_gemm), bound at cuda.cplus:55-56.
 * y f32 [m, n] = sum_g float(P_g) * (sa[m,g] * sw[n,g]) with P_g the exact
 * int32 per-group partial of the int4 codes.  Weights in QIPACK layout (not
 * tiled).  Requires m % 128 == 0, n % 128 == 0, k % 256 == 0, exactly as the
 * reference does. */
int qi_w4a4_gemm(const void *a_codes, const void *a_scales, const void *w_codes, const void *w_scales,
                 float *y, int m, int n, int k);

/* Replaces gemm.cu:262 (qi_w4a16_gemm), bound at cuda.cplus:57-58.
 * y f32 [m, n] = x_half [m, k] . W^T with W = fp16(fmaf(code, scale, min)).
 * Weights in QIPACK layout.  Requires m % 128 == 0, n % 128 == 0,
 * k % 64 == 0, exactly as the reference does. */
int qi_w4a16_gemm(const void *x_half, const void *codes, const void *scales, const void *minimums, float *y,
                  int m, int n, int k);

/* Replaces qwen_image_cuda/cuda/ops.cu:209 (qi_f32_to_f16), bound at
 * cuda.cplus:45-46.  Round-to-nearest-even f32 -> fp16. */
int qi_f32_to_f16(const float *source, void *out, unsigned long long count);

/* ---------------------------------------------------------------------------
 * Extensions: stream-taking forms, tiled weights, fused epilogues, GEMV.
 * No reference counterpart unless cited.
 * ------------------------------------------------------------------------- */

/* Stream-taking forms of the four reference entry points (same semantics). */
int qi_hip_w4a4_quantize_activations(const float *x, void *codes, void *scales, int m, int k, void *stream);
int qi_hip_f32_to_f16(const float *source, void *out, unsigned long long count, void *stream);

/* fp16-input activation quantiser, same arithmetic after exact widening
 * (the reference's bench twin, qwen_image_cuda/cuda/bench/bench_w4a4.cu:30-66). */
int qi_hip_w4a4_quantize_activations_f16(const void *x_half, void *codes, void *scales, int m, int k,
                                         void *stream);

/* One-time re-layout at upload (see layouts above).  n % 16 == 0 and
 * k % 256 == 0 (W4A4) or k % 64 == 0 (W4A16). */
int qi_hip_relayout_w4a4(const void *codes, const void *scales, void *tiled_codes, void *tiled_scales, int n,
                         int k, void *stream);
int qi_hip_relayout_w4a4_inverse(const void *tiled_codes, const void *tiled_scales, void *codes, void *scales,
                                 int n, int k, void *stream);
int qi_hip_relayout_w4a16(const void *codes, const void *scales, const void *minimums, void *tiled_codes,
                          void *tiled_scales, int n, int k, void *stream);
int qi_hip_relayout_w4a16_inverse(const void *tiled_codes, const void *tiled_scales, void *codes, void *scales,
                                  void *minimums, int n, int k, void *stream);

/* Output element type and fused epilogue for the *_tiled GEMMs and GEMV.
 * The epilogue computes, in fp32, v = acc (+ bias[n]) then optionally
 * gelu_tanh(v) (ops.cu:156-160 formula), then stores fp32 or RNE fp16. */
#define QI_HIP_OUT_F32 0
#define QI_HIP_OUT_F16 1
#define QI_HIP_EPILOGUE_NONE 0
#define QI_HIP_EPILOGUE_GELU_TANH 1

/* W4A4 GEMM on tiled weights.  a_codes/a_scales as produced by the
 * quantiser (QIPACK activation layout [m, k/2], [m, k/64]).  bias is an
 * fp32 [n] vector or NULL.  Any m >= 1; n % 16 == 0; k % 256 == 0. */
int qi_hip_w4a4_gemm_tiled(const void *a_codes, const void *a_scales, const void *w_tiled_codes,
                           const void *w_tiled_scales, const float *bias, void *y, int out_type, int epilogue,
                           int m, int n, int k, void *stream);

/* W4A16 GEMM on tiled weights.  x_half fp16 [m, k]; any m >= 1;
 * n % 16 == 0; k % 64 == 0.  Dispatches to the GEMV kernel for m <= 16. */
int qi_hip_w4a16_gemm_tiled(const void *x_half, const void *w_tiled_codes, const void *w_tiled_scales,
                            const float *bias, void *y, int out_type, int epilogue, int m, int n, int k,
                            void *stream);
/* The same GEMM over a fused record: several records of one input (the
 * reference's reuse_input group, transformer.cplus:759-762 -- to_q, to_k,
 * to_v) concatenated along n at upload, so their n outputs are
 * n / n_part consecutive parts of n_part outputs each, and y holds the parts
 * as consecutive [m, n_part] arrays (q, then k, then v).  One launch in
 * place of one per record.  n_part % 16 == 0, n % n_part == 0; n_part == n
 * is qi_hip_w4a16_gemm_tiled.  The kernel shape is chosen for the fused n,
 * so outputs agree with per-record calls within the W4A16 tolerance (bit
 * for bit when the same kernel shape is chosen). */
int qi_hip_w4a16_gemm_tiled_parts(const void *x_half, const void *w_tiled_codes, const void *w_tiled_scales,
                                  const float *bias, void *y, int out_type, int epilogue, int m, int n, int k,
                                  int n_part, void *stream);
/* Both streams of an MMDiT dual-stream block in one call (the W4A16 twin of
 * qi_hip_w4a4_gemm_fp6_dual): x_half [m, k] holds stream 0's rows
 * [0, m_split) then stream 1's; the tiled weight and scale arrays hold 2n
 * rows, stream 0's record then stream 1's; bias NULL or fp32 [2n]; y is n /
 * n_part parts of [m, n_part], each row with its own stream's outputs.  One
 * launch over both streams' tiles when the kernel shape chosen for (m, n)
 * tiles both blocks, else one launch per stream; outputs agree with the
 * per-stream calls within the W4A16 tolerance.  Each stream has more than
 * 16 rows. */
int qi_hip_w4a16_gemm_tiled_dual(const void *x_half, const void *w_tiled_codes, const void *w_tiled_scales,
                                 const float *bias, void *y, int out_type, int epilogue, int m, int m_split, int n,
                                 int k, int n_part, void *stream);

/* The tiled W4A16 GEMM with a caller workspace: m_split == 0 is
 * qi_hip_w4a16_gemm_tiled_parts (n outputs), m_split > 0 is
 * qi_hip_w4a16_gemm_tiled_dual (n outputs per stream, 2n weight rows).
 * Where few output tiles would leave most CUs walking all of K alone
 * (short m: the text stream, an encoder's prompt rows), the call splits K
 * over workgroups: fp32 partial tiles go to the workspace, and a second
 * kernel adds them in a fixed order (so results do not depend on timing)
 * and applies the epilogue.  From 2048 rows per stream (128 x 192,
 * 256 x 256 and 128 x 128 tiles) the workspace instead receives the
 * weights dequantised once to fp16 (n k * 2 bytes, the reference's
 * values), which the tiled kernel reads in place of the codes.  Outputs
 * agree with the workspace-free entries within the W4A16 tolerance (bit for
 * bit when no split is chosen).  workspace: 16-byte aligned device memory
 * of workspace_bytes, used only while the call's kernels run on `stream`
 * (calls on one stream may share it); with less than
 * qi_hip_w4a16_workspace_bytes(m, m_split, n, k) the call runs as the
 * workspace-free entry does.  No counterpart in the reference, whose one
 * W4A16 kernel has a fixed tile, no K split and dequantises in its loop
 * (gemm.cu:191-268). */
int qi_hip_w4a16_gemm_tiled_ws(const void *x_half, const void *w_tiled_codes, const void *w_tiled_scales,
                               const float *bias, void *y, int out_type, int epilogue, int m, int m_split, int n,
                               int k, int n_part, void *workspace, long long workspace_bytes, void *stream);
/* Workspace bytes the call above uses for (m, m_split, n, k); 0 when it
 * needs none (or the arguments are invalid).  A query only: no device
 * work. */
long long qi_hip_w4a16_workspace_bytes(int m, int m_split, int n, int k);

/* The kernel shape the W4A16 GEMMs above choose for m rows and n_out
 * outputs per stream: 0 GEMV (m <= 16), 1 K-split 64 x 64 tiles, 3 tiled
 * 64 x 64, 4 tiled 128 x 192, 5 tiled 256 x 256, 6 tiled 128 x 128, 7 tiled
 * 64 x 128; -1 for
 * m or n_out <= 0.  A query only (tests and tuning): no
 * device work.  No counterpart in the reference, whose one W4A16 kernel has
 * a fixed tile (gemm.cu:191-268). */
int qi_hip_w4a16_tiles(int m, int n_out);

/* Bandwidth-bound W4A16 GEMV for 1 <= m <= 16 (the adaLN / timestep
 * modulation linears).  Same arithmetic and layouts as above.  The
 * reference runs these linears as BF16 -> fp32 SGEMM
 * (qwen_image_cuda/src/transformer.cplus:716-730, cuda/blas.cu:138-142). */
int qi_hip_w4a16_gemv(const void *x_half, const void *w_tiled_codes, const void *w_tiled_scales,
                      const float *bias, void *y, int out_type, int epilogue, int m, int n, int k, void *stream);

/* fp6 operand path for W4A4.  The int4 codes -7..7 are exact in FP6 E2M3, so
 * the gfx950 f8f6f4 MFMA (32x32x64: K = one g64 group) yields the same exact
 * per-group integer partials as the int8 MFMA, already in fp32.  Layout of
 * both operands (7/8 byte per input): per 32-row tile T and 64-group g, 1792
 * bytes = half 0 (64 lanes x 16 bytes) then half 1 (64 lanes x 12 bytes);
 * lane l of half h holds the E2M3 codes (6 bits each, little-endian) of
 * inputs 32*(l/32) + 16h .. + 15 of the group, row 32T + l%32, and bytes
 * 12..15 of a half-0 slot hold that row's fp16 group scale, zero-extended.
 * The optional separate scale arrays are [rows/32][G][32] fp16 (tile, group,
 * row); pass NULL to skip them.
 *
 * Quantiser (same arithmetic and codes as qi_w4a4_quantize_activations):
 * x is f32 (x_is_half = 0) or fp16 [m, k]; codes6 holds ceil(m/32) * 32 rows
 * (rows past m get the codes of zeros, and the GEMM stores nothing from
 * them); k % 256 == 0; codes6 16-byte aligned. */
int qi_hip_w4a4_quantize_activations_fp6(const void *x, int x_is_half, void *codes6, void *scales_tiled, int m,
                                         int k, void *stream);
/* One-time re-layout of QIPACK W4A4 weights (codes [n, k/2], scales [n, G])
 * into the fp6 operand layout above, plus (unless NULL) tiled scales.
 * n % 32 == 0, k % 256 == 0. */
int qi_hip_relayout_w4a4_fp6(const void *codes, const void *scales, void *codes6, void *tiled_scales, int n, int k,
                             void *stream);
/* W4A4 GEMM on the fp6 operands (scales read from the code blocks); same
 * result, bit for bit, as qi_hip_w4a4_gemm_tiled on the same codes.  Any
 * m >= 1; n % 32 == 0; k % 256 == 0; both code buffers 16-byte aligned; y
 * aligned to 16 bytes (f32) or 8 bytes (f16). */
int qi_hip_w4a4_gemm_fp6(const void *a_codes6, const void *w_codes6, const float *bias, void *y, int out_type,
                         int epilogue, int m, int n, int k, void *stream);
/* The fp6 W4A4 GEMM over a fused record (parts as for
 * qi_hip_w4a16_gemm_tiled_parts; n_part % 32 == 0, n % n_part == 0).  Every
 * output is bit-identical to the per-record call's. */
int qi_hip_w4a4_gemm_fp6_parts(const void *a_codes6, const void *w_codes6, const float *bias, void *y,
                               int out_type, int epilogue, int m, int n, int k, int n_part, void *stream);
/* The tile shape qi_hip_w4a4_gemm_fp6[_parts] chooses for m rows and n
 * outputs: 0 = 128 x 128 tiles, one per workgroup; 1 = the same tiles walked
 * by the persistent kernel (m, n multiples of 128); 3 = 64 x 128 tiles; 4 =
 * single-wave 32 x 32 tiles; -1 for m or n <= 0.  A query only: no device
 * work.  No counterpart in the reference (fixed tile, gemm.cu:59-189). */
int qi_hip_w4a4_fp6_tiles(int m, int n);
/* Both streams of an MMDiT dual-stream block in one call (the reference
 * runs the image and the text stream's linear as two
 * transformer::linear calls on their own rows).  a_codes6: m rows of fp6
 * activation blocks, rows [0, m_split) of stream 0 and [m_split, m) of
 * stream 1 (one quantiser pass over the stacked rows); w_codes6: 2n weight
 * rows, the first n stream 0's record, the next n stream 1's (each possibly
 * a fused record with n / n_part parts); bias NULL or fp32 [2n].  y: n /
 * n_part parts of [m, n_part], every row holding its own stream's outputs.
 * Every output bit-identical to the per-stream calls.  0 < m_split < m,
 * m_split % 32 == 0, n % 32 == 0, n_part as above.  One persistent launch
 * when m, m_split and n are multiples of 128, else one launch per stream. */
int qi_hip_w4a4_gemm_fp6_dual(const void *a_codes6, const void *w_codes6, const float *bias, void *y,
                              int out_type, int epilogue, int m, int m_split, int n, int k, int n_part, void *stream);

/* Producers fused with the activation quantiser.  The reference runs the
 * LayerNorm-with-modulation-scale (qi_layer_norm_scale, ops.cu:56-59) and
 * SwiGLU (qi_swiglu, ops.cu:141-144) as kernels writing fp32 activations
 * that the quantiser then reads back (transformer.cplus:759-760, 808-813).
 *
 * qi_hip_layer_norm_scale: the reference's LayerNorm (affine-free, two-pass
 * variance, eps 1e-6) times (1 + scale[i]) with scale row 1 (at
 * scale + scale_stride) for rows < split and row 0 otherwise; fp32 or fp16
 * (RNE) output -- the fp16 form is the W4A16 path's input conversion fused
 * in.  width % 4 == 0; x, scale, out 16-byte aligned; scale_stride % 4 == 0.
 *
 * qi_hip_layer_norm_scale_quantize_fp6: the same values quantised straight
 * into the fp6 operand layout of qi_hip_w4a4_quantize_activations_fp6
 * (codes bit-identical to quantising qi_hip_layer_norm_scale's fp32
 * output).  row_stats is caller scratch of m * 8 bytes (per row: mean and
 * 1 / sqrt(variance + eps) as two floats).  k % 256 == 0.
 *
 * qi_hip_swiglu: out = gate / (1 + exp(-gate)) * up over count elements
 * (count % 4 == 0), fp32 or fp16 output.  qi_hip_swiglu_quantize_fp6: the
 * same values [m, k] quantised into the fp6 layout (bit-identical to
 * quantising qi_hip_swiglu's fp32 output); k % 256 == 0.
 *
 * Outputs agree with the reference formulas within a few fp32 ulps (the
 * reduction order and the rsqrt / exp implementations are this library's). */
int qi_hip_layer_norm_scale(const float *x, const float *scale, int scale_stride, void *out, int out_type, int rows,
                            int width, int split, void *stream);
int qi_hip_layer_norm_scale_quantize_fp6(const float *x, const float *scale, int scale_stride, int split,
                                         void *row_stats, void *codes6, int m, int k, void *stream);
/* qi_hip_layer_norm_scale_quantize_fp6 without a caller workspace, for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation).  No counterpart in
 * the reference.  Same arguments, kernels and codes as
 * qi_hip_layer_norm_scale_quantize_fp6 minus row_stats: the row statistics
 * live in a fixed device array of QI_HIP_NOALLOC_MAX_ROWS rows (8 bytes per
 * row) that the library holds on each GPU it runs on until the process
 * ends.  It calls no allocator.  m > QI_HIP_NOALLOC_MAX_ROWS returns
 * hipErrorInvalidValue before any launch.  All calls on one GPU share that
 * array: calls that overlap on one GPU (concurrent streams or threads) race
 * and must be serialised by the caller. */
#define QI_HIP_NOALLOC_MAX_ROWS 65536
int qi_hip_layer_norm_scale_quantize_fp6_noalloc(const float *x, const float *scale, int scale_stride, int split,
                                                 void *codes6, int m, int k, void *stream);
int qi_hip_swiglu(const float *gate, const float *up, void *out, int out_type, unsigned long long count,
                  void *stream);
int qi_hip_swiglu_quantize_fp6(const float *gate, const float *up, void *codes6, int m, int k, void *stream);

/* Fused attention (the reference's qi_flash_attention, qwen_image_cuda/
 * cuda/flash.cu:237-244, same arguments and layouts): head dim 128; q and
 * out fp32 [queries, heads * 128], k_half and v_half fp16 [keys, heads *
 * 128]; row r (global r + query_offset) sees keys [0, visible_keys[r]) when
 * visible_keys (device int array indexed by global row) is given, else
 * [0, r + 1) when r < causal_rows, else every key; rows with nothing visible
 * get 0.  Q is scaled by log2(e) / sqrt(128) and rounded to fp16, the
 * softmax runs online in the log2 domain with fp16 probabilities in the
 * P V product.  Pointers 16-byte aligned.  qi_flash_attention runs on the
 * null stream, as the reference does. */
int qi_flash_attention(const float *q, const void *k_half, const void *v_half, float *out, int queries, int keys,
                       int heads, int query_offset, int causal_rows, const int *visible_keys);
int qi_hip_flash_attention(const float *q, const void *k_half, const void *v_half, float *out, int queries, int keys,
                           int heads, int query_offset, int causal_rows, const int *visible_keys, void *stream);
/* The attention above with a caller workspace.  A call in which every row
 * sees every key (visible_keys NULL and causal_rows <= query_offset) and
 * whose (head, 256-query block) units leave a last round of CUs that its
 * units, each cut into 2-16 aligned key segments, fill in one round of
 * parts runs the whole rounds in lockstep, one workgroup per CU, then
 * those parts; each part's O, offset and sum go to the workspace and the
 * block's last part to finish merges them in segment order (so results
 * do not depend on timing).  Outputs agree with qi_hip_flash_attention within the
 * attention tolerance.  Masked calls, calls the split would not speed up,
 * and calls with less than
 * qi_hip_flash_attention_workspace_bytes(queries, keys, heads) run as
 * qi_hip_flash_attention does.  workspace: 16-byte aligned device memory
 * used only while the call's kernels run on `stream` (calls on one stream
 * may share it; its contents need no initialisation).  No counterpart in
 * the reference, whose grid is one workgroup per query block and head
 * (flash.cu:237-244). */
int qi_hip_flash_attention_ws(const float *q, const void *k_half, const void *v_half, float *out, int queries,
                              int keys, int heads, int query_offset, int causal_rows, const int *visible_keys,
                              void *workspace, long long workspace_bytes, void *stream);
/* Workspace bytes the call above uses for a mask-free call of (queries,
 * keys, heads) on the current device; 0 when it would not split (or the
 * arguments are invalid).  A query only: no device work. */
long long qi_hip_flash_attention_workspace_bytes(int queries, int keys, int heads);

/* Device-side QIPACK quantiser (int4_pack.cplus:237-468 arithmetic, bit-exact):
 * w_half fp16 [n, k] -> QIPACK arrays.  scheme 5 = W4A16 affine (minimums
 * required), scheme 6 = W4A4 H256 symmetric (minimums ignored).  group must
 * be 64; clip selects the 7-candidate range-shrink search. */
int qi_hip_pack_weights(const void *w_half, void *codes, void *scales, void *minimums, int n, int k, int scheme,
                        int clip, void *stream);

/* ---- QIPACK1 container, host side ------------------------------------------
 * Reading and checking a pack before its INT4 records are uploaded and
 * re-laid (layout int4_pack.cplus:55-95; the loader's header and policy test
 * transformer.cplus:342-375; the packer's verify int4_pack.cplus:733-850).
 * These functions do host file I/O only and return the QI_PACK_* codes below
 * (0 = success), not hipError_t. */
#define QI_PACK_OK 0
#define QI_PACK_EINVAL 1    /* bad argument or index */
#define QI_PACK_EIO 2       /* open / read failed */
#define QI_PACK_EFORMAT 3   /* not a QIPACK1 file, wrong size, unknown policy, wrong inventory */
#define QI_PACK_ELAYOUT 4   /* record geometry, alignment, order or bounds */
#define QI_PACK_EMETADATA 5 /* metadata checksum */
#define QI_PACK_ETENSOR 6   /* a tensor checksum */
#define QI_PACK_EPAYLOAD 7  /* payload checksum */

typedef struct qi_pack qi_pack; /* an open pack: header, directory, file */
typedef struct {                /* one 256-byte directory record, decoded */
    char name[129];
    uint32_t scheme, rank;
    uint64_t dims[4];
    uint32_t group_axis, group_size, scale_type, zero_type;
    uint64_t weights_offset, weights_length, scales_offset, scales_length, zeros_offset, zeros_length;
    uint64_t elements, tensor_checksum;
} qi_pack_record;

/* FNV-1a 64 over count bytes, continuing from hash (int4_pack.cplus:151-159). */
uint64_t qi_fnv1a(uint64_t hash, const void *bytes, uint64_t count);
/* Open: header (magic, size, directory placement) and directory. */
int qi_pack_open(const char *path, qi_pack **pack);
void qi_pack_close(qi_pack *pack);
/* policy33 receives the 32-byte policy string plus a terminating zero. */
int qi_pack_info(const qi_pack *pack, uint32_t *tensor_count, char *policy33, uint64_t *data_offset,
                 uint64_t *file_bytes);
int qi_pack_record_at(const qi_pack *pack, uint32_t index, qi_pack_record *record);
/* Index of the record named `name`, or -1. */
int qi_pack_find(const qi_pack *pack, const char *name);
/* length bytes from file offset into host memory dst. */
int qi_pack_read(const qi_pack *pack, uint64_t offset, uint64_t length, void *dst);
/* The verify of int4_pack.cplus:733-850: policy, metadata placement and
 * checksum, INT4 record geometry, 256-aligned monotonic tensors inside the
 * data section ending at the file end, every tensor checksum, the payload
 * checksum; expect_transformer != 0 also requires the full transformer
 * inventory (297 tensors, 224 INT4 matrices). */
int qi_pack_verify(const qi_pack *pack, int expect_transformer);

#ifdef __cplusplus
}
#endif
#endif /* QWEN_IMAGE_HIP_H */
