"""Torch-tensor wrappers over the C ABI.  torch supplies device memory and the
current HIP stream; every computation happens in the gfx950 kernels.

Shapes and dtypes follow the QIPACK arrays: codes are uint8 [N, K/2], scales
and minimums are fp16 [N, K/64]; activation codes/scales use the same layout
with M rows.  fp16 tensors are passed as torch.float16.
"""
from __future__ import annotations

import torch

from ._lib import check, load

OUT_F32 = 0
OUT_F16 = 1
EPILOGUE_NONE = 0
EPILOGUE_GELU_TANH = 1
GROUP = 64


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("qwen_image_hip ops take device tensors")
    if not t.is_contiguous():
        raise ValueError("qwen_image_hip ops take contiguous tensors")
    return t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _empty(shape, dtype, like: torch.Tensor) -> torch.Tensor:
    return torch.empty(shape, dtype=dtype, device=like.device)


# ----------------------------------------------------------- activations --


def quantize_activations(x: torch.Tensor, codes: torch.Tensor | None = None, scales: torch.Tensor | None = None):
    """H256-rotate and int4-quantise rows of x (fp32 or fp16) -> (codes, scales).

    Reference: qwen_image_cuda/cuda/gemm.cu:22-57.
    """
    m, k = x.shape
    codes = codes if codes is not None else _empty((m, k // 2), torch.uint8, x)
    scales = scales if scales is not None else _empty((m, k // GROUP), torch.float16, x)
    lib = load()
    if x.dtype == torch.float32:
        st = lib.qi_hip_w4a4_quantize_activations(_ptr(x), _ptr(codes), _ptr(scales), m, k, _stream())
    elif x.dtype == torch.float16:
        st = lib.qi_hip_w4a4_quantize_activations_f16(_ptr(x), _ptr(codes), _ptr(scales), m, k, _stream())
    else:
        raise TypeError("activations must be float32 or float16")
    check(st, "activation quantization")
    return codes, scales


def f32_to_f16(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """RNE fp32 -> fp16 (reference qwen_image_cuda/cuda/ops.cu:204-212)."""
    out = out if out is not None else _empty(x.shape, torch.float16, x)
    check(load().qi_hip_f32_to_f16(_ptr(x), _ptr(out), x.numel(), _stream()), "activation conversion")
    return out


# ------------------------------------------------------------------ packing --


def pack_weights(w_half: torch.Tensor, scheme: int, clip: bool = False):
    """QIPACK-quantise an fp16 [N, K] matrix on the device.

    scheme 5 -> (codes, scales, minimums) W4A16 affine; scheme 6 -> (codes,
    scales, None) W4A4 with the H256 rotation.  Same arithmetic as the
    reference packer (qwen_image_cuda/src/int4_pack.cplus:237-468).
    """
    n, k = w_half.shape
    codes = _empty((n, k // 2), torch.uint8, w_half)
    scales = _empty((n, k // GROUP), torch.float16, w_half)
    mins = _empty((n, k // GROUP), torch.float16, w_half) if scheme == 5 else None
    st = load().qi_hip_pack_weights(_ptr(w_half), _ptr(codes), _ptr(scales), _ptr(mins), n, k, scheme,
                                    1 if clip else 0, _stream())
    check(st, "weight packing")
    return codes, scales, mins


def relayout_w4a4(codes: torch.Tensor, scales: torch.Tensor):
    n, half_k = codes.shape
    k = half_k * 2
    tc = torch.empty_like(codes)
    ts = torch.empty_like(scales)
    check(load().qi_hip_relayout_w4a4(_ptr(codes), _ptr(scales), _ptr(tc), _ptr(ts), n, k, _stream()), "relayout")
    return tc, ts


def relayout_w4a4_inverse(tiled_codes: torch.Tensor, tiled_scales: torch.Tensor):
    n, half_k = tiled_codes.shape
    k = half_k * 2
    c = torch.empty_like(tiled_codes)
    s = torch.empty_like(tiled_scales)
    check(load().qi_hip_relayout_w4a4_inverse(_ptr(tiled_codes), _ptr(tiled_scales), _ptr(c), _ptr(s), n, k,
                                              _stream()), "relayout inverse")
    return c, s


def relayout_w4a16(codes: torch.Tensor, scales: torch.Tensor, minimums: torch.Tensor):
    n, half_k = codes.shape
    k = half_k * 2
    tc = torch.empty_like(codes)
    ts = _empty((n, 2 * (k // GROUP)), torch.float16, codes)
    check(load().qi_hip_relayout_w4a16(_ptr(codes), _ptr(scales), _ptr(minimums), _ptr(tc), _ptr(ts), n, k,
                                       _stream()), "relayout")
    return tc, ts


def relayout_w4a16_inverse(tiled_codes: torch.Tensor, tiled_scales: torch.Tensor):
    n, half_k = tiled_codes.shape
    k = half_k * 2
    c = torch.empty_like(tiled_codes)
    s = _empty((n, k // GROUP), torch.float16, tiled_codes)
    mn = _empty((n, k // GROUP), torch.float16, tiled_codes)
    check(load().qi_hip_relayout_w4a16_inverse(_ptr(tiled_codes), _ptr(tiled_scales), _ptr(c), _ptr(s), _ptr(mn),
                                               n, k, _stream()), "relayout inverse")
    return c, s, mn


# -------------------------------------------------------------------- GEMMs --


def w4a4_gemm_reference(a_codes, a_scales, w_codes, w_scales, y=None):
    """Reference-ABI W4A4 GEMM (QIPACK weight layout, fp32 out, null stream).

    Reference: qwen_image_cuda/cuda/gemm.cu:183-189.
    """
    m, n, k = a_codes.shape[0], w_codes.shape[0], a_codes.shape[1] * 2
    y = y if y is not None else _empty((m, n), torch.float32, a_codes)
    torch.cuda.current_stream().synchronize()
    check(load().qi_w4a4_gemm(_ptr(a_codes), _ptr(a_scales), _ptr(w_codes), _ptr(w_scales), _ptr(y), m, n, k),
          "w4a4 gemm")
    torch.cuda.synchronize()
    return y


def w4a16_gemm_reference(x_half, codes, scales, minimums, y=None):
    """Reference-ABI W4A16 GEMM (gemm.cu:262-268), null stream."""
    m, k = x_half.shape
    n = codes.shape[0]
    y = y if y is not None else _empty((m, n), torch.float32, x_half)
    torch.cuda.current_stream().synchronize()
    check(load().qi_w4a16_gemm(_ptr(x_half), _ptr(codes), _ptr(scales), _ptr(minimums), _ptr(y), m, n, k),
          "w4a16 gemm")
    torch.cuda.synchronize()
    return y


def w4a4_gemm(a_codes, a_scales, w_tiled_codes, w_tiled_scales, bias=None, out_dtype=torch.float32,
              gelu=False, y=None):
    m, n, k = a_codes.shape[0], w_tiled_codes.shape[0], a_codes.shape[1] * 2
    out_type = OUT_F16 if out_dtype == torch.float16 else OUT_F32
    y = y if y is not None else _empty((m, n), out_dtype, a_codes)
    st = load().qi_hip_w4a4_gemm_tiled(_ptr(a_codes), _ptr(a_scales), _ptr(w_tiled_codes), _ptr(w_tiled_scales),
                                       _ptr(bias), _ptr(y), out_type, EPILOGUE_GELU_TANH if gelu else EPILOGUE_NONE,
                                       m, n, k, _stream())
    check(st, "w4a4 gemm")
    return y


def _out_shape(m: int, n: int, n_part: int | None):
    if n_part is None or n_part == n:
        return (m, n)
    if n_part <= 0 or n % n_part:
        raise ValueError(f"n_part {n_part} does not divide n {n}")
    return (n // n_part, m, n_part)


def _w4a16_call(x_half, w_tiled_codes, w_tiled_scales, bias, y, out_type, gelu, m, m_split, n, k, n_part,
                split_k):
    lib = load()
    epi = EPILOGUE_GELU_TANH if gelu else EPILOGUE_NONE
    n_part = n if n_part is None else n_part
    if not split_k:
        if m_split:
            return lib.qi_hip_w4a16_gemm_tiled_dual(_ptr(x_half), _ptr(w_tiled_codes), _ptr(w_tiled_scales),
                                                    _ptr(bias), _ptr(y), out_type, epi, m, m_split, n, k, n_part,
                                                    _stream())
        return lib.qi_hip_w4a16_gemm_tiled_parts(_ptr(x_half), _ptr(w_tiled_codes), _ptr(w_tiled_scales), _ptr(bias),
                                                 _ptr(y), out_type, epi, m, n, k, n_part, _stream())
    # The K-split workspace comes from torch's caching allocator on the
    # current stream (so it is also valid under graph capture).
    ws_bytes = lib.qi_hip_w4a16_workspace_bytes(m, m_split, n, k)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=x_half.device) if ws_bytes > 0 else None
    return lib.qi_hip_w4a16_gemm_tiled_ws(_ptr(x_half), _ptr(w_tiled_codes), _ptr(w_tiled_scales), _ptr(bias),
                                          _ptr(y), out_type, epi, m, m_split, n, k, n_part, _ptr(ws), ws_bytes,
                                          _stream())


def w4a16_gemm(x_half, w_tiled_codes, w_tiled_scales, bias=None, out_dtype=torch.float32, gelu=False, y=None,
               n_part=None, split_k=True):
    """y = x . W^T for tiled W4A16 weights; with n_part, y is [n / n_part, m, n_part]
    (the parts of a fused record).  split_k: qi_hip_w4a16_gemm_tiled_ws with a
    workspace (K split over workgroups where the library chooses one), else
    qi_hip_w4a16_gemm_tiled_parts."""
    m, k = x_half.shape
    n = w_tiled_codes.shape[0]
    out_type = OUT_F16 if out_dtype == torch.float16 else OUT_F32
    y = y if y is not None else _empty(_out_shape(m, n, n_part), out_dtype, x_half)
    check(_w4a16_call(x_half, w_tiled_codes, w_tiled_scales, bias, y, out_type, gelu, m, 0, n, k, n_part, split_k),
          "w4a16 gemm")
    return y


def w4a16_gemm_dual(x_half, w_tiled_codes, w_tiled_scales, m_split: int, bias=None, out_dtype=torch.float32,
                    gelu=False, y=None, n_part=None, split_k=True):
    """Both streams of a dual-stream block: rows < m_split use the first half
    of the weight rows, the others the second; y is [m, n] (or [n / n_part,
    m, n_part]), n = weight rows / 2.  split_k as in w4a16_gemm (else
    qi_hip_w4a16_gemm_tiled_dual)."""
    m, k = x_half.shape
    n = w_tiled_codes.shape[0] // 2
    if m_split <= 0:
        raise ValueError("m_split must be positive")
    out_type = OUT_F16 if out_dtype == torch.float16 else OUT_F32
    y = y if y is not None else _empty(_out_shape(m, n, n_part), out_dtype, x_half)
    check(_w4a16_call(x_half, w_tiled_codes, w_tiled_scales, bias, y, out_type, gelu, m, m_split, n, k, n_part,
                      split_k), "w4a16 gemm")
    return y


def w4a16_gemv(x_half, w_tiled_codes, w_tiled_scales, bias=None, out_dtype=torch.float32, gelu=False, y=None):
    m, k = x_half.shape
    n = w_tiled_codes.shape[0]
    out_type = OUT_F16 if out_dtype == torch.float16 else OUT_F32
    y = y if y is not None else _empty((m, n), out_dtype, x_half)
    st = load().qi_hip_w4a16_gemv(_ptr(x_half), _ptr(w_tiled_codes), _ptr(w_tiled_scales), _ptr(bias), _ptr(y),
                                  out_type, EPILOGUE_GELU_TANH if gelu else EPILOGUE_NONE, m, n, k, _stream())
    check(st, "w4a16 gemv")
    return y


# ------------------------------------------------------------ fp6 W4A4 path --


def fp6_rows(m: int) -> int:
    """Rows an fp6 activation buffer holds for m rows (whole 32-row tiles)."""
    return (m + 31) // 32 * 32


def fp6_row_bytes(k: int) -> int:
    """Bytes of one row of an fp6 operand buffer: 1792 per 32 rows and group."""
    return k // GROUP * 56


def quantize_activations_fp6(x: torch.Tensor, codes6: torch.Tensor | None = None,
                             scales: torch.Tensor | None = None, want_scales: bool = False):
    """Quantise rows of x into the fp6 MFMA-operand layout.

    Returns (codes6 uint8 [ceil(m/32)*32, 7k/8], scales) in tile order (see
    qwen_image_hip.h); the code blocks carry the scales.  ``scales`` (fp16
    [ceil(m/32)*32, k/64], tile order) is also written when given or when
    ``want_scales``, else None.  Same codes as quantize_activations.
    """
    m, k = x.shape
    rows = fp6_rows(m)
    codes6 = codes6 if codes6 is not None else _empty((rows, fp6_row_bytes(k)), torch.uint8, x)
    if scales is None and want_scales:
        scales = _empty((rows, k // GROUP), torch.float16, x)
    if x.dtype not in (torch.float32, torch.float16):
        raise TypeError("activations must be float32 or float16")
    st = load().qi_hip_w4a4_quantize_activations_fp6(_ptr(x), 1 if x.dtype == torch.float16 else 0, _ptr(codes6),
                                                     _ptr(scales), m, k, _stream())
    check(st, "activation quantization")
    return codes6, scales


def relayout_w4a4_fp6(codes: torch.Tensor, scales: torch.Tensor, want_scales: bool = False):
    """QIPACK W4A4 arrays -> (fp6 operand blocks [n, 7k/8], tiled scales or None)."""
    n, half_k = codes.shape
    k = half_k * 2
    c6 = _empty((n, fp6_row_bytes(k)), torch.uint8, codes)
    ts = torch.empty_like(scales) if want_scales else None
    check(load().qi_hip_relayout_w4a4_fp6(_ptr(codes), _ptr(scales), _ptr(c6), _ptr(ts), n, k, _stream()),
          "relayout")
    return c6, ts


def w4a4_gemm_fp6(a_codes6, w_codes6, m: int, bias=None, out_dtype=torch.float32, gelu=False, y=None,
                  n_part=None):
    """fp6-operand W4A4 GEMM; with n_part, y is [n / n_part, m, n_part]
    (qi_hip_w4a4_gemm_fp6_parts)."""
    n, k = w_codes6.shape[0], w_codes6.shape[1] // 56 * GROUP
    out_type = OUT_F16 if out_dtype == torch.float16 else OUT_F32
    y = y if y is not None else _empty(_out_shape(m, n, n_part), out_dtype, w_codes6)
    st = load().qi_hip_w4a4_gemm_fp6_parts(_ptr(a_codes6), _ptr(w_codes6), _ptr(bias), _ptr(y), out_type,
                                           EPILOGUE_GELU_TANH if gelu else EPILOGUE_NONE, m, n, k,
                                           n if n_part is None else n_part, _stream())
    check(st, "w4a4 gemm")
    return y



def w4a4_gemm_fp6_dual(a_codes6, w_codes6, m: int, m_split: int, bias=None, out_dtype=torch.float32, gelu=False,
                       y=None, n_part=None):
    """Both streams of a dual-stream block (qi_hip_w4a4_gemm_fp6_dual): rows
    < m_split use the first half of w_codes6's rows, the others the second;
    y is [m, n] (or [n / n_part, m, n_part]) with n = w_codes6 rows / 2."""
    n2, k = w_codes6.shape[0], w_codes6.shape[1] // 56 * GROUP
    n = n2 // 2
    out_type = OUT_F16 if out_dtype == torch.float16 else OUT_F32
    y = y if y is not None else _empty(_out_shape(m, n, n_part), out_dtype, w_codes6)
    st = load().qi_hip_w4a4_gemm_fp6_dual(_ptr(a_codes6), _ptr(w_codes6), _ptr(bias), _ptr(y), out_type,
                                          EPILOGUE_GELU_TANH if gelu else EPILOGUE_NONE, m, m_split, n, k,
                                          n if n_part is None else n_part, _stream())
    check(st, "w4a4 gemm")
    return y

# ------------------------------------------------- producers + quantiser --


def layer_norm_scale(x: torch.Tensor, scale: torch.Tensor, split: int = 0, out_dtype=torch.float32,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """The reference's LayerNorm with modulation scale (ops.cu:37-59) on fp32
    x [rows, width]; scale is fp32 [2, width] (row 1 for rows < split)."""
    rows, width = x.shape
    if x.dtype != torch.float32 or scale.dtype != torch.float32 or scale.shape != (2, width):
        raise ValueError("x fp32 [rows, width] and scale fp32 [2, width]")
    out = out if out is not None else _empty((rows, width), out_dtype, x)
    out_type = OUT_F16 if out.dtype == torch.float16 else OUT_F32
    check(load().qi_hip_layer_norm_scale(_ptr(x), _ptr(scale), width, _ptr(out), out_type, rows, width, split,
                                         _stream()), "layer norm")
    return out


def layer_norm_scale_quantize_fp6(x: torch.Tensor, scale: torch.Tensor, split: int = 0,
                                  codes6: torch.Tensor | None = None, row_stats: torch.Tensor | None = None):
    """layer_norm_scale fused with quantize_activations_fp6: codes only."""
    m, k = x.shape
    if x.dtype != torch.float32 or scale.dtype != torch.float32 or scale.shape != (2, k):
        raise ValueError("x fp32 [m, k] and scale fp32 [2, k]")
    codes6 = codes6 if codes6 is not None else _empty((fp6_rows(m), fp6_row_bytes(k)), torch.uint8, x)
    row_stats = row_stats if row_stats is not None else _empty((m, 2), torch.float32, x)
    check(load().qi_hip_layer_norm_scale_quantize_fp6(_ptr(x), _ptr(scale), k, split, _ptr(row_stats),
                                                      _ptr(codes6), m, k, _stream()), "layer norm quantization")
    return codes6


def swiglu(gate: torch.Tensor, up: torch.Tensor, out_dtype=torch.float32, out: torch.Tensor | None = None):
    """silu(gate) * up on fp32 tensors (ops.cu:134-144)."""
    if gate.dtype != torch.float32 or up.shape != gate.shape or up.dtype != torch.float32:
        raise ValueError("gate and up: fp32 tensors of one shape")
    out = out if out is not None else _empty(gate.shape, out_dtype, gate)
    out_type = OUT_F16 if out.dtype == torch.float16 else OUT_F32
    check(load().qi_hip_swiglu(_ptr(gate), _ptr(up), _ptr(out), out_type, gate.numel(), _stream()), "swiglu")
    return out


def swiglu_quantize_fp6(gate: torch.Tensor, up: torch.Tensor, codes6: torch.Tensor | None = None):
    """swiglu fused with quantize_activations_fp6: codes only."""
    m, k = gate.shape
    if gate.dtype != torch.float32 or up.shape != gate.shape or up.dtype != torch.float32:
        raise ValueError("gate and up: fp32 tensors of one shape")
    codes6 = codes6 if codes6 is not None else _empty((fp6_rows(m), fp6_row_bytes(k)), torch.uint8, gate)
    check(load().qi_hip_swiglu_quantize_fp6(_ptr(gate), _ptr(up), _ptr(codes6), m, k, _stream()),
          "swiglu quantization")
    return codes6


# --------------------------------------------------------------- attention --


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, heads: int, query_offset: int = 0,
                    causal_rows: int = 0, visible_keys: torch.Tensor | None = None,
                    out: torch.Tensor | None = None, balanced: bool = True) -> torch.Tensor:
    """Fused attention, head dim 128 (reference qi_flash_attention,
    qwen_image_cuda/cuda/flash.cu): q fp32 [queries, heads*128], k and v fp16
    [keys, heads*128]; visible_keys an int32 device tensor indexed by global row.
    balanced: mask-free calls spread their key tiles evenly over the CUs
    (qi_hip_flash_attention_ws, workspace from torch's caching allocator);
    False runs the one-workgroup-per-query-block grid."""
    nq, width = q.shape
    if q.dtype != torch.float32 or k.dtype != torch.float16 or v.dtype != torch.float16:
        raise TypeError("q fp32, k and v fp16")
    if width != heads * 128 or k.shape[1] != width or v.shape != k.shape:
        raise ValueError("q, k, v must be [rows, heads * 128]")
    if visible_keys is not None and visible_keys.dtype != torch.int32:
        raise TypeError("visible_keys must be int32")
    out = out if out is not None else _empty((nq, width), torch.float32, q)
    lib = load()
    mask_free = visible_keys is None and causal_rows <= query_offset
    ws_bytes = lib.qi_hip_flash_attention_workspace_bytes(nq, k.shape[0], heads) if balanced and mask_free else 0
    if ws_bytes > 0:
        ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=q.device)
        check(lib.qi_hip_flash_attention_ws(_ptr(q), _ptr(k), _ptr(v), _ptr(out), nq, k.shape[0], heads,
                                            query_offset, causal_rows, None, _ptr(ws), ws_bytes, _stream()),
              "attention")
        return out
    check(lib.qi_hip_flash_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(out), nq, k.shape[0], heads, query_offset,
                                     causal_rows, _ptr(visible_keys), _stream()), "attention")
    return out
