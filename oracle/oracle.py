"""numpy-facing ctypes binding of the CPU oracle (oracle/qi_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker / CPU baseline.  The product
never imports this module.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libqi_oracle.so"

_lib = None
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.qo_half_to_f32.argtypes = [ctypes.c_uint16]
        L.qo_half_to_f32.restype = ctypes.c_float
        L.qo_half_from_f32.argtypes = [ctypes.c_float]
        L.qo_half_from_f32.restype = ctypes.c_uint16
        L.qo_half_round.argtypes = [ctypes.c_float]
        L.qo_half_round.restype = ctypes.c_float
        L.qo_f32_to_f16.argtypes = [_P, _P, ctypes.c_uint64]
        L.qo_hadamard256.argtypes = [_P]
        L.qo_quantize_affine_group.argtypes = [_P, _I, _I, _P, _P, _P]
        L.qo_quantize_symmetric_group.argtypes = [_P, _I, _I, _P, _P]
        L.qo_quantize_matrix.argtypes = [_P, _I64, _I64, _I, _I, _I, _P, _P, _P]
        L.qo_quantize_matrix.restype = _I
        L.qo_quantize_activations_f32.argtypes = [_P, _P, _P, _I64, _I]
        L.qo_quantize_activations_f16.argtypes = [_P, _P, _P, _I64, _I]
        L.qo_rotate_rows.argtypes = [_P, _I64, _I]
        L.qo_w4a4_partials.argtypes = [_P, _P, _P, _I64, _I64, _I64]
        L.qo_w4a4_gemm.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64]
        L.qo_w4a4_gemm_f64.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64]
        L.qo_w4a16_dequantize.argtypes = [_P, _P, _P, _P, _I64, _I64]
        L.qo_gemm_f16.argtypes = [_P, _P, _P, _I64, _I64, _I64, _I]
        L.qo_sgemm_nt.argtypes = [_P, _P, _P, _I64, _I64, _I64]
        L.qo_w4a16_gemv.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64]
        L.qo_gelu_tanh.argtypes = [ctypes.c_float]
        L.qo_gelu_tanh.restype = ctypes.c_float
        L.qo_fnv1a.argtypes = [ctypes.c_uint64, _P, ctypes.c_uint64]
        L.qo_fnv1a.restype = ctypes.c_uint64
        L.qo_num_threads.restype = _I
        _lib = L
    return _lib


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


# fp16 bits are carried as uint16 arrays throughout.

def half_from_f32(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().qo_f32_to_f16(_p(x), _p(out), x.size)
    return out


def half_to_f32(bits) -> np.ndarray:
    bits = _c(bits, np.uint16)
    return np.vectorize(lambda b: lib().qo_half_to_f32(int(b)), otypes=[np.float32])(bits) if bits.size < 4096 \
        else bits.view(np.float16).astype(np.float32)


def hadamard256(v) -> np.ndarray:
    v = _c(v, np.float32).copy()
    assert v.size == 256
    lib().qo_hadamard256(_p(v))
    return v


def rotate_rows(x) -> np.ndarray:
    x = _c(x, np.float32).copy()
    m, k = x.shape
    lib().qo_rotate_rows(_p(x), m, k)
    return x


def quantize_affine_group(values, clip=False):
    v = _c(values, np.float32)
    codes = np.zeros(v.size, np.uint8)
    s = np.zeros(1, np.uint16)
    mn = np.zeros(1, np.uint16)
    lib().qo_quantize_affine_group(_p(v), v.size, int(clip), _p(codes), _p(s), _p(mn))
    return codes, int(s[0]), int(mn[0])


def quantize_symmetric_group(values, clip=False):
    v = _c(values, np.float32)
    codes = np.zeros(v.size, np.uint8)
    s = np.zeros(1, np.uint16)
    lib().qo_quantize_symmetric_group(_p(v), v.size, int(clip), _p(codes), _p(s))
    return codes, int(s[0])


def quantize_matrix(w_half_bits, scheme: int, clip: bool = False, group: int = 64):
    """fp16 bits [n, k] -> (codes u8 [n, k/2], scales u16 [n, G], minimums u16 [n, G] or None)."""
    w = _c(w_half_bits, np.uint16)
    n, k = w.shape
    codes = np.zeros((n, k // 2), np.uint8)
    scales = np.zeros((n, k // group), np.uint16)
    mins = np.zeros((n, k // group), np.uint16)
    rc = lib().qo_quantize_matrix(_p(w), n, k, scheme, group, int(clip), _p(codes), _p(scales), _p(mins))
    if rc != 0:
        raise ValueError(f"quantize_matrix rejected the shape (rc={rc})")
    return codes, scales, (mins if scheme == 5 else None)


def quantize_activations(x):
    """fp32 [m, k] or fp16 bits (uint16) [m, k] -> (codes [m, k/2], scales u16 [m, k/64])."""
    m, k = x.shape
    codes = np.zeros((m, k // 2), np.uint8)
    scales = np.zeros((m, k // 64), np.uint16)
    if x.dtype == np.uint16:
        xx = _c(x, np.uint16)
        lib().qo_quantize_activations_f16(_p(xx), _p(codes), _p(scales), m, k)
    else:
        xx = _c(x, np.float32)
        lib().qo_quantize_activations_f32(_p(xx), _p(codes), _p(scales), m, k)
    return codes, scales


def w4a4_partials(a_codes, w_codes) -> np.ndarray:
    a = _c(a_codes, np.uint8)
    w = _c(w_codes, np.uint8)
    m, n, k = a.shape[0], w.shape[0], a.shape[1] * 2
    out = np.zeros((m, n, k // 64), np.int32)
    lib().qo_w4a4_partials(_p(a), _p(w), _p(out), m, n, k)
    return out


def w4a4_gemm(a_codes, a_scales, w_codes, w_scales, f64=False) -> np.ndarray:
    a, sa, w, sw = _c(a_codes, np.uint8), _c(a_scales, np.uint16), _c(w_codes, np.uint8), _c(w_scales, np.uint16)
    m, n, k = a.shape[0], w.shape[0], a.shape[1] * 2
    if f64:
        y = np.zeros((m, n), np.float64)
        lib().qo_w4a4_gemm_f64(_p(a), _p(sa), _p(w), _p(sw), _p(y), m, n, k)
    else:
        y = np.zeros((m, n), np.float32)
        lib().qo_w4a4_gemm(_p(a), _p(sa), _p(w), _p(sw), _p(y), m, n, k)
    return y


def w4a16_dequantize(codes, scales, mins) -> np.ndarray:
    c, s, mn = _c(codes, np.uint8), _c(scales, np.uint16), _c(mins, np.uint16)
    n, k = c.shape[0], c.shape[1] * 2
    w = np.zeros((n, k), np.uint16)
    lib().qo_w4a16_dequantize(_p(c), _p(s), _p(mn), _p(w), n, k)
    return w


def gemm_f16(x_bits, w_bits, precise=True) -> np.ndarray:
    x, w = _c(x_bits, np.uint16), _c(w_bits, np.uint16)
    m, k = x.shape
    n = w.shape[0]
    y = np.zeros((m, n), np.float32)
    lib().qo_gemm_f16(_p(x), _p(w), _p(y), m, n, k, int(precise))
    return y


def w4a16_gemm(x_bits, codes, scales, mins, precise=True) -> np.ndarray:
    return gemm_f16(x_bits, w4a16_dequantize(codes, scales, mins), precise)


def w4a16_gemv(x_bits, codes, scales, mins) -> np.ndarray:
    """W4A16 for a few rows with per-row dequantisation and fp32 dots (the
    CPU baseline of the modulation linears)."""
    x, c, s, mn = _c(x_bits, np.uint16), _c(codes, np.uint8), _c(scales, np.uint16), _c(mins, np.uint16)
    m, k = x.shape
    n = c.shape[0]
    y = np.zeros((m, n), np.float32)
    lib().qo_w4a16_gemv(_p(x), _p(c), _p(s), _p(mn), _p(y), m, n, k)
    return y


def gelu_tanh(v) -> np.ndarray:
    f = np.vectorize(lambda t: lib().qo_gelu_tanh(float(t)), otypes=[np.float32])
    return f(_c(v, np.float32))


def fnv1a(data: bytes, h: int = 14695981039346656037) -> int:
    buf = np.frombuffer(data, np.uint8)
    return int(lib().qo_fnv1a(h, _p(buf), buf.size))


def num_threads() -> int:
    return int(lib().qo_num_threads())


def layer_norm_scale(x, scale, split=0) -> np.ndarray:
    """The reference's LayerNorm with modulation scale in float64
    (qwen_image_cuda/cuda/ops.cu:37-53): per row, mean, mean of squared
    deviations (two passes), (x - mean) / sqrt(var + 1e-6) * (1 + s) with s =
    scale[1] for rows < split, else scale[0].  float64 result."""
    x = np.asarray(x, np.float64)
    scale = np.asarray(scale, np.float64)
    mean = x.mean(axis=1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=1, keepdims=True)
    rows = np.arange(x.shape[0])[:, None]
    s = np.where(rows < split, scale[1][None, :], scale[0][None, :])
    return (x - mean) / np.sqrt(var + 1e-6) * (1.0 + s)


def swiglu(gate, up) -> np.ndarray:
    """silu(gate) * up in float64 (qwen_image_cuda/cuda/ops.cu:134-139)."""
    g = np.asarray(gate, np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(up, np.float64)


def flash_attention(q, k_bits, v_bits, heads: int, query_offset: int = 0, causal_rows: int = 0,
                    visible_keys=None, round_p: bool = True) -> np.ndarray:
    """The reference's fused attention in float64 (qwen_image_cuda/cuda/flash.cu:
    1-244): head dim 128; q fp32 [Q, heads*128] is scaled by log2(e)/sqrt(128) in
    fp32 and rounded to fp16 (:86-97); k, v are fp16 bits [K, heads*128]; row r
    (global r + query_offset) sees keys [0, visible_keys[r]) or, without that
    array, [0, r + 1) when r < causal_rows, else all (:46-49); softmax in the
    log2 domain; the P V product uses fp16 probabilities (round_p) while the
    sum adds the unrounded ones (:178-186); rows with nothing visible give 0."""
    d = 128
    q = np.asarray(q, np.float32)
    nq, nk = q.shape[0], np.asarray(k_bits).shape[0]
    scale = np.float32(1.4426950408889634) / np.sqrt(np.float32(d))
    qs = half_to_f32(half_from_f32(q * scale)).astype(np.float64)
    k = half_to_f32(k_bits).astype(np.float64)
    v = half_to_f32(v_bits).astype(np.float64)
    rows = np.arange(nq) + query_offset
    if visible_keys is not None:
        vis = np.minimum(np.asarray(visible_keys)[rows], nk)
    else:
        vis = np.where(rows < causal_rows, rows + 1, nk)
    mask = np.arange(nk)[None, :] < vis[:, None]
    out = np.zeros((nq, heads * d))
    for h in range(heads):
        sl = slice(h * d, (h + 1) * d)
        s = qs[:, sl] @ k[:, sl].T
        s = np.where(mask, s, -np.inf)
        m = s.max(axis=1, keepdims=True)
        m = np.where(np.isfinite(m), m, 0.0)
        p = np.exp2(s - m)
        tot = p.sum(axis=1, keepdims=True)
        pv = half_to_f32(half_from_f32(p.astype(np.float32))).astype(np.float64) if round_p else p
        o = pv @ v[:, sl]
        out[:, sl] = np.where(tot > 0, o / np.where(tot > 0, tot, 1.0), 0.0)
    return out
