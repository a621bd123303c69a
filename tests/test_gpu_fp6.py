"""GPU parity of the fp6-operand W4A4 path: quantiser codes, weight re-layout,
and the GEMM (bit-exact with the oracle's reference-order fp32 formula, and
exposing exact int32 group partials)."""
import numpy as np
import pytest
import torch

import oracle
from _data import heavy_tailed, weights_f16

pytestmark = pytest.mark.gpu

_MAG = {0: 0, 8: 1, 16: 2, 20: 3, 24: 4, 26: 5, 28: 6, 30: 7}


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _h(bits, dev):
    return _dev(np.ascontiguousarray(bits).view(np.float16), dev)


def _u16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def fp6_blocks(buf: np.ndarray, rows: int, k: int):
    """fp6 operand blocks [rows/32][G][1792 B] -> (code bytes [rows/32, G, 2, 64, 12],
    half-0 slot tails [rows/32, G, 64, 4]).

    Per block: half 0 = 64 lanes x 16 B (12 code bytes, then the row's fp16
    scale and two zero bytes), half 1 = 64 lanes x 12 code bytes.
    """
    G = k // 64
    blk = buf.reshape(rows // 32, G, 1792)
    h0 = blk[..., :1024].reshape(rows // 32, G, 64, 16)
    h1 = blk[..., 1024:].reshape(rows // 32, G, 64, 12)
    return np.stack([h0[..., :12], h1], axis=2), h0[..., 12:]


def fp6_scales(buf: np.ndarray, rows: int, k: int) -> np.ndarray:
    """The scales carried by fp6 blocks, as [rows, G] fp16 bits (lanes 0..31
    and 32..63 must agree; the two pad bytes must be zero)."""
    _, tail = fp6_blocks(buf, rows, k)
    t = np.ascontiguousarray(tail).view(np.uint16)          # [T, G, 64, 2]
    assert (t[..., 1] == 0).all()
    np.testing.assert_array_equal(t[:, :, :32, 0], t[:, :, 32:, 0])
    return t[:, :, :32, 0].transpose(0, 2, 1).reshape(rows, k // 64)


def set_fp6_scales(buf: np.ndarray, rows: int, k: int, scales: np.ndarray) -> np.ndarray:
    """Copy of fp6 blocks with the carried scales replaced by [rows, G] fp16 bits."""
    G = k // 64
    out = buf.copy().reshape(rows // 32, G, 1792)
    h0 = out[..., :1024].reshape(rows // 32, G, 64, 16)
    s = np.ascontiguousarray(scales.reshape(rows // 32, 32, G).transpose(0, 2, 1)).astype(np.uint16)
    for half in range(2):
        h0[:, :, 32 * half:32 * half + 32, 12:14] = s.view(np.uint8).reshape(rows // 32, G, 32, 2)
    out[..., :1024] = h0.reshape(rows // 32, G, 1024)
    return out.reshape(buf.shape)


def decode_fp6_tiles(buf: np.ndarray, rows: int, k: int) -> np.ndarray:
    """fp6 operand blocks -> int codes [rows, k].

    Lane l of half h holds inputs 32 * (l // 32) + 16h .. + 15 of row l % 32.
    """
    G = k // 64
    b = fp6_blocks(buf, rows, k)[0].astype(np.uint32)
    b = np.concatenate([b, np.zeros(b.shape[:-1] + (1,), np.uint32)], axis=-1)
    vals = np.zeros(b.shape[:-1] + (16,), np.int64)
    lut = np.zeros(64, np.int64)
    for code, mag in _MAG.items():
        lut[code] = mag
        lut[code | 32] = -mag
    for j in range(16):
        bit = 6 * j
        byte, shift = bit // 8, bit % 8
        word = b[..., byte] | (b[..., byte + 1] << 8)
        vals[..., j] = lut[(word >> shift) & 63]
    # [t, g, h, lhi, r, j] -> [t, r, g, lhi, h, j]
    v = vals.reshape(rows // 32, G, 2, 2, 32, 16).transpose(0, 4, 1, 3, 2, 5)
    return v.reshape(rows, k)


def unpack_nibbles(codes: np.ndarray) -> np.ndarray:
    v = np.stack([codes & 15, codes >> 4], -1).reshape(codes.shape[0], -1).astype(np.int64)
    return np.where(v > 7, v - 16, v)


def tiled_scales(scales: np.ndarray, rows: int) -> np.ndarray:
    """[rows, G] -> [rows/32][G][32] as stored by the fp6 path."""
    G = scales.shape[1]
    return scales.reshape(rows // 32, 32, G).transpose(0, 2, 1).reshape(rows, G)


@pytest.mark.parametrize("m,k,half", [(16, 256, False), (37, 768, True), (128, 3072, False), (1056, 512, True),
                                      (2100, 1024, True), (2083, 768, False)])
def test_fp6_quantizer_matches_codes(dev, m, k, half):
    import qwen_image_hip.ops as ops
    x = heavy_tailed(m, k, 31 + m)
    xin = x.astype(np.float16) if half else x
    want_c, want_s = oracle.quantize_activations(xin.view(np.uint16) if half else xin)
    c6, s6 = ops.quantize_activations_fp6(_dev(xin, dev), want_scales=True)
    rows = ops.fp6_rows(m)
    buf = c6.cpu().numpy()
    codes = decode_fp6_tiles(buf, rows, k)[:m]
    np.testing.assert_array_equal(codes, unpack_nibbles(want_c))
    np.testing.assert_array_equal(fp6_scales(buf, rows, k)[:m], want_s)
    got_s = _u16(s6).reshape(rows // 32, k // 64, 32).transpose(0, 2, 1).reshape(rows, k // 64)
    np.testing.assert_array_equal(got_s[:m], want_s)


@pytest.mark.parametrize("half", [False, True])
def test_quantizers_round_exact_ties(dev, half):
    """Rows alpha e_i + beta e_j with alpha = 60 + 8t, beta = 52 - 8t rotate
    (H256, exact in fp32) to +-7 and +-(t + 0.5): the group scale is exactly
    1 and every other value is an exact rint tie, so both quantisers' division
    and rounding (to even) are compared bit for bit with the oracle where a
    quotient one ulp off would change the code."""
    import qwen_image_hip.ops as ops
    m, k = 64, 512
    x = np.zeros((m, k), np.float32)
    g = np.random.default_rng(91)
    for r in range(m):
        t = r % 7
        c = g.integers(0, k // 256)
        i, j = g.choice(256, 2, replace=False)
        x[r, c * 256 + i] = 60 + 8 * t
        x[r, c * 256 + j] = (52 - 8 * t) * (1 if r % 2 else -1)
    xin = x.astype(np.float16) if half else x
    want_c, want_s = oracle.quantize_activations(xin.view(np.uint16) if half else xin)
    c6, _ = ops.quantize_activations_fp6(_dev(xin, dev))
    np.testing.assert_array_equal(decode_fp6_tiles(c6.cpu().numpy(), m, k), unpack_nibbles(want_c))
    np.testing.assert_array_equal(fp6_scales(c6.cpu().numpy(), m, k), want_s)
    c4, s4 = ops.quantize_activations(_dev(xin, dev))
    np.testing.assert_array_equal(c4.cpu().numpy(), want_c)
    np.testing.assert_array_equal(_u16(s4), want_s)


def test_fp6_weight_relayout(dev):
    import qwen_image_hip.ops as ops
    n, k = 64, 512
    w = weights_f16(n, k, 41)
    c, s, _ = oracle.quantize_matrix(w, 6, clip=True)
    c6, ts = ops.relayout_w4a4_fp6(_dev(c, dev), _h(s, dev), want_scales=True)
    buf = c6.cpu().numpy()
    np.testing.assert_array_equal(decode_fp6_tiles(buf, n, k), unpack_nibbles(c))
    np.testing.assert_array_equal(fp6_scales(buf, n, k), s)
    np.testing.assert_array_equal(_u16(ts).reshape(n, k // 64), tiled_scales(s, n))
    c6b, none = ops.relayout_w4a4_fp6(_dev(c, dev), _h(s, dev))
    assert none is None
    np.testing.assert_array_equal(c6b.cpu().numpy(), buf)


# Shapes cover every tile configuration the dispatcher picks: single-wave
# 32 x 32 tiles (short M), 64 x 128 tiles (short M, N >= 8192) and 128 x 128
# tiles (at least 512 of them).
@pytest.mark.parametrize("m,n,k", [(1, 32, 256), (5, 96, 512), (100, 256, 768), (263, 128, 1024),
                                   (640, 1024, 512), (1024, 512, 3072), (100, 8192, 512), (2048, 4096, 256)])
def test_fp6_gemm_bit_exact(dev, m, n, k):
    print(f"fp6 gemm m={m} n={n} k={k}", flush=True)
    import qwen_image_hip.ops as ops
    x = heavy_tailed(m, k, 500 + m)
    w = weights_f16(n, k, 501 + n)
    ac, as_ = oracle.quantize_activations(x)
    wc, ws, _ = oracle.quantize_matrix(w, 6, clip=True)
    a6, _ = ops.quantize_activations_fp6(_dev(x, dev))
    w6, _ = ops.relayout_w4a4_fp6(_dev(wc, dev), _h(ws, dev))
    got = ops.w4a4_gemm_fp6(a6, w6, m).cpu().numpy()
    want = oracle.w4a4_gemm(ac, as_, wc, ws)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_fp6_group_partials_exact(dev):
    """Scales 1 on one group and 0 elsewhere expose each exact partial."""
    import qwen_image_hip.ops as ops
    m, n, k = 64, 64, 512
    x = heavy_tailed(m, k, 600)
    x[:2] = 1000.0                                   # saturated rows
    w = weights_f16(n, k, 601)
    ac, _ = oracle.quantize_activations(x)
    wc, _, _ = oracle.quantize_matrix(w, 6)
    wc[:4] = 0x77
    partials = oracle.w4a4_partials(ac, wc)
    a6, _ = ops.quantize_activations_fp6(_dev(x, dev))
    a6_host = a6.cpu().numpy()
    G = k // 64
    for g in range(G):
        s_act = np.zeros((m, G), np.uint16)
        s_w = np.zeros((n, G), np.uint16)
        s_act[:, g] = 0x3C00
        s_w[:, g] = 0x3C00
        w6, _ = ops.relayout_w4a4_fp6(_dev(wc, dev), _h(s_w, dev))
        a6_g = _dev(set_fp6_scales(a6_host, m, k, s_act), dev)  # m is a multiple of 32
        got = ops.w4a4_gemm_fp6(a6_g, w6, m).cpu().numpy()
        np.testing.assert_array_equal(got, partials[:, :, g].astype(np.float32))


# Shapes on the persistent 128 x 128 path (M, N multiples of 128, at least
# 512 tiles).  With two workgroups on each of the MI355X's 256 CUs (512
# slots): 768 tiles = one full round + 256 tiles run as 512 halves (XCD
# pairing); 1856 tiles = several tiles per workgroup, no halves (320 left
# over); 612 tiles = one round + 100 tiles as 200 halves (plain pairing).
# K = 256 is one ring of groups per tile, so every ring switches tiles.
@pytest.mark.parametrize("m,n,k", [(2048, 6144, 256), (2048, 6144, 768), (2048, 14848, 256), (512, 19584, 512)])
def test_fp6_gemm_persistent_bit_exact(dev, m, n, k):
    print(f"fp6 persistent gemm m={m} n={n} k={k}", flush=True)
    import qwen_image_hip.ops as ops
    x = heavy_tailed(m, k, 700 + k)
    w = weights_f16(n, k, 701 + n)
    ac, as_ = oracle.quantize_activations(x)
    wc, ws, _ = oracle.quantize_matrix(w, 6, clip=True)
    a6, _ = ops.quantize_activations_fp6(_dev(x, dev))
    w6, _ = ops.relayout_w4a4_fp6(_dev(wc, dev), _h(ws, dev))
    got = ops.w4a4_gemm_fp6(a6, w6, m).cpu().numpy()
    want = oracle.w4a4_gemm(ac, as_, wc, ws)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_fp6_gemm_persistent_epilogue(dev):
    """Bias + GELU + fp16 stores at every tile switch of the persistent path."""
    import qwen_image_hip.ops as ops
    m, n, k = 2048, 6144, 512
    print(f"fp6 persistent epilogue m={m} n={n} k={k}", flush=True)
    x = heavy_tailed(m, k, 710)
    w = weights_f16(n, k, 711)
    bias = np.random.default_rng(712).normal(0, 0.5, size=n).astype(np.float32)
    ac, as_ = oracle.quantize_activations(x)
    wc, ws, _ = oracle.quantize_matrix(w, 6, clip=True)
    a6, _ = ops.quantize_activations_fp6(_dev(x, dev))
    w6, _ = ops.relayout_w4a4_fp6(_dev(wc, dev), _h(ws, dev))
    got = ops.w4a4_gemm_fp6(a6, w6, m, bias=_dev(bias, dev), out_dtype=torch.float16, gelu=True)
    got = got.float().cpu().numpy()
    v = oracle.gelu_tanh(oracle.w4a4_gemm(ac, as_, wc, ws) + bias[None, :])
    want = oracle.half_to_f32(oracle.half_from_f32(v))
    # fp16 output of a GELU on the hardware exp2 / reciprocal: within two
    # fp16 ulps of the correctly rounded value.
    np.testing.assert_allclose(got, want, rtol=2 * 2.0 ** -10, atol=2.0 ** -20)


@pytest.mark.parametrize("m", [7, 300, 4096])
def test_fused_qkv_record_matches_separate_records(dev, m):
    """A fused (q, k, v) record writes each part bit-identical to the part's
    own call (the reference's to_q / to_k / to_v with reuse_input)."""
    import qwen_image_hip as q
    n, k = 1024, 768  # m = 4096: 768 fused 128 x 128 tiles, the persistent kernel
    print(f"fp6 fused qkv m={m} n={n} k={k}", flush=True)
    x = _dev(heavy_tailed(m, k, 720 + m), dev)
    recs = [q.PackedLinear.from_fp16(q.SCHEME_W4A4_H256, _dev(weights_f16(n, k, 721 + i), dev).view(torch.float16),
                                     clip=True) for i in range(3)]
    fused = q.PackedLinear.fuse(recs)
    work = q.Work(m, k, dev)
    got = q.linear(fused, work, x, out_dtype=torch.float16, gelu=True)
    assert got.shape == (3, m, n)
    for i, r in enumerate(recs):
        want = q.linear(r, work, x, reuse_input=True, out_dtype=torch.float16, gelu=True)
        torch.testing.assert_close(got[i], want, rtol=0, atol=0)


@pytest.mark.parametrize("m_img,m_txt,fuse", [(4096, 256, True), (640, 128, False), (320, 37, True)])
def test_dual_stream_record_matches_per_stream_calls(dev, m_img, m_txt, fuse):
    """The image and text streams' linears as one dual-stream call on the
    stacked rows: every output bit-identical to each stream's own call
    (4096 + 256, 640 + 128: one persistent launch; 320 + 37: one launch per
    stream)."""
    import qwen_image_hip as q
    n, k = 1024, 512
    m = m_img + m_txt
    print(f"fp6 dual stream m={m_img}+{m_txt} fuse={fuse}", flush=True)
    x = _dev(heavy_tailed(m, k, 740 + m), dev)
    bias = [_dev(np.random.default_rng(742 + s).normal(0, 0.5, size=(3 if fuse else 1) * n).astype(np.float32), dev)
            for s in range(2)]
    recs = []
    for s in range(2):
        parts = [q.PackedLinear.from_fp16(q.SCHEME_W4A4_H256,
                                          _dev(weights_f16(n, k, 743 + 10 * s + i), dev).view(torch.float16),
                                          clip=True) for i in range(3 if fuse else 1)]
        r = q.PackedLinear.fuse(parts) if fuse else parts[0]
        r.bias = bias[s]
        recs.append(r)
    pair = q.PackedLinear.dual(recs)
    work = q.Work(m, k, dev)
    got = q.linear(pair, work, x, out_dtype=torch.float16, gelu=True, split_rows=m_img)
    w1 = q.Work(m_txt, k, dev)
    want0 = q.linear(recs[0], work, x[:m_img], out_dtype=torch.float16, gelu=True)
    want1 = q.linear(recs[1], w1, x[m_img:].contiguous(), out_dtype=torch.float16, gelu=True)
    if fuse:
        torch.testing.assert_close(got[:, :m_img], want0, rtol=0, atol=0)
        torch.testing.assert_close(got[:, m_img:], want1, rtol=0, atol=0)
    else:
        torch.testing.assert_close(got[:m_img], want0, rtol=0, atol=0)
        torch.testing.assert_close(got[m_img:], want1, rtol=0, atol=0)
    # Each stream of the pair, taken back out as a view, is the stream's record.
    again = q.linear(pair.stream(1), w1, x[m_img:].contiguous(), out_dtype=torch.float16, gelu=True)
    torch.testing.assert_close(again, want1, rtol=0, atol=0)
