"""GPU parity: W4A4 GEMM, W4A16 GEMM, W4A16 GEMV, fused epilogues, linear().

Bars (north star): int32 per-group partials bit-exact; W4A4 fp32 outputs are
bit-exact with the oracle's reference-order fp32 formula (the kernel keeps
that order); W4A16 / GEMV fp32 outputs within rel-L2 <= 1e-3 and
max-abs <= 2e-2 * rms(out) of the float64 oracle; fp16 outputs are the same
value rounded once more, so they get the same tolerance.
"""
import numpy as np
import pytest
import torch

import oracle
from _data import (MAX_ABS_RMS_TOL, REL_L2_TOL, f16_bits, heavy_tailed, max_abs_over_rms, normal_f32, rel_l2,
                   weights_f16)

pytestmark = pytest.mark.gpu


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _h(bits, dev):
    return _dev(np.ascontiguousarray(bits).view(np.float16), dev)


def _close(got, want):
    """Within the north-star tolerance; the measured margin is printed (the
    GEMV's factored form keeps every weight c * s + min in fp32 instead of
    rounding it to fp16 first, which shows as a rel-L2 of a few 1e-4)."""
    e, a = rel_l2(got, want), max_abs_over_rms(got, want)
    print(f"  rel-L2 {e:.3e} (bar {REL_L2_TOL:g}), max-abs/rms {a:.3e} (bar {MAX_ABS_RMS_TOL:g})", flush=True)
    assert e <= REL_L2_TOL, e
    assert a <= MAX_ABS_RMS_TOL, a


def _w4a4_case(m, n, k, seed):
    x = heavy_tailed(m, k, seed)
    w = weights_f16(n, k, seed + 1)
    a_codes, a_scales = oracle.quantize_activations(x)
    w_codes, w_scales, _ = oracle.quantize_matrix(w, 6, clip=True)
    return a_codes, a_scales, w_codes, w_scales


# ------------------------------------------------------------------- W4A4 --

@pytest.mark.parametrize("m,n,k", [(128, 128, 256), (256, 384, 768), (128, 256, 3072)])
def test_w4a4_reference_abi_bit_exact(dev, m, n, k):
    print(f"w4a4 reference abi m={m} n={n} k={k}", flush=True)
    import qwen_image_hip.ops as ops
    ac, as_, wc, ws = _w4a4_case(m, n, k, 100 + k)
    want = oracle.w4a4_gemm(ac, as_, wc, ws)
    got = ops.w4a4_gemm_reference(_dev(ac, dev), _h(as_, dev), _dev(wc, dev), _h(ws, dev)).cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    want64 = oracle.w4a4_gemm(ac, as_, wc, ws, f64=True)
    _close(got, want64)


def test_w4a4_reference_abi_rejects_shapes(dev):
    import qwen_image_hip as q
    lib = q.load()
    assert lib.qi_w4a4_gemm(1, 1, 1, 1, 1, 100, 128, 256) == 1
    assert lib.qi_w4a4_gemm(1, 1, 1, 1, 1, 128, 100, 256) == 1
    assert lib.qi_w4a4_gemm(1, 1, 1, 1, 1, 128, 128, 320) == 1
    assert lib.qi_w4a16_gemm(1, 1, 1, 1, 1, 128, 128, 96) == 1


@pytest.mark.parametrize("m,n,k", [(1, 16, 256), (5, 48, 512), (100, 256, 768), (263, 128, 1024),
                                   (640, 1024, 512)])
def test_w4a4_tiled_bit_exact(dev, m, n, k):
    print(f"w4a4 tiled m={m} n={n} k={k}", flush=True)
    import qwen_image_hip.ops as ops
    ac, as_, wc, ws = _w4a4_case(m, n, k, 200 + m)
    tc, ts = ops.relayout_w4a4(_dev(wc, dev), _h(ws, dev))
    got = ops.w4a4_gemm(_dev(ac, dev), _h(as_, dev), tc, ts).cpu().numpy()
    want = oracle.w4a4_gemm(ac, as_, wc, ws)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_w4a4_group_partials_exact(dev):
    """Expose each int32 group partial: scales 1 on group g, 0 elsewhere."""
    import qwen_image_hip.ops as ops
    m, n, k = 64, 64, 512
    ac, _, wc, _ = _w4a4_case(m, n, k, 300)
    # Saturated codes too: every nibble -7 or 7 in the first rows.
    ac[:2] = 0x77
    ac[2:4] = 0x99
    wc[:4] = 0x77
    partials = oracle.w4a4_partials(ac, wc)          # [m, n, G]
    assert np.abs(partials).max() == 64 * 49          # the int32 range is reached
    tc_src = _dev(wc, dev)
    G = k // 64
    one = np.uint16(0x3C00)
    for g in range(G):
        sa = np.zeros((m, G), np.uint16)
        sw = np.zeros((n, G), np.uint16)
        sa[:, g] = one
        sw[:, g] = one
        tc, ts = ops.relayout_w4a4(tc_src, _h(sw, dev))
        got = ops.w4a4_gemm(_dev(ac, dev), _h(sa, dev), tc, ts).cpu().numpy()
        np.testing.assert_array_equal(got, partials[:, :, g].astype(np.float32))


@pytest.mark.parametrize("gelu", [False, True])
def test_w4a4_epilogue_f16_bias_gelu(dev, gelu):
    import qwen_image_hip.ops as ops
    m, n, k = 96, 128, 768
    ac, as_, wc, ws = _w4a4_case(m, n, k, 400)
    bias = np.random.default_rng(401).normal(0, 0.5, size=n).astype(np.float32)
    tc, ts = ops.relayout_w4a4(_dev(wc, dev), _h(ws, dev))
    got = ops.w4a4_gemm(_dev(ac, dev), _h(as_, dev), tc, ts, bias=_dev(bias, dev), out_dtype=torch.float16,
                        gelu=gelu).float().cpu().numpy()
    v = oracle.w4a4_gemm(ac, as_, wc, ws) + bias[None, :]
    if gelu:
        v = oracle.gelu_tanh(v)
    want = oracle.half_to_f32(oracle.half_from_f32(v))
    _close(got, want)


# ------------------------------------------------------------------ W4A16 --

def _w4a16_case(m, n, k, seed, clip=False):
    xb = f16_bits(normal_f32(m, k, seed))
    w = weights_f16(n, k, seed + 1)
    codes, scales, mins = oracle.quantize_matrix(w, 5, clip=clip)
    return xb, codes, scales, mins


@pytest.mark.parametrize("m,n,k", [(128, 128, 64), (256, 256, 640), (128, 384, 3072)])
def test_w4a16_reference_abi(dev, m, n, k):
    print(f"w4a16 reference abi m={m} n={n} k={k}", flush=True)
    import qwen_image_hip.ops as ops
    xb, c, s, mn = _w4a16_case(m, n, k, 500 + k)
    got = ops.w4a16_gemm_reference(_h(xb, dev), _dev(c, dev), _h(s, dev), _h(mn, dev)).cpu().numpy()
    want = oracle.w4a16_gemm(xb, c, s, mn, precise=True)
    _close(got, want)


# m <= 256 with few column tiles runs the K-split kernel (17, 100, 256
# rows here), larger m the tiled kernel.  The M = 300 rows are the
# text-encoder shapes of config 4 (Qwen2.5-VL-7B: hidden 3584, MLP 18944).
# 600 x 18432 runs the 128 x 192 tiles on a ragged last row band.
@pytest.mark.parametrize("m,n,k,clip", [(17, 16, 64, False), (100, 48, 192, True), (256, 192, 3072, False),
                                        (300, 512, 3584 // 64 * 64, False), (1024, 256, 1024, True),
                                        (300, 2048, 3584, False), (300, 1024, 18944, False),
                                        (600, 18432, 256, False)])
def test_w4a16_tiled(dev, m, n, k, clip):
    print(f"w4a16 tiled m={m} n={n} k={k}", flush=True)
    import qwen_image_hip.ops as ops
    xb, c, s, mn = _w4a16_case(m, n, k, 600 + m, clip)
    tc, ts = ops.relayout_w4a16(_dev(c, dev), _h(s, dev), _h(mn, dev))
    got = ops.w4a16_gemm(_h(xb, dev), tc, ts).cpu().numpy()
    want = oracle.w4a16_gemm(xb, c, s, mn, precise=True)
    _close(got, want)


def test_gelu_epilogue_accuracy(dev):
    """The fused GELU on outputs spanning [-12, 12] (x = identity, so each
    output is one dequantised weight), fp32 out, against the oracle's tanhf
    form: within a few fp32 ulp of max(1, |v|)."""
    import qwen_image_hip.ops as ops
    n, k = 128, 128
    g = np.random.default_rng(17)
    codes = g.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scales = np.full((n, k // 64), 1.6, np.float16).view(np.uint16)
    mins = (g.random((n, k // 64)) * 12.0 - 12.0).astype(np.float16).view(np.uint16)
    w = oracle.w4a16_dequantize(codes, scales, mins).view(np.float16).astype(np.float32)   # [n, k]
    tc, ts = ops.relayout_w4a16(_dev(codes, dev), _h(scales, dev), _h(mins, dev))
    got = ops.w4a16_gemm(_dev(np.eye(k, dtype=np.float16), dev), tc, ts, gelu=True).cpu().numpy()  # [k, n]
    want = oracle.gelu_tanh(w.T)
    err = np.abs(got - want) / np.maximum(1.0, np.abs(w.T))
    assert w.min() < -11 and w.max() > 11
    assert err.max() <= 4e-6, err.max()


@pytest.mark.parametrize("gelu", [False, True])
def test_w4a16_epilogue_f16_bias_gelu(dev, gelu):
    import qwen_image_hip.ops as ops
    m, n, k = 160, 128, 512
    xb, c, s, mn = _w4a16_case(m, n, k, 700)
    bias = np.random.default_rng(701).normal(0, 0.5, size=n).astype(np.float32)
    tc, ts = ops.relayout_w4a16(_dev(c, dev), _h(s, dev), _h(mn, dev))
    got = ops.w4a16_gemm(_h(xb, dev), tc, ts, bias=_dev(bias, dev), out_dtype=torch.float16,
                         gelu=gelu).float().cpu().numpy()
    v = oracle.w4a16_gemm(xb, c, s, mn, precise=True) + bias[None, :]
    if gelu:
        v = oracle.gelu_tanh(v)
    _close(got, oracle.half_to_f32(oracle.half_from_f32(v)))


# m = 1, 2 also at group counts that leave waves idle (1, 13 groups) or a
# ragged last chunk (56, 100 groups over four waves of four-group chunks).
@pytest.mark.parametrize("m,n,k", [(1, 18432, 3072), (2, 18432, 3072), (3, 64, 256), (16, 512, 3584 // 64 * 64),
                                   (1, 96, 64), (2, 160, 832), (1, 48, 6400), (2, 32, 3584)])
def test_w4a16_gemv(dev, m, n, k):
    print(f"gemv m={m} n={n} k={k}", flush=True)
    import qwen_image_hip.ops as ops
    xb, c, s, mn = _w4a16_case(m, n, k, 800 + m)
    tc, ts = ops.relayout_w4a16(_dev(c, dev), _h(s, dev), _h(mn, dev))
    got = ops.w4a16_gemv(_h(xb, dev), tc, ts).cpu().numpy()
    want = oracle.w4a16_gemm(xb, c, s, mn, precise=True)
    _close(got, want)
    # The kernels' own arithmetic, apart from the choice of weights: the
    # dequantising form (x too large for LDS) uses the reference's fp16
    # weights, so against the oracle only its fp32 sums differ; the factored
    # forms (vector unit for m <= 2, matrix core otherwise) keep c s + min in
    # fp32, so they are checked against the float64 product with those
    # weights (a cancelled 1024 X term would show here as about 1.5e-5).
    if m > 2 and m * k * 2 > 48 * 1024:
        own = rel_l2(got, want)
    else:
        nib = np.stack([c & 15, c >> 4], -1).reshape(n, k).astype(np.float64)
        w = (nib * np.repeat(s.view(np.float16).astype(np.float64), 64, axis=1)
             + np.repeat(mn.view(np.float16).astype(np.float64), 64, axis=1))
        own = rel_l2(got, xb.view(np.float16).astype(np.float64) @ w.T)
    print(f"  arithmetic rel-L2 {own:.3e} (bar 2e-6)", flush=True)
    assert own <= 2e-6, own
    # The tiled GEMM entry point dispatches m <= 16 to the same kernel.
    got2 = ops.w4a16_gemm(_h(xb, dev), tc, ts).cpu().numpy()
    np.testing.assert_array_equal(got, got2)


# ---------------------------------------------------------------- linear() --

@pytest.mark.parametrize("operand", ["fp6", "int8"])
def test_linear_dispatch_and_reuse(dev, operand):
    """transformer.cplus:669-713 call pattern: Q quantises, K and V reuse it."""
    import qwen_image_hip as q
    rows, k, n = 136, 512, 256
    x = heavy_tailed(rows, k, 900)
    ws = [weights_f16(n, k, 901 + i) for i in range(3)]
    work = q.Work(rows_max=256, k_max=1024, device=dev)
    recs = [q.PackedLinear.from_fp16(q.SCHEME_W4A4_H256, _h(w, dev), clip=True, operand=operand) for w in ws]
    xd = _dev(x, dev)
    outs = [q.linear(recs[0], work, xd)]
    outs += [q.linear(r, work, xd, reuse_input=True) for r in recs[1:]]
    ac, as_ = oracle.quantize_activations(x)
    for w, o in zip(ws, outs):
        wc, wsc, _ = oracle.quantize_matrix(w, 6, clip=True)
        np.testing.assert_array_equal(o.cpu().numpy(), oracle.w4a4_gemm(ac, as_, wc, wsc))

    rec16 = q.PackedLinear.from_fp16(q.SCHEME_W4A16, _h(ws[0], dev))
    y16 = q.linear(rec16, work, xd).cpu().numpy()
    c, s, mn = oracle.quantize_matrix(ws[0], 5)
    _close(y16, oracle.w4a16_gemm(oracle.half_from_f32(x), c, s, mn))


# ------------------------------------------------- dequantisation exactness --

def _double_rounding_cases(count, seed=0):
    """(scale, minimum) fp16 pairs for which fp16(fmaf(c, s, m)) (the
    reference's two roundings, gemm.cu:229-230) differs from a single rounding
    of c*s + m for some code c, with every code's weight finite."""
    g = np.random.default_rng(seed)
    n = 2_000_000
    s = g.integers(1, 0x7C00, n).astype(np.uint16)
    m = g.integers(0, 0x10000, n).astype(np.uint16)
    ok = (m & 0x7C00) != 0x7C00
    s, m = s[ok], m[ok]
    sf = s.view(np.float16).astype(np.float64)
    mf = m.view(np.float16).astype(np.float64)
    codes = np.arange(16, dtype=np.float64)[:, None]
    exact = codes * sf[None, :] + mf[None, :]
    with np.errstate(over="ignore"):
        single = exact.astype(np.float16)
        double = exact.astype(np.float32).astype(np.float16)
    finite = np.all(np.isfinite(double), axis=0) & np.all(np.isfinite(single), axis=0)
    differs = np.any(single.view(np.uint16) != double.view(np.uint16), axis=0)
    idx = np.nonzero(finite & differs)[0][:count]
    return s[idx], m[idx]


@pytest.mark.parametrize("path", ["tiled", "reference", "gemv", "gemv1", "gemv2"])
def test_w4a16_dequant_bit_exact_identity(dev, path):
    """x = identity makes y = W^T exactly (one nonzero product per output), so
    the kernels' dequantised weights are compared bit for bit with the oracle,
    on (scale, minimum) pairs where double and single rounding disagree."""
    import qwen_image_hip.ops as ops
    n, k = 128, 128
    s_adv, m_adv = _double_rounding_cases(n * 2)
    assert len(s_adv) == n * 2
    scales = s_adv.reshape(n, 2)
    mins = m_adv.reshape(n, 2)
    codes = np.random.default_rng(3).integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    want = oracle.w4a16_dequantize(codes, scales, mins).view(np.float16).astype(np.float32)   # [n, k]
    eye = np.eye(k, dtype=np.float16)
    if path == "reference":
        got = ops.w4a16_gemm_reference(_dev(eye, dev), _dev(codes, dev), _h(scales, dev), _h(mins, dev))
        got = got.cpu().numpy().T
    else:
        tc, ts = ops.relayout_w4a16(_dev(codes, dev), _h(scales, dev), _h(mins, dev))
        if path == "tiled":
            got = ops.w4a16_gemm(_dev(eye, dev), tc, ts).cpu().numpy().T
        else:
            # 16 rows per call (matrix-core form); 1 or 2 rows (vector form)
            rows = {"gemv": 16, "gemv1": 1, "gemv2": 2}[path]
            got = np.concatenate([ops.w4a16_gemv(_dev(eye[r:r + rows], dev), tc, ts).cpu().numpy()
                                  for r in range(0, k, rows)], axis=0).T
            # The GEMV keeps each weight c * s + minimum in fp32 (one
            # rounding of the exact value) instead of rounding it to fp16.
            nib = np.stack([codes & 15, codes >> 4], -1).reshape(n, k).astype(np.float64)
            s64 = np.repeat(scales.view(np.float16).astype(np.float64), 64, axis=1)
            m64 = np.repeat(mins.view(np.float16).astype(np.float64), 64, axis=1)
            want = (nib * s64 + m64).astype(np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("m,n,k,tiles", [(1152, 18432, 128, 4), (4096, 12288, 64, 5)])
@pytest.mark.parametrize("mixed", [False, True])
def test_w4a16_dequant_bit_exact_large_tiles(dev, mixed, m, n, k, tiles):
    """The large-M tile shapes (m > 1024: 128 x 192 tiles, and 256 x 256
    tiles once they give 768 workgroups): x repeats the identity, so every
    output is one dequantised weight, compared bit for bit on double-rounding
    (scale, minimum) pairs -- in every group, or mixed with ordinary groups so
    both dequantisation paths run in one launch."""
    import qwen_image_hip as q
    import qwen_image_hip.ops as ops
    assert q.load().qi_hip_w4a16_tiles(m, n) == tiles
    G = k // 64
    s_adv, m_adv = _double_rounding_cases(n * G, seed=5)   # ~17k distinct pairs; repeated to fill n * G
    scales = np.resize(s_adv, n * G).reshape(n, G).copy()
    mins = np.resize(m_adv, n * G).reshape(n, G).copy()
    if mixed:
        g = np.random.default_rng(6)
        plain = g.random((n, G)) < 0.5
        scales[plain] = (g.random(plain.sum()) * 0.01 + 0.001).astype(np.float16).view(np.uint16)
        mins[plain] = (-(g.random(plain.sum()) * 0.05)).astype(np.float16).view(np.uint16)
    codes = np.random.default_rng(7).integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    want = oracle.w4a16_dequantize(codes, scales, mins).view(np.float16).astype(np.float32)   # [n, k]
    x = np.tile(np.eye(k, dtype=np.float16), (m // k, 1))
    tc, ts = ops.relayout_w4a16(_dev(codes, dev), _h(scales, dev), _h(mins, dev))
    got = ops.w4a16_gemm(_dev(x, dev), tc, ts).cpu().numpy()                                  # [m, n]
    np.testing.assert_array_equal(got.view(np.uint32), np.tile(want.T, (m // k, 1)).view(np.uint32))


# ------------------------------------------------------- QIPACK file upload --

@pytest.mark.parametrize("scheme", [5, 6])
def test_linear_from_qipack_file(dev, tmp_path, scheme):
    """Quantise on the device, write a QIPACK1 file, verify it, load the
    record back through the upload re-layout: the linear's output equals the
    in-memory record's bit for bit (the arrays round-trip exactly)."""
    import qwen_image_hip as q
    from qwen_image_hip import qipack
    import qwen_image_hip.ops as ops
    n, k, rows = 256, 512, 96
    w = weights_f16(n, k, 950 + scheme)
    codes, scales, mins = ops.pack_weights(_h(w, dev), scheme, clip=scheme == 6)
    host = lambda t: None if t is None else t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)  # noqa
    path = tmp_path / "w.qipack"
    qipack.write_pack(path, [("transformer_blocks.0.img_mlp.net.0.proj.weight", codes.cpu().numpy(),
                              host(scales), host(mins))], scheme)
    direct = q.PackedLinear.from_qipack(scheme, codes, scales, mins)
    with qipack.Pack(path) as p:
        p.verify()
        loaded = q.PackedLinear.from_pack(p, "transformer_blocks.0.img_mlp.net.0.proj.weight", dev)
    x = _dev(heavy_tailed(rows, k, 951), dev)
    if scheme == 5:
        x = x.half()
    work = q.Work(rows_max=rows, k_max=k, device=dev)
    a = q.linear(direct, work, x).cpu().numpy()
    b = q.linear(loaded, work, x).cpu().numpy()
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


# m = 1, 2: the vector-unit GEMV; 5: the factored matrix-core GEMV; 16 at
# k = 2048: the dequantising GEMV (x too large for LDS).
@pytest.mark.parametrize("m,k", [(1, 640), (2, 640), (5, 640), (16, 2048), (300, 640), (4096, 640)])
def test_w4a16_fused_record_matches_separate_records(dev, m, k):
    """A fused (q, k, v) W4A16 record: each part within the W4A16 tolerance of
    the part's own call, and bit-identical on the GEMV path (m <= 16), which
    runs the same kernel as the part's own call in one launch over all parts,
    writing the parts layout."""
    import qwen_image_hip as q
    n = 1024
    print(f"w4a16 fused qkv m={m} n={n} k={k}", flush=True)
    x = _h(f16_bits(normal_f32(m, k, 730 + m)), dev)
    recs = [q.PackedLinear.from_fp16(q.SCHEME_W4A16, _h(weights_f16(n, k, 731 + i), dev)) for i in range(3)]
    fused = q.PackedLinear.fuse(recs)
    work = q.Work(m, k, dev)
    got = q.linear(fused, work, x, out_dtype=torch.float32)
    assert got.shape == (3, m, n)
    for i, r in enumerate(recs):
        want = q.linear(r, work, x, out_dtype=torch.float32)
        if m <= 16:
            torch.testing.assert_close(got[i], want, rtol=0, atol=0)
        else:
            _close(got[i].cpu().numpy(), want.cpu().numpy())


@pytest.mark.parametrize("m_img,m_txt", [(4096, 256), (320, 40)])
def test_w4a16_dual_stream_record_matches_per_stream_calls(dev, m_img, m_txt):
    """The image and text streams' fused W4A16 records as one dual-stream
    call on the stacked rows, against each stream's own call: within the
    W4A16 tolerance (the kernel shape is chosen for the stacked rows; 320 +
    40 runs one launch over both streams), and bit-identical for the image
    rows at 4096 + 256, which runs one launch per stream."""
    import qwen_image_hip as q
    n, k = 1536, 1024
    m = m_img + m_txt
    print(f"w4a16 dual stream m={m_img}+{m_txt}", flush=True)
    x = _h(f16_bits(normal_f32(m, k, 760 + m)), dev)
    recs = []
    for s in range(2):
        parts = [q.PackedLinear.from_fp16(q.SCHEME_W4A16, _h(weights_f16(n, k, 761 + 10 * s + i), dev))
                 for i in range(3)]
        recs.append(q.PackedLinear.fuse(parts))
    pair = q.PackedLinear.dual(recs)
    work = q.Work(m, k, dev)
    got = q.linear(pair, work, x, out_dtype=torch.float32, split_rows=m_img)
    want0 = q.linear(recs[0], work, x[:m_img], out_dtype=torch.float32)
    want1 = q.linear(recs[1], work, x[m_img:].contiguous(), out_dtype=torch.float32)
    _close(got[:, :m_img].cpu().numpy(), want0.cpu().numpy())
    _close(got[:, m_img:].cpu().numpy(), want1.cpu().numpy())
    if m_img == 4096:
        torch.testing.assert_close(got[:, :m_img], want0, rtol=0, atol=0)
