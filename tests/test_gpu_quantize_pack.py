"""GPU parity: activation quantiser, f32->f16, device packer, re-layout.

All of these are integer / bit outputs, so the bar is bit-exact equality with
the CPU oracle on the same seeded inputs.
"""
import numpy as np
import pytest
import torch

import oracle
from _data import f16_bits, heavy_tailed, normal_f32, weights_f16

pytestmark = pytest.mark.gpu


def _to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _u16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _special_rows(k):
    rows = np.zeros((6, k), np.float32)
    rows[1, 5] = 1000.0                                   # one spike
    rows[2] = np.linspace(-3, 3, k, dtype=np.float32)     # ramp
    rows[3, ::64] = 1e-30                                 # subnormal-scale group
    rows[4] = 0.5                                         # constant row
    rows[5] = np.float32(2.0 ** -20) * (np.arange(k) % 7 - 3)
    return rows


@pytest.mark.parametrize("m,k,dist", [(1, 256, "n"), (3, 768, "n"), (128, 3072, "t"), (37, 12288, "t"),
                                      (6, 1024, "special")])
def test_quantize_f32_bit_exact(dev, m, k, dist):
    print(f"quantize f32 m={m} k={k} {dist}", flush=True)
    x = {"n": lambda: normal_f32(m, k, 11), "t": lambda: heavy_tailed(m, k, 12),
         "special": lambda: _special_rows(k)}[dist]()
    m = x.shape[0]
    codes, scales = oracle.quantize_activations(x)
    import qwen_image_hip.ops as ops
    gc, gs = ops.quantize_activations(_to_dev(x, dev))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(gc.cpu().numpy(), codes)
    np.testing.assert_array_equal(_u16(gs), scales)


@pytest.mark.parametrize("m,k", [(2, 256), (64, 3072), (5, 18944)])
def test_quantize_f16_bit_exact(dev, m, k):
    print(f"quantize f16 m={m} k={k}", flush=True)
    xb = f16_bits(heavy_tailed(m, k, 13))
    codes, scales = oracle.quantize_activations(xb)
    import qwen_image_hip.ops as ops
    xt = _to_dev(xb.view(np.float16), dev)
    gc, gs = ops.quantize_activations(xt)
    np.testing.assert_array_equal(gc.cpu().numpy(), codes)
    np.testing.assert_array_equal(_u16(gs), scales)


def test_reference_abi_quantizer_null_stream(dev):
    import qwen_image_hip as q
    m, k = 4, 512
    x = normal_f32(m, k, 14)
    codes, scales = oracle.quantize_activations(x)
    xt = _to_dev(x, dev)
    gc = torch.empty((m, k // 2), dtype=torch.uint8, device=dev)
    gs = torch.empty((m, k // 64), dtype=torch.float16, device=dev)
    torch.cuda.synchronize()
    assert q.load().qi_w4a4_quantize_activations(xt.data_ptr(), gc.data_ptr(), gs.data_ptr(), m, k) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(gc.cpu().numpy(), codes)
    np.testing.assert_array_equal(_u16(gs), scales)
    # k not a multiple of 256 is rejected before launch.
    assert q.load().qi_w4a4_quantize_activations(xt.data_ptr(), gc.data_ptr(), gs.data_ptr(), m, 320) == 1


def test_f32_to_f16_bit_exact(dev):
    g = np.random.default_rng(15)
    x = np.concatenate([
        g.normal(size=4099).astype(np.float32),
        (g.normal(size=1000) * 1e-6).astype(np.float32),          # fp16 subnormals
        np.array([65504, 65519.996, 65520, 1e6, -1e6, 0.0, -0.0, 2 ** -25, 3 * 2 ** -26], np.float32),
        (np.arange(2048, dtype=np.float32) + 0.5) * np.float32(2 ** -10),  # exact ties
    ]).astype(np.float32)
    expect = oracle.half_from_f32(x)
    import qwen_image_hip.ops as ops
    got = ops.f32_to_f16(_to_dev(x, dev))
    np.testing.assert_array_equal(_u16(got), expect)


@pytest.mark.parametrize("scheme,clip,n,k", [(5, False, 64, 256), (5, True, 48, 1024), (6, False, 32, 512),
                                             (6, True, 80, 3072), (5, True, 16, 64)])
def test_pack_bit_exact(dev, scheme, clip, n, k):
    print(f"pack scheme={scheme} clip={clip} n={n} k={k}", flush=True)
    w = weights_f16(n, k, 20 + n)
    w[0, :64] = f16_bits(np.zeros(64))          # all-zero group
    w[1, :64] = f16_bits(np.full(64, 0.25))      # constant group
    codes, scales, mins = oracle.quantize_matrix(w, scheme, clip)
    import qwen_image_hip.ops as ops
    gc, gs, gm = ops.pack_weights(_to_dev(w.view(np.float16), dev), scheme, clip)
    np.testing.assert_array_equal(gc.cpu().numpy(), codes)
    np.testing.assert_array_equal(_u16(gs), scales)
    if scheme == 5:
        np.testing.assert_array_equal(_u16(gm), mins)


def _expected_w4a4_tiles(codes, scales):
    n, hk = codes.shape
    G = hk * 2 // 64
    c = codes.reshape(n // 16, 16, G, 4, 8).transpose(0, 2, 3, 1, 4).reshape(n, hk)
    s = scales.reshape(n // 16, 16, G).transpose(0, 2, 1).reshape(n, G)
    return c, s


def _permute_nibbles(words):
    # element 2i -> nibble i, element 2i+1 -> nibble 4+i, within each dword
    out = np.zeros_like(words)
    for e in range(8):
        slot = 4 + e // 2 if e % 2 else e // 2
        out |= ((words >> np.uint32(4 * e)) & np.uint32(15)) << np.uint32(4 * slot)
    return out


def _expected_w4a16_tiles(codes, scales, mins):
    n, hk = codes.shape
    G = hk * 2 // 64
    c = codes.reshape(n // 16, 16, G, 2, 4, 4).transpose(0, 2, 4, 1, 3, 5).reshape(n, hk)
    c = _permute_nibbles(np.ascontiguousarray(c).view(np.uint32)).view(np.uint8).reshape(n, hk)
    sm = np.stack([scales, mins], axis=-1).reshape(n // 16, 16, G, 2).transpose(0, 2, 1, 3).reshape(n, 2 * G)
    return c, sm


@pytest.mark.parametrize("n,k", [(16, 256), (48, 768), (256, 3072)])
def test_relayout_permutation_and_inverse(dev, n, k):
    import qwen_image_hip.ops as ops
    g = np.random.default_rng(n + k)
    codes = g.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scales = g.integers(0, 0x7C00, size=(n, k // 64), dtype=np.uint16)
    mins = g.integers(0, 0xFC00, size=(n, k // 64), dtype=np.uint16)
    dc, ds, dm = _to_dev(codes, dev), _to_dev(scales.view(np.float16), dev), _to_dev(mins.view(np.float16), dev)

    tc, ts = ops.relayout_w4a4(dc, ds)
    ec, es = _expected_w4a4_tiles(codes, scales)
    np.testing.assert_array_equal(tc.cpu().numpy(), ec)
    np.testing.assert_array_equal(_u16(ts), es)
    ic, is_ = ops.relayout_w4a4_inverse(tc, ts)
    np.testing.assert_array_equal(ic.cpu().numpy(), codes)
    np.testing.assert_array_equal(_u16(is_), scales)

    tc, ts = ops.relayout_w4a16(dc, ds, dm)
    ec, es = _expected_w4a16_tiles(codes, scales, mins)
    np.testing.assert_array_equal(tc.cpu().numpy(), ec)
    np.testing.assert_array_equal(_u16(ts), es)
    ic, is_, im = ops.relayout_w4a16_inverse(tc, ts)
    np.testing.assert_array_equal(ic.cpu().numpy(), codes)
    np.testing.assert_array_equal(_u16(is_), scales)
    np.testing.assert_array_equal(_u16(im), mins)
