"""The HIP path against the committed golden vectors (tests/golden/*.npz):
every W4A4 route and the device packer bit-exact; W4A16 within the north-star
tolerance (rel-L2 <= 1e-3, max-abs <= 2e-2 * rms) of the double-precision
product, with its device dequantisation bit-exact."""
from pathlib import Path

import numpy as np
import pytest
import torch

from _data import MAX_ABS_RMS_TOL, REL_L2_TOL, max_abs_over_rms, rel_l2

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _d(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _h(bits, dev):
    return _d(np.ascontiguousarray(bits).view(np.float16), dev)


def _u16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def test_golden_w4a4_all_routes(dev):
    import qwen_image_hip as q
    from qwen_image_hip import ops
    g = _load("w4a4_h256_g64.npz")
    m, k = g["x"].shape
    x = _d(g["x"], dev)
    # activation quantiser, reference ABI layout
    c, s = ops.quantize_activations(x)
    np.testing.assert_array_equal(c.cpu().numpy(), g["a_codes"])
    np.testing.assert_array_equal(_u16(s), g["a_scales"])
    # device weight packer
    wc, ws, _ = ops.pack_weights(_h(g["w_f16"], dev), 6, clip=True)
    np.testing.assert_array_equal(wc.cpu().numpy(), g["w_codes"])
    np.testing.assert_array_equal(_u16(ws), g["w_scales"])
    want = g["y"].view(np.uint32)
    # reference ABI GEMM on QIPACK layout; its rows are a multiple of 128,
    # padded with zero rows by the caller (transformer.cplus:100-102,660)
    cp = torch.zeros((128, k // 2), dtype=torch.uint8, device=dev)
    sp = torch.zeros((128, k // 64), dtype=torch.float16, device=dev)
    cp[:m], sp[:m] = c, s
    y = ops.w4a4_gemm_reference(cp, sp, _d(g["w_codes"], dev), _h(g["w_scales"], dev))[:m]
    np.testing.assert_array_equal(y.cpu().numpy().view(np.uint32), want)
    # linear() on both operand formats
    work = q.Work(m, k, dev)
    for operand in (q.W4A4_FP6, q.W4A4_INT8):
        rec = q.PackedLinear.from_qipack(6, _d(g["w_codes"], dev), _h(g["w_scales"], dev), operand=operand)
        y = q.linear(rec, work, x)
        np.testing.assert_array_equal(y.cpu().numpy().view(np.uint32), want, err_msg=operand)


def test_golden_w4a16(dev):
    import qwen_image_hip as q
    from qwen_image_hip import ops
    g = _load("w4a16_g64.npz")
    m, k = g["x_f16"].shape
    c, s, mn = ops.pack_weights(_h(g["w_f16"], dev), 5)
    np.testing.assert_array_equal(c.cpu().numpy(), g["codes"])
    np.testing.assert_array_equal(_u16(s), g["scales"])
    np.testing.assert_array_equal(_u16(mn), g["minimums"])
    x = _h(g["x_f16"], dev)
    rec = q.PackedLinear.from_qipack(5, c, s, mn)
    work = q.Work(m, k, dev)
    # identity input rows expose dequantised weights exactly: y = x . W^T with
    # x = e_i gives the fp16 dequantised column, exactly representable in fp32
    eye = torch.zeros((k, k), dtype=torch.float16, device=dev)
    eye.fill_diagonal_(1.0)
    wt = q.linear(rec, q.Work(k, k, dev), eye).cpu().numpy()
    np.testing.assert_array_equal(wt.T.astype(np.float16).view(np.uint16), g["w_dequant"])
    xp = torch.zeros((128, k), dtype=torch.float16, device=dev)
    xp[:m] = x
    y_ref_abi = ops.w4a16_gemm_reference(xp, _d(g["codes"], dev), _h(g["scales"], dev), _h(g["minimums"], dev))[:m]
    for y in (q.linear(rec, work, x), y_ref_abi):
        y = y.cpu().numpy()
        assert rel_l2(y, g["y"]) <= REL_L2_TOL
        assert max_abs_over_rms(y, g["y"]) <= MAX_ABS_RMS_TOL
    yv = q.linear(rec, work, x[:2]).cpu().numpy()  # m <= 16: the GEMV
    assert rel_l2(yv, g["y"][:2]) <= REL_L2_TOL
