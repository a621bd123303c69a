"""The CPU oracle still reproduces the committed golden vectors bit for bit
(tests/golden/make_golden.py wrote them)."""
from pathlib import Path

import numpy as np

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_w4a4_golden_reproduced():
    g = _load("w4a4_h256_g64.npz")
    ac, as_ = oracle.quantize_activations(g["x"])
    np.testing.assert_array_equal(ac, g["a_codes"])
    np.testing.assert_array_equal(as_, g["a_scales"])
    wc, ws, _ = oracle.quantize_matrix(g["w_f16"], 6, clip=True)
    np.testing.assert_array_equal(wc, g["w_codes"])
    np.testing.assert_array_equal(ws, g["w_scales"])
    np.testing.assert_array_equal(oracle.w4a4_partials(ac, wc), g["partials"])
    y = oracle.w4a4_gemm(ac, as_, wc, ws)
    np.testing.assert_array_equal(y.view(np.uint32), g["y"].view(np.uint32))
    # special rows: the zero row quantises to scale 2^-24 (fp16 bits 0x0001) and codes 0
    assert (g["a_scales"][3] == 1).all() and (g["a_codes"][3] == 0).all()


def test_w4a16_golden_reproduced():
    g = _load("w4a16_g64.npz")
    c, s, mn = oracle.quantize_matrix(g["w_f16"], 5)
    for a, b in ((c, "codes"), (s, "scales"), (mn, "minimums")):
        np.testing.assert_array_equal(a, g[b])
    np.testing.assert_array_equal(oracle.w4a16_dequantize(c, s, mn), g["w_dequant"])
    y = oracle.w4a16_gemm(g["x_f16"], c, s, mn)
    np.testing.assert_array_equal(y.view(np.uint32), g["y"].view(np.uint32))
