"""GPU parity of the producers fused with the fp6 quantiser: the reference's
LayerNorm with modulation scale (ops.cu:37-59) and SwiGLU (ops.cu:134-144)
against the float64 oracle, and the fused codes bit-identical to quantising
the plain producers' fp32 outputs."""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("m,k,split", [(1, 256, 0), (300, 3072, 37), (64, 12288, 64), (2100, 3072, 2048)])
def test_layer_norm_scale_and_fused_quantiser(dev, m, k, split):
    print(f"layer norm m={m} k={k} split={split}", flush=True)
    import qwen_image_hip.ops as ops
    rng = np.random.default_rng(900 + m)
    x = (rng.standard_t(3, size=(m, k)) * 2.0 + 0.5).astype(np.float32)
    scale = rng.normal(0.0, 0.3, size=(2, k)).astype(np.float32)
    xd, sd = _dev(x, dev), _dev(scale, dev)
    got = ops.layer_norm_scale(xd, sd, split)
    want = oracle.layer_norm_scale(x, scale, split)
    g = got.cpu().numpy()
    # fp32 statistics over k inputs and three fp32 roundings per output
    np.testing.assert_allclose(g, want, rtol=2e-5, atol=2e-5)
    # fp16 output: the fp32 value rounded once
    h = ops.layer_norm_scale(xd, sd, split, out_dtype=torch.float16)
    np.testing.assert_array_equal(h.cpu().numpy().view(np.uint16), oracle.half_from_f32(g))
    # fused: the same codes as quantising the plain output
    fused = ops.layer_norm_scale_quantize_fp6(xd, sd, split)
    plain, _ = ops.quantize_activations_fp6(got)
    np.testing.assert_array_equal(fused.cpu().numpy(), plain.cpu().numpy())


@pytest.mark.parametrize("m,k", [(5, 256), (300, 12288), (2050, 1024)])
def test_swiglu_and_fused_quantiser(dev, m, k):
    print(f"swiglu m={m} k={k}", flush=True)
    import qwen_image_hip.ops as ops
    rng = np.random.default_rng(950 + m)
    gate = (rng.normal(0.0, 3.0, size=(m, k))).astype(np.float32)
    up = (rng.normal(0.0, 1.0, size=(m, k))).astype(np.float32)
    gd, ud = _dev(gate, dev), _dev(up, dev)
    got = ops.swiglu(gd, ud)
    want = oracle.swiglu(gate, up)
    # exp, one division and one product in fp32
    np.testing.assert_allclose(got.cpu().numpy(), want, rtol=1e-6, atol=1e-30)
    h = ops.swiglu(gd, ud, out_dtype=torch.float16)
    np.testing.assert_array_equal(h.cpu().numpy().view(np.uint16), oracle.half_from_f32(got.cpu().numpy()))
    fused = ops.swiglu_quantize_fp6(gd, ud)
    plain, _ = ops.quantize_activations_fp6(got)
    np.testing.assert_array_equal(fused.cpu().numpy(), plain.cpu().numpy())
