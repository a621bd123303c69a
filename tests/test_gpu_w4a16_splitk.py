"""GPU parity of the W4A16 K split over workgroups (qi_hip_w4a16_gemm_tiled_ws).

Short-M shapes (the text stream, an encoder's 300 prompt rows) split K into
slices whose fp32 partial tiles a second kernel adds in slice order before
the epilogue.  Checked against the float64 oracle on sampled rows (W4A16
bar: rel-L2 <= 1e-3, max-abs <= 2e-2 * rms, gemm.cu:191-268), against the
workspace-free entry (same tolerance: only the summation order differs),
for the bias + GELU epilogue, fp16 and fp32 output, the parts layout of a
fused record, both streams of a dual call, run-to-run identity, and a
workspace too small for the split (then bit-identical to the unsplit call).

From 2048 rows the workspace instead holds the weights dequantised once to
fp16 (the reference's values, in the order the tiled kernel reads them):
the same MFMAs in the same order, so the outputs equal the workspace-free
call's bit for bit.
"""
import numpy as np
import pytest
import torch

import oracle
from _data import MAX_ABS_RMS_TOL, REL_L2_TOL, max_abs_over_rms, rel_l2, weights_f16
from test_gpu_block_shapes import _dev, _h, _rows_host, normal_f16_dev, sample_rows

pytestmark = pytest.mark.gpu


def _close(got, want, what):
    e, a = rel_l2(got, want), max_abs_over_rms(got, want)
    print(f"  {what}: rel-L2 {e:.3e} (bar {REL_L2_TOL:g}), max-abs/rms {a:.3e} (bar {MAX_ABS_RMS_TOL:g})",
          flush=True)
    assert e <= REL_L2_TOL and a <= MAX_ABS_RMS_TOL, (e, a)


def _record(n, k, seed, dev):
    import qwen_image_hip.ops as ops
    w = weights_f16(n, k, seed)
    c, s, mn = oracle.quantize_matrix(w, 5)
    tc, ts = ops.relayout_w4a16(_dev(c, dev), _h(s, dev), _h(mn, dev))
    return (c, s, mn), tc, ts


def _want(x, rows, qw, bias=None, gelu=False):
    want = oracle.w4a16_gemm(_rows_host(x, rows).view(np.uint16), *qw, precise=True)
    if bias is not None:
        want = want + bias.cpu().numpy()[None, :]
    return oracle.gelu_tanh(want) if gelu else want


# (m, n, k, expected slices): slices = workspace / (m * n * 4)
SPLIT_CASES = [
    (300, 1024, 3584, 3),    # encoder k + v (fused), 80 tiles
    (300, 4608, 3584, 3),    # encoder q + k + v (fused), 56 groups: 160-row tiles, 2 x 72 tiles
    (300, 3584, 18944, 4),   # encoder down, K = 18944: 160-row tiles, 2 x 56 tiles
    (288, 3584, 9472, 4),    # 160-row tiles, ragged second row tile
    (320, 3072, 12288, 5),   # 160-row tiles, 2 x 48 tiles
    (256, 3072, 12288, 5),   # text-stream MLP down: 128-row tiles, 2 x 48 tiles
    (64, 3072, 12288, 12),   # 48 tiles, long K
    (200, 2048, 8192, 8),    # 128-row tiles, ragged last row tile
]


@pytest.mark.parametrize("m,n,k,slices", SPLIT_CASES)
def test_w4a16_splitk_oracle(dev, m, n, k, slices):
    import qwen_image_hip as q
    import qwen_image_hip.ops as ops
    print(f"w4a16 split-K m={m} n={n} k={k}", flush=True)
    assert q.load().qi_hip_w4a16_workspace_bytes(m, 0, n, k) == slices * m * n * 4
    x = normal_f16_dev(m, k, 40 + m, dev)
    qw, tc, ts = _record(n, k, 41 + n, dev)
    g = torch.Generator(device=dev).manual_seed(m + n)
    bias = torch.randn(n, generator=g, device=dev)
    y = ops.w4a16_gemm(x, tc, ts, bias=bias, gelu=True)
    y_ref = ops.w4a16_gemm(x, tc, ts, bias=bias, gelu=True, split_k=False)
    rows = sample_rows(m, m + k)
    _close(_rows_host(y, rows), _want(x, rows, qw, bias, gelu=True), f"split vs oracle, {len(rows)} rows")
    _close(y.cpu().numpy(), y_ref.cpu().numpy(), "split vs unsplit, all rows")
    # Deterministic: the slices are added in a fixed order.
    assert torch.equal(ops.w4a16_gemm(x, tc, ts, bias=bias, gelu=True), y)


def test_w4a16_splitk_f16_parts(dev):
    """A fused k + v record (parts layout) with fp16 output through the
    split: every part matches the oracle's columns."""
    import qwen_image_hip.ops as ops
    m, n_part, k = 300, 512, 3584
    n = 2 * n_part
    x = normal_f16_dev(m, k, 77, dev)
    qw, tc, ts = _record(n, k, 78, dev)
    y = ops.w4a16_gemm(x, tc, ts, out_dtype=torch.float16, n_part=n_part)
    assert y.shape == (2, m, n_part)
    rows = sample_rows(m, 79)
    want = _want(x, rows, qw)
    for p in range(2):
        _close(_rows_host(y[p].contiguous(), rows).astype(np.float32), want[:, p * n_part:(p + 1) * n_part],
               f"part {p}")


def test_w4a16_splitk_dual(dev):
    """Both streams of the block's MLP down (4096 + 256 rows, 12288 -> 3072):
    two launches, the image stream's on fp16 weights dequantised into the
    workspace, the text stream's split K; the image stream's rows equal the
    workspace-free call bit for bit, the text rows match the oracle."""
    import qwen_image_hip as q
    import qwen_image_hip.ops as ops
    m_img, m_txt, n, k = 4096, 256, 3072, 12288
    m = m_img + m_txt
    assert q.load().qi_hip_w4a16_workspace_bytes(m, m_img, n, k) == n * k * 2
    x = normal_f16_dev(m, k, 90, dev)
    qw0, tc0, ts0 = _record(n, k, 91, dev)
    qw1, tc1, ts1 = _record(n, k, 92, dev)
    tc, ts = torch.cat([tc0, tc1]), torch.cat([ts0, ts1])
    y = ops.w4a16_gemm_dual(x, tc, ts, m_img, out_dtype=torch.float16)
    y_ref = ops.w4a16_gemm_dual(x, tc, ts, m_img, out_dtype=torch.float16, split_k=False)
    assert torch.equal(y[:m_img], y_ref[:m_img])
    rows = sample_rows(m_txt, 93)
    _close(_rows_host(y[m_img:].contiguous(), rows).astype(np.float32),
           _want(x[m_img:].contiguous(), rows, qw1), "text stream vs oracle")


def test_w4a16_splitk_small_workspace(dev):
    """With less workspace than the split needs the call runs unsplit and
    equals the workspace-free entry bit for bit."""
    import qwen_image_hip as q
    import qwen_image_hip.ops as ops
    from qwen_image_hip.ops import _ptr, _stream
    m, n, k = 300, 1024, 3584
    need = q.load().qi_hip_w4a16_workspace_bytes(m, 0, n, k)
    assert need > 0
    x = normal_f16_dev(m, k, 5, dev)
    _, tc, ts = _record(n, k, 6, dev)
    ws = torch.empty(need - 16, dtype=torch.uint8, device=dev)
    y = torch.empty(m, n, device=dev)
    st = q.load().qi_hip_w4a16_gemm_tiled_ws(_ptr(x), _ptr(tc), _ptr(ts), None, _ptr(y), 0, 0, m, 0, n, k, n,
                                             _ptr(ws), need - 16, _stream())
    assert st == 0
    assert torch.equal(y, ops.w4a16_gemm(x, tc, ts, split_k=False))


# (m, n, k, tile choice): 128 x 192, 256 x 256 and 128 x 128 tiles, a
# ragged last row tile.
F16W_CASES = [(2048, 9216, 3072, 4), (4096, 12288, 3072, 5), (2048, 2176, 1024, 6), (3000, 12288, 3072, 4)]


@pytest.mark.parametrize("m,n,k,cfg", F16W_CASES)
def test_w4a16_f16w(dev, m, n, k, cfg):
    import qwen_image_hip as q
    import qwen_image_hip.ops as ops
    print(f"w4a16 fp16-weight path m={m} n={n} k={k}", flush=True)
    L = q.load()
    assert L.qi_hip_w4a16_tiles(m, n) == cfg
    assert L.qi_hip_w4a16_workspace_bytes(m, 0, n, k) == n * k * 2
    x = normal_f16_dev(m, k, 60 + m, dev)
    qw, tc, ts = _record(n, k, 61 + n, dev)
    g = torch.Generator(device=dev).manual_seed(m * n)
    bias = torch.randn(n, generator=g, device=dev)
    y = ops.w4a16_gemm(x, tc, ts, bias=bias, gelu=True, out_dtype=torch.float16)
    y_ref = ops.w4a16_gemm(x, tc, ts, bias=bias, gelu=True, out_dtype=torch.float16, split_k=False)
    assert torch.equal(y, y_ref)
    rows = sample_rows(m, m + n)
    _close(_rows_host(y, rows).astype(np.float32), _want(x, rows, qw, bias, gelu=True),
           f"fp16 weights vs oracle, {len(rows)} rows")


# Ragged shapes on each workspace path: tall 128-row and 160-row K splits
# (rows 161..320, >= 128 groups) and the fp16-weight path on 128 x 128 tiles
# with a ragged last row tile -- against the oracle on sampled rows and the
# workspace-free entry (bit for bit on the fp16-weight path).
RAGGED_CASES = [(161, 1024, 8192, "tall"), (255, 2048, 8192, "tall"), (257, 1024, 8192, "tall"),
                (319, 512, 16384, "tall"), (2085, 1408, 1024, "f16w"), (2085, 1408, 3072, "f16w")]


@pytest.mark.parametrize("m,n,k,path", RAGGED_CASES)
def test_w4a16_workspace_paths_ragged(dev, m, n, k, path):
    import qwen_image_hip as q
    import qwen_image_hip.ops as ops
    print(f"w4a16 workspace path {path} m={m} n={n} k={k}", flush=True)
    ws = q.load().qi_hip_w4a16_workspace_bytes(m, 0, n, k)
    # fp16 weights (n k halves), or whole fp32 K slices of the output.
    assert ws == n * k * 2 if path == "f16w" else (ws > 0 and ws % (m * n * 4) == 0)
    x = normal_f16_dev(m, k, 3 * m + k, dev)
    qw, tc, ts = _record(n, k, m + n, dev)
    y = ops.w4a16_gemm(x, tc, ts)
    y_ref = ops.w4a16_gemm(x, tc, ts, split_k=False)
    if path == "f16w":
        assert torch.equal(y, y_ref)
    else:
        _close(y.cpu().numpy(), y_ref.cpu().numpy(), "split vs unsplit, all rows")
    rows = sample_rows(m, m + k)
    _close(_rows_host(y, rows), _want(x, rows, qw), f"vs oracle, {len(rows)} rows")
