"""GPU parity at the MMDiT block's own shapes (configs 2, 3 and 5).

The block's linears: per stream q, k, v, out 3072 x 3072, MLP up
3072 -> 12288 (GELU), down 12288 -> 3072; image rows 4096 (12288 for an edit
with two reference images), text rows 256 (512).  Every kernel shape the
dispatcher picks for these linears runs here at its full K, so the multi-group
rings, the interleaved dequantisation and the persistent tile walk are
compared with the oracle at real depth.

The GPU computes every row; the oracle recomputes a sample of rows (both
streams' first and last rows, rows either side of 128- and 256-row tile
boundaries, the rest random), which bounds the CPU time while covering every
column tile.  W4A4 outputs must be bit-identical to the reference's fp32
group order (gemm.cu:137-168); W4A16 outputs within rel-L2 <= 1e-3 and
max-abs <= 2e-2 * rms(out) of the float64 oracle (gemm.cu:191-268).
"""
import numpy as np
import pytest
import torch

import oracle
from _data import MAX_ABS_RMS_TOL, REL_L2_TOL, max_abs_over_rms, rel_l2, weights_f16

pytestmark = pytest.mark.gpu

SAMPLE = 192


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _h(bits, dev):
    return _dev(np.ascontiguousarray(bits).view(np.float16), dev)


def _close(got, want, what):
    e, a = rel_l2(got, want), max_abs_over_rms(got, want)
    print(f"  {what}: rel-L2 {e:.3e} (bar {REL_L2_TOL:g}), max-abs/rms {a:.3e} (bar {MAX_ABS_RMS_TOL:g})",
          flush=True)
    assert e <= REL_L2_TOL and a <= MAX_ABS_RMS_TOL, (e, a)


def heavy_tailed_dev(m, k, seed, dev):
    """Student-t (3 degrees of freedom) with 1 % of the channels scaled by
    20, generated on the device (the config-3 activation distribution)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    z = torch.randn(m, k, generator=g, device=dev)
    c = torch.randn(3, m, k, generator=g, device=dev).square_().sum(0)
    t = z / torch.sqrt(c / 3.0)
    idx = torch.randperm(k, generator=g, device=dev)[: max(1, -(-k // 100))]
    t[:, idx] *= 20.0
    return t.contiguous()


def normal_f16_dev(m, k, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(m, k, generator=g, device=dev).half()


def sample_rows(m, seed, splits=()):
    """Sorted distinct rows of [0, m): both ends, random rows either side of
    128-row tile edges, every stream edge and 32 rows of the stream after
    it, the rest uniform."""
    g = np.random.default_rng(seed)
    edges = np.arange(128, m, 128)
    edges = g.choice(edges, size=min(len(edges), SAMPLE // 4), replace=False) if len(edges) else edges
    fixed = [0, 1, m - 2, m - 1, *edges - 1, *edges]
    for s in splits:
        fixed += [s - 2, s - 1, s, s + 1, *g.choice(np.arange(s, m), size=min(32, m - s), replace=False)]
    rows = np.unique(np.concatenate([np.array(fixed, np.int64), g.choice(m, size=min(SAMPLE // 2, m), replace=False)]))
    return rows[(rows >= 0) & (rows < m)]


def _rows_host(t, rows):
    return t[torch.from_numpy(rows).to(t.device)].cpu().numpy()


# ------------------------------------------------------------------ W4A16 --

# (m, n, k, tiles): every tiled kernel shape the block's W4A16 linears use,
# at the block's K.  Tile ids as qi_hip_w4a16_tiles returns them.
W4A16_CASES = [
    (4096, 12288, 3072, 5),   # MLP up: 256 x 256 tiles
    (4096, 3072, 12288, 4),   # MLP down: 128 x 192 tiles at K = 12288
    (4096, 9216, 3072, 4),    # fused QKV: 128 x 192
    (4096, 3072, 3072, 4),    # out projection: 128 x 192
    (600, 18432, 3072, 4),    # 128 x 192 on a ragged last row band
    (256, 12288, 3072, 3),    # text MLP up: 64 x 64 tiles
    (240, 9216, 1024, 3),     # 64 x 64 tiles, ragged rows
    (64, 12288, 3072, 1),     # K-split on a wide N
    (256, 3072, 12288, 1),    # text MLP down: K-split
    (1152, 1024, 256, 6),     # 128 x 128 tiles
    (1152, 18432, 128, 4),    # 128 x 192 tiles, two groups
    (300, 32768, 512, 7),     # 64 x 128 tiles (an encoder's gate + up shape), ragged rows
    (300, 4608, 3584, 3),     # an encoder's fused q + k + v (3 K slices with a workspace)
    (300, 3584, 18944, 3),    # an encoder's MLP down (160 x 64 tiles, 4 K slices, with a workspace)
]


@pytest.mark.parametrize("m,n,k,tiles", W4A16_CASES)
def test_w4a16_block_shape(dev, m, n, k, tiles):
    import qwen_image_hip as q
    import qwen_image_hip.ops as ops
    print(f"w4a16 block shape m={m} n={n} k={k} tiles={tiles}", flush=True)
    assert q.load().qi_hip_w4a16_tiles(m, n) == tiles
    x = normal_f16_dev(m, k, 10 + m + k, dev)
    w = weights_f16(n, k, 11 + n + k)
    c, s, mn = oracle.quantize_matrix(w, 5)
    tc, ts = ops.relayout_w4a16(_dev(c, dev), _h(s, dev), _h(mn, dev))
    y = ops.w4a16_gemm(x, tc, ts)
    rows = sample_rows(m, m + n)
    xr = _rows_host(x, rows).view(np.uint16)
    _close(_rows_host(y, rows), oracle.w4a16_gemm(xr, c, s, mn, precise=True), f"{len(rows)} rows")


def test_w4a16_dual_stream_block_qkv(dev):
    """The block's fused QKV for both streams (4096 + 256 rows, 3 x 3072
    outputs per stream, K = 3072) as one dual-stream record through
    linear(), against the oracle on sampled rows of each stream."""
    import qwen_image_hip as q
    m_img, m_txt, n, k = 4096, 256, 3072, 3072
    m = m_img + m_txt
    x = normal_f16_dev(m, k, 20, dev)
    host, recs = [], []
    for s in range(2):
        ws = [weights_f16(n, k, 21 + 3 * s + i) for i in range(3)]
        qs = [oracle.quantize_matrix(w, 5) for w in ws]
        host.append(qs)
        recs.append(q.PackedLinear.fuse([q.PackedLinear.from_qipack(q.SCHEME_W4A16, _dev(c, dev), _h(sc, dev),
                                                                    _h(mn, dev)) for c, sc, mn in qs]))
    work = q.Work(m, k, dev)
    y = q.linear(q.PackedLinear.dual(recs), work, x, split_rows=m_img)      # [3, m, n]
    rows = sample_rows(m, 22, splits=(m_img,))
    xr = _rows_host(x, rows).view(np.uint16)
    for s, sel in enumerate((rows < m_img, rows >= m_img)):
        for p, (c, sc, mn) in enumerate(host[s]):
            got = y[p][torch.from_numpy(rows[sel]).to(dev)].cpu().numpy()
            _close(got, oracle.w4a16_gemm(xr[sel], c, sc, mn, precise=True), f"stream {s} part {p}")


# ------------------------------------------------------------------- W4A4 --

def _w4a4_record(q, n, k, seed, dev, parts=1):
    hs, recs = [], []
    for i in range(parts):
        w = weights_f16(n, k, seed + i)
        c, s, _ = oracle.quantize_matrix(w, 6, clip=True)
        hs.append((c, s))
        recs.append(q.PackedLinear.from_qipack(q.SCHEME_W4A4_H256, _dev(c, dev), _h(s, dev)))
    return hs, (recs[0] if parts == 1 else q.PackedLinear.fuse(recs))


def _w4a4_check(y_rows, x_rows, c, s):
    ac, as_ = oracle.quantize_activations(x_rows)
    want = oracle.w4a4_gemm(ac, as_, c, s)
    np.testing.assert_array_equal(y_rows.view(np.uint32), want.view(np.uint32))


# The persistent fp6 kernel at the block's K (48 and 192 groups: 12 and 48
# ring passes per tile) and widths, and the text stream's short-M tiles.
@pytest.mark.parametrize("m,n,k", [(4096, 3072, 3072), (4096, 12288, 3072), (4096, 3072, 12288),
                                   (256, 12288, 3072), (256, 3072, 12288)])
def test_w4a4_block_shape_bit_exact(dev, m, n, k):
    import qwen_image_hip as q
    print(f"w4a4 block shape m={m} n={n} k={k} tiles={q.load().qi_hip_w4a4_fp6_tiles(m, n)}", flush=True)
    x = heavy_tailed_dev(m, k, 30 + m + k, dev)
    (hs,), rec = _w4a4_record(q, n, k, 31 + n + k, dev)
    work = q.Work(m, k, dev)
    y = q.linear(rec, work, x)
    rows = sample_rows(m, m + n + 1)
    _w4a4_check(_rows_host(y, rows), _rows_host(x, rows), *hs)


def test_w4a4_block_mlp_up_epilogue(dev):
    """MLP up with bias, GELU-tanh and fp16 outputs at the block's shape:
    the exact fp32 accumulator (checked bit for bit above) through the
    epilogue, within two fp16 ulps of the correctly rounded value."""
    import qwen_image_hip as q
    m, n, k = 4096, 12288, 3072
    x = heavy_tailed_dev(m, k, 40, dev)
    (hs,), rec = _w4a4_record(q, n, k, 41, dev)
    bias = np.random.default_rng(42).normal(0, 0.5, size=n).astype(np.float32)
    rec.bias = _dev(bias, dev)
    y = q.linear(rec, q.Work(m, k, dev), x, gelu=True, out_dtype=torch.float16)
    rows = sample_rows(m, 43)
    ac, as_ = oracle.quantize_activations(_rows_host(x, rows))
    v = oracle.gelu_tanh(oracle.w4a4_gemm(ac, as_, *hs) + bias[None, :])
    want = oracle.half_to_f32(oracle.half_from_f32(v))
    np.testing.assert_allclose(_rows_host(y, rows).astype(np.float32), want, rtol=2 * 2.0 ** -10, atol=2.0 ** -20)


@pytest.mark.parametrize("m_img,m_txt", [(4096, 256), (12288, 512)])
def test_w4a4_dual_stream_fused_qkv(dev, m_img, m_txt):
    """The block's fused QKV (3 x 3072 outputs per stream, K = 3072) for both
    streams as one dual-stream call through linear(split_rows=m_img): config
    3's 4096 + 256 rows, the headline launch, and config 5's 12288 + 512 rows
    (an edit with two reference images), bit for bit against the oracle on
    sampled rows of each stream."""
    import qwen_image_hip as q
    n, k = 3072, 3072
    m = m_img + m_txt
    print(f"w4a4 dual-stream fused qkv {m_img}+{m_txt} x 3x{n} x {k}", flush=True)
    x = heavy_tailed_dev(m, k, 50 + m, dev)
    hs0, r0 = _w4a4_record(q, n, k, 51, dev, parts=3)
    hs1, r1 = _w4a4_record(q, n, k, 61, dev, parts=3)
    y = q.linear(q.PackedLinear.dual([r0, r1]), q.Work(m, k, dev), x, split_rows=m_img)   # [3, m, n]
    rows = sample_rows(m, 52 + m, splits=(m_img,))
    xr = _rows_host(x, rows)
    for hs, sel in ((hs0, rows < m_img), (hs1, rows >= m_img)):
        r = torch.from_numpy(rows[sel]).to(dev)
        for p, (c, s) in enumerate(hs):
            _w4a4_check(y[p][r].cpu().numpy(), xr[sel], c, s)


def test_w4a4_dual_stream_mlp_down(dev):
    """MLP down (12288 -> 3072) for both streams in one dual-stream launch,
    K = 12288 (192 groups per tile), bit for bit on sampled rows."""
    import qwen_image_hip as q
    m_img, m_txt, n, k = 4096, 256, 3072, 12288
    m = m_img + m_txt
    x = heavy_tailed_dev(m, k, 70, dev)
    (h0,), r0 = _w4a4_record(q, n, k, 71, dev)
    (h1,), r1 = _w4a4_record(q, n, k, 72, dev)
    y = q.linear(q.PackedLinear.dual([r0, r1]), q.Work(m, k, dev), x, split_rows=m_img)
    rows = sample_rows(m, 73, splits=(m_img,))
    xr = _rows_host(x, rows)
    for h, sel in ((h0, rows < m_img), (h1, rows >= m_img)):
        _w4a4_check(y[torch.from_numpy(rows[sel]).to(dev)].cpu().numpy(), xr[sel], *h)
