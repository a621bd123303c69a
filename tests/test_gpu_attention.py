"""GPU parity of the fused attention (reference qi_flash_attention,
qwen_image_cuda/cuda/flash.cu) against the float64 oracle on small shapes
(every mask form, ragged tiles, rows with nothing visible) and against a
torch fp32 restatement at the 1024x1024 block's full size."""
import numpy as np
import pytest
import torch

import oracle
from _data import MAX_ABS_RMS_TOL, REL_L2_TOL, max_abs_over_rms, rel_l2

pytestmark = pytest.mark.gpu


def _case(nq, nk, heads, seed):
    rng = np.random.default_rng(seed)
    q = rng.normal(0, 1.5, size=(nq, heads * 128)).astype(np.float32)
    k = oracle.half_from_f32(rng.normal(0, 1, size=(nk, heads * 128)).astype(np.float32))
    v = oracle.half_from_f32(rng.normal(0, 1, size=(nk, heads * 128)).astype(np.float32))
    return q, k, v


def _run(dev, q, k, v, heads, **kw):
    import qwen_image_hip.ops as ops
    vis = kw.pop("visible_keys", None)
    vd = None if vis is None else torch.from_numpy(np.asarray(vis, np.int32)).to(dev)
    return ops.flash_attention(torch.from_numpy(q).to(dev), torch.from_numpy(k).to(dev).view(torch.float16),
                               torch.from_numpy(v).to(dev).view(torch.float16), heads, visible_keys=vd,
                               **kw).cpu().numpy()


def _close(got, want):
    e, a = rel_l2(got, want), max_abs_over_rms(got, want)
    print(f"  rel-L2 {e:.3e} (bar {REL_L2_TOL:g}), max-abs/rms {a:.3e} (bar {MAX_ABS_RMS_TOL:g})", flush=True)
    assert e <= REL_L2_TOL, e
    assert a <= MAX_ABS_RMS_TOL, a


@pytest.mark.parametrize("nq,nk,heads", [(1, 64, 1), (200, 300, 3), (129, 1000, 2)])
def test_attention_unmasked(dev, nq, nk, heads):
    print(f"attention nq={nq} nk={nk} heads={heads}", flush=True)
    q, k, v = _case(nq, nk, heads, 1000 + nq)
    _close(_run(dev, q, k, v, heads), oracle.flash_attention(q, k, v, heads))


@pytest.mark.parametrize("step", [0.05, 0.5, 3.0])
def test_attention_rising_scores(dev, step):
    """Scores that rise from key tile to key tile (by `step` per key in the
    log2 domain, so the running maximum grows by less than, about, and far
    more than the kernel's rescaling threshold per 64-key tile), against
    the oracle."""
    rng = np.random.default_rng(1400)
    nq, nk, heads = 96, 700, 1
    u = rng.normal(0, 1, size=128).astype(np.float32)
    u /= np.linalg.norm(u)
    # q_i . k_j ~ 3 c_j + noise; in the kernel's log2 domain (scale
    # log2(e) / sqrt(128)) the score of key j is about step * j.
    c = step * np.arange(nk, dtype=np.float32) / (3.0 * 1.4426950408889634 / np.sqrt(128.0))
    q = (rng.normal(0, 0.3, size=(nq, 128)) + 3.0 * u).astype(np.float32)
    k = oracle.half_from_f32((rng.normal(0, 0.3, size=(nk, 128)) + c[:, None] * u).astype(np.float32))
    v = oracle.half_from_f32(rng.normal(0, 1, size=(nk, 128)).astype(np.float32))
    _close(_run(dev, q, k, v, heads), oracle.flash_attention(q, k, v, heads))


def test_attention_causal_and_offset(dev):
    q, k, v = _case(257, 400, 2, 1100)
    got = _run(dev, q, k, v, 2, query_offset=50, causal_rows=200)
    want = oracle.flash_attention(q, k, v, 2, query_offset=50, causal_rows=200)
    _close(got, want)
    # global row 50 + 0 < 200 sees 51 keys; rows from 150 on see all 400
    np.testing.assert_allclose(got[0], want[0], rtol=5e-3, atol=5e-3)


def test_attention_visible_keys_and_empty_rows(dev):
    q, k, v = _case(96, 130, 2, 1200)
    vis = np.random.default_rng(1201).integers(0, 131, size=96)
    vis[[0, 7, 40]] = 0                       # nothing visible: output 0
    vis[[1, 2]] = 1                           # one key: its value row
    got = _run(dev, q, k, v, 2, visible_keys=vis)
    want = oracle.flash_attention(q, k, v, 2, visible_keys=vis)
    assert (got[[0, 7, 40]] == 0).all()
    np.testing.assert_array_equal(got[1], oracle.half_to_f32(v[0]))
    _close(got, want)


def test_attention_full_block_size_vs_torch_fp32(dev):
    """4352 tokens (4096 image + 256 text), 24 heads: against torch fp32 on
    the same fp16-rounded scaled q and fp16 k, v (softmax in fp32)."""
    import qwen_image_hip.ops as ops
    n, heads = 4352, 24
    g = torch.Generator(device=dev)
    g.manual_seed(1300)
    q = torch.randn((n, heads * 128), generator=g, device=dev) * 1.5
    k = torch.randn((n, heads * 128), generator=g, device=dev).half()
    v = torch.randn((n, heads * 128), generator=g, device=dev).half()
    got = ops.flash_attention(q, k, v, heads)
    scale = np.float32(1.4426950408889634) / np.sqrt(np.float32(128))
    qs = (q * float(scale)).half().float().view(n, heads, 128).transpose(0, 1)
    s = torch.bmm(qs, k.float().view(n, heads, 128).permute(1, 2, 0))          # log2-domain scores
    p = torch.softmax(s * float(np.log(2.0)), dim=-1)
    want = torch.bmm(p, v.float().view(n, heads, 128).transpose(0, 1)).transpose(0, 1).reshape(n, heads * 128)
    _close(got.cpu().numpy(), want.cpu().numpy())


def _split_bytes(nq, nk, heads):
    import qwen_image_hip
    return qwen_image_hip.load().qi_hip_flash_attention_workspace_bytes(nq, nk, heads)


def test_attention_split_choice(dev):
    """The balanced split is taken where whole rounds of query blocks would
    leave CUs idle, and not where the query blocks fill the CUs evenly."""
    import qwen_image_hip
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    assert _split_bytes(256 * (cus + cus // 16), 4352, 1) > 0  # one round and 1/16 of another
    assert _split_bytes(256 * cus, 4352, 1) == 0               # exactly one round
    assert _split_bytes(300, 4100, 3) > 0                      # 6 blocks: keys spread over CUs
    assert _split_bytes(129, 192, 2) == 0                      # 3 key tiles: too short to split
    assert _split_bytes(4352, 4352, 24) == 0                   # 152 blocks left: parts over several rounds
    assert _split_bytes(0, 1000, 2) == 0 and _split_bytes(10, 0, 2) == 0
    assert _split_bytes(10, 10, 0) == 0


@pytest.mark.parametrize("nq,nk,heads,offset", [(2000, 2100, 40, 0), (300, 4100, 3, 0), (1000, 2000, 5, 64)])
def test_attention_split_vs_oracle(dev, nq, nk, heads, offset):
    """A lockstep round then the blocks left split in 4 key segments, 6
    blocks in 6 segments with ragged key and query tiles, and a query
    offset with no causal row: the balanced split against the oracle and
    against the one-block-per-workgroup grid."""
    print(f"attention split nq={nq} nk={nk} heads={heads} offset={offset}", flush=True)
    assert _split_bytes(nq, nk, heads) > 0
    q, k, v = _case(nq, nk, heads, 1500 + nq)
    got = _run(dev, q, k, v, heads, query_offset=offset, causal_rows=offset)
    plain = _run(dev, q, k, v, heads, query_offset=offset, causal_rows=offset, balanced=False)
    want = oracle.flash_attention(q, k, v, heads, query_offset=offset, causal_rows=offset)
    _close(got, want)
    _close(plain, want)
    # The parts form their fp16 probabilities at their own offsets, so the
    # two grids round differently: equal within the attention tolerance.
    d = rel_l2(got, plain)
    print(f"  split vs plain rel-L2 {d:.3e}", flush=True)
    assert d <= REL_L2_TOL


def test_attention_split_deterministic_and_small_workspace(dev):
    """Two balanced calls give identical bits (parts merge in workgroup
    order, whatever order they finish in); a workspace one byte short runs
    the plain grid, bit for bit."""
    import qwen_image_hip
    from qwen_image_hip import ops
    L = qwen_image_hip.load()
    n, heads = 4352, 16
    g = torch.Generator(device=dev)
    g.manual_seed(1600)
    q = torch.randn((n, heads * 128), generator=g, device=dev)
    k = torch.randn((n, heads * 128), generator=g, device=dev).half()
    v = torch.randn((n, heads * 128), generator=g, device=dev).half()
    a = ops.flash_attention(q, k, v, heads)
    b = ops.flash_attention(q, k, v, heads)
    plain = ops.flash_attention(q, k, v, heads, balanced=False)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert ((a - plain).norm() / plain.norm()).item() <= REL_L2_TOL
    ws_bytes = L.qi_hip_flash_attention_workspace_bytes(n, n, heads)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    short = torch.empty_like(q)
    s = torch.cuda.current_stream().cuda_stream
    assert L.qi_hip_flash_attention_ws(q.data_ptr(), k.data_ptr(), v.data_ptr(), short.data_ptr(), n, n, heads, 0, 0,
                                       None, ws.data_ptr(), ws_bytes - 1, s) == 0
    torch.cuda.synchronize()
    assert torch.equal(short, plain)
