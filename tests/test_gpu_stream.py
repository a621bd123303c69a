"""GPU test of block streaming (qwen_image_hip.BlockStream, the reference's
two-slot asynchronous block upload, transformer.cplus:503-598): a small
stack of blocks run through the two device slots gives every block's outputs
bit-identical to the same blocks resident in HBM, over two passes of the
cyclic walk (the prefix pass, then a step)."""
import numpy as np
import pytest
import torch

from _data import heavy_tailed, weights_f16

pytestmark = pytest.mark.gpu


def _h(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits)).to(dev).view(torch.float16)


def test_streamed_blocks_match_resident(dev):
    import qwen_image_hip as q
    blocks_n, m_img, m_txt, k, n = 5, 96, 64, 512, 256
    m = m_img + m_txt
    print(f"block stream {blocks_n} blocks m={m_img}+{m_txt} k={k} n={n}", flush=True)
    g = np.random.default_rng(3)
    blocks = []
    for b in range(blocks_n):
        streams = []
        for s in range(2):
            parts = [q.PackedLinear.from_fp16(q.SCHEME_W4A4_H256, _h(weights_f16(n, k, 100 * b + 10 * s + i), dev),
                                              clip=True) for i in range(3)]
            rec = q.PackedLinear.fuse(parts)
            rec.bias = torch.from_numpy(g.normal(0, 0.5, 3 * n).astype(np.float32)).to(dev)
            streams.append(rec)
        w16 = q.PackedLinear.from_fp16(q.SCHEME_W4A16, _h(weights_f16(n, k, 100 * b + 50), dev))
        blocks.append({"qkv": q.PackedLinear.dual(streams), "w16": w16})
    x = torch.from_numpy(heavy_tailed(m, k, 7)).to(dev)
    x16 = x.half()
    work = q.Work(m, k, dev)

    def run(recs):
        y = q.linear(recs["qkv"], work, x, split_rows=m_img, out_dtype=torch.float16, gelu=True)
        z = q.linear(recs["w16"], work, x16)
        return y.clone(), z.clone()

    want = [run(blk) for blk in blocks]
    stream = q.BlockStream(blocks, dev)
    for _ in range(2):
        for b in range(blocks_n):
            got = run(stream.begin(b))
            stream.end(b)
            for a, w in zip(got, want[b]):
                assert torch.equal(a, w), f"block {b} differs when streamed"
    torch.cuda.synchronize()


def test_stream_rejects_out_of_order_blocks(dev):
    import qwen_image_hip as q
    w = torch.zeros((64, 256), dtype=torch.float16, device=dev)
    blocks = [{"a": q.PackedLinear.from_fp16(q.SCHEME_W4A16, w)} for _ in range(3)]
    stream = q.BlockStream(blocks, dev)
    stream.begin(0)
    stream.end(0)
    with pytest.raises(ValueError):
        stream.begin(2)
    torch.cuda.synchronize()
