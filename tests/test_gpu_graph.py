"""The linear paths under HIP graph capture: a captured sequence of linear()
calls (W4A4 on both operand formats with input reuse, W4A16 GEMM, W4A16 GEMV)
is replayed several times, with eager work in between, and every replay must
equal the eager results bit for bit."""
import numpy as np
import pytest
import torch

from _data import heavy_tailed, weights_f16

pytestmark = pytest.mark.gpu


def _h(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.float16)).to(dev)


def test_linear_graph_replay(dev):
    import qwen_image_hip as q
    rows, k, n = 200, 512, 384
    x = torch.from_numpy(heavy_tailed(rows, k, 1200)).to(dev).half()
    work = q.Work(rows, k, dev)
    w = [weights_f16(n, k, 1201 + i) for i in range(4)]
    r6 = q.PackedLinear.from_fp16(q.SCHEME_W4A4_H256, _h(w[0], dev), clip=True)
    r6b = q.PackedLinear.from_fp16(q.SCHEME_W4A4_H256, _h(w[1], dev), clip=True)
    r8 = q.PackedLinear.from_fp16(q.SCHEME_W4A4_H256, _h(w[2], dev), clip=True, operand=q.W4A4_INT8)
    r5 = q.PackedLinear.from_fp16(q.SCHEME_W4A16, _h(w[3], dev))
    outs = [torch.empty((rows, n), dtype=torch.float16, device=dev) for _ in range(4)]
    gemv_out = torch.empty((2, n), dtype=torch.float32, device=dev)

    def step():
        q.linear(r6, work, x, outs[0], out_dtype=torch.float16)
        q.linear(r6b, work, x, outs[1], reuse_input=True, out_dtype=torch.float16, gelu=True)
        q.linear(r8, work, x, outs[2], out_dtype=torch.float16)
        q.linear(r5, work, x, outs[3], out_dtype=torch.float16)
        q.linear(r5, work, x[:2], gemv_out)

    step()
    torch.cuda.synchronize()
    want = [o.clone() for o in outs] + [gemv_out.clone()]
    capture = torch.cuda.Stream()
    capture.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=capture):
        step()
    torch.cuda.synchronize()
    for it in range(4):
        for o in outs + [gemv_out]:
            o.zero_()           # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(want, outs + [gemv_out]):
            assert torch.equal(a, b), f"replay {it} differs"
