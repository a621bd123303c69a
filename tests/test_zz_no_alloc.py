"""GPU test of the no-allocation entry point
qi_hip_layer_norm_scale_quantize_fp6_noalloc (row statistics in the
library's fixed device array instead of a caller workspace): through the C
ABI, its fp6 codes equal those of qi_hip_layer_norm_scale_quantize_fp6 with
a caller-supplied workspace, bit for bit, on two calls in a row (the second
on fewer rows, so stale statistics from the first call would show)."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _codes_bytes(m, k):
    return ((m + 31) // 32 * 32, k // 64 * 56)


@pytest.mark.parametrize("first,second", [((4096, 3072, 4000), (300, 3072, 0)), ((1056, 12288, 0), (37, 256, 20))])
def test_noalloc_layer_norm_quantize_matches_workspace_form(dev, first, second):
    import qwen_image_hip as q
    lib = q.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    g = torch.Generator(device=dev).manual_seed(5)
    for m, k, split in (first, second):
        print(f"noalloc layer norm quantize m={m} k={k} split={split}", flush=True)
        x = torch.randn((m, k), generator=g, device=dev) * 3.0 + 0.5
        scale = torch.randn((2, k), generator=g, device=dev) * 0.3
        want = torch.full(_codes_bytes(m, k), 0xA5, dtype=torch.uint8, device=dev)
        got = torch.full(_codes_bytes(m, k), 0x5A, dtype=torch.uint8, device=dev)
        stats = torch.empty((m, 2), dtype=torch.float32, device=dev)
        assert lib.qi_hip_layer_norm_scale_quantize_fp6(x.data_ptr(), scale.data_ptr(), k, split, stats.data_ptr(),
                                                        want.data_ptr(), m, k, stream) == 0
        assert lib.qi_hip_layer_norm_scale_quantize_fp6_noalloc(x.data_ptr(), scale.data_ptr(), k, split,
                                                                got.data_ptr(), m, k, stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_noalloc_rejects_rows_beyond_the_array(dev):
    import qwen_image_hip as q
    lib = q.load()
    assert lib.qi_hip_layer_norm_scale_quantize_fp6_noalloc(16, 16, 256, 0, 16, 65537, 256, None) == 1
