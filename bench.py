"""QIPACK W4A4 / W4A16 linear benchmark on one MI355X.

A step is one pass of one Qwen-Image MMDiT dual-stream block's linears at
1024x1024 (image stream M = 4096 tokens, text stream M = 256 tokens; per
stream to_q, to_k, to_v, to_out 3072x3072, MLP up 3072->12288 with fused
GELU-tanh, down 12288->3072), W4A4 with H256/g64: every
distinct input is quantised online (Q/K/V share one quantisation, as the
reference's reuse_input does) and all seven GEMMs run.  value = block TOPS
(2*M*N*K int ops per GEMM, quantiser work not counted).  The same pass with
W4A16 weights (config 2), the same W4A4 pass on the int8 operand path and
the M=1/M=2 modulation GEMV (config 4) are reported beside it.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu] [--no-extra]
    python bench.py --library-only   # calibration: hipBLASLt plain fp16 / int8 GEMMs, same shapes
    python bench.py --kernel-only    # the dominant GEMM x 20 + a 512 MiB copy,
                                     # the workload of the counter runs
    python bench.py --gemv-only      # the all-blocks modulation GEMV x 10 + a
                                     # 512 MiB copy, for the GEMV's counter runs
    python bench.py --w4a16-only     # the W4A16 MLP-up GEMM x 11 + a 512 MiB copy
    python bench.py --probe-overlap  # matrix-core / vector-unit co-execution micro-benchmark
    python bench.py --ablate-w4a4    # the roofline kernel with parts of its work removed
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "qwen-image-cplus_amd"))

HIDDEN, MLP = 3072, 12288
STREAMS = {"image": 4096, "text": 256}
MODULATION_N = 18432
PEAK_INT8_OPS = 5.0e15      # MI355X dense int8 MFMA
PEAK_FP16_FLOPS = 2.5e15    # MI355X dense fp16 MFMA
PEAK_HBM = 8.0e12           # MI355X HBM3E bytes/s
TRAFFIC_FILE = ROOT / "profiles" / "w4a4_gemm_traffic.json"
# The roofline kernel: its traffic record counts only when measured on it.
DOMINANT_WORKLOAD = "w4a4 fp6 dual-stream GEMM M=4096+256 N=9216 per stream K=3072 (fused qkv), fp16 out"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def block_shapes():
    """(name, N, K) of one stream's block linears."""
    return [("to_q", HIDDEN, HIDDEN), ("to_k", HIDDEN, HIDDEN), ("to_v", HIDDEN, HIDDEN),
            ("to_out", HIDDEN, HIDDEN), ("mlp_up", MLP, HIDDEN), ("mlp_down", HIDDEN, MLP)]


def block_ops() -> float:
    params = sum(n * k for _, n, k in block_shapes())
    return 2.0 * params * sum(STREAMS.values())


class Block:
    """Random-init weights of one block (both streams), packed on the device."""

    def __init__(self, scheme: int, seed: int, operand: str = "fp6"):
        import torch
        import qwen_image_hip as q

        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.layers = {}
        for stream in STREAMS:
            for name, n, k in block_shapes():
                w = (torch.randn((n, k), generator=g, device="cuda") * 0.02).half()
                # W4A4 packs use the clip search; W4A16 packs do not (the
                # reference's published packs, README.md:38).
                self.layers[(stream, name)] = q.PackedLinear.from_fp16(
                    scheme, w, clip=(scheme == q.SCHEME_W4A4_H256), operand=operand)
                del w
            # to_q, to_k and to_v read one input: one fused record, one GEMM
            # (the int8 operand path keeps three calls).
            if operand == "fp6" or scheme == q.SCHEME_W4A16:
                self.layers[(stream, "qkv")] = q.PackedLinear.fuse(
                    [self.layers[(stream, name)] for name in ("to_q", "to_k", "to_v")])
        # fp6 W4A4 and W4A16: each linear's image and text records as one
        # dual-stream record (both streams in one launch over their stacked
        # rows).
        if operand == "fp6" or scheme == q.SCHEME_W4A16:
            for name in ("qkv", "to_out", "mlp_up", "mlp_down"):
                self.layers[("dual", name)] = q.PackedLinear.dual(
                    [self.layers[(stream, name)] for stream in STREAMS])
        torch.cuda.synchronize()


def heavy_tailed(m, k, g):
    """Student-t (3 dof) fp16 activations, 1% of channels scaled by 20."""
    import torch

    z = torch.randn((m, k), generator=g, device="cuda")
    chi2 = sum(torch.randn((m, k), generator=g, device="cuda") ** 2 for _ in range(3))
    t = z / torch.sqrt(chi2 / 3.0)
    idx = torch.randperm(k, generator=g, device="cuda")[: -(-k // 100)]
    t[:, idx] *= 20.0
    return t.half()


def two_streams(run_phase, side):
    """Run each phase of the block (QKV, output projection, MLP) with the text
    stream's linears on `side` and the image stream's on the current stream,
    forked and joined with stream waits per phase (a captured graph gets two
    parallel branches per phase).  Within a phase the two streams are
    independent (in the model they meet at the joint attention, between the
    phases); the small text-stream kernels fill CUs beside the image
    stream's.  side=None runs everything on the current stream in order."""
    import torch

    for phase in PHASES:
        if side is None:
            for stream in STREAMS:
                run_phase(stream, phase)
            continue
        main = torch.cuda.current_stream()
        side.wait_stream(main)
        with torch.cuda.stream(side):
            run_phase("text", phase)
        run_phase("image", phase)
        main.wait_stream(side)


PHASES = ("qkv", "out", "mlp")


class StepW4A4:
    """One block's W4A4 linears through the transformer::linear mirror: every
    distinct input quantised once, MLP up with the fused GELU, its fp16
    output quantised again for MLP down.  fp6 records: the image and text
    streams' rows stacked (image first) and each linear run as one
    dual-stream record (to_q/to_k/to_v fused), so a step is four quantiser
    and four GEMM launches.  int8 records: per stream, K/V reusing Q's codes."""

    def __init__(self, block: Block, seed: int, one_stream: bool = True):
        import torch
        import qwen_image_hip as q

        self.q = q
        self.side = None if one_stream else torch.cuda.Stream()
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.block = block
        self.dual = ("dual", "qkv") in block.layers
        self.bufs = {}
        for stream, m in STREAMS.items():
            self.bufs[stream] = {
                "x_qkv": heavy_tailed(m, HIDDEN, g), "x_out": heavy_tailed(m, HIDDEN, g),
                "x_mlp": heavy_tailed(m, HIDDEN, g),
                "work": q.Work(m, MLP, "cuda"),
                "y": torch.empty((m, HIDDEN), dtype=torch.float16, device="cuda"),
                "qkv": torch.empty((3, m, HIDDEN), dtype=torch.float16, device="cuda"),
                "h": torch.empty((m, MLP), dtype=torch.float16, device="cuda"),
            }
        if self.dual:
            m = sum(STREAMS.values())
            b = {name: torch.cat([self.bufs[st][name] for st in STREAMS], 0)
                 for name in ("x_qkv", "x_out", "x_mlp")}
            b.update({"work": q.Work(m, MLP, "cuda"),
                      "y": torch.empty((m, HIDDEN), dtype=torch.float16, device="cuda"),
                      "qkv": torch.empty((3, m, HIDDEN), dtype=torch.float16, device="cuda"),
                      "h": torch.empty((m, MLP), dtype=torch.float16, device="cuda")})
            self.bufs["stacked"] = b

    def outputs(self):
        """Copies of the buffers the step writes last (MLP hidden h, down output y)."""
        keys = ["stacked"] if self.dual else list(STREAMS)
        return [self.bufs[st][name].clone() for st in keys for name in ("h", "y")]

    def __call__(self):
        import torch

        lin = self.q.linear
        f16 = torch.float16
        if self.dual:
            b, w = self.bufs["stacked"], self.bufs["stacked"]["work"]
            L = lambda name: self.block.layers[("dual", name)]  # noqa: E731
            split = STREAMS["image"]
            lin(L("qkv"), w, b["x_qkv"], b["qkv"], out_dtype=f16, split_rows=split)
            lin(L("to_out"), w, b["x_out"], b["y"], out_dtype=f16, split_rows=split)
            lin(L("mlp_up"), w, b["x_mlp"], b["h"], out_dtype=f16, gelu=True, split_rows=split)
            lin(L("mlp_down"), w, b["h"], b["y"], out_dtype=f16, split_rows=split)
            return

        def run_phase(stream, phase):
            b = self.bufs[stream]
            L = lambda name: self.block.layers[(stream, name)]  # noqa: E731
            w = b["work"]
            if phase == "qkv" and (stream, "qkv") in self.block.layers:
                lin(L("qkv"), w, b["x_qkv"], b["qkv"], out_dtype=f16)
            elif phase == "qkv":
                lin(L("to_q"), w, b["x_qkv"], b["y"], out_dtype=f16)
                lin(L("to_k"), w, b["x_qkv"], b["y"], reuse_input=True, out_dtype=f16)
                lin(L("to_v"), w, b["x_qkv"], b["y"], reuse_input=True, out_dtype=f16)
            elif phase == "out":
                lin(L("to_out"), w, b["x_out"], b["y"], out_dtype=f16)
            else:
                lin(L("mlp_up"), w, b["x_mlp"], b["h"], out_dtype=f16, gelu=True)
                lin(L("mlp_down"), w, b["h"], b["y"], out_dtype=f16)

        two_streams(run_phase, self.side)


class StepW4A16:
    """One block's W4A16 linears: the image and text streams' rows stacked
    (image first), each linear one dual-stream record (to_q/to_k/to_v
    fused), fp16 activations, MLP up with the fused GELU feeding MLP down."""

    def __init__(self, block: Block, seed: int, one_stream: bool = True):
        import torch
        from qwen_image_hip import ops

        self.ops = ops
        self.side = None if one_stream else torch.cuda.Stream()
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.block = block
        m = sum(STREAMS.values())
        self.b = {
            "x": torch.randn((m, HIDDEN), generator=g, device="cuda").half(),
            "y": torch.empty((m, HIDDEN), dtype=torch.float16, device="cuda"),
            "qkv": torch.empty((3, m, HIDDEN), dtype=torch.float16, device="cuda"),
            "h": torch.empty((m, MLP), dtype=torch.float16, device="cuda"),
        }
        # Two streams: each stream's rows of the same buffers, its own records.
        rows, r0 = {}, 0
        for stream, ms in STREAMS.items():
            rows[stream] = (r0, r0 + ms)
            r0 += ms
        self.rows = rows
        self.qkv_s = {stream: torch.empty((3, ms, HIDDEN), dtype=torch.float16, device="cuda")
                      for stream, ms in STREAMS.items()}

    def _two_streams(self):
        ops, b, f16 = self.ops, self.b, self.ops.torch.float16

        def run_phase(stream, phase):
            r0, r1 = self.rows[stream]
            L = lambda name: self.block.layers[(stream, name)]  # noqa: E731
            x, y, h = b["x"][r0:r1], b["y"][r0:r1], b["h"][r0:r1]
            if phase == "qkv":
                r = L("qkv")
                ops.w4a16_gemm(x, r.tiled_codes, r.tiled_scales, out_dtype=f16, y=self.qkv_s[stream], n_part=HIDDEN)
            elif phase == "out":
                r = L("to_out")
                ops.w4a16_gemm(x, r.tiled_codes, r.tiled_scales, out_dtype=f16, y=y)
            else:
                r = L("mlp_up")
                ops.w4a16_gemm(x, r.tiled_codes, r.tiled_scales, out_dtype=f16, gelu=True, y=h)
                r = L("mlp_down")
                ops.w4a16_gemm(h, r.tiled_codes, r.tiled_scales, out_dtype=f16, y=y)

        two_streams(run_phase, self.side)

    def __call__(self):
        if self.side is not None:
            return self._two_streams()
        ops, b, f16 = self.ops, self.b, self.ops.torch.float16
        L = lambda name: self.block.layers[("dual", name)]  # noqa: E731
        split = STREAMS["image"]
        r = L("qkv")
        ops.w4a16_gemm_dual(b["x"], r.tiled_codes, r.tiled_scales, split, out_dtype=f16, y=b["qkv"], n_part=HIDDEN)
        r = L("to_out")
        ops.w4a16_gemm_dual(b["x"], r.tiled_codes, r.tiled_scales, split, out_dtype=f16, y=b["y"])
        r = L("mlp_up")
        ops.w4a16_gemm_dual(b["x"], r.tiled_codes, r.tiled_scales, split, out_dtype=f16, gelu=True, y=b["h"])
        r = L("mlp_down")
        ops.w4a16_gemm_dual(b["h"], r.tiled_codes, r.tiled_scales, split, out_dtype=f16, y=b["y"])


def device_peaks():
    """The box's own peaks: reported CU count x peak engine clock x per-CU
    dense rate (gfx950: 8192 int8 ops, 4096 fp16 flops per CU per clock),
    beside the published figures the roofline fractions use."""
    import ctypes

    import torch

    hip = ctypes.CDLL("libamdhip64.so")
    clock_khz, cus = ctypes.c_int(0), ctypes.c_int(0)
    # hipDeviceAttributeClockRate = 5, hipDeviceAttributeMultiprocessorCount = 63 (hip_runtime_api.h).
    if hip.hipDeviceGetAttribute(ctypes.byref(clock_khz), 5, 0) or hip.hipDeviceGetAttribute(ctypes.byref(cus), 63, 0):
        return None
    hz = clock_khz.value * 1e3
    return {"cus": cus.value, "peak_sclk_mhz": round(hz / 1e6), "name": torch.cuda.get_device_properties(0).name,
            "int8_tops_at_clock": round(cus.value * hz * 8192 / 1e12, 1),
            "fp16_tflops_at_clock": round(cus.value * hz * 4096 / 1e12, 1),
            "int8_tops_published": PEAK_INT8_OPS / 1e12, "fp16_tflops_published": PEAK_FP16_FLOPS / 1e12,
            "hbm_gb_s_published": PEAK_HBM / 1e9}


WARM_S = 0.05  # untimed work before every timed region: the clock drops while the GPU idles between sections


def time_fn(fn, iters, warmup):
    """Mean ms per call with HIP events on the current stream (the one every
    op is launched on), after `warmup` untimed calls and at least WARM_S
    seconds of untimed calls (the GPU clock settles again after the host-side
    set-up between sections)."""
    import time

    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0, n = time.perf_counter(), 0
    while time.perf_counter() - t0 < WARM_S and n < 10000:
        fn()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        fn()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / iters


def dominant_kernel(block: Block, step: StepW4A4):
    """The step's largest launch, the dual-stream fused QKV W4A4 GEMM (image
    M=4096 and text M=256 rows stacked, N=3x3072 per stream, K=3072), timed
    alone with HIP events on the stream it is launched on."""
    import torch

    b = step.bufs["stacked"]
    L = block.layers[("dual", "qkv")]
    lin = step.q.linear
    split = STREAMS["image"]
    lin(L, b["work"], b["x_qkv"], b["qkv"], out_dtype=torch.float16, split_rows=split)
    fn = lambda: lin(L, b["work"], b["x_qkv"], b["qkv"], reuse_input=True, out_dtype=torch.float16,  # noqa: E731
                     split_rows=split)
    ms = time_fn(fn, 50, 5)
    ops_per_launch = 2.0 * sum(STREAMS.values()) * (3 * HIDDEN) * HIDDEN
    return ms, ops_per_launch


def kernel_only():
    """The dominant W4A4 GEMM (dual-stream fused QKV, 4096 + 256 rows x 2 x 9216
    x 3072) x 20, then a plain 512 MiB copy x 5 whose known byte count
    calibrates the FETCH_SIZE / WRITE_SIZE counters."""
    import torch
    import qwen_image_hip as q

    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    pairs = []
    for _ in STREAMS:
        recs = []
        for _ in range(3):
            w = (torch.randn((HIDDEN, HIDDEN), generator=g, device="cuda") * 0.02).half()
            recs.append(q.PackedLinear.from_fp16(q.SCHEME_W4A4_H256, w, clip=True))
        pairs.append(q.PackedLinear.fuse(recs))
    rec = q.PackedLinear.dual(pairs)
    m = sum(STREAMS.values())
    work = q.Work(m, HIDDEN, "cuda")
    x = heavy_tailed(m, HIDDEN, g)
    y = torch.empty((3, m, HIDDEN), dtype=torch.float16, device="cuda")
    split = STREAMS["image"]
    q.linear(rec, work, x, y, out_dtype=torch.float16, split_rows=split)
    for _ in range(20):
        q.linear(rec, work, x, y, reuse_input=True, out_dtype=torch.float16, split_rows=split)
    src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("kernel-only: 20 x dual-stream w4a4 GEMM (4096+256)x(2x9216)x3072 (fused qkv), 5 x copy 536870912 B")
    return 0


def gemv_only():
    """The HBM-bound kernel's counter workload: all 60 blocks' modulation
    linears (image + text stream, 120 x 3072->18432, m = 1) as one fused GEMV
    launch: one, untimed launches for at least WARM_S seconds, 10 timed, then a
    plain 512 MiB copy x 5 whose known byte count calibrates the FETCH_SIZE /
    WRITE_SIZE counters."""
    import torch
    import qwen_image_hip as q
    from qwen_image_hip import ops

    n, k, parts = MODULATION_N, HIDDEN, 120
    g = torch.Generator(device="cuda")
    g.manual_seed(77)
    pool = []
    for _ in range(8):
        w = (torch.randn((n, k), generator=g, device="cuda") * 0.02).half()
        pool.append(q.PackedLinear.from_fp16(q.SCHEME_W4A16, w))
        del w
    codes_all = torch.cat([pool[i % 8].tiled_codes for i in range(parts)], 0)
    scales_all = torch.cat([pool[i % 8].tiled_scales for i in range(parts)], 0)
    del pool
    x = torch.randn((1, k), generator=g, device="cuda").half()
    y = torch.empty((1, parts * n), dtype=torch.float16, device="cuda")
    ops.w4a16_gemv(x, codes_all, scales_all, out_dtype=torch.float16, y=y)
    ms = time_fn(lambda: ops.w4a16_gemv(x, codes_all, scales_all, out_dtype=torch.float16, y=y), 10, 0)
    src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    total = parts * (n * k // 2 + n * (k // 64) * 4) + k * 2 + parts * n * 2
    log(f"gemv-only: fused modulation GEMV m=1 n={parts}x{n} k={k} ({total} algorithmic bytes), "
        f"{ms * 1e3:.1f} us per launch by HIP events over the 10; 5 x copy 536870912 B")
    return 0


def w4a16_only():
    """The fp16-MFMA kernel's counter workload: the image stream's W4A16 MLP
    up linear (4096 x 12288 x 3072, GELU-tanh, fp16 out): one call, untimed
    calls for at least WARM_S seconds, 10 timed calls, then a plain 512 MiB
    copy x 5 for the counter calibration."""
    import torch
    import qwen_image_hip as q
    from qwen_image_hip import ops

    m, n, k = STREAMS["image"], MLP, HIDDEN
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    w = (torch.randn((n, k), generator=g, device="cuda") * 0.02).half()
    rec = q.PackedLinear.from_fp16(q.SCHEME_W4A16, w)
    del w
    x = torch.randn((m, k), generator=g, device="cuda").half()
    y = torch.empty((m, n), dtype=torch.float16, device="cuda")

    def fn():
        ops.w4a16_gemm(x, rec.tiled_codes, rec.tiled_scales, out_dtype=torch.float16, gelu=True, y=y)

    fn()
    ms = time_fn(fn, 10, 0)
    src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    total = n * k // 2 + n * (k // 64) * 4 + m * k * 2 + m * n * 2
    log(f"w4a16-only: W4A16 GEMM m={m} n={n} k={k} gelu fp16 out ({total} algorithmic bytes, "
        f"{2 * m * n * k} flops), {ms * 1e3:.1f} us per launch by HIP events over the 10; 5 x copy 536870912 B")
    return 0


def time_block(operand: str, seed: int, steps: int, warmup: int):
    """ms per W4A4 block step with the given operand format."""
    import qwen_image_hip as q

    blk = Block(q.SCHEME_W4A4_H256, seed, operand)
    step = StepW4A4(blk, seed + 1)
    return time_fn(step, steps, warmup)


def bench_gemv(iters=200):
    """M=1 and M=2 modulation GEMV 3072->18432 over a rotating pool of weight
    copies larger than the 256 MB MALL, so every launch reads HBM."""
    import torch
    import qwen_image_hip as q
    from qwen_image_hip import ops

    n, k = MODULATION_N, HIDDEN
    g = torch.Generator(device="cuda")
    g.manual_seed(77)
    pool = []
    for i in range(10):
        w = (torch.randn((n, k), generator=g, device="cuda") * 0.02).half()
        pool.append(q.PackedLinear.from_fp16(q.SCHEME_W4A16, w))
        del w
    bytes_per = n * k // 2 + n * (k // 64) * 4  # codes + scales + minimums
    out = {}
    for m in (1, 2):
        x = torch.randn((m, k), generator=g, device="cuda").half()
        y = torch.empty((m, n), dtype=torch.float16, device="cuda")
        idx = [0]

        def fn():
            r = pool[idx[0] % len(pool)]
            idx[0] += 1
            ops.w4a16_gemv(x, r.tiled_codes, r.tiled_scales, out_dtype=torch.float16, y=y)

        ms = time_fn(fn, iters, 20)
        total = bytes_per + m * k * 2 + m * n * 2
        out[f"m{m}"] = {"us": round(ms * 1e3, 3), "GB_s": round(total / (ms * 1e-3) / 1e9, 1),
                        "frac_hbm": round(total / (ms * 1e-3) / PEAK_HBM, 4), "bytes": total}

    # Every block's modulation linears (60 blocks x image and text stream)
    # read the same timestep embedding, so with all blocks resident they run
    # as one GEMV over the stacked tiled weights (a fused record of 120
    # parts, m = 1: one launch), against one launch per matrix.  The 120
    # matrices are 8 packed random matrices repeated (distinct memory; the
    # bytes read are what is timed).
    parts = 120
    reps = [pool[i % 8] for i in range(parts)]
    codes_all = torch.cat([r.tiled_codes for r in reps], 0)
    scales_all = torch.cat([r.tiled_scales for r in reps], 0)
    del reps
    x = torch.randn((1, k), generator=g, device="cuda").half()
    y_all = torch.empty((1, parts * n), dtype=torch.float16, device="cuda")
    ms_one = time_fn(lambda: ops.w4a16_gemv(x, codes_all, scales_all, out_dtype=torch.float16, y=y_all), 20, 3)

    def per_matrix():
        for p in range(parts):
            ops.w4a16_gemv(x, codes_all[p * n:(p + 1) * n], scales_all[p * n:(p + 1) * n],
                           out_dtype=torch.float16, y=y_all[:, p * n:(p + 1) * n])

    ms_each = time_fn(per_matrix, 5, 1)
    total = parts * bytes_per + k * 2 + parts * n * 2
    out["m1_all_blocks"] = {"matrices": parts, "bytes": total, "one_launch_us": round(ms_one * 1e3, 1),
                            "GB_s": round(total / (ms_one * 1e-3) / 1e9, 1),
                            "frac_hbm": round(total / (ms_one * 1e-3) / PEAK_HBM, 4),
                            "per_matrix_launches_us": round(ms_each * 1e3, 1)}
    x2 = torch.randn((2, k), generator=g, device="cuda").half()
    y2 = torch.empty((2, parts * n), dtype=torch.float16, device="cuda")
    ms_two = time_fn(lambda: ops.w4a16_gemv(x2, codes_all, scales_all, out_dtype=torch.float16, y=y2), 20, 3)
    total2 = parts * bytes_per + 2 * k * 2 + 2 * parts * n * 2
    out["m2_all_blocks"] = {"matrices": parts, "bytes": total2, "one_launch_us": round(ms_two * 1e3, 1),
                            "GB_s": round(total2 / (ms_two * 1e-3) / 1e9, 1),
                            "frac_hbm": round(total2 / (ms_two * 1e-3) / PEAK_HBM, 4)}
    del codes_all, scales_all
    return out


def bench_producers(iters=50):
    """The producers in front of the quantiser at the image stream's shapes:
    LayerNorm with modulation scale (M=4096, K=3072, fp32 hidden) and SwiGLU
    (M=4096, K=12288, fp32 gate/up), each as the reference runs it (producer
    kernel writing fp32, then the quantiser reading it back) and fused (one
    quantiser pass applying the producer to what it loads)."""
    import torch
    from qwen_image_hip import ops

    g = torch.Generator(device="cuda")
    g.manual_seed(88)
    m = STREAMS["image"]
    out = {}
    x = torch.randn((m, HIDDEN), generator=g, device="cuda") * 2.0
    scale = torch.randn((2, HIDDEN), generator=g, device="cuda") * 0.3
    normed = torch.empty_like(x)
    codes = torch.empty((ops.fp6_rows(m), ops.fp6_row_bytes(MLP)), dtype=torch.uint8, device="cuda")
    c3 = codes[:, : ops.fp6_row_bytes(HIDDEN)].contiguous()
    stats = torch.empty((m, 2), dtype=torch.float32, device="cuda")

    def ln_separate():
        ops.layer_norm_scale(x, scale, 0, out=normed)
        ops.quantize_activations_fp6(normed, c3)

    def ln_fused():
        ops.layer_norm_scale_quantize_fp6(x, scale, 0, c3, stats)

    out["layer_norm_quantize"] = {"shape": f"{m}x{HIDDEN}", "separate_us": round(time_fn(ln_separate, iters, 5) * 1e3, 2),
                                  "fused_us": round(time_fn(ln_fused, iters, 5) * 1e3, 2)}
    gate = torch.randn((m, MLP), generator=g, device="cuda") * 3.0
    up = torch.randn((m, MLP), generator=g, device="cuda")
    act = torch.empty_like(gate)

    def sw_separate():
        ops.swiglu(gate, up, out=act)
        ops.quantize_activations_fp6(act, codes)

    def sw_fused():
        ops.swiglu_quantize_fp6(gate, up, codes)

    out["swiglu_quantize"] = {"shape": f"{m}x{MLP}", "separate_us": round(time_fn(sw_separate, iters, 5) * 1e3, 2),
                              "fused_us": round(time_fn(sw_fused, iters, 5) * 1e3, 2)}
    return out


def bench_attention(iters=20):
    """The block's joint attention at 1024x1024: 4096 image + 256 text tokens,
    24 heads of 128, no mask (qi_flash_attention's work in the reference,
    transformer.cplus:802-803); FLOPs = 4 * tokens^2 * 128 * heads."""
    import torch
    from qwen_image_hip import ops

    n, heads = sum(STREAMS.values()), HIDDEN // 128
    g = torch.Generator(device="cuda")
    g.manual_seed(77)
    q = torch.randn((n, HIDDEN), generator=g, device="cuda")
    k = torch.randn((n, HIDDEN), generator=g, device="cuda").half()
    v = torch.randn((n, HIDDEN), generator=g, device="cuda").half()
    out = torch.empty_like(q)
    ms = time_fn(lambda: ops.flash_attention(q, k, v, heads, out=out), iters, 3)
    flops = 4.0 * n * n * 128 * heads
    return {"tokens": n, "heads": heads, "us": round(ms * 1e3, 1), "TFLOP_s": round(flops / (ms * 1e-3) / 1e12, 1),
            "frac_fp16_peak": round(flops / (ms * 1e-3) / PEAK_FP16_FLOPS, 4)}


ENCODER_ROWS = 300  # config 4: prompt tokens through the Qwen2.5-VL-7B-shaped text encoder
ENCODER_SHAPES = [("q+k+v fused", 3584 + 2 * 512, 3584), ("gate+up fused", 2 * 18944, 3584), ("down", 3584, 18944)]


def bench_encoder(iters=30):
    """Config 4's encoder linears, W4A16 g64 at M=300 (q, k and v, gate and up
    as fused records: one input each), fp16 in / fp16 out; per linear us and
    the total fp16 TFLOP/s."""
    import torch
    import qwen_image_hip as q
    from qwen_image_hip import ops

    g = torch.Generator(device="cuda")
    g.manual_seed(300)
    x = {k: torch.randn((ENCODER_ROWS, k), generator=g, device="cuda").half() for k in (3584, 18944)}
    out, total_ms, flops = {}, 0.0, 0.0
    for name, n, k in ENCODER_SHAPES:
        w = (torch.randn((n, k), generator=g, device="cuda") * 0.02).half()
        rec = q.PackedLinear.from_fp16(q.SCHEME_W4A16, w)
        del w
        y = torch.empty((ENCODER_ROWS, n), dtype=torch.float16, device="cuda")
        ms = time_fn(lambda: ops.w4a16_gemm(x[k], rec.tiled_codes, rec.tiled_scales,  # noqa: B023
                                            out_dtype=torch.float16, y=y), iters, 5)
        f = 2.0 * ENCODER_ROWS * n * k
        out[name] = {"n": n, "k": k, "us": round(ms * 1e3, 2), "TFLOP_s": round(f / (ms * 1e-3) / 1e12, 1)}
        total_ms += ms
        flops += f
        del rec
    out["total"] = {"us": round(total_ms * 1e3, 2), "TFLOP_s": round(flops / (total_ms * 1e-3) / 1e12, 1),
                    "frac_fp16_peak": round(flops / (total_ms * 1e-3) / PEAK_FP16_FLOPS, 4)}
    return out


STACK_STREAMS = {"image": 3 * 4096, "text": 512}  # config 5: 1024^2 edit with 2 reference images
STACK_BLOCKS = 60


def bench_stack(blocks=STACK_BLOCKS, steps=4):
    """Config 5: the full 60-block MMDiT linear stack, W4A4 H256 g64, image
    stream M=12288 + text stream M=512, every block with its own random-init
    weights packed by the device QIPACK quantiser (fp6 operand records, Q/K/V
    fused, each linear's two streams as one dual-stream record over the
    stacked rows), heavy-tailed fp16 activations quantised online before
    every distinct input.  The block inputs are the same buffers in every
    block (their values do not change the work).  One denoising step = the
    60 blocks; `steps` steps are timed one by one with HIP events, the first
    reported separately as the warm-up."""
    import torch
    import qwen_image_hip as q

    g = torch.Generator(device="cuda")
    g.manual_seed(500)
    layers = []
    for _ in range(blocks):
        per = {}
        for stream in STACK_STREAMS:
            qkv = []
            for name, n, k in block_shapes():
                w = (torch.randn((n, k), generator=g, device="cuda") * 0.02).half()
                rec = q.PackedLinear.from_fp16(q.SCHEME_W4A4_H256, w, clip=True)
                del w
                if name in ("to_q", "to_k", "to_v"):
                    qkv.append(rec)
                else:
                    per[(stream, name)] = rec
            per[(stream, "qkv")] = q.PackedLinear.fuse(qkv)
            del qkv
        layers.append({name: q.PackedLinear.dual([per[(st, name)] for st in STACK_STREAMS])
                       for name in ("qkv", "to_out", "mlp_up", "mlp_down")})
        del per
    m = sum(STACK_STREAMS.values())
    split = STACK_STREAMS["image"]
    b = {"x_qkv": heavy_tailed(m, HIDDEN, g), "x_out": heavy_tailed(m, HIDDEN, g),
         "x_mlp": heavy_tailed(m, HIDDEN, g), "work": q.Work(m, MLP, "cuda"),
         "y": torch.empty((m, HIDDEN), dtype=torch.float16, device="cuda"),
         "qkv": torch.empty((3, m, HIDDEN), dtype=torch.float16, device="cuda"),
         "h": torch.empty((m, MLP), dtype=torch.float16, device="cuda")}
    torch.cuda.synchronize()
    lin, f16 = q.linear, torch.float16

    def denoise_step():
        w = b["work"]
        for blk in layers:
            lin(blk["qkv"], w, b["x_qkv"], b["qkv"], out_dtype=f16, split_rows=split)
            lin(blk["to_out"], w, b["x_out"], b["y"], out_dtype=f16, split_rows=split)
            lin(blk["mlp_up"], w, b["x_mlp"], b["h"], out_dtype=f16, gelu=True, split_rows=split)
            lin(blk["mlp_down"], w, b["h"], b["y"], out_dtype=f16, split_rows=split)

    times = []
    for _ in range(steps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        denoise_step()
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1))
    ops_step = blocks * 2.0 * sum(n * k for _, n, k in block_shapes()) * sum(STACK_STREAMS.values())
    ms = sum(times[1:]) / max(1, len(times) - 1)
    tops = ops_step / (ms * 1e-3) / 1e12
    result = {"workload": f"config 5: {blocks}-block W4A4 stack, image M={STACK_STREAMS['image']} + text "
                          f"M={STACK_STREAMS['text']}", "ms_per_step": round(ms, 3),
              "first_step_ms": round(times[0], 3), "TOPS": round(tops, 1),
              "frac_int8_peak": round(tops * 1e12 / PEAK_INT8_OPS, 4), "steps_timed": len(times) - 1}
    result["streamed_variant"] = _stack_streamed_variant(q, layers, b, split, denoise_step_body=lin)
    del b
    result["prefix_variant"] = _stack_prefix_variant(q, layers, g, steps)
    del layers
    torch.cuda.empty_cache()
    return result


def _stack_streamed_variant(q, layers, b, split, denoise_step_body, steps=2):
    """The same stack with the blocks streamed from pinned host memory
    through two device slots (qwen_image_hip.BlockStream, the reference's
    asynchronous block upload, transformer.cplus:503-598): per step every
    block's 198 MB of fp6 records crosses PCIe while the previous block
    computes.  `steps` steps timed one by one after one warm-up step."""
    import torch

    lin, f16 = denoise_step_body, torch.float16
    t0 = time.perf_counter()
    stream = q.BlockStream(layers)
    pin_s = time.perf_counter() - t0

    def step():
        w = b["work"]
        for i in range(len(layers)):
            blk = stream.begin(i)
            lin(blk["qkv"], w, b["x_qkv"], b["qkv"], out_dtype=f16, split_rows=split)
            lin(blk["to_out"], w, b["x_out"], b["y"], out_dtype=f16, split_rows=split)
            lin(blk["mlp_up"], w, b["x_mlp"], b["h"], out_dtype=f16, gelu=True, split_rows=split)
            lin(blk["mlp_down"], w, b["h"], b["y"], out_dtype=f16, split_rows=split)
            stream.end(i)

    times = []
    for _ in range(steps + 1):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        step()
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1))
    ms = sum(times[1:]) / steps
    gb = stream.block_bytes * len(layers) / 1e9
    del stream
    return {"workload": f"the same {len(layers)} blocks streamed from pinned host memory through two device slots",
            "ms_per_step": round(ms, 3), "first_step_ms": round(times[0], 3), "GB_per_step": round(gb, 2),
            "host_to_device_GB_s": round(gb / (ms * 1e-3), 1), "pinning_s": round(pin_s, 1)}


def _stack_prefix_variant(q, layers, g, steps):
    """The reference's own call pattern for the same edit
    (qwen_image_cuda/src/transformer.cplus:822-1017): the prefix rows (512
    text + 2 x 4096 condition-image rows) run through the 60 blocks once,
    their keys and values cached, and each denoising step then runs only the
    4096 rows of the image being generated.  Here: the prefix as one
    dual-stream pass (condition rows on the image stream's weights, text rows
    on the text stream's), timed once; each step the image stream's records
    alone at M = 4096; `steps` steps timed one by one, the first reported
    apart.  Linears only, as the stack above."""
    import torch

    m_img = STACK_STREAMS["image"] // 3
    m_pre = STACK_STREAMS["image"] - m_img + STACK_STREAMS["text"]
    split = STACK_STREAMS["image"] - m_img
    lin, f16 = q.linear, torch.float16

    def buffers(m):
        return {"x_qkv": heavy_tailed(m, HIDDEN, g), "x_out": heavy_tailed(m, HIDDEN, g),
                "x_mlp": heavy_tailed(m, HIDDEN, g), "work": q.Work(m, MLP, "cuda"),
                "y": torch.empty((m, HIDDEN), dtype=f16, device="cuda"),
                "qkv": torch.empty((3, m, HIDDEN), dtype=f16, device="cuda"),
                "h": torch.empty((m, MLP), dtype=f16, device="cuda")}

    def run(recs, b, split_rows):
        w = b["work"]
        for blk in recs:
            lin(blk["qkv"], w, b["x_qkv"], b["qkv"], out_dtype=f16, split_rows=split_rows)
            lin(blk["to_out"], w, b["x_out"], b["y"], out_dtype=f16, split_rows=split_rows)
            lin(blk["mlp_up"], w, b["x_mlp"], b["h"], out_dtype=f16, gelu=True, split_rows=split_rows)
            lin(blk["mlp_down"], w, b["h"], b["y"], out_dtype=f16, split_rows=split_rows)

    def timed(fn):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1)

    bp = buffers(m_pre)
    prefix_ms = timed(lambda: run(layers, bp, split))
    del bp
    image_layers = [{name: rec.stream(0) for name, rec in blk.items()} for blk in layers]
    bi = buffers(m_img)
    times = [timed(lambda: run(image_layers, bi, None)) for _ in range(steps)]
    del bi
    per_block = 2.0 * sum(n * k for _, n, k in block_shapes())
    ms = sum(times[1:]) / max(1, len(times) - 1)
    tops = len(layers) * per_block * m_img / (ms * 1e-3) / 1e12
    pre_tops = len(layers) * per_block * m_pre / (prefix_ms * 1e-3) / 1e12
    return {"workload": f"prefix {m_pre} rows ({split} condition + {STACK_STREAMS['text']} text) once, then "
                        f"{m_img} image rows per step, {len(layers)} blocks",
            "prefix_ms": round(prefix_ms, 3), "prefix_TOPS": round(pre_tops, 1),
            "ms_per_step": round(ms, 3), "first_step_ms": round(times[0], 3), "TOPS": round(tops, 1),
            "frac_int8_peak": round(tops * 1e12 / PEAK_INT8_OPS, 4),
            "ms_for_4_steps_with_prefix": round(prefix_ms + 4 * ms, 3)}


def cpu_baseline(budget_s=20.0):
    """The CPU oracle (C, OpenMP over the host cores) on a bounded sample of
    the same workload: the block's W4A4 linears (quantise + GEMM per linear,
    K/V reusing Q's codes) in step order, image stream first, stopping once
    about budget_s seconds of CPU work have run.  TOPS = 2*M*N*K of the
    GEMMs that ran / their time (weights packed outside the timed part)."""
    import numpy as np

    oracle = _cpu_oracle()
    from _data import heavy_tailed as ht, weights_f16

    done_ops, spent, ran = 0.0, 0.0, []
    seed = 10
    for stream, m in STREAMS.items():
        x_in = None
        for name, n, k in block_shapes():
            if spent >= budget_s:
                break
            seed += 1
            wc, ws, _ = oracle.quantize_matrix(weights_f16(n, k, seed), 6, clip=True)
            if name in ("to_q", "to_out", "mlp_up", "mlp_down"):
                x_in = ht(m, k, seed + 100)
            t0 = time.perf_counter()
            if name not in ("to_k", "to_v"):
                ac, as_ = oracle.quantize_activations(x_in)
            oracle.w4a4_gemm(ac, as_, wc, ws)
            spent += time.perf_counter() - t0
            done_ops += 2.0 * m * n * k
            ran.append(f"{stream}.{name}")
    return {"value": round(done_ops / spent / 1e12, 6), "unit": "TOPS", "cores": oracle.num_threads(),
            "kind": "port",
            "sample": f"CPU oracle W4A4 quantise + GEMM over {len(ran)} of the block's 12 linears "
                      f"({', '.join(ran)}), {done_ops / 1e9:.1f} G int-ops in {spent:.1f} s on "
                      f"{oracle.num_threads()} threads ({platform.processor() or platform.machine()})"}


PROBE_BODIES = {0: "fp6 MFMA x4 (4 chains)", 1: "fp32 FMA x64", 2: "MFMA x4 + FMA x64 interleaved, independent",
                3: "W4A4 per-group mix: fp6 MFMA x4 + f32 outer MFMA x2 + FMA x64 on their results",
                4: "FMA x32, MFMA x2, FMA x32, MFMA x2 (independent)",
                5: "body 3 in the product kernel's order (partial tiles two tiles behind their FMAs)",
                6: "ds_read_b128 x8 (1 KiB per wave each): LDS read throughput",
                7: "fp32 FMA x64 on 16 accumulators (few registers)",
                8: "direct-to-LDS loads 4 x 1 KiB per wave (L2-resident): L2 -> LDS throughput",
                9: "f32 32x32x1 2-block MFMA x4 (2048 outputs each)",
                10: "f16 32x32x4 2-block MFMA x4 (2048 outputs each)",
                11: "f16 32x32x8 MFMA x4 (1024 outputs each)",
                12: "f16 16x16x4 4-block MFMA x4 (1024 outputs each)",
                13: "f16 4x4x4 16-block MFMA x4 (256 outputs each)",
                14: "body 2 held to two waves per SIMD (<= 256 registers: AGPR results in the AGPR build)",
                15: "body 0 held to two waves per SIMD",
                16: "body 14 with MFMA results in AGPRs (inline asm)",
                17: "body 15 with MFMA results in AGPRs (inline asm)",
                18: "f16 32x32x16 MFMA x4 (the attention's)",
                19: "f16 16x16x32 MFMA x4 (the W4A16 GEMM's)"}


def probe_overlap(iters=2000):
    """Matrix-core / vector-unit co-execution on this MI355X
    (probe/mfma_valu_probe.hip): shader clocks per loop iteration and wave
    for each body, at one and two waves per SIMD, with MFMA results in
    ordinary VGPRs (the product's build) and in accumulator registers."""
    import ctypes

    import torch

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    seed = torch.randint(0, 1 << 30, (64,), dtype=torch.int32, device="cuda")
    out = {"cus": cus, "iters": iters, "unit": "shader clocks per iteration per wave (s_memtime)",
           "bodies": PROBE_BODIES}
    for form in ("vgpr", "agpr"):
        lib = ctypes.CDLL(str(ROOT / "qwen-image-cplus_amd" / "probe" / f"libqi_probe_{form}.so"))
        lib.qi_probe_run.argtypes = [ctypes.c_int] * 3 + [ctypes.c_void_p] * 4
        for waves in (1, 2, 4, 8):
            blocks = cus * waves  # four-wave workgroups: `waves` waves per SIMD
            res = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
            cyc = torch.empty(blocks * 4, dtype=torch.int64, device="cuda")
            for body in PROBE_BODIES:
                st = lib.qi_probe_run(body, blocks, iters, seed.data_ptr(), res.data_ptr(), cyc.data_ptr(),
                                      ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
                if st:
                    raise RuntimeError(f"probe body {body} failed ({st})")
                ms = time_fn(lambda: lib.qi_probe_run(body, blocks, iters, seed.data_ptr(), res.data_ptr(),  # noqa
                                                      cyc.data_ptr(), ctypes.c_void_p(
                                                          torch.cuda.current_stream().cuda_stream)), 3, 1)
                c = cyc.double()
                out[f"{form}_w{waves}_body{body}"] = {
                    "clk_per_iter_mean": round(float(c.mean()) / iters, 1),
                    "clk_per_iter_max": round(float(c.max()) / iters, 1),
                    "kernel_ms": round(ms, 3)}
                log(f"probe {form} waves/SIMD={waves} body {body}: {out[f'{form}_w{waves}_body{body}']}")
    return out


def _cpu_oracle():
    sys.path.insert(0, str(ROOT / "oracle"))
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle

    oracle.lib()
    return oracle


def cpu_baseline_w4a16(budget_s=10.0):
    """The CPU oracle's W4A16 path (dequantise to fp16 as gemm.cu:229-230,
    then a blocked fp32 matmul, OpenMP over the host cores): config 1 (one
    linear, M=256, N=K=3072) in full, then config 2's image-stream linears in
    block order until about budget_s seconds have run.  TFLOP/s = 2*M*N*K of
    the GEMMs that ran / their time (dequantisation inside the timing, weight
    packing outside)."""
    import numpy as np

    oracle = _cpu_oracle()
    from _data import normal_f32, weights_f16

    def one(m, n, k, seed):
        c, sc, mn = oracle.quantize_matrix(weights_f16(n, k, seed), 5)
        xb = oracle.half_from_f32(normal_f32(m, k, seed + 1))
        t0 = time.perf_counter()
        oracle.gemm_f16(xb, oracle.w4a16_dequantize(c, sc, mn), precise=False)
        return time.perf_counter() - t0

    t1 = one(256, HIDDEN, HIDDEN, 1)
    c1 = 2.0 * 256 * HIDDEN * HIDDEN
    spent, flops, ran = 0.0, 0.0, []
    for name, n, k in block_shapes():
        if spent >= budget_s:
            break
        spent += one(STREAMS["image"], n, k, 20 + len(ran))
        flops += 2.0 * STREAMS["image"] * n * k
        ran.append(f"image.{name}")
    cores = oracle.num_threads()
    cpu = platform.processor() or platform.machine()
    return {"value": round(flops / spent / 1e12, 6), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"CPU oracle W4A16 dequantise + blocked fp32 matmul over {len(ran)} of config 2's image-stream "
                      f"linears ({', '.join(ran)}, M=4096), {flops / 1e9:.1f} GFLOP in {spent:.1f} s on {cores} "
                      f"threads ({cpu})",
            "config1_m256_n3072_k3072": {"ms": round(t1 * 1e3, 2), "TFLOP_s": round(c1 / t1 / 1e12, 6)}}


def cpu_baseline_gemv(reps=5):
    """The CPU oracle's W4A16 path on config 4's modulation linear
    (3072 -> 18432) at M=1 and M=2: each weight row dequantised to fp16
    (gemm.cu:229-230) and dotted with the input rows in fp32, OpenMP over the
    rows; mean of `reps` calls, GB/s over the same algorithmic bytes as the
    GPU figure."""
    oracle = _cpu_oracle()
    from _data import normal_f32, weights_f16

    n, k = MODULATION_N, HIDDEN
    c, sc, mn = oracle.quantize_matrix(weights_f16(n, k, 6), 5)
    out = {"kind": "port", "cores": oracle.num_threads(), "unit": "us",
           "sample": f"CPU oracle per-row dequantise + fp32 dots, {n}x{k} weights, mean of {reps} calls, "
                     f"{oracle.num_threads()} threads ({platform.processor() or platform.machine()})"}
    for m in (1, 2):
        xb = oracle.half_from_f32(normal_f32(m, k, 7))
        t0 = time.perf_counter()
        for _ in range(reps):
            oracle.w4a16_gemv(xb, c, sc, mn)
        t = (time.perf_counter() - t0) / reps
        total = n * k // 2 + n * (k // 64) * 4 + m * k * 2 + m * n * 2
        out[f"m{m}"] = {"us": round(t * 1e6, 1), "GB_s": round(total / t / 1e9, 2)}
    out["value"] = out["m1"]["us"]
    return out


ABLATION_NAMES = ("none", "dma", "lds", "barrier", "vmwait", "fma", "mfma", "memory", "arith_only")


def ablate_w4a4(iters=20, reps=5):
    """The roofline kernel's workload (dual-stream fused QKV, 4352 x 2 x 9216 x
    3072) on the W4A4 GEMM built with parts of its work removed
    (csrc/w4a4_fp6.hip QI_ABLATE_*, probe/libqi_fp6_ablate_*.so; outputs
    wrong by design): median us per launch by HIP events over `reps` x
    `iters` launches, the variants interleaved over two passes after a
    warm-up of the unmodified build."""
    import ctypes
    import statistics

    import torch
    import qwen_image_hip as q
    from qwen_image_hip import ops

    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    pairs = []
    for _ in STREAMS:
        recs = [q.PackedLinear.from_fp16(q.SCHEME_W4A4_H256,
                                         (torch.randn((HIDDEN, HIDDEN), generator=g, device="cuda") * 0.02).half(),
                                         clip=True) for _ in range(3)]
        pairs.append(q.PackedLinear.fuse(recs))
    rec = q.PackedLinear.dual(pairs)
    m, n, k, split = sum(STREAMS.values()), 3 * HIDDEN, HIDDEN, STREAMS["image"]
    work = q.Work(m, k, "cuda")
    a6 = work.fp6_views(m, k)
    ops.quantize_activations_fp6(heavy_tailed(m, k, g), a6)
    y = torch.empty((m, n), dtype=torch.float16, device="cuda")
    fns = {}
    for name in ABLATION_NAMES:
        f = ctypes.CDLL(str(ROOT / "qwen-image-cplus_amd" / "probe" / f"libqi_fp6_ablate_{name}.so"),
                        mode=ctypes.RTLD_LOCAL).qi_hip_w4a4_gemm_fp6_dual
        f.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 7 + [ctypes.c_void_p]
        fns[name] = f
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def call(name):
        if fns[name](a6.data_ptr(), rec.tiled_codes.data_ptr(), None, y.data_ptr(), 1, 0, m, split, n, k, n, st):
            raise RuntimeError(f"ablation build {name} failed to launch")

    for _ in range(2000):
        call("none")
    torch.cuda.synchronize()
    times = {name: [] for name in ABLATION_NAMES}
    for _ in range(2):
        for name in ABLATION_NAMES:
            for _ in range(5):
                call(name)
            for _ in range(reps):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(iters):
                    call(name)
                e1.record()
                e1.synchronize()
                times[name].append(e0.elapsed_time(e1) / iters * 1e3)
    med = {name: statistics.median(t) for name, t in times.items()}
    return {"workload": DOMINANT_WORKLOAD, "unit": "us per launch (median)",
            "removed": {"none": "nothing (the product kernel)", "dma": "direct-to-LDS operand loads",
                        "lds": "fragment reads after the first group", "barrier": "per-group workgroup barrier",
                        "fma": "exact fp32 group steps", "mfma": "matrix-core partials and scale products",
                        "memory": "loads and fragment reads", "arith_only": "loads, fragment reads and barriers"},
            "us": {name: round(v, 1) for name, v in med.items()},
            "saved_us": {name: round(med["none"] - v, 1) for name, v in med.items() if name != "none"}}


def bench_library(iters=50):
    """Calibration, not the product: the vendor library's plain GEMMs
    (torch.matmul fp16 and torch._int_mm int8 through hipBLASLt, no group
    structure, no quantisation) at the block's image-stream shapes and the
    dual-stream QKV shape, against the same peaks as this build's kernels."""
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(99)
    shapes = [(4096, 3 * HIDDEN, HIDDEN), (4096, HIDDEN, HIDDEN), (4096, 4 * HIDDEN, HIDDEN),
              (4096, HIDDEN, 4 * HIDDEN), (4352, 3 * HIDDEN, HIDDEN), (4352, 4 * HIDDEN, HIDDEN),
              (4352, HIDDEN, 4 * HIDDEN)]
    out = {}
    for m, n, k in shapes:
        x = torch.randn((m, k), generator=g, device="cuda").half()
        w = torch.randn((n, k), generator=g, device="cuda").half()
        ms = time_fn(lambda: x @ w.t(), iters, 5)
        a = torch.randint(-7, 8, (m, k), generator=g, device="cuda", dtype=torch.int8)
        b = torch.randint(-7, 8, (n, k), generator=g, device="cuda", dtype=torch.int8)
        ms8 = time_fn(lambda: torch._int_mm(a, b.t()), iters, 5)
        ops = 2.0 * m * n * k
        out[f"{m}x{n}x{k}"] = {
            "fp16_us": round(ms * 1e3, 1), "fp16_frac": round(ops / (ms * 1e-3) / PEAK_FP16_FLOPS, 4),
            "int8_us": round(ms8 * 1e3, 1), "int8_frac": round(ops / (ms8 * 1e-3) / PEAK_INT8_OPS, 4)}
        del x, w, a, b
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=200,
                    help="untimed steps first (the GPU clock settles over the first ~100 steps: 0.80 -> 0.74 ms)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="only the headline W4A4 block")
    ap.add_argument("--no-stack", action="store_true", help="skip the 60-block stack (config 5)")
    ap.add_argument("--stack-only", action="store_true", help="only the 60-block stack (config 5), printed as JSON")
    ap.add_argument("--no-graph", action="store_true", help="time the eager step (one Python call per linear)")
    ap.add_argument("--two-streams", action="store_true",
                    help="run each phase's text-stream linears on a second HIP stream beside the image stream's "
                         "(measured no faster with the joins between phases)")
    ap.add_argument("--kernel-only", action="store_true",
                    help="run only the dominant GEMM (20 launches) and a 512 MiB device copy (5 launches), "
                         "for hardware-counter runs")
    ap.add_argument("--gemv-only", action="store_true",
                    help="run only the all-blocks modulation GEMV (11 launches) and a 512 MiB device copy "
                         "(5 launches), for hardware-counter runs")
    ap.add_argument("--w4a16-only", action="store_true",
                    help="run only the W4A16 MLP-up GEMM (11 launches) and a 512 MiB device copy (5 launches), "
                         "for hardware-counter runs")
    ap.add_argument("--probe-overlap", action="store_true",
                    help="only the matrix-core / vector-unit co-execution micro-benchmark (probe/)")
    ap.add_argument("--ablate-w4a4", action="store_true",
                    help="only the roofline kernel's ablation builds (probe/libqi_fp6_ablate_*.so), printed as JSON")
    ap.add_argument("--w4a16-block-only", action="store_true",
                    help="only the W4A16 block (config 2), printed as JSON (for kernel traces)")
    ap.add_argument("--attention-only", action="store_true",
                    help="only the attention extra (4352 tokens x 24 heads) and the encoder's W4A16 linears, "
                         "printed as JSON (for kernel traces)")
    ap.add_argument("--library-only", action="store_true",
                    help="only the calibration: the vendor library's plain fp16 / int8 GEMMs at the block's shapes")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        return 2

    import torch
    import qwen_image_hip as q

    q.load()
    torch.cuda.set_device(0)
    if args.kernel_only:
        return kernel_only()
    if args.gemv_only:
        return gemv_only()
    if args.w4a16_only:
        return w4a16_only()
    if args.stack_only:
        print(json.dumps(bench_stack()), flush=True)
        return 0
    if args.library_only:
        print(json.dumps({"library_gemm": bench_library()}), flush=True)
        return 0
    if args.ablate_w4a4:
        print(json.dumps({"w4a4_ablation": ablate_w4a4()}), flush=True)
        return 0
    if args.attention_only:
        print(json.dumps({"attention": bench_attention(), "encoder_w4a16_m300": bench_encoder()}), flush=True)
        return 0
    if args.w4a16_block_only:
        blk16 = Block(q.SCHEME_W4A16, 3)
        out = {}
        for name, one in (("one_stream", True), ("two_streams", False)):
            step16 = StepW4A16(blk16, 4, one_stream=one)
            ms16 = time_fn(step16, args.steps, args.warmup)
            tf16 = block_ops() / (ms16 * 1e-3) / 1e12
            out[name] = {"ms_per_step": round(ms16, 4), "TFLOP_s": round(tf16, 1),
                         "frac_fp16_peak": round(tf16 * 1e12 / PEAK_FP16_FLOPS, 4)}
            torch.cuda.synchronize()
            out[name]["y_checksum"] = float(step16.b["y"].float().abs().sum())
        print(json.dumps({"w4a16_block": out}), flush=True)
        return 0
    if args.probe_overlap:
        print(json.dumps({"mfma_valu_probe": probe_overlap()}), flush=True)
        return 0
    log("packing W4A4 block weights (fp6 operands)")
    blk4 = Block(q.SCHEME_W4A4_H256, 1)
    step4 = StepW4A4(blk4, 2, one_stream=not args.two_streams)

    # Eager: one Python call per linear.
    ms_eager = time_fn(step4, args.steps, args.warmup)
    eager_out = step4.outputs()

    # Graph: the step's 20 launches captured once into a HIP graph and
    # replayed, as a serving loop would, so the host's per-launch cost is not
    # on the GPU's critical path.  Every replay must reproduce the eager
    # outputs bit for bit.
    graph = None
    if not args.no_graph:
        capture = torch.cuda.Stream()
        capture.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(capture):
            step4()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=capture):
            step4()
        torch.cuda.synchronize()
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            for a, b in zip(eager_out, step4.outputs()):
                if not torch.equal(a, b):
                    raise RuntimeError("graph replay differs from the eager step")
    run = graph.replay if graph is not None else step4
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        run()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = start.elapsed_time(stop) / args.steps
    tops = block_ops() / (ms_step * 1e-3) / 1e12
    log(f"w4a4 block: {ms_step:.3f} ms/step ({'graph' if graph else 'eager'}), {tops:.1f} TOPS "
        f"(wall {wall:.3f} s); eager {ms_eager:.3f} ms/step")
    del graph

    dom_ms, dom_ops = dominant_kernel(blk4, step4)
    achieved = dom_ops / (dom_ms * 1e-3) / 1e12
    traffic = None
    if TRAFFIC_FILE.exists():
        try:
            rec = json.loads(TRAFFIC_FILE.read_text())
            traffic = rec.get("bytes_per_launch") if rec.get("workload") == DOMINANT_WORKLOAD else None
        except (ValueError, OSError):
            traffic = None
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_INT8_OPS / 1e12, "unit": "TFLOP/s",
                "frac": round(achieved * 1e12 / PEAK_INT8_OPS, 4), "traffic": traffic,
                "kernel": "w4a4_fp6_persistent_kernel, " + DOMINANT_WORKLOAD + " (int ops vs dense int8 MFMA peak)",
                "ms_per_launch": round(dom_ms, 4)}
    del step4, blk4
    torch.cuda.empty_cache()

    extra = {}
    if not args.no_extra:
        log("W4A4 block on the int8 operand path")
        ms8 = time_block("int8", 5, args.steps, args.warmup)
        extra["w4a4_int8_block"] = {"ms_per_step": round(ms8, 4), "TOPS": round(block_ops() / (ms8 * 1e-3) / 1e12, 1)}
        torch.cuda.empty_cache()
        log("packing W4A16 block weights")
        blk16 = Block(q.SCHEME_W4A16, 3)
        step16 = StepW4A16(blk16, 4, one_stream=not args.two_streams)
        ms16 = time_fn(step16, args.steps, args.warmup)
        tf16 = block_ops() / (ms16 * 1e-3) / 1e12
        extra["w4a16_block"] = {"ms_per_step": round(ms16, 4), "TFLOP_s": round(tf16, 1),
                                "frac_fp16_peak": round(tf16 * 1e12 / PEAK_FP16_FLOPS, 4)}
        log(f"w4a16 block: {ms16:.3f} ms/step, {tf16:.1f} TFLOP/s")
        del step16, blk16
        torch.cuda.empty_cache()
        extra["modulation_gemv"] = bench_gemv()
        log(f"gemv: {extra['modulation_gemv']}")
        extra["producers"] = bench_producers()
        log(f"producers: {extra['producers']}")
        extra["attention"] = bench_attention()
        log(f"attention: {extra['attention']}")
        extra["encoder_w4a16_m300"] = bench_encoder()
        log(f"encoder: {extra['encoder_w4a16_m300']}")
        if not args.no_stack:
            log("packing the 60-block stack (config 5)")
            extra["stack60_w4a4"] = bench_stack()
            log(f"stack: {extra['stack60_w4a4']}")

    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        cpu = cpu_baseline()
        log(f"cpu: {cpu}")
        if "w4a16_block" in extra:
            extra["w4a16_block"]["cpu_baseline"] = cpu_baseline_w4a16()
            log(f"cpu w4a16: {extra['w4a16_block']['cpu_baseline']}")
        if "modulation_gemv" in extra:
            extra["modulation_gemv"]["cpu_baseline"] = cpu_baseline_gemv()
            log(f"cpu gemv: {extra['modulation_gemv']['cpu_baseline']}")

    line = {
        "metric": "QIPACK W4A4/W4A16 linear TOPS + % roofline, MMDiT block @1024^2 (M=4352)",
        "value": round(tops, 2), "unit": "TOPS", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4), "ms_per_step_eager": round(ms_eager, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int4 x int4 exact group partials (fp6 E2M3 MFMA operands), fp32 epilogue, fp16 out", "data": "synthetic",
        "config": {"workload": "W4A4 H256 g64 one MMDiT dual-stream block linears (config 3): image M=4096 + "
                               "text M=256, hidden 3072, MLP 12288, heavy-tailed fp16 activations, online quantiser",
                   "global_batch": 1, "seq_len": sum(STREAMS.values()), "parallelism": "single-gpu", "streams": 2 if args.two_streams else 1},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "peaks": device_peaks(),
    }
    line.update(extra)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
