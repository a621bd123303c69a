"""Host-side mirror of the reference's backend linear-op interface.

The reference engine calls one function per linear layer,
``transformer::linear(model, work, index, input, output, rows, reuse_input)``
(qwen_image_cuda/src/transformer.cplus:669-713), which dispatches on the pack
record's scheme:

* scheme 6 (W4A4 H256): quantise ``input`` into ``work.codes`` /
  ``work.code_scales`` unless ``reuse_input``, then ``qi_w4a4_gemm``;
* scheme 5 (W4A16): convert ``input`` to fp16 into ``work.halves`` unless
  ``reuse_input``, then ``qi_w4a16_gemm``.

This module keeps that shape.  ``PackedLinear`` is one uploaded INT4 record,
re-laid out once into MFMA-tile order (the load-time hook the reference's
``transformer::load``, transformer.cplus:342-501, would call).  ``Work`` holds
the activation scratch the reference sizes in ``allocate_work``
(transformer.cplus:638-667).  Unlike the reference, rows need not be a
multiple of 128, outputs may be fp16 with a fused bias/GELU epilogue, and
m <= 16 dispatches to the bandwidth-bound GEMV.

W4A4 records run on one of two operand formats, both bit-identical to the
reference's arithmetic (gemm.cu:137-168):

* ``W4A4_FP6`` (default): the int4 codes are widened once to 6-bit E2M3
  floats in MFMA-operand tiles and multiplied on the f8f6f4 matrix core,
  which returns the exact group partials already in fp32;
* ``W4A4_INT8``: nibble tiles multiplied on the int8 matrix core.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops

SCHEME_W4A16 = 5
SCHEME_W4A4_H256 = 6
W4A4_FP6 = "fp6"
W4A4_INT8 = "int8"


@dataclass
class PackedLinear:
    """One INT4 block matrix resident in HBM in tiled order."""

    scheme: int
    n: int
    k: int
    tiled_codes: torch.Tensor
    tiled_scales: torch.Tensor | None  # None for fp6 operands (scales inside the code blocks)
    bias: torch.Tensor | None = None  # fp32 [n] or None (the reference has none)
    operand: str = W4A4_FP6  # W4A4 records only
    parts: int = 1  # > 1: records fused along n (fuse()); outputs [parts, rows, n / parts]
    streams: int = 1  # 2: a dual-stream pair (dual()); n is per stream

    @classmethod
    def dual(cls, records: "list[PackedLinear]") -> "PackedLinear":
        """The image and text streams' records of one MMDiT block linear
        (same shape), run by one call over the stacked rows of both streams
        (``linear(..., split_rows=image_rows)``); fp6 W4A4 or W4A16 records."""
        if len(records) != 2:
            raise ValueError("a dual-stream record pairs exactly two records")
        a, b = records
        if (a.scheme, a.n, a.k, a.operand, a.parts, a.streams) != (b.scheme, b.n, b.k, b.operand, b.parts, 1) \
                or a.streams != 1:
            raise ValueError("dual-stream records need one scheme, shape and operand format")
        if a.scheme == SCHEME_W4A4_H256 and a.operand != W4A4_FP6:
            raise ValueError("dual-stream W4A4 records run on the fp6 operand format")
        if (a.bias is None) != (b.bias is None):
            raise ValueError("either both records have a bias or neither has")
        bias = None if a.bias is None else torch.cat([a.bias, b.bias], 0)
        ts = None if a.tiled_scales is None else torch.cat([a.tiled_scales, b.tiled_scales], 0)
        return cls(a.scheme, a.n, a.k, torch.cat([a.tiled_codes, b.tiled_codes], 0), ts, bias, a.operand,
                   a.parts, 2)

    def stream(self, index: int) -> "PackedLinear":
        """Stream `index` (0 or 1) of a dual-stream record, as a view of its
        arrays (no copy)."""
        if self.streams != 2 or index not in (0, 1):
            raise ValueError("stream() takes stream 0 or 1 of a dual-stream record")
        half = lambda t: None if t is None else t[index * (t.shape[0] // 2):(index + 1) * (t.shape[0] // 2)]  # noqa
        return PackedLinear(self.scheme, self.n, self.k, half(self.tiled_codes), half(self.tiled_scales),
                            half(self.bias), self.operand, self.parts, 1)

    @classmethod
    def fuse(cls, records: "list[PackedLinear]") -> "PackedLinear":
        """One record for several records that read the same input (the
        reference's reuse_input group: to_q, to_k, to_v after one
        quantisation, transformer.cplus:759-762), concatenated along n so
        one GEMM launch computes all of them.  The tiled layouts are per
        16- or 32-row tile, so the fused arrays are the concatenations.
        """
        first = records[0]
        for r in records:
            if (r.scheme, r.n, r.k, r.operand, r.parts) != (first.scheme, first.n, first.k, first.operand, 1):
                raise ValueError("fused records need one scheme, shape and operand format")
            if (r.bias is None) != (first.bias is None):
                raise ValueError("either every fused record has a bias or none has")
        tc = torch.cat([r.tiled_codes for r in records], 0)
        ts = None if first.tiled_scales is None else torch.cat([r.tiled_scales for r in records], 0)
        bias = None if first.bias is None else torch.cat([r.bias for r in records], 0)
        return cls(first.scheme, first.n * len(records), first.k, tc, ts, bias, first.operand, len(records))

    @classmethod
    def from_qipack(cls, scheme: int, codes: torch.Tensor, scales: torch.Tensor,
                    minimums: torch.Tensor | None = None, bias: torch.Tensor | None = None,
                    operand: str = W4A4_FP6) -> "PackedLinear":
        """Upload hook: re-lay the QIPACK arrays of one record (device tensors)."""
        n, half_k = codes.shape
        if scheme == SCHEME_W4A4_H256:
            if operand == W4A4_FP6:
                tc, ts = ops.relayout_w4a4_fp6(codes, scales)
            elif operand == W4A4_INT8:
                tc, ts = ops.relayout_w4a4(codes, scales)
            else:
                raise ValueError(f"unknown W4A4 operand format {operand!r}")
        elif scheme == SCHEME_W4A16:
            if minimums is None:
                raise ValueError("W4A16 records carry a minimums (zeros) array")
            tc, ts = ops.relayout_w4a16(codes, scales, minimums)
        else:
            raise ValueError(f"unsupported INT4 scheme {scheme}")
        return cls(scheme, n, half_k * 2, tc, ts, bias, operand)

    @classmethod
    def from_pack(cls, pack, name: str, device: torch.device | str = "cuda", bias: torch.Tensor | None = None,
                  operand: str = W4A4_FP6) -> "PackedLinear":
        """Load one INT4 record of an open ``qipack.Pack`` (the upload step of
        transformer.cplus:386-392): its codes, scales and zeros go to the
        device and are re-laid once; the staging copies are dropped."""
        r = pack.record(name)
        if r.scheme not in (SCHEME_W4A4_H256, SCHEME_W4A16) or r.group_size != ops.GROUP:
            raise ValueError(f"{name}: scheme {r.scheme} group {r.group_size} is not an INT4 g64 record")
        codes, scales, zeros = pack.arrays(name)
        dev = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
        return cls.from_qipack(r.scheme, dev(codes), dev(scales).view(torch.float16),
                               None if zeros is None else dev(zeros).view(torch.float16), bias, operand)

    @classmethod
    def from_fp16(cls, scheme: int, w_half: torch.Tensor, clip: bool = False,
                  bias: torch.Tensor | None = None, operand: str = W4A4_FP6) -> "PackedLinear":
        """Quantise an fp16 [N, K] matrix with the QIPACK quantiser, then re-lay it."""
        codes, scales, mins = ops.pack_weights(w_half, scheme, clip)
        return cls.from_qipack(scheme, codes, scales, mins, bias, operand)


class Work:
    """Activation scratch shared by consecutive linears (the reference's Work)."""

    def __init__(self, rows_max: int, k_max: int, device: torch.device | str = "cuda"):
        self.rows_max = rows_max
        self.k_max = k_max
        # Sized for the fp6 operand blocks (whole 32-row tiles, 7/8 byte per
        # input, scales included), which also hold the nibble layout (1/2
        # byte per input).
        rows32 = ops.fp6_rows(rows_max)
        self.codes = torch.empty(rows32 * ops.fp6_row_bytes(k_max), dtype=torch.uint8, device=device)
        self.code_scales = torch.empty(rows_max * k_max // ops.GROUP, dtype=torch.float16, device=device)
        self.halves = torch.empty(rows_max * k_max, dtype=torch.float16, device=device)

    def views(self, rows: int, k: int):
        if rows > self.rows_max or k > self.k_max:
            raise ValueError("work buffers are smaller than this linear")
        return (self.codes[: rows * k // 2].view(rows, k // 2),
                self.code_scales[: rows * k // ops.GROUP].view(rows, k // ops.GROUP),
                self.halves[: rows * k].view(rows, k))

    def fp6_views(self, rows: int, k: int):
        if rows > self.rows_max or k > self.k_max:
            raise ValueError("work buffers are smaller than this linear")
        r32 = ops.fp6_rows(rows)
        return self.codes[: r32 * ops.fp6_row_bytes(k)].view(r32, ops.fp6_row_bytes(k))


def linear(record: PackedLinear, work: Work, input: torch.Tensor, output: torch.Tensor | None = None,
           rows: int | None = None, reuse_input: bool = False, gelu: bool = False,
           out_dtype: torch.dtype = torch.float32, split_rows: int | None = None) -> torch.Tensor:
    """output[rows, N] = input[rows, K] . W^T (+ bias, GELU) for one record.

    ``input`` is fp32 (the engine's activations) or fp16.  ``reuse_input``
    skips the quantisation / conversion when the previous linear already
    processed the same input (Q/K/V and gate/up in the reference).  A fused
    record (``PackedLinear.fuse``) writes ``output[parts, rows, N / parts]``.
    A dual-stream record (``PackedLinear.dual``) takes the two streams' rows
    stacked in ``input`` (the first ``split_rows`` rows are stream 0's).
    """
    n_part = record.n // record.parts if record.parts > 1 else None
    rows = input.shape[0] if rows is None else rows
    k = record.k
    if input.shape[-1] != k:
        raise ValueError(f"input width {input.shape[-1]} != record inputs {k}")
    codes, code_scales, halves = work.views(rows, k)
    if record.scheme == SCHEME_W4A4_H256 and record.operand == W4A4_FP6:
        codes6 = work.fp6_views(rows, k)
        if not reuse_input:
            ops.quantize_activations_fp6(input[:rows], codes6)
        if record.streams == 2:
            if split_rows is None:
                raise ValueError("a dual-stream record needs split_rows")
            return ops.w4a4_gemm_fp6_dual(codes6, record.tiled_codes, rows, split_rows, record.bias, out_dtype, gelu,
                                          output, n_part)
        return ops.w4a4_gemm_fp6(codes6, record.tiled_codes, rows, record.bias, out_dtype, gelu, output, n_part)
    if record.parts > 1 and record.scheme == SCHEME_W4A4_H256:
        raise ValueError("fused W4A4 records run on the fp6 operand format")
    if record.scheme == SCHEME_W4A4_H256:
        if not reuse_input:
            ops.quantize_activations(input[:rows], codes, code_scales)
        return ops.w4a4_gemm(codes, code_scales, record.tiled_codes, record.tiled_scales, record.bias,
                             out_dtype, gelu, output)
    if record.scheme == SCHEME_W4A16:
        if input.dtype == torch.float16:
            x_half = input[:rows]
        else:
            if not reuse_input:
                ops.f32_to_f16(input[:rows], halves)
            x_half = halves
        if record.streams == 2:
            if split_rows is None:
                raise ValueError("a dual-stream record needs split_rows")
            return ops.w4a16_gemm_dual(x_half, record.tiled_codes, record.tiled_scales, split_rows, record.bias,
                                       out_dtype, gelu, output, n_part)
        return ops.w4a16_gemm(x_half, record.tiled_codes, record.tiled_scales, record.bias, out_dtype, gelu,
                              output, n_part)
    raise ValueError(f"unsupported scheme {record.scheme}")
