"""Block streaming: the weights of a model that does not stay resident in HBM
run through two device slots, each block uploaded on a copy stream while the
previous block computes.

Mirror of the reference's asynchronous block upload
(qwen_image_cuda/src/transformer.cplus:503-598): the blocks live in pinned
host memory; a block uses one of two slots; ``begin(b)`` makes the compute stream
wait for the block's upload (``begin_block``, :556-563) and ``end(b)``
records that the slot's kernels are queued, then queues the block two ahead
in the walk (cyclic, so the prefix pass and every denoising step reuse the
same walk) into the freed slot once those kernels finish (``end_block`` /
``queue_upload``, :539-554, :565-572).  Blocks are taken in walk order, 0,
1, ..., n - 1, 0, 1, ...; the slot is the walk position's parity (block
parity, as in the reference, when n is even).  Where the reference streams
the QIPACK bytes of a block and reads records at their pack offsets, this
streams the block's re-laid records (the bytes the kernels read), so nothing
is re-laid per step.

On MI355X a whole 60-block model is about 12.6 GB of fp6 records and fits the
288 GB of HBM many times over, so the resident path is the default; this is
for hosts that share the GPU or larger models.
"""
from __future__ import annotations

import torch

from .linear import PackedLinear

_ALIGN = 256  # bytes; every array of a block starts on this boundary


def _arrays(rec: PackedLinear):
    return [("tiled_codes", rec.tiled_codes), ("tiled_scales", rec.tiled_scales), ("bias", rec.bias)]


class BlockStream:
    """Two device slots fed from pinned host copies of ``blocks`` (a list of
    dicts name -> PackedLinear, every block with the same names and array
    sizes, as the blocks of one transformer are)."""

    def __init__(self, blocks: "list[dict[str, PackedLinear]]", device: torch.device | str = "cuda"):
        if len(blocks) < 2:
            raise ValueError("block streaming needs at least two blocks")
        self.device = torch.device(device)
        names = list(blocks[0])
        self.layout = {}  # name -> (record template, [(field, offset, shape, dtype) or None])
        offset = 0
        for name in names:
            rec = blocks[0][name]
            fields = []
            for field, t in _arrays(rec):
                if t is None:
                    fields.append((field, None))
                    continue
                fields.append((field, (offset, tuple(t.shape), t.dtype)))
                offset += -(-t.numel() * t.element_size() // _ALIGN) * _ALIGN
            self.layout[name] = (rec, fields)
        self.block_bytes = offset
        # Pinned host copies (allocated pinned, not registered afterwards).
        self.host = []
        for b, blk in enumerate(blocks):
            if list(blk) != names:
                raise ValueError(f"block {b} does not have the records of block 0")
            buf = torch.empty(self.block_bytes, dtype=torch.uint8, pin_memory=True)
            for name in names:
                rec, fields = self.layout[name]
                other = blk[name]
                if (other.scheme, other.n, other.k, other.operand, other.parts, other.streams) != \
                        (rec.scheme, rec.n, rec.k, rec.operand, rec.parts, rec.streams):
                    raise ValueError(f"block {b} record {name} differs in shape from block 0's")
                for (field, spec), (_, t) in zip(fields, _arrays(other)):
                    if (spec is None) != (t is None):
                        raise ValueError(f"block {b} record {name}: {field} present in one block only")
                    if spec is None:
                        continue
                    off, shape, dtype = spec
                    if tuple(t.shape) != shape or t.dtype != dtype:
                        raise ValueError(f"block {b} record {name}: {field} shape or dtype differs")
                    n = t.numel() * t.element_size()
                    buf[off:off + n].copy_(t.contiguous().view(torch.uint8).reshape(-1))
            self.host.append(buf)
        self.slots = [torch.empty(self.block_bytes, dtype=torch.uint8, device=self.device) for _ in range(2)]
        self.copy_stream = torch.cuda.Stream(device=self.device)
        self.uploaded = [torch.cuda.Event() for _ in range(2)]
        self.computed = [torch.cuda.Event() for _ in range(2)]
        self.views = [self._views(slot) for slot in self.slots]
        self.position = 0  # walk position of the next begin()
        self._queue(0)
        self._queue(1)

    def __len__(self) -> int:
        return len(self.host)

    def _views(self, slot: torch.Tensor) -> "dict[str, PackedLinear]":
        out = {}
        for name, (rec, fields) in self.layout.items():
            arrays = {}
            for field, spec in fields:
                if spec is None:
                    arrays[field] = None
                    continue
                off, shape, dtype = spec
                n = 1
                for d in shape:
                    n *= d
                arrays[field] = slot[off:off + n * torch.empty((), dtype=dtype).element_size()].view(dtype).view(shape)
            out[name] = PackedLinear(rec.scheme, rec.n, rec.k, arrays["tiled_codes"], arrays["tiled_scales"],
                                     arrays["bias"], rec.operand, rec.parts, rec.streams)
        return out

    def _queue(self, position: int) -> None:
        """queue_upload: the block at walk position `position` -> slot
        position % 2 on the copy stream, after the kernels that last read
        that slot."""
        s = position % 2
        self.copy_stream.wait_event(self.computed[s])
        with torch.cuda.stream(self.copy_stream):
            self.slots[s].copy_(self.host[position % len(self.host)], non_blocking=True)
        self.uploaded[s].record(self.copy_stream)

    def _check(self, block: int) -> None:
        if block != self.position % len(self.host):
            raise ValueError(f"blocks are streamed in walk order: expected block "
                             f"{self.position % len(self.host)}, got {block}")

    def begin(self, block: int) -> "dict[str, PackedLinear]":
        """begin_block: the current stream waits for the block's upload; the
        block's records, as views of its slot."""
        self._check(block)
        s = self.position % 2
        torch.cuda.current_stream(self.device).wait_event(self.uploaded[s])
        return self.views[s]

    def end(self, block: int) -> None:
        """end_block: the slot is free once the kernels queued so far finish;
        queue the block two ahead in the walk into it."""
        self._check(block)
        s = self.position % 2
        self.computed[s].record(torch.cuda.current_stream(self.device))
        self._queue(self.position + 2)
        self.position += 1
