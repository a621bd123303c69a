"""QIPACK1 container: header / record parsing and writing, FNV-1a checksums.

Layout (qwen_image_cuda/src/int4_pack.cplus:55-95; field offsets as read by
qwen_image/src/pack_info.cplus and tools/evaluate_int4_quantization.py:48-64):

header, 256 bytes, little-endian
  0  magic "QIPACK1\\0"   8  version u32   12 header_bytes u32   16 tensor_count u32
  20 scope u32           24 directory_offset u64   32 data_offset u64
  40 file_bytes u64      48 payload_checksum u64   56 model_snapshot[40]
  96 diffusers_commit[40]  136 policy[32]  168 metadata_offset u64
  176 metadata_bytes u32   180 metadata_version u32   184 metadata_checksum u64
  192 reserved[64]
record, 256 bytes
  0 name[128]  128 scheme u32  132 rank u32  136 dims[4] u64  168 group_axis u32
  172 group_size u32  176 scale_type u32  180 zero_type u32
  184 weights_offset u64  192 weights_length  200 scales_offset  208 scales_length
  216 zeros_offset  224 zeros_length  232 elements  240 tensor_checksum  248 reserved[8]

Tensors start on 256-byte boundaries (:36-38, plan_record :476-518).  This
module handles the container only; the INT4 payload goes to the device and
through ``PackedLinear.from_qipack``.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

MAGIC = b"QIPACK1\x00"
HEADER_BYTES = 256
RECORD_BYTES = 256
TENSOR_ALIGNMENT = 256
FNV_OFFSET = 14695981039346656037
FNV_PRIME = 1099511628211
SCHEME_BF16, SCHEME_FP16, SCHEME_W4A16, SCHEME_W4A4_H256 = 0, 1, 5, 6
TYPE_NONE, TYPE_F16 = 0, 1

_HEADER = struct.Struct("<8sIIII QQQQ 40s40s32s QIIQ 64s")
_RECORD = struct.Struct("<128sII4QIIII QQQQQQ QQ 8s")
assert _HEADER.size == HEADER_BYTES and _RECORD.size == RECORD_BYTES


def fnv1a(data: bytes | memoryview, h: int = FNV_OFFSET) -> int:
    """FNV-1a 64 (int4_pack.cplus:151-159)."""
    mask = (1 << 64) - 1
    for b in bytes(data):
        h = ((h ^ b) * FNV_PRIME) & mask
    return h


def align_up(value: int, alignment: int = TENSOR_ALIGNMENT) -> int:
    return (value + alignment - 1) // alignment * alignment


def policy_name(scheme: int, group: int = 64) -> str:
    """int4_pack.cplus:108-113."""
    return {SCHEME_W4A16: f"transformer:w4a16-g{group}-v6",
            SCHEME_W4A4_H256: f"transformer:w4a4-h256-g{group}-v6"}[scheme]


@dataclass
class Record:
    name: str
    scheme: int
    dims: tuple
    group_size: int = 0
    scale_type: int = TYPE_NONE
    zero_type: int = TYPE_NONE
    weights_offset: int = 0
    weights_length: int = 0
    scales_offset: int = 0
    scales_length: int = 0
    zeros_offset: int = 0
    zeros_length: int = 0
    elements: int = 0
    tensor_checksum: int = 0
    rank: int = 2
    group_axis: int = 1

    def pack(self) -> bytes:
        dims = tuple(self.dims) + (0,) * (4 - len(self.dims))
        return _RECORD.pack(self.name.encode().ljust(128, b"\0"), self.scheme, self.rank, *dims, self.group_axis,
                            self.group_size, self.scale_type, self.zero_type, self.weights_offset,
                            self.weights_length, self.scales_offset, self.scales_length, self.zeros_offset,
                            self.zeros_length, self.elements, self.tensor_checksum, b"\0" * 8)

    @classmethod
    def unpack(cls, raw: bytes) -> "Record":
        f = _RECORD.unpack(raw)
        return cls(name=f[0].rstrip(b"\0").decode(), scheme=f[1], rank=f[2], dims=tuple(f[3:7]), group_axis=f[7],
                   group_size=f[8], scale_type=f[9], zero_type=f[10], weights_offset=f[11], weights_length=f[12],
                   scales_offset=f[13], scales_length=f[14], zeros_offset=f[15], zeros_length=f[16],
                   elements=f[17], tensor_checksum=f[18])


@dataclass
class Header:
    tensor_count: int
    directory_offset: int
    data_offset: int
    file_bytes: int
    payload_checksum: int
    policy: str
    metadata_offset: int = 0
    metadata_bytes: int = 0
    metadata_version: int = 1
    metadata_checksum: int = FNV_OFFSET
    version: int = 1
    scope: int = 0
    model_snapshot: bytes = field(default=b"")
    diffusers_commit: bytes = field(default=b"")

    def pack(self) -> bytes:
        return _HEADER.pack(MAGIC, self.version, HEADER_BYTES, self.tensor_count, self.scope, self.directory_offset,
                            self.data_offset, self.file_bytes, self.payload_checksum,
                            self.model_snapshot.ljust(40, b"\0"), self.diffusers_commit.ljust(40, b"\0"),
                            self.policy.encode().ljust(32, b"\0"), self.metadata_offset, self.metadata_bytes,
                            self.metadata_version, self.metadata_checksum, b"\0" * 64)

    @classmethod
    def unpack(cls, raw: bytes) -> "Header":
        f = _HEADER.unpack(raw[:HEADER_BYTES])
        if f[0] != MAGIC:
            raise ValueError("not a QIPACK1 file")
        return cls(version=f[1], tensor_count=f[3], scope=f[4], directory_offset=f[5], data_offset=f[6],
                   file_bytes=f[7], payload_checksum=f[8], model_snapshot=f[9].rstrip(b"\0"),
                   diffusers_commit=f[10].rstrip(b"\0"), policy=f[11].rstrip(b"\0").decode(),
                   metadata_offset=f[12], metadata_bytes=f[13], metadata_version=f[14], metadata_checksum=f[15])


def int4_record(name: str, scheme: int, n: int, k: int, group: int = 64) -> Record:
    """Record fields of one INT4 block matrix (int4_pack.cplus:483-503)."""
    groups = n * (k // group)
    return Record(name=name, scheme=scheme, dims=(n, k), group_size=group, scale_type=TYPE_F16,
                  zero_type=TYPE_F16 if scheme == SCHEME_W4A16 else TYPE_NONE, weights_length=n * k // 2,
                  scales_length=groups * 2, zeros_length=groups * 2 if scheme == SCHEME_W4A16 else 0,
                  elements=n * k)


def plan(records: list[Record], data_offset: int) -> int:
    """Assign 256-aligned offsets in record order (int4_pack.cplus:504-517); returns file bytes."""
    cursor = data_offset
    for r in records:
        cursor = align_up(cursor)
        r.weights_offset = cursor
        cursor += r.weights_length
        if r.scales_length:
            cursor = align_up(cursor)
            r.scales_offset = cursor
            cursor += r.scales_length
        if r.zeros_length:
            cursor = align_up(cursor)
            r.zeros_offset = cursor
            cursor += r.zeros_length
    return align_up(cursor)


def tensor_arrays(blob: bytes | memoryview, r: Record):
    """(codes, scales, zeros) byte views of one record inside a mapped pack."""
    mv = memoryview(blob)
    w = mv[r.weights_offset: r.weights_offset + r.weights_length]
    s = mv[r.scales_offset: r.scales_offset + r.scales_length] if r.scales_length else None
    z = mv[r.zeros_offset: r.zeros_offset + r.zeros_length] if r.zeros_length else None
    return w, s, z


def record_checksum(blob, r: Record) -> int:
    """Tensor checksum over weights, scales, zeros in that order (:715-720)."""
    h = FNV_OFFSET
    for part in tensor_arrays(blob, r):
        if part is not None and len(part):
            h = fnv1a(part, h)
    return h
