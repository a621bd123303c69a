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

import ctypes
import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

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


def fnv1a(data, h: int = FNV_OFFSET) -> int:
    """FNV-1a 64 (int4_pack.cplus:151-159), by the library's qi_fnv1a."""
    from ._lib import load

    buf = np.ascontiguousarray(np.frombuffer(memoryview(data).cast("B"), np.uint8))
    return int(load().qi_fnv1a(h, buf.ctypes.data if buf.size else None, buf.size))


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


# ---------------------------------------------------------------- writing --

def write_pack(path, matrices, scheme: int, group: int = 64, metadata: bytes = b"",
               model_snapshot: bytes = b"", diffusers_commit: bytes = b"") -> Header:
    """Write a QIPACK1 file of INT4 records (the packer's layout,
    int4_pack.cplus:476-518 and :620-720): header, directory, metadata in the
    directory padding, then every record's codes, scales and (W4A16) zeros on
    256-byte boundaries, with tensor, metadata and payload checksums.

    ``matrices``: (name, codes uint8 [n, k/2], scales fp16 bits [n, k/g],
    zeros fp16 bits [n, k/g] or None) in record order, host arrays.
    """
    records, arrays = [], []
    for name, codes, scales, zeros in matrices:
        n, half_k = codes.shape
        r = int4_record(name, scheme, n, half_k * 2, group)
        parts = [np.ascontiguousarray(codes, np.uint8), np.ascontiguousarray(scales).view(np.uint16)]
        if scheme == SCHEME_W4A16:
            if zeros is None:
                raise ValueError(f"{name}: W4A16 records carry a zeros (minimums) array")
            parts.append(np.ascontiguousarray(zeros).view(np.uint16))
        for a, length in zip(parts, (r.weights_length, r.scales_length, r.zeros_length)):
            if a.nbytes != length:
                raise ValueError(f"{name}: array of {a.nbytes} bytes, record expects {length}")
        records.append(r)
        arrays.append(parts)
    directory_offset = HEADER_BYTES
    metadata_offset = directory_offset + RECORD_BYTES * len(records)
    data_offset = align_up(metadata_offset + len(metadata))
    file_bytes = plan(records, data_offset)
    blob = np.zeros(file_bytes, np.uint8)
    for r, parts in zip(records, arrays):
        h = FNV_OFFSET
        for a, off in zip(parts, (r.weights_offset, r.scales_offset, r.zeros_offset)):
            raw = a.view(np.uint8).reshape(-1)
            blob[off: off + raw.size] = raw
            h = fnv1a(raw, h)
        r.tensor_checksum = h
    blob[metadata_offset: metadata_offset + len(metadata)] = np.frombuffer(metadata, np.uint8)
    header = Header(tensor_count=len(records), directory_offset=directory_offset, data_offset=data_offset,
                    file_bytes=file_bytes, payload_checksum=fnv1a(blob[data_offset:]),
                    policy=policy_name(scheme, group), metadata_offset=metadata_offset,
                    metadata_bytes=len(metadata), metadata_checksum=fnv1a(metadata),
                    model_snapshot=model_snapshot, diffusers_commit=diffusers_commit)
    blob[:HEADER_BYTES] = np.frombuffer(header.pack(), np.uint8)
    for i, r in enumerate(records):
        o = directory_offset + i * RECORD_BYTES
        blob[o: o + RECORD_BYTES] = np.frombuffer(r.pack(), np.uint8)
    Path(path).write_bytes(blob.tobytes())
    return header


# ---------------------------------------------------------------- reading --

PACK_ERRORS = {1: "bad argument", 2: "I/O error", 3: "not a QIPACK1 pack of a known policy",
               4: "record layout", 5: "metadata checksum", 6: "tensor checksum", 7: "payload checksum"}


class QipackError(RuntimeError):
    def __init__(self, what: str, status: int):
        super().__init__(f"qipack: {what}: {PACK_ERRORS.get(status, status)}")
        self.status = status


class _CRecord(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 129), ("scheme", ctypes.c_uint32), ("rank", ctypes.c_uint32),
                ("dims", ctypes.c_uint64 * 4), ("group_axis", ctypes.c_uint32), ("group_size", ctypes.c_uint32),
                ("scale_type", ctypes.c_uint32), ("zero_type", ctypes.c_uint32),
                ("weights_offset", ctypes.c_uint64), ("weights_length", ctypes.c_uint64),
                ("scales_offset", ctypes.c_uint64), ("scales_length", ctypes.c_uint64),
                ("zeros_offset", ctypes.c_uint64), ("zeros_length", ctypes.c_uint64),
                ("elements", ctypes.c_uint64), ("tensor_checksum", ctypes.c_uint64)]


class Pack:
    """An open QIPACK1 file (qi_pack_open): header, directory, verify, and
    each INT4 record's arrays for the upload re-layout."""

    def __init__(self, path):
        from ._lib import load

        self._lib = load()
        self._h = ctypes.c_void_p()
        st = self._lib.qi_pack_open(str(path).encode(), ctypes.byref(self._h))
        if st:
            raise QipackError(f"open {path}", st)
        count, policy = ctypes.c_uint32(), ctypes.create_string_buffer(33)
        data_offset, file_bytes = ctypes.c_uint64(), ctypes.c_uint64()
        self._lib.qi_pack_info(self._h, ctypes.byref(count), policy, ctypes.byref(data_offset),
                               ctypes.byref(file_bytes))
        self.policy = policy.value.decode()
        self.data_offset, self.file_bytes = data_offset.value, file_bytes.value
        self.records = []
        for i in range(count.value):
            c = _CRecord()
            self._lib.qi_pack_record_at(self._h, i, ctypes.byref(c))
            self.records.append(Record(name=c.name.decode(), scheme=c.scheme, rank=c.rank, dims=tuple(c.dims),
                                       group_axis=c.group_axis, group_size=c.group_size, scale_type=c.scale_type,
                                       zero_type=c.zero_type, weights_offset=c.weights_offset,
                                       weights_length=c.weights_length, scales_offset=c.scales_offset,
                                       scales_length=c.scales_length, zeros_offset=c.zeros_offset,
                                       zeros_length=c.zeros_length, elements=c.elements,
                                       tensor_checksum=c.tensor_checksum))
        self._index = {r.name: i for i, r in enumerate(self.records)}

    def close(self):
        if self._h:
            self._lib.qi_pack_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter teardown
            pass

    def verify(self, expect_transformer: bool = False) -> None:
        """qi_pack_verify (int4_pack.cplus:733-850); raises QipackError."""
        st = self._lib.qi_pack_verify(self._h, 1 if expect_transformer else 0)
        if st:
            raise QipackError("verify", st)

    def read(self, offset: int, length: int) -> np.ndarray:
        out = np.empty(length, np.uint8)
        st = self._lib.qi_pack_read(self._h, offset, length, out.ctypes.data if length else None)
        if st:
            raise QipackError(f"read {length} bytes at {offset}", st)
        return out

    def record(self, name: str) -> Record:
        if name not in self._index:
            raise KeyError(f"no record {name!r} in the pack")
        return self.records[self._index[name]]

    def arrays(self, name: str):
        """(codes uint8 [n, k/2], scales fp16 bits [n, G], zeros or None) of an INT4 record."""
        r = self.record(name)
        n, k = r.dims[0], r.dims[1]
        g = k // r.group_size
        codes = self.read(r.weights_offset, r.weights_length).reshape(n, k // 2)
        scales = self.read(r.scales_offset, r.scales_length).view(np.uint16).reshape(n, g)
        zeros = (self.read(r.zeros_offset, r.zeros_length).view(np.uint16).reshape(n, g)
                 if r.zeros_length else None)
        return codes, scales, zeros
