"""qi-quantize, the pack writer / verifier command
(qwen_image_quantize/src/main.cplus:9-55, int4_pack.cplus:472-850).

The expected output pack is built here from the oracle's quantisers and the
reference writer's layout rules (int4_pack.cplus:476-518 planning, :563-580
metadata, :620-680 header and payload checksum, :682-731 tensor checksums);
the GPU test requires the command's file to equal it byte for byte.  The CPU
tests cover the argument handling and the verify command on packs written
here (a valid one, the FP16 source, a damaged one)."""
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle
from qwen_image_hip import qipack

CLI = Path(qipack.__file__).resolve().parent / "qi-quantize"
SOURCE_POLICY = "transformer:all-matrix-f16-v4"
SOURCE_META = b"model=synthetic\nsnapshot=test\n"
# Per block: seven rank-2 FP16 matrices (input widths multiples of 256) and
# two rank-1 vectors; nine global vectors first: 9 + 32 * 9 = 297 records.
BLOCK_SHAPES = [(16, 256), (32, 256), (16, 512), (48, 256), (16, 256), (32, 512), (16, 768)]


def _run(*args):
    return subprocess.run([str(CLI), *map(str, args)], capture_output=True, text=True, timeout=600)


def _source_pack(path: Path, seed: int = 0) -> bytes:
    """An all-FP16 v4 QIPACK with the transformer inventory, tiny matrices."""
    rng = np.random.default_rng(seed)
    records, payloads = [], []

    def add(name, arr):
        arr = np.ascontiguousarray(arr)
        r = qipack.Record(name=name, scheme=1, dims=arr.shape, rank=arr.ndim, weights_length=arr.nbytes,
                          elements=arr.size, group_axis=0)
        records.append(r)
        payloads.append(arr.view(np.uint8).reshape(-1))

    def halves(shape, scale):
        return oracle.half_from_f32(rng.standard_normal(shape).astype(np.float32) * scale)

    for i in range(9):
        add(f"global.{i}", halves((64 + 8 * i,), 0.5))
    for b in range(32):
        for j, (n, k) in enumerate(BLOCK_SHAPES):
            w = halves((n, k), 0.05)
            if j == 3:
                w[0, :64] = 0  # an all-zero group
            add(f"transformer_blocks.{b}.m{j}.weight", w)
        add(f"transformer_blocks.{b}.v0", halves((48,), 1.0))
        add(f"transformer_blocks.{b}.v1", halves((40,), 1.0))
    directory_end = 256 + 256 * len(records)
    data_offset = qipack.align_up(directory_end + len(SOURCE_META) + 4096)
    file_bytes = qipack.plan(records, data_offset)
    blob = np.zeros(file_bytes, np.uint8)
    for r, p in zip(records, payloads):
        blob[r.weights_offset: r.weights_offset + p.size] = p
        r.tensor_checksum = qipack.fnv1a(p)
    blob[directory_end: directory_end + len(SOURCE_META)] = np.frombuffer(SOURCE_META, np.uint8)
    h = qipack.Header(tensor_count=len(records), directory_offset=256, data_offset=data_offset,
                      file_bytes=file_bytes, payload_checksum=qipack.fnv1a(blob[data_offset:]),
                      policy=SOURCE_POLICY, metadata_offset=directory_end, metadata_bytes=len(SOURCE_META),
                      metadata_checksum=qipack.fnv1a(SOURCE_META), model_snapshot=b"snap", diffusers_commit=b"dc")
    blob[:256] = np.frombuffer(h.pack(), np.uint8)
    for i, r in enumerate(records):
        blob[256 + 256 * i: 512 + 256 * i] = np.frombuffer(r.pack(), np.uint8)
    raw = blob.tobytes()
    path.write_bytes(raw)
    return raw


def _expected_pack(source: bytes, scheme: int, clip: bool) -> bytes:
    """The output the reference writer produces for `source`."""
    src = np.frombuffer(source, np.uint8)
    header = qipack.Header.unpack(source[:256])
    recs = [qipack.Record.unpack(source[header.directory_offset + 256 * i: header.directory_offset + 256 * (i + 1)])
            for i in range(header.tensor_count)]
    meta = source[header.metadata_offset: header.metadata_offset + header.metadata_bytes]
    base = "w4a16-g64" if scheme == 5 else "w4a4-h256-g64"
    meta += f"quant={base}{'-clip' if clip else ''}\nquant_source={SOURCE_POLICY}\n".encode()
    out_recs, parts = [], []
    for r in recs:
        data = src[r.weights_offset: r.weights_offset + r.weights_length]
        if r.scheme == 1 and r.rank == 2:
            n, k = r.dims[:2]
            codes, scales, mins = oracle.quantize_matrix(data.view(np.uint16).reshape(n, k), scheme, clip)
            o = qipack.int4_record(r.name, scheme, n, k)
            o.rank, o.dims, o.elements = r.rank, r.dims, r.elements
            arrays = [codes, scales] + ([mins] if scheme == 5 else [])
        else:
            o = qipack.Record(**{**r.__dict__, "tensor_checksum": 0})
            arrays = [data]
        out_recs.append(o)
        parts.append([np.ascontiguousarray(a).view(np.uint8).reshape(-1) for a in arrays])
    file_bytes = qipack.plan(out_recs, header.data_offset)
    blob = np.zeros(file_bytes, np.uint8)
    for o, arrays in zip(out_recs, parts):
        h = qipack.FNV_OFFSET
        for a, off in zip(arrays, (o.weights_offset, o.scales_offset, o.zeros_offset)):
            blob[off: off + a.size] = a
            h = qipack.fnv1a(a, h)
        o.tensor_checksum = h
    directory_end = header.directory_offset + 256 * len(out_recs)
    out_h = qipack.Header.unpack(source[:256])
    out_h.policy = qipack.policy_name(scheme)
    out_h.file_bytes = file_bytes
    out_h.payload_checksum = qipack.fnv1a(blob[header.data_offset:])
    out_h.metadata_offset, out_h.metadata_bytes = directory_end, len(meta)
    out_h.metadata_version, out_h.metadata_checksum = 1, qipack.fnv1a(meta)
    blob[:256] = np.frombuffer(out_h.pack(), np.uint8)
    for i, o in enumerate(out_recs):
        blob[header.directory_offset + 256 * i: header.directory_offset + 256 * (i + 1)] = \
            np.frombuffer(o.pack(), np.uint8)
    blob[directory_end: directory_end + len(meta)] = np.frombuffer(meta, np.uint8)
    return blob.tobytes()


def test_usage_and_group_are_rejected_with_status_2(tmp_path):
    assert _run().returncode == 2
    assert _run("w4a8", "a", "b").returncode == 2
    assert _run("w4a4", "a").returncode == 2
    assert _run("w4a4", "a", "b", "96").returncode == 2
    r = _run("w4a16", "a", "b", "128")
    assert r.returncode == 2 and "g64" in r.stderr
    assert _run("verify").returncode == 2


def test_bad_sources_fail_with_status_1(tmp_path):
    assert _run("w4a4", tmp_path / "missing.qipack", tmp_path / "o").returncode == 1
    junk = tmp_path / "junk.qipack"
    junk.write_bytes(b"\0" * 4096)
    assert _run("w4a4", junk, tmp_path / "o").returncode == 1
    assert not (tmp_path / "o").exists() and not (tmp_path / "o.tmp").exists()


def test_verify_command(tmp_path):
    src = tmp_path / "src.qipack"
    source = _source_pack(src, seed=1)
    # The FP16 source is not an INT4 pack.
    assert _run("verify", src).returncode == 1
    good = tmp_path / "good.qipack"
    blob = bytearray(_expected_pack(source, 6, clip=False))
    good.write_bytes(bytes(blob))
    r = _run("verify", good)
    assert r.returncode == 0, r.stderr
    # One flipped code byte in the last matrix: its tensor checksum fails.
    h = qipack.Header.unpack(bytes(blob[:256]))
    last = qipack.Record.unpack(bytes(blob[h.directory_offset + 256 * 296: h.directory_offset + 256 * 297]))
    mats = [qipack.Record.unpack(bytes(blob[h.directory_offset + 256 * i: h.directory_offset + 256 * (i + 1)]))
            for i in range(297)]
    m = [r for r in mats if r.scheme == 6][-1]
    blob[m.weights_offset + 3] ^= 0x10
    bad = tmp_path / "bad.qipack"
    bad.write_bytes(bytes(blob))
    assert _run("verify", bad).returncode == 1
    assert last.scheme == 1  # the last record is a copied vector


@pytest.mark.gpu
@pytest.mark.parametrize("scheme,name,clip", [(6, "w4a4", False), (5, "w4a16", False), (6, "w4a4", True),
                                              (5, "w4a16", True)])
def test_writes_the_reference_pack_byte_for_byte(tmp_path, scheme, name, clip):
    print(f"qi-quantize {name} clip={clip}", flush=True)
    src = tmp_path / "src.qipack"
    source = _source_pack(src, seed=2 + scheme)
    out = tmp_path / f"{name}.qipack"
    args = [name, src, out] + (["clip"] if clip else [])
    r = _run(*args)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "block 32/32" in r.stdout
    got = out.read_bytes()
    want = _expected_pack(source, scheme, clip)
    assert len(got) == len(want)
    if got != want:
        diff = np.flatnonzero(np.frombuffer(got, np.uint8) != np.frombuffer(want, np.uint8))
        pytest.fail(f"{diff.size} bytes differ, first at {diff[0]}")
    assert _run("verify", out).returncode == 0
