"""QIPACK1 container: header/record layout, FNV-1a, 256-byte planning."""
import numpy as np

import oracle
from qwen_image_hip import qipack


def test_fnv1a_known_answers():
    # Published FNV-1a 64 test vectors.
    assert qipack.fnv1a(b"") == 0xCBF29CE484222325
    assert qipack.fnv1a(b"a") == 0xAF63DC4C8601EC8C
    assert qipack.fnv1a(b"foobar") == 0x85944171F73967E8
    data = np.random.default_rng(0).integers(0, 256, 4096, dtype=np.uint8).tobytes()
    assert qipack.fnv1a(data) == oracle.fnv1a(data)


def test_header_and_record_round_trip():
    h = qipack.Header(tensor_count=297, directory_offset=256, data_offset=1 << 20, file_bytes=123 << 20,
                      payload_checksum=0xDEADBEEF, policy=qipack.policy_name(6))
    raw = h.pack()
    assert len(raw) == 256 and raw[:8] == b"QIPACK1\x00"
    assert raw[136:168].rstrip(b"\0") == b"transformer:w4a4-h256-g64-v6"
    h2 = qipack.Header.unpack(raw)
    assert (h2.tensor_count, h2.data_offset, h2.policy) == (297, 1 << 20, "transformer:w4a4-h256-g64-v6")
    r = qipack.int4_record("transformer_blocks.0.attn.to_q.weight", 5, 3072, 3072)
    raw = r.pack()
    assert len(raw) == 256
    # field offsets as the NumPy reader reads them (evaluate_int4_quantization.py:58-63)
    import struct
    assert struct.unpack_from("<II", raw, 128) == (5, 2)
    assert struct.unpack_from("<4Q", raw, 136)[:2] == (3072, 3072)
    assert struct.unpack_from("<IIII", raw, 168) == (1, 64, 1, 1)
    r2 = qipack.Record.unpack(raw)
    assert r2.name == r.name and r2.weights_length == 3072 * 1536 and r2.zeros_length == 3072 * 48 * 2


def test_plan_aligns_every_tensor_to_256():
    recs = [qipack.int4_record(f"m{i}", s, n, k) for i, (s, n, k) in
            enumerate([(5, 48, 256), (6, 16, 512), (5, 3072, 3072)])]
    end = qipack.plan(recs, data_offset=4096 + 17)
    for r in recs:
        for off, ln in ((r.weights_offset, r.weights_length), (r.scales_offset, r.scales_length),
                        (r.zeros_offset, r.zeros_length)):
            if ln:
                assert off % 256 == 0
    assert end % 256 == 0 and end >= recs[-1].zeros_offset + recs[-1].zeros_length
    assert recs[1].zeros_length == 0 and recs[1].zeros_offset == 0


def test_record_checksum_order():
    r = qipack.int4_record("x", 5, 16, 256)
    end = qipack.plan([r], 0)
    blob = bytearray(np.random.default_rng(1).integers(0, 256, end, dtype=np.uint8).tobytes())
    w, s, z = qipack.tensor_arrays(blob, r)
    want = qipack.fnv1a(bytes(z), qipack.fnv1a(bytes(s), qipack.fnv1a(bytes(w))))
    assert qipack.record_checksum(blob, r) == want


# ------------------------------------------------- container write / verify --

import pytest  # noqa: E402


def _pack_file(tmp_path, scheme=5, shapes=((64, 256), (32, 512)), metadata=b'{"source": "synthetic"}'):
    g = np.random.default_rng(7)
    mats = []
    for i, (n, k) in enumerate(shapes):
        codes = g.integers(0, 256, (n, k // 2), dtype=np.uint8)
        scales = (g.random((n, k // 64)) * 0.01 + 0.001).astype(np.float16).view(np.uint16)
        zeros = (-(g.random((n, k // 64)) * 0.05)).astype(np.float16).view(np.uint16) if scheme == 5 else None
        mats.append((f"transformer_blocks.{i}.attn.to_q.weight", codes, scales, zeros))
    path = tmp_path / "model.qipack"
    qipack.write_pack(path, mats, scheme, metadata=metadata)
    return path, mats


@pytest.mark.parametrize("scheme", [5, 6])
def test_write_open_verify_round_trip(tmp_path, scheme):
    path, mats = _pack_file(tmp_path, scheme)
    with qipack.Pack(path) as p:
        p.verify()
        assert p.policy == qipack.policy_name(scheme)
        assert [r.name for r in p.records] == [m[0] for m in mats]
        for name, codes, scales, zeros in mats:
            c, s, z = p.arrays(name)
            np.testing.assert_array_equal(c, codes)
            np.testing.assert_array_equal(s, scales)
            if scheme == 5:
                np.testing.assert_array_equal(z, zeros)
            else:
                assert z is None
            r = p.record(name)
            assert r.weights_offset % 256 == 0 and r.scales_offset % 256 == 0
            assert r.tensor_checksum == oracle.fnv1a(zeros.tobytes() if zeros is not None else b"",
                                                     oracle.fnv1a(scales.tobytes(), oracle.fnv1a(codes.tobytes())))
        with pytest.raises(qipack.QipackError, match="not a QIPACK1"):
            p.verify(expect_transformer=True)  # 2 records, not the 297-tensor transformer


def _corrupt(path, offset, value=None):
    b = bytearray(path.read_bytes())
    b[offset] = (b[offset] ^ 0x5A) if value is None else value
    path.write_bytes(bytes(b))


def test_verify_catches_each_kind_of_damage(tmp_path):
    path, mats = _pack_file(tmp_path)
    with qipack.Pack(path) as p:
        r0, meta_off, data_off = p.records[0], 256 + 256 * len(mats), p.data_offset
    cases = {
        "tensor checksum": r0.scales_offset + 3,        # a scale byte
        "metadata checksum": meta_off + 2,              # a metadata byte
        "payload checksum": 48,                         # the header's payload checksum field
    }
    for what, off in cases.items():
        bad = tmp_path / f"bad_{off}.qipack"
        bad.write_bytes(path.read_bytes())
        _corrupt(bad, off)
        with qipack.Pack(bad) as p, pytest.raises(qipack.QipackError, match=what):
            p.verify()
    # a record's weights moved off its 256-byte boundary
    bad = tmp_path / "misaligned.qipack"
    bad.write_bytes(path.read_bytes())
    _corrupt(bad, 256 + 184, (r0.weights_offset + 16) & 0xFF)
    with qipack.Pack(bad) as p, pytest.raises(qipack.QipackError, match="record layout"):
        p.verify()
    # not a pack, and a truncated one
    bad = tmp_path / "magic.qipack"
    bad.write_bytes(path.read_bytes())
    _corrupt(bad, 0, ord("X"))
    with pytest.raises(qipack.QipackError, match="not a QIPACK1"):
        qipack.Pack(bad)
    bad = tmp_path / "short.qipack"
    bad.write_bytes(path.read_bytes()[:-256])
    with pytest.raises(qipack.QipackError, match="not a QIPACK1"):
        qipack.Pack(bad)
    with pytest.raises(qipack.QipackError, match="I/O"):
        qipack.Pack(tmp_path / "absent.qipack")
