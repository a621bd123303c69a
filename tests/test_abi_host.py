"""CPU tests of the boundary: the C-ABI library loads, exports every symbol
the header declares, and rejects bad shapes before touching the GPU (the
reference returns cudaErrorInvalidValue the same way, gemm.cu:185,264)."""
import ctypes
import re
from pathlib import Path

import pytest

import qwen_image_hip
from qwen_image_hip import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "qwen_image_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|void|uint64_t|long long)\s+(qi_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_reference_entry_points():
    names = declared_functions()
    for ref in ("qi_w4a4_quantize_activations", "qi_w4a4_gemm", "qi_w4a16_gemm", "qi_f32_to_f16"):
        assert ref in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared_functions()) == set(_lib.SIGNATURES) | set(_lib.RESTYPES), \
        "ctypes table out of sync with the header"


def test_abi_version():
    assert qwen_image_hip.load().qi_hip_abi_version() == _lib.ABI_VERSION


INVALID = 1  # hipErrorInvalidValue


@pytest.mark.parametrize("m,n,k", [(100, 128, 256), (128, 100, 256), (128, 128, 320), (129, 128, 256)])
def test_reference_w4a4_shape_rules(m, n, k):
    assert qwen_image_hip.load().qi_w4a4_gemm(8, 8, 8, 8, 8, m, n, k) == INVALID


@pytest.mark.parametrize("m,n,k", [(100, 128, 64), (128, 100, 64), (128, 128, 96)])
def test_reference_w4a16_shape_rules(m, n, k):
    assert qwen_image_hip.load().qi_w4a16_gemm(8, 8, 8, 8, 8, m, n, k) == INVALID


def test_extension_argument_checks():
    L = qwen_image_hip.load()
    assert L.qi_w4a4_quantize_activations(16, 16, 16, 4, 300) == INVALID          # k % 256
    assert L.qi_hip_w4a4_quantize_activations_f16(16, 16, 16, 4, 255, None) == INVALID
    assert L.qi_hip_w4a4_gemm_tiled(8, 8, 8, 8, None, 8, 0, 0, 5, 24, 256, None) == INVALID  # n % 16
    assert L.qi_hip_w4a4_gemm_tiled(8, 8, 8, 8, None, 8, 2, 0, 5, 32, 256, None) == INVALID  # out type
    assert L.qi_hip_w4a16_gemm_tiled(16, 8, 8, None, 8, 0, 7, 5, 32, 64, None) == INVALID    # epilogue
    assert L.qi_hip_w4a16_gemv(16, 8, 8, None, 8, 0, 0, 17, 32, 64, None) == INVALID         # m > 16
    assert L.qi_hip_w4a16_gemv(16, 8, 8, None, 8, 0, 0, 0, 32, 64, None) == INVALID
    assert L.qi_hip_pack_weights(8, 8, 8, 8, 16, 320, 6, 0, None) == INVALID                 # k % 256
    assert L.qi_hip_pack_weights(8, 8, 8, None, 16, 256, 5, 0, None) == INVALID             # no minimums
    assert L.qi_hip_pack_weights(8, 8, 8, 8, 16, 256, 4, 0, None) == INVALID                 # scheme
    assert L.qi_hip_relayout_w4a4(8, 8, 8, 8, 24, 256, None) == INVALID
    assert L.qi_hip_relayout_w4a16(8, 8, 8, 8, 8, 16, 96, None) == INVALID
    # misaligned operand pointers are refused, not faulted on
    assert L.qi_hip_w4a4_gemm_tiled(9, 8, 8, 8, None, 8, 0, 0, 5, 32, 256, None) == INVALID
    assert L.qi_w4a4_quantize_activations(18, 16, 16, 4, 256) == INVALID
    # fused-record parts: n_part must divide n and keep whole tiles
    assert L.qi_hip_w4a4_gemm_fp6_parts(16, 16, None, 16, 0, 0, 4, 96, 256, 48, None) == INVALID
    assert L.qi_hip_w4a4_gemm_fp6_parts(16, 16, None, 16, 0, 0, 4, 96, 256, 64, None) == INVALID
    assert L.qi_hip_w4a4_gemm_fp6_parts(16, 16, None, 16, 0, 0, 4, 96, 256, 0, None) == INVALID
    assert L.qi_hip_w4a16_gemm_tiled_parts(16, 8, 8, None, 8, 0, 0, 5, 96, 64, 24, None) == INVALID
    assert L.qi_hip_w4a16_gemm_tiled_parts(16, 8, 8, None, 8, 0, 0, 5, 96, 64, 64, None) == INVALID
    # dual-stream split must be inside (0, m) and on a 32-row tile
    assert L.qi_hip_w4a4_gemm_fp6_dual(16, 16, None, 16, 0, 0, 256, 0, 64, 256, 64, None) == INVALID
    assert L.qi_hip_w4a4_gemm_fp6_dual(16, 16, None, 16, 0, 0, 256, 256, 64, 256, 64, None) == INVALID
    assert L.qi_hip_w4a4_gemm_fp6_dual(16, 16, None, 16, 0, 0, 256, 40, 64, 256, 64, None) == INVALID
    # W4A16 dual-stream: each stream needs more than 16 rows
    assert L.qi_hip_w4a16_gemm_tiled_dual(16, 8, 8, None, 16, 0, 0, 100, 16, 64, 64, 64, None) == INVALID
    assert L.qi_hip_w4a16_gemm_tiled_dual(16, 8, 8, None, 16, 0, 0, 100, 90, 64, 64, 64, None) == INVALID
    # producers: widths, alignment, output types, scratch
    assert L.qi_hip_layer_norm_scale(16, 16, 16, 16, 0, 4, 30, 0, None) == INVALID          # width % 4
    assert L.qi_hip_layer_norm_scale(16, 16, 16, 16, 2, 4, 32, 0, None) == INVALID          # out type
    assert L.qi_hip_layer_norm_scale(16, 16, 16, 24, 0, 4, 32, 0, None) == INVALID          # out alignment
    assert L.qi_hip_layer_norm_scale_quantize_fp6(16, 16, 256, 0, 16, 16, 4, 320, None) == INVALID  # k % 256
    assert L.qi_hip_layer_norm_scale_quantize_fp6(16, 16, 256, 0, None, 16, 4, 256, None) == INVALID
    assert L.qi_hip_swiglu(16, 16, 16, 0, 6, None) == INVALID                               # count % 4
    assert L.qi_hip_swiglu_quantize_fp6(16, 16, 16, 4, 128, None) == INVALID               # k % 256
    # null pointers
    assert L.qi_w4a4_gemm(None, None, None, None, None, 128, 128, 256) == INVALID


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "absent.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(ImportError):
        _lib.load()


def test_error_wording_mirrors_reference():
    e = _lib.QiHipError("w4a4 gemm", 1)
    assert "w4a4 gemm failed" in str(e) and e.status == 1


# The tile choices the parity tests rely on (a query: no device work).  The
# MMDiT block's shapes: image rows 4096 (12288 for an edit with two reference
# images), text rows 256 (512), q/k/v/out 3072, MLP 12288, fused QKV 9216.
@pytest.mark.parametrize("m,n_out,cfg", [
    (1, 18432, 0), (16, 18432, 0),                 # GEMV
    (256, 3072, 1), (256, 3968, 1), (64, 12288, 1),  # K-split: under 256 64 x 64 tiles
    (256, 4096, 3), (256, 9216, 3), (256, 12288, 3), (128, 9216, 3), (200, 9216, 3),
    (1152, 192, 3), (300, 2048, 3), (1024, 256, 3),
    (4096, 9216, 4), (4096, 3072, 4), (1152, 18432, 4), (600, 18432, 4),
    (4096, 12288, 5), (12288, 12288, 5),
    (1152, 1024, 6),
    (300, 37888, 7), (256, 37888, 7), (512, 32768, 7), (600, 37888, 3),  # 64 x 128: short M, >= 2048 small tiles
])
def test_w4a16_tile_choice(m, n_out, cfg):
    assert qwen_image_hip.load().qi_hip_w4a16_tiles(m, n_out) == cfg


@pytest.mark.parametrize("m,n,cfg", [
    (4096, 9216, 1), (4096, 3072, 1), (4096, 12288, 1), (12288, 9216, 1), (2048, 6144, 1),
    (4100, 3072, 0), (256, 9216, 3), (256, 3072, 4), (512, 3072, 4), (100, 8192, 3),
])
def test_fp6_tile_choice(m, n, cfg):
    assert qwen_image_hip.load().qi_hip_w4a4_fp6_tiles(m, n) == cfg


@pytest.mark.parametrize("m,m_split,n,k,slices", [
    (300, 0, 1024, 3584, 3), (300, 0, 3584, 3584, 3), (300, 0, 3584, 18944, 4), (300, 0, 37888, 3584, 0),
    (300, 0, 4608, 3584, 3), (320, 0, 3072, 3072, 3),
    (288, 0, 3584, 9472, 4), (320, 0, 3072, 12288, 5),
    (256, 0, 3072, 12288, 5), (256, 0, 3072, 3072, 0), (64, 0, 3072, 12288, 12), (512, 0, 3072, 12288, 2),
    (1536, 0, 3072, 3072, 0), (1536, 0, 12288, 3072, 0), (16, 0, 3072, 12288, 0),
])
def test_w4a16_split_choice(m, m_split, n, k, slices):
    """K slices the W4A16 call with a workspace chooses (workspace bytes =
    slices * m * n * 4), at a 256-CU device's rule (the library's default
    when no GPU is visible)."""
    assert qwen_image_hip.load().qi_hip_w4a16_workspace_bytes(m, m_split, n, k) == slices * m * n * 4


@pytest.mark.parametrize("m,n,k,f16w", [
    (4096, 3072, 3072, True), (4096, 12288, 3072, True), (2048, 9216, 3072, True), (4096, 3072, 12288, True),
    (2047, 9216, 3072, False), (1536, 12288, 3072, False), (1152, 18432, 3072, False),
])
def test_w4a16_f16w_choice(m, n, k, f16w):
    """From 2048 rows (128 x 192, 256 x 256 and 128 x 128 tiles) a call with
    a workspace dequantises the weights once into it (n k fp16) instead of
    once per row tile."""
    assert qwen_image_hip.load().qi_hip_w4a16_workspace_bytes(m, 0, n, k) == (n * k * 2 if f16w else 0)


def test_w4a16_split_choice_dual():
    """A dual call run as two launches needs the larger stream's workspace:
    here the image stream's fp16 weights (against the text stream's four K
    slices, 256 x 3072 x 4 x 4 bytes, at K = 12288)."""
    L = qwen_image_hip.load()
    assert L.qi_hip_w4a16_workspace_bytes(4352, 4096, 3072, 12288) == 3072 * 12288 * 2
    assert L.qi_hip_w4a16_workspace_bytes(4352, 4096, 9216, 3072) == 9216 * 3072 * 2
    assert L.qi_hip_w4a16_workspace_bytes(1280, 1024, 3072, 12288) == 0  # one launch, 64 x 64 tiles
    assert L.qi_hip_w4a16_workspace_bytes(4352, 4352, 3072, 3072) == 0  # invalid m_split


def test_w4a16_ws_entry_checks():
    L = qwen_image_hip.load()
    # negative workspace size, unaligned workspace, negative m_split
    assert L.qi_hip_w4a16_gemm_tiled_ws(16, 16, 16, None, 16, 0, 0, 64, 0, 64, 64, 64, 16, -1, None) == INVALID
    assert L.qi_hip_w4a16_gemm_tiled_ws(16, 16, 16, None, 16, 0, 0, 64, 0, 64, 64, 64, 8, 64, None) == INVALID
    assert L.qi_hip_w4a16_gemm_tiled_ws(16, 16, 16, None, 16, 0, 0, 64, -1, 64, 64, 64, 16, 64, None) == INVALID


def test_tile_queries_reject_empty_shapes():
    L = qwen_image_hip.load()
    assert L.qi_hip_w4a16_tiles(0, 64) == -1 and L.qi_hip_w4a4_fp6_tiles(64, 0) == -1


def test_noalloc_entry_point_rejects_sizes_beyond_its_array():
    """The no-allocation LayerNorm -> quantise entry point refuses more rows
    than its fixed statistics array holds (65536), before touching a GPU."""
    L = qwen_image_hip.load()
    assert L.qi_hip_layer_norm_scale_quantize_fp6_noalloc(16, 16, 256, 0, 16, 65537, 256, None) == INVALID
    assert L.qi_hip_layer_norm_scale_quantize_fp6_noalloc(16, 16, 256, 0, 16, 4, 300, None) == INVALID  # k % 256
    assert L.qi_hip_layer_norm_scale_quantize_fp6_noalloc(16, 16, 256, 0, 16, 0, 256, None) == 0          # no rows


CPLUS = Path(__file__).resolve().parents[1] / "include" / "cplus" / "src" / "hip.cplus"


def _c_to_cplus(c: str) -> str:
    c = " ".join(c.replace("const ", "").split())
    ptr, base = c.count("*"), c.replace("*", "").strip()
    return "*" * ptr + {"void": "u8", "float": "f32", "int": "i32", "char": "u8", "uint32_t": "u32",
                        "uint64_t": "u64", "long long": "i64", "unsigned long long": "u64", "qi_pack": "u8",
                        "qi_pack_record": "u8"}[base]


def test_cplus_binding_matches_the_header():
    """include/cplus/src/hip.cplus (the C+ declarations a reference-side
    package binds) declares every function of the header, with the same
    parameter names, order and C+ types, and the reference's own four
    declarations (cuda.cplus:45-46,53-58) unchanged."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    header = {}
    for m in re.finditer(r"^\s*((?:const\s+)?(?:int|void|uint64_t|long long|unsigned long long)\s*\**)\s*(qi_\w+)"
                         r"\s*\(([^)]*)\)\s*;", text, flags=re.M | re.S):
        args = " ".join(m.group(3).split())
        params = [] if args == "void" else [
            (re.match(r"(.*?)(\w+)$", a.strip()).group(2), _c_to_cplus(re.match(r"(.*?)(\w+)$", a.strip()).group(1)))
            for a in args.split(",")]
        ret = None if m.group(1).strip() == "void" else _c_to_cplus(m.group(1))
        header[m.group(2)] = (params, ret)
    cplus = {}
    for m in re.finditer(r'#\[link_name = "(qi_\w+)"\]\nextern fn (qi_\w+)\(([^)]*)\)(?: -> (\S+))?;',
                         CPLUS.read_text()):
        assert m.group(1) == m.group(2)
        params = [tuple(p.strip().split(": ")) for p in m.group(3).split(",")] if m.group(3).strip() else []
        cplus[m.group(1)] = (params, m.group(4))
    assert set(cplus) == set(header) == set(declared_functions())
    for name, sig in header.items():
        assert cplus[name] == sig, name
    # The reference's declarations, verbatim in meaning.
    assert cplus["qi_w4a4_gemm"][0] == [("a_codes", "*u8"), ("a_scales", "*u8"), ("w_codes", "*u8"),
                                        ("w_scales", "*u8"), ("y", "*f32"), ("m", "i32"), ("n", "i32"), ("k", "i32")]
    assert cplus["qi_f32_to_f16"] == ([("source", "*f32"), ("out", "*u8"), ("count", "u64")], "i32")


def _att_split_bytes(tail, segs):
    """Counters (4 bytes per split unit, 256-byte rounded), then one part
    slot per segment of each split unit: 512 threads x (offset, sum, 64 O
    floats)."""
    return (tail * 4 + 255) // 256 * 256 + tail * segs * 512 * (8 + 256)


@pytest.mark.parametrize("nq,nk,heads,tail,segs", [
    (4352, 4352, 16, 16, 7),    # 272 query blocks: one lockstep round, 16 left in 7 segments
    (4352, 4352, 20, 84, 3),    # 340 blocks: 84 left in 3 segments (252 parts, one round of CUs)
    (4352, 4352, 32, 32, 7),    # 544 blocks: two rounds, 32 left
    (4352, 4352, 48, 48, 5),    # 816 blocks: three rounds, 48 left
    (300, 4100, 3, 6, 6),       # 6 blocks x 65 key tiles, no whole round
    (129, 1000, 2, 2, 4),       # 2 blocks x 16 key tiles
    (4352, 4352, 24, 0, 0),     # 408 blocks: 152 left would need parts over several rounds
    (4352, 4352, 8, 0, 0),      # 136 blocks: likewise
    (4352, 4352, 12, 0, 0),     # 204 blocks in one round
    (256 * 256, 4352, 1, 0, 0), # exactly one round
    (129, 192, 2, 0, 0),        # 3 key tiles: too short to split
    (0, 64, 1, 0, 0), (64, 0, 1, 0, 0), (64, 64, 0, 0, 0),
])
def test_attention_split_choice(nq, nk, heads, tail, segs):
    """The attention's balanced split (qi_hip_flash_attention_ws) and its
    workspace at a 256-CU device's rule (the library's default when no GPU
    is visible): whole rounds of 256-query blocks in lockstep, then the
    `tail` blocks left, each cut into `segs` aligned key segments, all parts
    in one round of CUs; taken where the tail costs at most 85 % of a round
    of whole blocks."""
    got = qwen_image_hip.load().qi_hip_flash_attention_workspace_bytes(nq, nk, heads)
    assert got == (_att_split_bytes(tail, segs) if tail else 0)
