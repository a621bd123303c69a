"""Pin the CPU oracle: reference known-answer tests, closed forms, brute force.

Each check is chosen so that a plausible slip in the oracle (a wrong rounding
mode, a transposed butterfly, a dropped clip candidate, a wrong nibble order)
fails it.  The reference's own #[test] functions are ported first, with their
file:line.
"""
import numpy as np
import pytest

import oracle
from _data import f16_bits, heavy_tailed, normal_f32, weights_f16


# ------------------------------------------------------------------ fp16 --

def test_half_known_answers():
    """half.cplus:81-90 (half_round_trip_is_exact_for_representable_values)."""
    L = oracle.lib()
    assert L.qo_half_to_f32(L.qo_half_from_f32(1.0)) == 1.0
    assert L.qo_half_to_f32(L.qo_half_from_f32(-2.5)) == -2.5
    assert L.qo_half_to_f32(L.qo_half_from_f32(0.000061035156)) == np.float32(0.000061035156)
    assert L.qo_half_from_f32(0.000000059604645) == 1
    assert L.qo_half_from_f32(0.000000029802322) == 0
    assert L.qo_half_from_f32(65504.0) == 0x7BFF


def test_half_exhaustive_round_trip_and_widening():
    """Every finite fp16: to_f32 equals IEEE widening, and from_f32 inverts it."""
    L = oracle.lib()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = (bits & 0x7C00) != 0x7C00
    ieee = bits.view(np.float16).astype(np.float32)
    sample = bits[finite][::7]
    ours = np.array([L.qo_half_to_f32(int(b)) for b in sample], np.float32)
    np.testing.assert_array_equal(ours.view(np.uint32), ieee[finite][::7].view(np.uint32))
    back = oracle.half_from_f32(ieee[finite])
    np.testing.assert_array_equal(back, bits[finite])


def test_half_rounding_matches_ieee_rne():
    """from_f32 is IEEE round-to-nearest-even, ties and subnormals included."""
    g = np.random.default_rng(1)
    x = np.concatenate([
        g.normal(size=20000).astype(np.float32),
        (g.normal(size=20000) * 1e-5).astype(np.float32),
        # exact midpoints between adjacent fp16 values (normal and subnormal)
        ((np.arange(1, 4000, dtype=np.float64) + 0.5) * 2.0 ** -24).astype(np.float32),
        ((np.arange(1024, 2048, dtype=np.float64) + 0.5) * 2.0 ** -10).astype(np.float32),
        np.array([65504, 65519, 65520, 70000, -65520, 1e-9, -1e-9], np.float32),
    ])
    with np.errstate(over="ignore"):
        ieee = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(oracle.half_from_f32(x), ieee)


# ------------------------------------------------------------------ H256 --

H4 = 0.5 * np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], np.float64)


def test_hadamard_involution():
    """int4_pack.cplus:854-869 (hadamard_256_is_an_involution)."""
    v = (np.arange(256, dtype=np.float32) * np.float32(0.01) - np.float32(1.0)).astype(np.float32)
    twice = oracle.hadamard256(oracle.hadamard256(v))
    assert np.max(np.abs(twice - v)) < 1e-5


def test_hadamard_equals_dense_kronecker():
    """Stride 1 mixes the lowest base-4 digit, stride 64 the highest, so the
    256x256 matrix is H4 (x) H4 (x) H4 (x) H4 with the first factor acting on
    the highest digit.  A transposed or mis-strided butterfly fails this."""
    H = np.kron(np.kron(H4, H4), np.kron(H4, H4))
    g = np.random.default_rng(2)
    for _ in range(8):
        v = g.normal(size=256).astype(np.float32)
        np.testing.assert_allclose(oracle.hadamard256(v), H @ v.astype(np.float64), atol=2e-6, rtol=1e-6)
    # basis vectors map to matrix columns
    for i in (0, 1, 5, 64, 255):
        e = np.zeros(256, np.float32)
        e[i] = 1.0
        np.testing.assert_array_equal(oracle.hadamard256(e), H[:, i].astype(np.float32))


def test_hadamard_orthonormal_norm():
    v = np.random.default_rng(3).normal(size=256).astype(np.float32)
    r = oracle.hadamard256(v)
    assert abs(np.linalg.norm(r) - np.linalg.norm(v)) < 1e-4 * np.linalg.norm(v)


def test_rotate_rows_is_per_chunk():
    x = normal_f32(3, 768, 4)
    r = oracle.rotate_rows(x)
    for row in range(3):
        for c in range(3):
            np.testing.assert_array_equal(r[row, 256 * c:256 * (c + 1)], oracle.hadamard256(x[row, 256 * c:256 * (c + 1)]))


# ------------------------------------------------------------ quantisers --

def _snib(codes):
    c = codes.astype(np.int32)
    return np.where(c > 7, c - 16, c)


def test_affine_group_reconstructs_within_half_a_step():
    """int4_pack.cplus:871-892."""
    values = (np.arange(64, dtype=np.float32) * np.float32(0.003) - np.float32(0.05)).astype(np.float32)
    codes, sb, mb = oracle.quantize_affine_group(values, clip=False)
    L = oracle.lib()
    s, m = L.qo_half_to_f32(sb), L.qo_half_to_f32(mb)
    assert codes.max() <= 15
    rec = codes.astype(np.float32) * np.float32(s) + np.float32(m)
    assert np.all(np.abs(rec - values) <= np.float32(s) * 0.5 + 1e-4)


def test_symmetric_group_uses_signed_nibbles():
    """int4_pack.cplus:894-908 known answer: scale 0.1, codes 9, 7, 1, 0."""
    values = np.zeros(64, np.float32)
    values[0], values[1], values[2] = -0.7, 0.7, 0.1
    codes, sb = oracle.quantize_symmetric_group(values, clip=False)
    assert abs(oracle.lib().qo_half_to_f32(sb) - 0.1) < 1e-4
    assert list(codes[:4]) == [9, 7, 1, 0]


def test_clipping_never_increases_group_error():
    """int4_pack.cplus:910-938."""
    values = np.array([((i * 7) % 13) * 0.01 for i in range(64)], np.float32)
    values[5] = 2.0
    L = oracle.lib()
    pc, ps = oracle.quantize_symmetric_group(values, clip=False)
    cc, cs = oracle.quantize_symmetric_group(values, clip=True)
    pe = np.sum((_snib(pc) * np.float32(L.qo_half_to_f32(ps)) - values) ** 2)
    ce = np.sum((_snib(cc) * np.float32(L.qo_half_to_f32(cs)) - values) ** 2)
    assert ce <= pe


def _candidate_errors(values, affine):
    """float64 squared error of every clip candidate, from the format's closed
    form (codes = clamp(rint(...)), fp16-rounded scale / minimum)."""
    v = values.astype(np.float64)
    out = []
    for c in (1.0, 0.95, 0.9, 0.85, 0.8, 0.75, 0.7):
        if affine:
            lo, hi = np.float32(values.min()), np.float32(values.max())
            center = np.float32((hi + lo) * np.float32(0.5))
            half = np.float32((hi - lo) * np.float32(0.5 * c))
            mn = np.float32(np.float16(np.float32(center - half)))
            s = np.float32(np.float16(max(np.float32(np.float32(center + half) - mn) / np.float32(15), np.float32(2 ** -24))))
            q = np.clip(np.rint((values - mn) / s), 0, 15)
            rec = q.astype(np.float64) * s + mn
        else:
            peak = np.float32(np.abs(values).max())
            s = np.float32(np.float16(max(np.float32(peak * np.float32(c / 7.0)), np.float32(2 ** -24))))
            q = np.clip(np.rint(values / s), -7, 7)
            rec = q.astype(np.float64) * s
        out.append((np.sum((rec - v) ** 2), s, q))
    return out


@pytest.mark.parametrize("affine", [False, True])
def test_clip_search_picks_a_minimal_candidate(affine):
    """Brute force over all 7 candidates: the chosen scale is (to fp32
    summation noise) the error minimum, and codes are the rint/clamp of it."""
    g = np.random.default_rng(5)
    L = oracle.lib()
    for trial in range(300):
        values = (g.standard_t(3, size=64) * 0.02).astype(np.float32)
        if trial % 3 == 0:
            values[g.integers(64)] *= 10
        if affine:
            codes, sb, mb = oracle.quantize_affine_group(values, clip=True)
        else:
            codes, sb = oracle.quantize_symmetric_group(values, clip=True)
        cands = _candidate_errors(values, affine)
        best = min(e for e, _, _ in cands)
        chosen = [i for i, (_, s, _) in enumerate(cands) if s == np.float32(L.qo_half_to_f32(sb))]
        assert chosen, "scale is not one of the candidates"
        assert min(cands[i][0] for i in chosen) <= best * (1 + 1e-5) + 1e-12
        q = cands[chosen[0]][2]
        want = q.astype(np.int64) & 15 if not affine else q.astype(np.int64)
        np.testing.assert_array_equal(codes.astype(np.int64), want)


def test_zero_and_constant_groups():
    zero = np.zeros(64, np.float32)
    codes, sb = oracle.quantize_symmetric_group(zero, clip=True)
    assert sb == 0x0001 and not codes.any()        # scale floor 2^-24 (int4_pack.cplus:53)
    codes, sb, mb = oracle.quantize_affine_group(zero, clip=True)
    assert sb == 0x0001 and mb == 0 and not codes.any()
    const = np.full(64, 0.25, np.float32)
    codes, sb, mb = oracle.quantize_affine_group(const, clip=False)
    assert mb == 0x3400 and sb == 0x0001 and not codes.any()


def test_quantize_matrix_layout_and_rotation():
    """Even k in the low nibble (int4_pack.cplus:414-418); W4A4 rows are rotated first."""
    w = weights_f16(8, 512, 6)
    codes, scales, mins = oracle.quantize_matrix(w, 5)
    row = w[3].view(np.float16).astype(np.float32)
    c0, s0, m0 = oracle.quantize_affine_group(row[64:128])
    assert scales[3, 1] == s0 and mins[3, 1] == m0
    np.testing.assert_array_equal(codes[3, 32:64] & 15, c0[0::2])
    np.testing.assert_array_equal(codes[3, 32:64] >> 4, c0[1::2])
    codes6, scales6, none = oracle.quantize_matrix(w, 6)
    assert none is None
    rot = oracle.rotate_rows(row[None, :])[0]
    c1, s1 = oracle.quantize_symmetric_group(rot[256:320])
    assert scales6[3, 4] == s1
    np.testing.assert_array_equal(codes6[3, 128:160] & 15, c1[0::2])
    with pytest.raises(ValueError):
        oracle.quantize_matrix(weights_f16(4, 320, 7), 6)


# --------------------------------------------------- activation quantiser --

def test_activation_quantizer_closed_form():
    """gemm.cu:41-51 on identical rotated inputs, restated with numpy's IEEE
    float32 division and rint (vectorised, independent of the C loops)."""
    x = heavy_tailed(64, 1024, 8)
    codes, scales = oracle.quantize_activations(x)
    r = oracle.rotate_rows(x).reshape(64, 16, 64)
    peak = np.abs(r).max(axis=-1)
    s16 = np.maximum(peak / np.float32(7.0), np.float32(5.9604645e-08)).astype(np.float32).astype(np.float16)
    np.testing.assert_array_equal(scales, s16.view(np.uint16))
    q = np.clip(np.rint(r / s16.astype(np.float32)[..., None]), -7, 7).astype(np.int64)
    nib = (q & 15).reshape(64, 512, 2)
    np.testing.assert_array_equal(codes, (nib[..., 0] | (nib[..., 1] << 4)).astype(np.uint8))


def test_activation_quantizer_special_rows():
    k = 256
    x = np.zeros((3, k), np.float32)
    x[1, 0] = 7.0            # rotates to +-3.5/4 ... one spike spreads over the chunk
    codes, scales = oracle.quantize_activations(x)
    assert (scales[0] == 1).all() and not codes[0].any()    # zero rows: 2^-24 floor, code 0
    # A spike of 7 at k=0 rotates to +-7/16 everywhere: scale 1/16, every code +-7.
    assert (scales[1] == np.float16(0.0625).view(np.uint16)).all()
    assert set(np.unique(codes[1])) <= {0x77, 0x79, 0x97, 0x99}


def test_activation_quantizer_ties_round_to_even():
    """Values at exact half-steps round to the even code (rint), not away."""
    # Build a chunk whose rotation is known: rotate a designed vector back.
    target = np.zeros(256, np.float32)
    target[:64] = np.float32(0.25) * np.array([7, 2.5, 1.5, -2.5, -1.5, 0.5, -0.5, 3.5] * 8, np.float32)
    x = oracle.hadamard256(target)          # H is its own inverse
    codes, scales = oracle.quantize_activations(x[None, :])
    # the rotation round trip is not exact, so only assert where it is
    back = oracle.hadamard256(x)
    if np.array_equal(back[:64], target[:64]):
        assert scales[0, 0] == np.float16(0.25).view(np.uint16)
        q = _snib(np.stack([codes[0, :32] & 15, codes[0, :32] >> 4], -1).reshape(-1))
        np.testing.assert_array_equal(q[:8], [7, 2, 2, -2, -2, 0, -0, 4])


def test_activation_f16_input_equals_widened_f32():
    xb = f16_bits(normal_f32(16, 768, 9))
    c16, s16 = oracle.quantize_activations(xb)
    c32, s32 = oracle.quantize_activations(xb.view(np.float16).astype(np.float32))
    np.testing.assert_array_equal(c16, c32)
    np.testing.assert_array_equal(s16, s32)


# ----------------------------------------------------------------- GEMMs --

def test_w4a4_partials_brute_force():
    g = np.random.default_rng(10)
    a = g.integers(0, 256, size=(7, 128), dtype=np.uint8)
    w = g.integers(0, 256, size=(5, 128), dtype=np.uint8)
    P = oracle.w4a4_partials(a, w)

    def unpack(c):
        v = np.stack([c & 15, c >> 4], -1).reshape(c.shape[0], -1).astype(np.int64)
        return np.where(v > 7, v - 16, v)

    A, W = unpack(a), unpack(w)
    want = np.einsum("mgk,ngk->mng", A.reshape(7, 4, 64), W.reshape(5, 4, 64))
    np.testing.assert_array_equal(P, want)


def test_w4a4_gemm_f32_vs_f64_and_formula():
    x = heavy_tailed(32, 512, 11)
    w = weights_f16(48, 512, 12)
    ac, as_ = oracle.quantize_activations(x)
    wc, ws, _ = oracle.quantize_matrix(w, 6, clip=True)
    y32 = oracle.w4a4_gemm(ac, as_, wc, ws)
    y64 = oracle.w4a4_gemm(ac, as_, wc, ws, f64=True)
    P = oracle.w4a4_partials(ac, wc).astype(np.float64)
    sa = as_.view(np.float16).astype(np.float64)
    sw = ws.view(np.float16).astype(np.float64)
    np.testing.assert_allclose(y64, np.einsum("mng,mg,ng->mn", P, sa, sw), rtol=1e-12, atol=1e-12)
    assert np.linalg.norm(y32 - y64) / np.linalg.norm(y64) < 1e-6
    # fp32 replay of gemm.cu:159-168 order: ascending g, fma(P, sa*sw, acc)
    acc = np.zeros((32, 48), np.float32)
    for gi in range(P.shape[2]):
        s = (sa[:, gi][:, None] * sw[:, gi][None, :]).astype(np.float32)   # exact in fp32
        acc = (P[:, :, gi] * s.astype(np.float64) + acc.astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(y32, acc)


def test_w4a4_end_to_end_approximates_float_linear():
    """Rotation + int4 both ways approximate x . W^T (sanity: not a bit test)."""
    x = normal_f32(64, 1024, 13)
    w = weights_f16(64, 1024, 14)
    ac, as_ = oracle.quantize_activations(x)
    wc, ws, _ = oracle.quantize_matrix(w, 6, clip=True)
    y = oracle.w4a4_gemm(ac, as_, wc, ws, f64=True)
    ref = x.astype(np.float64) @ w.view(np.float16).astype(np.float64).T
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 0.25


def test_w4a16_dequantize_closed_form():
    w = weights_f16(16, 256, 15)
    c, s, mn = oracle.quantize_matrix(w, 5, clip=True)
    deq = oracle.w4a16_dequantize(c, s, mn)
    codes = np.stack([c & 15, c >> 4], -1).reshape(16, 256).astype(np.float64)
    sc = np.repeat(s.view(np.float16).astype(np.float64), 64, axis=1)
    mi = np.repeat(mn.view(np.float16).astype(np.float64), 64, axis=1)
    # code*scale+min is exact in float64; one rounding to f32 = fmaf; then RNE fp16
    want = (codes * sc + mi).astype(np.float32).astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(deq, want)
    # without clipping it reconstructs the weights to within half a step
    c, s, mn = oracle.quantize_matrix(w, 5, clip=False)
    deq = oracle.w4a16_dequantize(c, s, mn).view(np.float16).astype(np.float32)
    sc = np.repeat(s.view(np.float16).astype(np.float32), 64, axis=1)
    err = np.abs(deq - w.view(np.float16).astype(np.float32))
    assert np.all(err <= sc * 0.5 + 1e-3)


def test_gemm_f16_precise_and_blocked():
    x = f16_bits(normal_f32(33, 320, 16))
    w = weights_f16(17, 320, 17)
    want = x.view(np.float16).astype(np.float64) @ w.view(np.float16).astype(np.float64).T
    np.testing.assert_allclose(oracle.gemm_f16(x, w, precise=True), want, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(oracle.gemm_f16(x, w, precise=False), want, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("m", [1, 2, 5])
def test_w4a16_gemv_baseline_matches_dequantised_matmul(m):
    """The CPU baseline of the modulation linears (per-group 16-entry weight
    tables, fp32 dots) against the closed-form dequantised weights
    (pinned above) times x in float64."""
    x = f16_bits(normal_f32(m, 640, 18))
    w = weights_f16(48, 640, 19)
    c, s, mn = oracle.quantize_matrix(w, 5)
    wd = oracle.w4a16_dequantize(c, s, mn).view(np.float16).astype(np.float64)
    want = x.view(np.float16).astype(np.float64) @ wd.T
    np.testing.assert_allclose(oracle.w4a16_gemv(x, c, s, mn), want, rtol=1e-5, atol=1e-5)


def test_gelu_tanh_formula():
    v = np.linspace(-6, 6, 101).astype(np.float32)
    want = 0.5 * v.astype(np.float64) * (1 + np.tanh(np.sqrt(2 / np.pi) * (v + 0.044715 * v.astype(np.float64) ** 3)))
    np.testing.assert_allclose(oracle.gelu_tanh(v), want, rtol=1e-5, atol=1e-6)


# ------------------------------------------- producers (LayerNorm, SwiGLU) --

def test_layer_norm_scale_oracle_closed_forms():
    import statistics
    rng = np.random.default_rng(11)
    x = rng.normal(3.0, 2.0, size=(6, 512))
    zero = np.zeros((2, 512))
    out = oracle.layer_norm_scale(x, zero)
    # zero scale: each row has mean 0 and population variance var / (var + eps)
    var = x.var(axis=1)
    np.testing.assert_allclose(out.mean(axis=1), 0.0, atol=1e-12)
    np.testing.assert_allclose(out.var(axis=1), var / (var + 1e-6), rtol=1e-12)
    # shift invariance, and one row against the statistics module
    np.testing.assert_allclose(oracle.layer_norm_scale(x + 100.0, zero), out, atol=1e-9)
    row = list(x[2])
    mu, pv = statistics.fmean(row), statistics.pvariance(row)
    np.testing.assert_allclose(out[2], [(v - mu) / (pv + 1e-6) ** 0.5 for v in row], rtol=1e-12)
    # the scale row: row 1 for rows < split, row 0 after; (1 + s) multiplies
    scale = np.stack([np.full(512, 0.5), np.full(512, -0.25)])
    got = oracle.layer_norm_scale(x, scale, split=2)
    np.testing.assert_allclose(got[:2], out[:2] * 0.75, rtol=1e-12)
    np.testing.assert_allclose(got[2:], out[2:] * 1.5, rtol=1e-12)


def test_swiglu_oracle_known_values():
    from scipy.special import expit
    g = np.array([0.0, 1.0, -1.0, 30.0, -30.0, 2.5])
    u = np.array([3.0, 2.0, 2.0, 1.0, 1.0, -4.0])
    np.testing.assert_allclose(oracle.swiglu(g, u), g * expit(g) * u, rtol=1e-14)
    assert oracle.swiglu(np.array([0.0]), np.array([5.0]))[0] == 0.0
    np.testing.assert_allclose(oracle.swiglu(np.array([40.0]), np.array([1.0])), [40.0], rtol=1e-15)


# ------------------------------------------------------------- attention --

def _att_inputs(nq, nk, heads, seed):
    rng = np.random.default_rng(seed)
    q = rng.normal(0, 1, size=(nq, heads * 128)).astype(np.float32)
    k = oracle.half_from_f32(rng.normal(0, 1, size=(nk, heads * 128)).astype(np.float32))
    v = oracle.half_from_f32(rng.normal(0, 1, size=(nk, heads * 128)).astype(np.float32))
    return q, k, v


def test_attention_oracle_closed_forms():
    from scipy.special import softmax
    q, k, v = _att_inputs(5, 7, 2, 21)
    vf = oracle.half_to_f32(v).astype(np.float64)
    # identical keys: uniform weights, out = mean of the visible values
    k_same = np.tile(k[:1], (7, 1))
    out = oracle.flash_attention(q, k_same, v, 2, round_p=False)
    np.testing.assert_allclose(out, np.tile(vf.mean(axis=0), (5, 1)), rtol=1e-12, atol=1e-12)
    # one visible key: out = that key's value row (p = 1 exactly)
    out = oracle.flash_attention(q, k, v, 2, visible_keys=np.ones(5, np.int64))
    np.testing.assert_allclose(out, np.tile(vf[0], (5, 1)), rtol=0, atol=0)
    # causal rows: row r sees r + 1 keys; nothing visible gives 0
    out = oracle.flash_attention(q, k, v, 2, causal_rows=5)
    np.testing.assert_allclose(out[0], vf[0], rtol=0, atol=0)
    vis = np.array([0, 3, 7, 2, 0])
    out = oracle.flash_attention(q, k, v, 2, visible_keys=vis)
    assert (out[0] == 0).all() and (out[4] == 0).all()
    # against scipy's softmax over the natural-log scores of the fp16 inputs
    qs = oracle.half_to_f32(oracle.half_from_f32(q * (np.float32(1.4426950408889634) / np.sqrt(np.float32(128)))))
    kf = oracle.half_to_f32(k).astype(np.float64)
    want = np.zeros((5, 256))
    for h in range(2):
        sl = slice(128 * h, 128 * h + 128)
        w = softmax((qs[:, sl].astype(np.float64) @ kf[:, sl].T) * np.log(2.0), axis=1)
        want[:, sl] = w @ vf[:, sl]
    np.testing.assert_allclose(oracle.flash_attention(q, k, v, 2, round_p=False), want, rtol=1e-10, atol=1e-12)
    # fp16 probabilities move the result by ~2^-11 relative at most
    np.testing.assert_allclose(oracle.flash_attention(q, k, v, 2), want, rtol=0, atol=2e-3)
