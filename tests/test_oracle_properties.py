"""Pin the CPU oracle where the reference's known answers leave it open.

Each check is independent of the oracle's code (numpy, closed forms, the
f64 reference semantics), and the planted-mistake tests show that a dropped
term, a wrong sign or a wrong index fails them.  A plant lives in a Python
copy of the formula, never in the oracle itself.
"""
import numpy as np
import pytest

from manta_amd import synth
from oracle import oracle as orc


# ------------------------------------------------------------------ f16
def test_f16_to_f32_all_values():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan], want[~nan])


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(3.0),
        (rng.standard_normal(50000) * 1e-6).astype(np.float32),     # f16 subnormals
        (rng.standard_normal(20000) * 70000.0).astype(np.float32),  # overflow to inf
        np.array([65504, 65519.99, 65520, -65520, 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26, 0.0, -0.0],
                 dtype=np.float32),
    ])
    got = orc.f32_to_f16(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)


# ------------------------------------------------------------- packing
def _round_half_away(v32):
    v = v32.astype(np.float64)
    return np.where(v >= 0, np.floor(v + 0.5), np.ceil(v - 0.5))


def numpy_pack_q8(x):
    x = x.astype(np.float32)
    maxabs = np.abs(x).max(axis=1)
    with np.errstate(divide="ignore", invalid="ignore"):
        v = (x * np.float32(127.0)) / maxabs[:, None]
    codes = np.clip(_round_half_away(v), -127, 127)
    codes[maxabs == 0] = 0
    scales = (maxabs / np.float32(127.0)).astype(np.float32)
    return codes.astype(np.int8), scales


def test_pack_q8_matches_numpy_restatement():
    x = synth.normal_f32(1, 0, 3000, 96, 1.0, normalize=True)
    x[7] = 0.0
    x[8, :] = 0.5  # ties at the clamp edge
    codes, scales = orc.pack_q8_rows(x)
    wc, ws = numpy_pack_q8(x)
    np.testing.assert_array_equal(codes, wc)
    np.testing.assert_array_equal(scales, ws)


def test_pack_q4_nibbles_and_scales():
    x = synth.normal_f32(2, 0, 500, 64, 1.0, normalize=True)
    packed, scales = orc.pack_q4_blocks(x)
    lo = (packed & 0xF).astype(np.int16)
    hi = (packed >> 4).astype(np.int16)
    lo[lo >= 8] -= 16
    hi[hi >= 8] -= 16
    codes = np.empty((500, 64), np.int16)
    codes[:, 0::2] = lo
    codes[:, 1::2] = hi
    blocks = x.reshape(500, 2, 32)
    maxabs = np.abs(blocks).max(axis=2)
    v = (blocks * np.float32(7.0)) / maxabs[:, :, None]
    want = np.clip(_round_half_away(v), -7, 7).reshape(500, 64)
    np.testing.assert_array_equal(codes, want)
    np.testing.assert_array_equal(scales, (maxabs / np.float32(7.0)).astype(np.float16).view(np.uint16))


# ------------------------------------------------------ integer sums
def test_q8_dot_accumulators_equal_int64_matmul():
    q = synth.normal_f16(3, 0, 5, 256, 1.0, normalize=True)
    codes, scales = synth.q8_rows(3, 1, 2000, 256, normalize=True)
    _, acc = orc.score_q8("dot", q, codes, scales, with_acc=True)
    qc = np.stack([orc.query_e8(q[i])[0] for i in range(5)]).astype(np.int64)
    np.testing.assert_array_equal(acc, qc @ codes.astype(np.int64).T)


def test_q8_e16_accumulators_equal_int64_matmul():
    q = synth.normal_f16(4, 0, 4, 128, 1.0)
    codes, scales = synth.q8_rows(4, 1, 1500, 128)
    _, acc = orc.score_q8("l2_distance", q, codes, scales, with_acc=True)
    qc = np.stack([orc.query_e16(q[i])[0] for i in range(4)]).astype(np.int64)
    np.testing.assert_array_equal(acc, qc @ codes.astype(np.int64).T)


def test_query_e16_digits_and_range():
    q = synth.normal_f16(5, 0, 50, 384, 3.0)
    for i in range(50):
        codes, qs, qn, qq = orc.query_e16(q[i])
        assert np.abs(codes).max() == 32639
        qf = orc.f16_to_f32(q[i]).astype(np.float64)
        # half a step, plus the f32 rounding of 32639/maxabs and of qs
        err = np.abs(codes * np.float64(qs) - qf)
        assert np.all(err <= 0.5 * qs + 4.0 * np.abs(qf) * 2.0 ** -23 + 1e-12)
        lo = ((codes.astype(np.int32) + 128) & 255) - 128
        hi = (codes.astype(np.int32) - lo) // 256
        assert lo.min() >= -128 and lo.max() <= 127 and hi.min() >= -128 and hi.max() <= 127


# --------------------------------------------------------- closed forms
def test_one_hot_query_dot_reads_one_coordinate():
    codes, scales = synth.q8_rows(6, 1, 300, 64, normalize=True)
    for j in (0, 17, 63):
        q = np.zeros((1, 64), np.float32)
        q[0, j] = 1.0
        got = orc.score_q8("dot", orc.f32_to_f16(q), codes, scales)[0]
        want = scales.astype(np.float64) * codes[:, j]
        assert np.all(np.abs(got - want) <= np.spacing(np.abs(want).astype(np.float32)) + 1e-30)


def test_orthonormal_candidates_cosine_and_l2():
    d = 32
    eye = np.eye(d, dtype=np.float32)
    codes, scales = orc.pack_q8_rows(eye)
    packed, s4 = orc.pack_q4_blocks(eye)
    q = orc.f32_to_f16(eye[[3]])
    for got in (orc.score_q8("cosine", q, codes, scales)[0], orc.score_q4("cosine", q, packed, s4, d)[0]):
        assert abs(got[3] - 1.0) < 1e-6
        assert np.all(got[np.arange(d) != 3] == 0.0)
    # |e3 - v*e_j| = sqrt(1 + v^2) with v the dequantized 1.0 of each format
    v8 = np.float64(scales[0]) * 127
    v4 = np.float64(s4.view(np.float16)[0, 0]) * 7
    for got, v in ((orc.score_q8("l2_distance", q, codes, scales)[0], v8),
                   (orc.score_q4("l2_distance", q, packed, s4, d)[0], v4)):
        # the expanded |q|^2 + |d|^2 - 2 q.d cancels near zero: absolute error
        # up to sqrt(4 ulp(|q|^2 + |d|^2)) ~ 7e-4 here (documented limitation)
        assert got[3] <= abs(1 - v) + np.sqrt(8 * 2.0 ** -24)
        np.testing.assert_allclose(got[np.arange(d) != 3], np.sqrt(1.0 + v * v), rtol=2e-6)


# ----------------------------------------- f64 semantics of the reference
def _dequant_q8(codes, scales):
    return codes.astype(np.float32) * scales[:, None].astype(np.float32)


def _dequant_q4(packed, scales, d):
    lo = (packed & 0xF).astype(np.int16)
    hi = (packed >> 4).astype(np.int16)
    lo[lo >= 8] -= 16
    hi[hi >= 8] -= 16
    codes = np.empty((packed.shape[0], d), np.float32)
    codes[:, 0::2] = lo
    codes[:, 1::2] = hi
    s = scales.view(np.float16).astype(np.float32)
    return codes * np.repeat(s, 32, axis=1)


def _semantic(op, qf, docs):
    """The reference's formulas (tensor_ops.go:1366-1490) in f64 numpy."""
    q = qf.astype(np.float64)
    dd = docs.astype(np.float64)
    if op == "dot":
        return q @ dd.T
    if op == "cosine":
        return (q @ dd.T) / (np.linalg.norm(q, axis=1)[:, None] * np.linalg.norm(dd, axis=1)[None, :])
    diff = qf[:, None, :].astype(np.float32) - docs[None, :, :]
    return np.sqrt((diff.astype(np.float64) ** 2).sum(-1))


# Bounds of the packed contract against the f64 semantics (query encoding
# error): E16 ~2^-15 relative per coordinate; E8 ~1/254.
BOUNDS = {("q8", "cosine"): 2e-4, ("q8", "l2_distance"): 2e-4, ("q4", "cosine"): 2e-4,
          ("q4", "l2_distance"): 2e-4, ("q4", "dot"): 2e-4, ("q8", "dot"): 2e-2}


def _check_against_semantics(fmt, op, got, qf, docs):
    want = _semantic(op, qf, docs)
    scale = np.abs(want).max()
    return np.max(np.abs(got - want)) <= BOUNDS[(fmt, op)] * max(scale, 1.0)


@pytest.mark.parametrize("op", ["dot", "cosine", "l2_distance"])
def test_packed_q8_scores_track_reference_semantics(op):
    q = synth.normal_f16(7, 0, 6, 128, 1.0, normalize=(op != "l2_distance"))
    codes, scales = synth.q8_rows(7, 1, 800, 128, normalize=(op != "l2_distance"))
    got = orc.score_q8(op, q, codes, scales)
    qf = orc.f16_to_f32(q)
    if op == "dot":  # E8: the query is itself quantized to 127 levels
        qf = np.stack([orc.query_e8(q[i])[0] for i in range(6)]).astype(np.float32) / 127.0
    assert _check_against_semantics("q8", op, got, qf, _dequant_q8(codes, scales))


@pytest.mark.parametrize("op", ["dot", "cosine", "l2_distance"])
def test_packed_q4_scores_track_reference_semantics(op):
    q = synth.normal_f16(8, 0, 6, 384, 1.0, normalize=True)
    packed, s4 = synth.q4_rows(8, 1, 600, 384, normalize=True)
    got = orc.score_q4(op, q, packed, s4, 384)
    assert _check_against_semantics("q4", op, got, orc.f16_to_f32(q), _dequant_q4(packed, s4, 384))


def _planted_l2(q, codes, scales, mistake):
    """Python copy of the q8 l2 contract with one planted mistake."""
    out = np.empty((q.shape[0], codes.shape[0]), np.float32)
    dn, dd = orc.q8_row_consts(codes, scales)
    for i in range(q.shape[0]):
        c16, qs, qn, qq = orc.query_e16(q[i])
        acc = codes.astype(np.int64) @ c16.astype(np.int64)
        qd = (scales * np.float32(qs)) * acc.astype(np.float32)
        if mistake == "sign":
            t = (np.float32(qq) + dd) + np.float32(2.0) * qd
        elif mistake == "drop_dd":
            t = np.float32(qq) - np.float32(2.0) * qd
        elif mistake == "index":
            t = (np.float32(qq) + np.roll(dd, 1)) - np.float32(2.0) * qd
        else:
            t = (np.float32(qq) + dd) - np.float32(2.0) * qd
        out[i] = np.sqrt(np.maximum(t, 0))
    return out


def test_planted_mistakes_fail_the_semantic_check():
    q = synth.normal_f16(9, 0, 4, 128, 1.0)
    codes, scales = synth.q8_rows(9, 1, 500, 128)
    qf = orc.f16_to_f32(q)
    docs = _dequant_q8(codes, scales)
    honest = _planted_l2(q, codes, scales, None)
    np.testing.assert_array_equal(honest, orc.score_q8("l2_distance", q, codes, scales))
    assert _check_against_semantics("q8", "l2_distance", honest, qf, docs)
    for m in ("sign", "drop_dd", "index"):
        assert not _check_against_semantics("q8", "l2_distance", _planted_l2(q, codes, scales, m), qf, docs), m


# ---------------------------------------------------------------- top-k
@pytest.mark.parametrize("smallest", [False, True])
def test_topk_matches_lexsort(smallest):
    rng = np.random.default_rng(11)
    s = (rng.integers(-50, 50, size=(5, 3000)) / 7.0).astype(np.float32)
    got = orc.topk(s, 37, smallest=smallest)
    for r in range(5):
        key = s[r] if smallest else -s[r]
        order = np.lexsort((np.arange(3000), key))
        np.testing.assert_array_equal(got[r], order[:37])


def test_topk_treats_signed_zeros_as_equal():
    s = np.array([0.0, -0.0, 0.0, -0.0, -1.0], np.float32)
    np.testing.assert_array_equal(orc.topk(s, 4), [0, 1, 2, 3])


# -------------------------------------------------------- embed pieces
def test_normalize_rows_unit_norm_and_zero_rows():
    x = synth.normal_f32(12, 0, 100, 384, 3.0)
    x[5] = 0.0
    y = orc.normalize_rows(x)
    n = np.linalg.norm(y.astype(np.float64), axis=1)
    assert np.all(np.abs(n[np.arange(100) != 5] - 1.0) < 1e-6)
    assert np.all(y[5] == 0)


def test_mean_pool_masked_constant_rows_and_numpy():
    b, t, c = 6, 20, 48
    x = synth.normal_f32(13, 0, b * t, c).reshape(b, t, c)
    x[1] = x[1, :1]  # constant sequence: the pool is that row
    mask = np.ones((b, t), np.int32)
    mask[2] = 0
    mask[3, 7:] = 0
    got = orc.mean_pool_masked(x, mask)
    np.testing.assert_allclose(got[1], x[1, 0], rtol=1e-6)
    assert np.all(got[2] == 0)
    want = (x.astype(np.float64) * mask[:, :, None]).sum(1) / np.maximum(mask.sum(1), 1)[:, None]
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_matmul_against_f64():
    a = synth.normal_f32(14, 0, 50, 384, 0.02)
    w = synth.normal_f32(14, 1, 384, 96, 0.05)
    got = orc.matmul(a, w)
    want = a.astype(np.float64) @ w.astype(np.float64)
    bound = 384 * 6e-8 * (np.abs(a.astype(np.float64)) @ np.abs(w.astype(np.float64)))
    assert np.all(np.abs(got - want) <= bound + 1e-12)


def test_embed_is_the_composition_of_the_steps():
    tokens, mask, table, proj = synth.config1(b=4, t=40, vocab=300, d=64, e=32)
    out16, out32 = orc.embed(tokens, mask, table, proj_f16=proj)
    g = orc.gather_rows(orc.f16_to_f32(table), tokens.reshape(-1)).reshape(4, 40, 64)
    y = orc.matmul(g, orc.f16_to_f32(proj))
    p = orc.normalize_rows(orc.mean_pool_masked(y, mask))
    np.testing.assert_array_equal(out32, p)
    np.testing.assert_array_equal(out16, orc.f32_to_f16(p))
