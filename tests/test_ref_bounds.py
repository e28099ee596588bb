"""The error bounds the reference-semantics top-k rests on, checked on the CPU.

The device ranks rows by a quantized-query score (E16 query codes) and proves
that its best kp rows hold the reference's best k with bounds on how far the
reference score (dotRows / cosineRows / l2DistanceRows on the dequantized
values) can lie from that score: [ref_lo(c), ref_hi(c)] around a scan score
c (manta_amd/csrc/ref_common.hpp).  Here the same bounds, computed from the
same quantities, are checked against the oracle's scan scores and reference
scores over every (query, row) of seeded inputs built to stress them: f16
queries with subnormal and large entries, rows of very different norms,
unnormalized and normalized data, d up to 1024.  A bound that is too tight
anywhere fails; a cosine margin without its query term is shown to fail.
"""
import math

import numpy as np
import pytest

from manta_amd import synth
from oracle import oracle as orc

U = 2.0 ** -24
UP = 1.0 + 2.0 ** -40


def _query_terms(q16):
    """G = |q - qs*code|, |q|, |q^| of one f16 query, as the finish computes
    them (f64, widened by 2^-40)."""
    x = orc.f16_to_f32(q16).astype(np.float64)
    codes, qs, _, _ = orc.query_e16(q16)
    qs = float(qs)
    c = codes.astype(np.float64)
    g = math.sqrt(float(((x - c * qs) ** 2).sum())) * UP
    qn = math.sqrt(float((x * x).sum())) * UP
    qh = math.sqrt(float((c * c).sum())) * qs * UP
    return g, qn, qh, float(np.abs(x).max())


def _bounds(op, g, qn, qh, e_qd, dn, bb, d):
    if op == "dot16":
        gam = d * U / (1 - d * U)
        m = (dn * (g * (1 + e_qd) + qn * (e_qd + U + 1.01 * gam)) + d * 1.401298464324817e-45) * UP
        return ("lin", m)
    if op == "cosine":
        m = ((2 * g / qn if qn > 0 else 0.0) + e_qd + 7.1 * U + 2.0 ** -40) * UP
        return ("lin", m)
    return ("l2", (g + U * dn) * UP, (5 * U + e_qd) * 1.02 * (qh * qh + bb) * UP)


def _hi(b, c):
    if b[0] == "lin":
        x = c + b[1]
        return x * np.where(x >= 0, UP, 1 / UP)
    s = c * (1 + 2.0 ** -23)
    return (np.sqrt(s * s + b[2]) + b[1]) * (1 + 2.1 * U) * UP


def _lo(b, c):
    if b[0] == "lin":
        x = c - b[1]
        return x * np.where(x >= 0, 1 / UP, UP)
    s = c * (1 - 2.0 ** -23)
    t = s * s - b[2]
    r = np.where(t > 0, np.sqrt(np.maximum(t, 0)), 0.0) - b[1]
    return np.where(r > 0, r * (1 - 2.1 * U) / UP, 0.0)


def _queries(seed, nq, d, normalize):
    q = synth.normal_f16(seed, 0, nq, d, 1.0, normalize=normalize).copy()
    rng = np.random.default_rng(seed)
    # stress the E16 rounding: subnormal f16 entries, and one large entry
    # that coarsens every other code
    q[0, :: 7] = orc.f32_to_f16(rng.uniform(-6e-5, 6e-5, size=q[0, ::7].shape).astype(np.float32))
    if nq > 1:
        q[1, 3] = orc.f32_to_f16(np.array([40.0], np.float32))[0]
    return q


def _rows_q8(seed, n, d, normalize):
    codes, scales = synth.q8_rows(seed, 1, n, d, normalize=normalize)
    scales = scales.copy()
    # rows of very different norms
    scales[::5] *= 1e-3
    scales[1::5] *= 1e3
    return codes, scales


def _check(op_scan, op_ref, q, scan, ref, fmt_err, dn, bb, d):
    viol = 0
    for i in range(q.shape[0]):
        g, qn, qh, maxabs = _query_terms(q[i])
        if maxabs == 0.0:
            continue
        b = _bounds(op_scan, g, qn, qh, fmt_err, dn, bb, d)
        c = scan[i].astype(np.float64)
        r = ref[i].astype(np.float64)
        viol += int((r > _hi(b, c)).sum() + (r < _lo(b, c)).sum())
    return viol


@pytest.mark.parametrize("op", ["dot", "cosine", "l2_distance"])
@pytest.mark.parametrize("d,normalize", [(64, True), (256, False), (384, True), (1024, False), (100, True)])
def test_q8_bounds_hold(op, d, normalize):
    nq, n = 6, 3000
    q = _queries(d + 11, nq, d, normalize)
    codes, scales = _rows_q8(d + 13, n, d, normalize)
    scan_op = "dot16" if op == "dot" else op
    scan = orc.score_q8(scan_op, q, codes, scales)
    ref = orc.ref_score_q8(op, q, codes, scales)
    dn, dd = orc.q8_row_consts(codes, scales)
    wide = 1 + 2.0 ** -22
    assert _check(scan_op, op, q, scan, ref, 3.1 * U, float(dn.max()) * wide, float(dd.max()) * wide, d) == 0


@pytest.mark.parametrize("op", ["dot", "cosine", "l2_distance"])
@pytest.mark.parametrize("d,normalize", [(32, True), (384, False), (1024, True)])
def test_q4_bounds_hold(op, d, normalize):
    nq, n = 6, 3000
    q = _queries(d + 17, nq, d, normalize)
    packed, s4 = synth.q4_rows(d + 19, 1, n, d, normalize=normalize)
    scan_op = "dot16" if op == "dot" else op
    scan = orc.score_q4("dot" if op == "dot" else op, q, packed, s4, d)
    ref = orc.ref_score_q4(op, q, packed, s4, d)
    dn, dd = orc.q4_row_consts(packed, s4, d)
    wide = 1 + 2.0 ** -22
    e_qd = (d // 32 + 1.2) * U
    assert _check(scan_op, op, q, scan, ref, e_qd, float(dn.max()) * wide, float(dd.max()) * wide, d) == 0


def test_cosine_margin_without_query_term_fails():
    """The check has teeth: without the query-quantization term 2G/|q| (only
    the rounding terms), reference cosines fall outside the bound on the same
    kind of data."""
    d, nq, n = 384, 6, 20000
    q = _queries(5, nq, d, True)
    codes, scales = _rows_q8(7, n, d, True)
    scan = orc.score_q8("cosine", q, codes, scales)
    ref = orc.ref_score_q8("cosine", q, codes, scales)
    viol = 0
    for i in range(nq):
        g, qn, qh, _ = _query_terms(q[i])
        b = ("lin", (3.1 * U + 7.1 * U) * UP)  # 2G/|q| left out
        c = scan[i].astype(np.float64)
        r = ref[i].astype(np.float64)
        viol += int((r > _hi(b, c)).sum() + (r < _lo(b, c)).sum())
    assert viol > 0


def test_reference_scores_of_packed_rows_equal_the_dequantized_matrix_form():
    """ref_score_q8 / ref_score_q4 (dequantizing row by row) are the
    reference restatements applied to the dequantized matrix, bit for bit,
    in both score layouts."""
    q = synth.normal_f16(3, 0, 3, 96, 1.0, normalize=False)
    codes, scales = synth.q8_rows(3, 1, 400, 96, normalize=False)
    packed, s4 = synth.q4_rows(3, 1, 400, 96, normalize=False)
    q32 = orc.f16_to_f32(q)
    fns = {"dot": orc.dot_rows, "cosine": orc.cosine_rows, "l2_distance": orc.l2_distance_rows}
    for op, fn in fns.items():
        np.testing.assert_array_equal(orc.ref_score_q8(op, q, codes, scales), fn(q32, orc.dequant_q8(codes, scales)))
        np.testing.assert_array_equal(orc.ref_score_q4(op, q, packed, s4, 96), fn(q32, orc.dequant_q4(packed, s4, 96)))
        # one candidate set per query: the reference's batched [Q,D] x [Q,N,D]
        c3 = np.stack([codes[:100], codes[100:200], codes[200:300]])
        s3 = np.stack([scales[:100], scales[100:200], scales[200:300]])
        np.testing.assert_array_equal(orc.ref_score_q8(op, q, c3, s3), fn(q32, orc.dequant_q8(c3, s3)))


def test_dequantized_values_are_the_f32_products():
    """q8 values are code*scale rounded once to f32; q4 values are exact
    (numpy's f32 multiply is the IEEE one)."""
    codes, scales = synth.q8_rows(4, 1, 50, 64, normalize=False)
    np.testing.assert_array_equal(orc.dequant_q8(codes, scales),
                                  codes.astype(np.float32) * scales[:, None].astype(np.float32))
    packed, s4 = synth.q4_rows(4, 1, 50, 64, normalize=False)
    lo = (packed & 0xF).astype(np.int8)
    hi = (packed >> 4).astype(np.int8)
    nib = np.empty((50, 64), np.int8)
    nib[:, 0::2] = np.where(lo >= 8, lo - 16, lo)
    nib[:, 1::2] = np.where(hi >= 8, hi - 16, hi)
    sc = orc.f16_to_f32(s4).astype(np.float64)
    want = (nib.astype(np.float64) * np.repeat(sc, 32, axis=1)).astype(np.float32)
    np.testing.assert_array_equal(orc.dequant_q4(packed, s4, 64), want)
