"""GPU parity of the default scores: the reference's own dotRows /
cosineRows / l2DistanceRows (runtime/backend/tensor_ops.go:1366-1490) on the
dequantized candidates, and topKTensor's ids (value desc, index asc).

Bar: ids and scores bit-exact with the oracle's restatement of those
functions (oracle.ref_score_q8 / ref_score_q4, pinned against the dequantized
matrix form in tests/test_oracle_properties.py) on identical seeded inputs,
through every device route: the streaming scans (per-wave lists and the
reservoir), the multi-query matrix-core passes, the q4 int8 shadow, the
reference finish and its full rescan (ties, duplicates, zero rows and
queries, scales outside the scans' range).
"""
import json
import os

import numpy as np
import pytest

from manta_amd import synth
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))


def _q8_case(seed, nq, n, d, sets=1, normalize=True):
    q = synth.normal_f16(500 + seed, 0, nq, d, 1.0, normalize=normalize)
    codes = np.empty((sets, n, d), np.int8)
    scales = np.empty((sets, n), np.float32)
    for s in range(sets):
        codes[s], scales[s] = synth.q8_rows(500 + seed, 1 + s, n, d, normalize=normalize)
    if sets == 1:
        return q, codes[0], scales[0]
    return q, codes, scales


def _q4_case(seed, nq, n, d, normalize=True):
    q = synth.normal_f16(600 + seed, 0, nq, d, 1.0, normalize=normalize)
    packed, s4 = synth.q4_rows(600 + seed, 1, n, d, normalize=normalize)
    return q, packed, s4


def _check_topk(rt, cands, op, q, want_s, k, smallest):
    ids, sc, _ = rt.score_topk(cands, op, rt.to_device(q), k, smallest=smallest)
    want_ids = orc.topk(want_s, k, smallest=smallest)
    np.testing.assert_array_equal(ids.download(), want_ids)
    np.testing.assert_array_equal(sc.download(), np.take_along_axis(want_s, want_ids, 1))
    return want_ids


def test_reference_runtime_vectors_on_device(rt):
    """The reference's runtime-level known answers (runtime_test.go), with
    the docs packed to q8: scores equal the oracle's reference restatement on
    the packed values and stay within the reference's 5e-4 of its f32
    answers; ids equal the reference's."""
    for case in GOLD["score_runtime"]:
        q = orc.f32_to_f16(np.asarray(case["q"], np.float32).reshape(1, -1))
        docs = np.asarray(case["docs"], np.float32)
        codes, scales = orc.pack_q8_rows(docs)
        cands = rt.bind_q8(codes, scales)
        qd = rt.to_device(q)
        got = rt.score(cands, case["op"], qd).download()[0]
        want = orc.ref_score_q8(case["op"], q, codes, scales)[0]
        np.testing.assert_array_equal(got, want)
        if "want" in case:
            np.testing.assert_allclose(got, case["want"], rtol=0, atol=5e-4)
        else:
            ids, sc, _ = rt.score_topk(cands, case["op"], qd, case["topk"])
            np.testing.assert_array_equal(ids.download()[0], case["want_ids"])
            np.testing.assert_allclose(sc.download()[0], case["want_scores"], rtol=0, atol=5e-4)
        cands.close()


@pytest.mark.parametrize("op", ["dot", "cosine", "l2_distance"])
@pytest.mark.parametrize("d,sets", [(64, 1), (256, 1), (384, 1), (100, 1), (48, 3), (256, 3)])
def test_q8_score_matrix_reference(rt, op, d, sets):
    nq, n = 3, 1500
    q, codes, scales = _q8_case(d + sets, nq, n, d, sets, normalize=(op != "l2_distance"))
    cands = rt.bind_q8(codes, scales)
    got = rt.score(cands, op, rt.to_device(q)).download()
    np.testing.assert_array_equal(got, orc.ref_score_q8(op, q, codes, scales))
    cands.close()


@pytest.mark.parametrize("op", ["dot", "cosine", "l2_distance"])
@pytest.mark.parametrize("d", [32, 384])
def test_q4_score_matrix_reference(rt, op, d):
    nq, n = 3, 2000
    q, packed, s4 = _q4_case(d, nq, n, d, normalize=(op != "l2_distance"))
    cands = rt.bind_q4(packed, s4, d)
    got = rt.score(cands, op, rt.to_device(q)).download()
    np.testing.assert_array_equal(got, orc.ref_score_q4(op, q, packed, s4, d))
    cands.close()


@pytest.mark.parametrize("op,smallest", [("dot", False), ("cosine", False), ("l2_distance", True),
                                         ("l2_distance", False), ("dot", True), ("cosine", True)])
@pytest.mark.parametrize("sets", [1, 4])
@pytest.mark.parametrize("n,k,d", [(1, 1, 256), (300, 7, 256), (4097, 10, 128), (20000, 48, 384),
                                   (20000, 100, 256), (5000, 1000, 100)])
def test_q8_topk_reference_streaming(rt, op, smallest, sets, n, k, d):
    """One query per workgroup (few queries, or one candidate set per query):
    per-wave lists (k <= 48) and the reservoir, then the finish."""
    nq = 4
    q, codes, scales = _q8_case(n + k + d, nq, n, d, sets, normalize=(op != "l2_distance"))
    cands = rt.bind_q8(codes, scales)
    _check_topk(rt, cands, op, q, orc.ref_score_q8(op, q, codes, scales), k, smallest)
    cands.close()


@pytest.mark.parametrize("op,smallest", [("dot", False), ("cosine", False), ("l2_distance", True),
                                         ("cosine", True), ("l2_distance", False)])
@pytest.mark.parametrize("nq,n,d,k", [(8, 5000, 128, 10), (33, 20000, 384, 50), (16, 30000, 128, 1000),
                                      (40, 4097, 256, 100), (64, 12345, 64, 1), (300, 4000, 256, 20)])
def test_q8_topk_reference_multi_query(rt, op, smallest, nq, n, d, k):
    """Many queries against one shared matrix: the matrix-core passes rank
    the rows, the finish rescores and proves."""
    q, codes, scales = _q8_case(nq + n + d + k, nq, n, d, 1, normalize=(op != "l2_distance"))
    cands = rt.bind_q8(codes, scales)
    _check_topk(rt, cands, op, q, orc.ref_score_q8(op, q, codes, scales), k, smallest)
    cands.close()


@pytest.mark.parametrize("op,smallest", [("cosine", False), ("l2_distance", True), ("dot", False), ("dot", True)])
@pytest.mark.parametrize("nq,n,d,k", [(3, 3000, 32, 50), (37, 5000, 128, 50), (129, 4097, 384, 100),
                                      (9, 2000, 64, 1)])
def test_q4_topk_reference(rt, op, smallest, nq, n, d, k):
    q, packed, s4 = _q4_case(nq + n + d + k, nq, n, d, normalize=(op != "l2_distance"))
    cands = rt.bind_q4(packed, s4, d)
    _check_topk(rt, cands, op, q, orc.ref_score_q4(op, q, packed, s4, d), k, smallest)
    cands.close()


@pytest.mark.parametrize("op,smallest", [("cosine", False), ("cosine", True), ("dot", False)])
@pytest.mark.parametrize("nq,n,d,k", [(256, 6000, 384, 100), (300, 5003, 128, 10), (520, 3000, 384, 300)])
def test_q4_shadow_topk_reference(rt, op, smallest, nq, n, d, k):
    """256 or more q4 cosine / dot queries: the int8 shadow ranks, the exact
    q4 scores select the candidates, the finish rescores with the reference
    arithmetic."""
    q, packed, s4 = _q4_case(nq + n + d + k, nq, n, d)
    cands = rt.bind_q4(packed, s4, d)
    _check_topk(rt, cands, op, q, orc.ref_score_q4(op, q, packed, s4, d), k, smallest)
    cands.close()


@pytest.mark.parametrize("op,smallest", [("dot", False), ("cosine", False), ("l2_distance", True)])
@pytest.mark.parametrize("nq", [2, 40])
def test_reference_all_ties_go_to_the_rescan(rt, op, smallest, nq):
    """Identical rows: every score ties, the finish cannot prove its set
    (the kp-th row ties the k-th), and the full rescan returns the k lowest
    indices."""
    n, d, k = 20000, 256, 64
    q, codes1, scale1 = _q8_case(3, nq, 1, d, 1)
    codes = np.repeat(codes1, n, axis=0)
    scales = np.repeat(scale1, n)
    cands = rt.bind_q8(codes, scales)
    want = _check_topk(rt, cands, op, q, orc.ref_score_q8(op, q, codes, scales), k, smallest)
    np.testing.assert_array_equal(want, np.tile(np.arange(k), (nq, 1)))
    cands.close()


@pytest.mark.parametrize("op,smallest", [("cosine", False), ("l2_distance", True), ("dot", False)])
def test_reference_duplicates_across_the_boundary(rt, op, smallest):
    """Clusters of duplicate rows around the k-th place: ties the scan
    cannot order are settled by index after the reference rescoring, with
    the rescan where the kp rows end inside a cluster."""
    nq, n, d, k = 12, 30000, 128, 50
    q, codes, scales = _q8_case(17, nq, n, d, 1, normalize=(op != "l2_distance"))
    codes, scales = codes.copy(), scales.copy()
    rng = np.random.default_rng(5)
    # each query's best few rows get 40 exact copies scattered over the matrix
    want_s = orc.ref_score_q8(op, q, codes, scales)
    for qi in range(nq):
        order = np.argsort(want_s[qi], kind="stable")
        src = order[k - 1] if smallest else order[-k]
        dst = rng.choice(n, 40, replace=False)
        codes[dst] = codes[src]
        scales[dst] = scales[src]
    cands = rt.bind_q8(codes, scales)
    _check_topk(rt, cands, op, q, orc.ref_score_q8(op, q, codes, scales), k, smallest)
    cands.close()


@pytest.mark.parametrize("op,smallest", [("cosine", False), ("l2_distance", True), ("dot", True)])
def test_reference_zero_rows_and_zero_query(rt, op, smallest):
    nq, n, d, k = 9, 6000, 128, 40
    q, codes, scales = _q8_case(23, nq, n, d, 1, normalize=(op != "l2_distance"))
    q, codes, scales = q.copy(), codes.copy(), scales.copy()
    q[4] = 0
    zero = np.arange(0, n, 7)
    codes[zero] = 0
    scales[zero[::2]] = 0.0
    cands = rt.bind_q8(codes, scales)
    _check_topk(rt, cands, op, q, orc.ref_score_q8(op, q, codes, scales), k, smallest)
    got = rt.score(cands, op, rt.to_device(q)).download()
    np.testing.assert_array_equal(got, orc.ref_score_q8(op, q, codes, scales))
    cands.close()


@pytest.mark.parametrize("op,smallest", [("cosine", False), ("l2_distance", True), ("dot", False)])
def test_reference_scales_outside_the_scan_range(rt, op, smallest):
    """A row scale below 2^-60 takes the candidates off the quantized-query
    scans (their error bounds assume no underflow): every query is rescanned
    with the reference arithmetic."""
    nq, n, d, k = 5, 8000, 64, 30
    q, codes, scales = _q8_case(29, nq, n, d, 1, normalize=(op != "l2_distance"))
    scales = scales.copy()
    scales[123] = 1e-30
    cands = rt.bind_q8(codes, scales)
    _check_topk(rt, cands, op, q, orc.ref_score_q8(op, q, codes, scales), k, smallest)
    cands.close()


@pytest.mark.parametrize("op,smallest", [("dot", False), ("l2_distance", True), ("cosine", False)])
def test_reference_adversarial_row_order(rt, op, smallest):
    """Rows ranked worst first for every query (same codes, scales growing
    with the index): the scans' regions fill and compact, many rows tie in
    the quantized scores, and the reference finish settles them."""
    nq, n, d, k = 24, 100000, 128, 100
    rng = np.random.default_rng(k)
    base = rng.standard_normal(d)
    q = orc.f32_to_f16((base + 0.05 * rng.standard_normal((nq, d))).astype(np.float32))
    codes1, scale1 = orc.pack_q8_rows((base / np.linalg.norm(base)).astype(np.float32).reshape(1, -1))
    codes = np.repeat(codes1, n, axis=0)
    if op == "l2_distance":
        smax = 0.9 * scale1[0] * np.linalg.norm(base)
        scales = (smax * (np.arange(n) + 1) / n).astype(np.float32)
    else:
        scales = (scale1[0] * (1.0 + np.arange(n) / n)).astype(np.float32)
    cands = rt.bind_q8(codes, scales)
    _check_topk(rt, cands, op, q, orc.ref_score_q8(op, q, codes, scales), k, smallest)
    cands.close()


def test_reference_repeated_calls(rt):
    """Per-call state (the finish's verdicts, tickets) is reset: calls in a
    row with different shapes each match the oracle."""
    for n, nq, k in ((20000, 32, 100), (5000, 3, 10), (9000, 40, 700)):
        q, codes, scales = _q8_case(n + nq, nq, n, 128, 1, normalize=False)
        cands = rt.bind_q8(codes, scales)
        _check_topk(rt, cands, "l2_distance", q, orc.ref_score_q8("l2_distance", q, codes, scales), k, True)
        cands.close()


def test_quantized_dot_differs_from_reference_dot(rt):
    """The two dot semantics on the same data: the default equals dotRows,
    the quantized-query flag BASELINE's formula, and they are not the same
    scores (a round(q*127) query is not the f16 query)."""
    q, codes, scales = _q8_case(31, 2, 3000, 256, 1)
    cands = rt.bind_q8(codes, scales)
    qd = rt.to_device(q)
    ref = rt.score(cands, "dot", qd).download()
    quant = rt.score(cands, "dot", qd, quantized=True).download()
    np.testing.assert_array_equal(ref, orc.ref_score_q8("dot", q, codes, scales))
    np.testing.assert_array_equal(quant, orc.score_q8("dot", q, codes, scales))
    assert not np.array_equal(ref, quant)
    cands.close()
