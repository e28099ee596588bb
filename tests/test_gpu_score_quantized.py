"""GPU parity of the quantized-query scores (MANTA_ROCM_QUANTIZED_QUERY)
and their top-k against the CPU oracle.

These are the scans that rank rows for the reference-semantics top-k (whose
proof rests on them returning their exact best kp rows), and BASELINE's q8
dot formula (configs 0 and 4).  Bar: scores, ids and integer accumulators
bit-exact with the oracle's restatement of the quantized-query formulas on
identical seeded inputs.
"""
import json
import os

import numpy as np
import pytest

from manta_amd import synth
from manta_amd._lib import MantaRocmError
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))


def _qscore(rt, *args, **kw):
    return rt.score(*args, quantized=True, **kw)


def _qtopk(rt, *args, **kw):
    return rt.score_topk(*args, quantized=True, **kw)


def _q8_case(seed, nq, n, d, sets, normalize=True):
    q = synth.normal_f16(100 + seed, 0, nq, d, 1.0, normalize=normalize)
    codes = np.empty((sets, n, d), np.int8)
    scales = np.empty((sets, n), np.float32)
    for s in range(sets):
        codes[s], scales[s] = synth.q8_rows(100 + seed, 1 + s, n, d, normalize=normalize)
    return q, codes, scales


def _oracle_codes(codes, sets):
    return codes[0] if sets == 1 else codes


@pytest.mark.parametrize("op", ["dot", "cosine", "l2_distance"])
@pytest.mark.parametrize("d", [64, 128, 256, 384, 100, 48])
def test_q8_score_matrix_bit_exact(rt, op, d):
    nq, n = 3, 1000
    q, codes, scales = _q8_case(d, nq, n, d, sets=1, normalize=(op != "l2_distance"))
    cands = rt.bind_q8(codes[0], scales[0])
    got = _qscore(rt, cands, op, rt.to_device(q)).download()
    want = orc.score_q8(op, q, codes[0], scales[0])
    np.testing.assert_array_equal(got, want)
    cands.close()


@pytest.mark.parametrize("op,smallest", [("dot", False), ("cosine", False), ("l2_distance", True),
                                         ("l2_distance", False), ("dot", True)])
@pytest.mark.parametrize("sets", [1, 4])
@pytest.mark.parametrize("n,k", [(1, 1), (300, 7), (4097, 10), (20000, 100)])
def test_q8_score_topk_bit_exact(rt, op, smallest, sets, n, k):
    nq, d = 4, 256
    q, codes, scales = _q8_case(n + k, nq, n, d, sets)
    cands = rt.bind_q8(codes[0] if sets == 1 else codes, scales[0] if sets == 1 else scales)
    ids, sc, acc = _qtopk(rt, cands, op, rt.to_device(q), k, smallest=smallest, with_acc=True)
    ids, sc, acc = ids.download(), sc.download(), acc.download()
    want_s, want_acc = orc.score_q8(op, q, _oracle_codes(codes, sets), scales[0] if sets == 1 else scales,
                                    with_acc=True)
    want_ids = orc.topk(want_s, k, smallest=smallest)
    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_array_equal(sc, np.take_along_axis(want_s, want_ids, 1))
    np.testing.assert_array_equal(acc, np.take_along_axis(want_acc, want_ids, 1))
    cands.close()


def _check_q8_topk(rt, op, smallest, q, codes, scales, k):
    """score_topk over per-query candidate sets against the oracle: ids,
    scores and integer accumulators bit-exact."""
    cands = rt.bind_q8(codes, scales)
    ids, sc, acc = _qtopk(rt, cands, op, rt.to_device(q), k, smallest=smallest, with_acc=True)
    ids, sc, acc = ids.download(), sc.download(), acc.download()
    want_s, want_acc = orc.score_q8(op, q, codes, scales, with_acc=True)
    want_ids = orc.topk(want_s, k, smallest=smallest)
    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_array_equal(sc, np.take_along_axis(want_s, want_ids, 1))
    np.testing.assert_array_equal(acc, np.take_along_axis(want_acc, want_ids, 1))
    cands.close()


@pytest.mark.parametrize("op,smallest", [("dot", False), ("cosine", False), ("l2_distance", True),
                                         ("dot", True)])
@pytest.mark.parametrize("d", [64, 128, 192, 384, 512, 768, 1024])
@pytest.mark.parametrize("k", [1, 33, 64])
def test_q8_wave_list_topk_bit_exact(rt, op, smallest, d, k):
    """k <= 64 keeps sorted per-wave lists in registers: every coalesced row
    width, with a row count that leaves a partial last round."""
    nq, n = 2, 5000 + d
    q, codes, scales = _q8_case(d + k, nq, n, d, nq)
    _check_q8_topk(rt, op, smallest, q, codes, scales, k)


@pytest.mark.parametrize("k", [10, 64])
def test_q8_wave_list_many_parts(rt, k):
    """One query over 300000 rows: over a thousand workgroups publish their
    lists, and the final merge walks all of them."""
    q, codes, scales = _q8_case(7 + k, 1, 300000, 128, 1)
    _check_q8_topk(rt, "dot", False, q, codes, scales, k)


@pytest.mark.parametrize("op,smallest", [("dot", False), ("dot", True), ("l2_distance", True)])
@pytest.mark.parametrize("k", [1, 10, 64])
def test_q8_wave_list_all_ties(rt, op, smallest, k):
    """Every row identical: every score ties, so the ids are the k lowest
    row indices in order."""
    n, d = 20000, 256
    q, codes, scales = _q8_case(11, 2, n, d, 2)
    codes[:] = codes[:, :1, :]
    scales[:] = scales[:, :1]
    _check_q8_topk(rt, op, smallest, q, codes, scales, k)
    cands = rt.bind_q8(codes, scales)
    ids, _, _ = _qtopk(rt, cands, op, rt.to_device(q), k, smallest=smallest)
    np.testing.assert_array_equal(ids.download(), np.tile(np.arange(k, dtype=np.int32), (2, 1)))
    cands.close()


@pytest.mark.parametrize("op", ["dot", "cosine", "l2_distance"])
@pytest.mark.parametrize("d", [32, 384])
def test_q4_score_and_topk_bit_exact(rt, op, d):
    nq, n, k = 3, 3000, 50
    q = synth.normal_f16(7, 0, nq, d, 1.0, normalize=True)
    packed, s4 = synth.q4_rows(7, 1, n, d, normalize=True)
    cands = rt.bind_q4(packed, s4, d)
    qd = rt.to_device(q)
    got = _qscore(rt, cands, op, qd).download()
    want = orc.score_q4(op, q, packed, s4, d)
    np.testing.assert_array_equal(got, want)
    smallest = op == "l2_distance"
    ids, sc, _ = _qtopk(rt, cands, op, qd, k, smallest=smallest)
    want_ids = orc.topk(want, k, smallest=smallest)
    np.testing.assert_array_equal(ids.download(), want_ids)
    np.testing.assert_array_equal(sc.download(), np.take_along_axis(want, want_ids, 1))
    cands.close()


@pytest.mark.parametrize("rows,cols,k", [(1, 4, 3), (2, 3, 2), (1, 65536, 10), (3, 100000, 1000),
                                         (7, 5000, 1), (2, 600, 600)])
@pytest.mark.parametrize("smallest", [False, True])
def test_topk_matrix_with_ties(rt, rows, cols, k, smallest):
    rng = np.random.default_rng(rows * 7919 + cols + k)
    # few distinct values -> many ties resolved by index; include -0.0 / +0.0
    vals = rng.integers(-20, 20, size=(rows, cols)).astype(np.float32) / 8.0
    vals[vals == 0] = np.where(rng.random((vals == 0).sum()) < 0.5, -0.0, 0.0)
    ids, v = rt.topk(rt.to_device(vals), k, smallest=smallest)
    want = orc.topk(vals, k, smallest=smallest)
    np.testing.assert_array_equal(ids.download(), want)
    np.testing.assert_array_equal(v.download(), np.take_along_axis(vals, want, 1))


def test_reference_topk_vectors_on_device(rt):
    for case in GOLD["topk"]:
        s = np.asarray(case["scores"], np.float32)
        s2 = s.reshape(1, -1) if s.ndim == 1 else s
        ids, _ = rt.topk(rt.to_device(s2), case["k"])
        np.testing.assert_array_equal(ids.download().reshape(np.shape(case["want"])), case["want"])


def test_errors_match_reference(rt):
    codes, scales = synth.q8_rows(1, 1, 10, 64, normalize=True)
    cands = rt.bind_q8(codes, scales)
    q = rt.to_device(synth.normal_f16(1, 0, 1, 64, 1.0, normalize=True))
    with pytest.raises(MantaRocmError, match="topk limit 11 out of range for row width 10"):
        rt.score_topk(cands, "dot", q, 11)
    with pytest.raises(MantaRocmError, match="topk limit 0 out of range"):
        rt.score_topk(cands, "dot", q, 0)
    s = rt.to_device(np.zeros((1, 4), np.float32))
    with pytest.raises(MantaRocmError, match="topk limit 5 out of range for 4 scores"):
        rt.topk(s, 5)
    per_query = rt.bind_q8(np.stack([codes, codes]), np.stack([scales, scales]))
    q3 = rt.to_device(synth.normal_f16(1, 0, 3, 64, 1.0, normalize=True))
    with pytest.raises(MantaRocmError, match="score mismatch"):
        rt.score(per_query, "dot", q3)
    cands.close()
    per_query.close()


@pytest.mark.slow
def test_config0_full_size_bit_exact(rt):
    """BASELINE config 0 at its full shape: ids, scores and int32
    accumulators bit-exact with the oracle."""
    q, codes, scales = synth.config0()
    cands = rt.bind_q8(codes[0], scales[0])
    ids, sc, acc = _qtopk(rt, cands, "dot", rt.to_device(q), 10, with_acc=True)
    want_s, want_acc = orc.score_q8("dot", q, codes[0], scales[0], with_acc=True)
    want_ids = orc.topk(want_s, 10)
    np.testing.assert_array_equal(ids.download(), want_ids)
    np.testing.assert_array_equal(sc.download(), np.take_along_axis(want_s, want_ids, 1))
    np.testing.assert_array_equal(acc.download(), np.take_along_axis(want_acc, want_ids, 1))
    assert np.all(np.abs(acc.download()) < 2 ** 31)
    cands.close()


# ---------------------------------------------------------------------------
# Many queries against one shared candidate matrix (the matrix-core path).

@pytest.mark.parametrize("op,smallest", [("dot", False), ("cosine", False), ("l2_distance", True),
                                         ("dot", True), ("l2_distance", False)])
@pytest.mark.parametrize("d", [64, 128, 256, 384, 512])
def test_multi_query_score_matrix_bit_exact(rt, op, smallest, d):
    nq, n = 37, 3000
    q, codes, scales = _q8_case(d + 1, nq, n, d, sets=1, normalize=(op != "l2_distance"))
    cands = rt.bind_q8(codes[0], scales[0])
    got = _qscore(rt, cands, op, rt.to_device(q)).download()
    want = orc.score_q8(op, q, codes[0], scales[0])
    np.testing.assert_array_equal(got, want)
    cands.close()


@pytest.mark.parametrize("op,smallest", [("dot", False), ("cosine", False), ("l2_distance", True),
                                         ("dot", True), ("l2_distance", False)])
@pytest.mark.parametrize("nq,n,d,k", [(8, 5000, 128, 10), (33, 20000, 384, 50), (16, 30000, 128, 1000),
                                      (40, 4097, 256, 100), (9, 700, 512, 700), (64, 12345, 64, 1)])
def test_multi_query_topk_bit_exact(rt, op, smallest, nq, n, d, k):
    q, codes, scales = _q8_case(nq + n + d + k, nq, n, d, sets=1, normalize=(op != "l2_distance"))
    cands = rt.bind_q8(codes[0], scales[0])
    ids, sc, acc = _qtopk(rt, cands, op, rt.to_device(q), k, smallest=smallest, with_acc=True)
    ids, sc, acc = ids.download(), sc.download(), acc.download()
    want_s, want_acc = orc.score_q8(op, q, codes[0], scales[0], with_acc=True)
    want_ids = orc.topk(want_s, k, smallest=smallest)
    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_array_equal(sc, np.take_along_axis(want_s, want_ids, 1))
    np.testing.assert_array_equal(acc, np.take_along_axis(want_acc, want_ids, 1))
    cands.close()


@pytest.mark.parametrize("op,smallest", [("dot", False), ("cosine", False), ("l2_distance", True),
                                         ("cosine", True), ("l2_distance", False)])
def test_multi_query_zero_rows_partial_group(rt, op, smallest):
    """All-zero rows (cosine's zero denominator) among normal ones, with a
    query count that leaves most of the last query group empty: the empty
    slots never append keys, and zero rows score like the oracle's."""
    nq, n, d, k = 19, 6000, 128, 40
    q, codes, scales = _q8_case(91, nq, n, d, sets=1, normalize=(op != "l2_distance"))
    codes, scales = codes[0].copy(), scales[0].copy()
    zero = np.arange(0, n, 7)
    codes[zero] = 0
    scales[zero[::2]] = 0.0
    cands = rt.bind_q8(codes, scales)
    ids, sc, _ = _qtopk(rt, cands, op, rt.to_device(q), k, smallest=smallest)
    want_s = orc.score_q8(op, q, codes, scales)
    want_ids = orc.topk(want_s, k, smallest=smallest)
    np.testing.assert_array_equal(ids.download(), want_ids)
    np.testing.assert_array_equal(sc.download(), np.take_along_axis(want_s, want_ids, 1))
    cands.close()


def test_multi_query_repeated_calls_are_identical(rt):
    """Thresholds and tickets are reset between calls: a second call with a
    smaller input reproduces the oracle too."""
    for n, nq in ((20000, 32), (5000, 8)):
        q, codes, scales = _q8_case(n, nq, n, 128, sets=1, normalize=False)
        cands = rt.bind_q8(codes[0], scales[0])
        ids, _, _ = _qtopk(rt, cands, "l2_distance", rt.to_device(q), 100, smallest=True)
        want = orc.topk(orc.score_q8("l2_distance", q, codes[0], scales[0]), 100, smallest=True)
        np.testing.assert_array_equal(ids.download(), want)
        cands.close()


def _ordered_case(op, nq, n, d, seed):
    """Every row holds the same codes; only the scale changes, so each query
    ranks the rows by index -- worst first.  Each pass's threshold then lets
    every later row through: regions fill up and are compacted inside the
    scan kernel, and the select streams more keys than its LDS buffer."""
    rng = np.random.default_rng(seed)
    base = rng.standard_normal(d)
    q = orc.f32_to_f16((base + 0.05 * rng.standard_normal((nq, d))).astype(np.float32))
    codes1, scale1 = orc.pack_q8_rows((base / np.linalg.norm(base)).astype(np.float32).reshape(1, -1))
    codes = np.repeat(codes1, n, axis=0)
    if op == "l2_distance":
        # scales below the distance minimum: distance falls with the index
        # the row is scale * codes ~ scale/scale1 * unit(base); its distance
        # to a query near base falls while scale/scale1 stays below |base|
        smax = 0.9 * scale1[0] * np.linalg.norm(base)
        scales = (smax * (np.arange(n) + 1) / n).astype(np.float32)
    else:
        scales = (scale1[0] * (1.0 + np.arange(n) / n)).astype(np.float32)
    return q, codes, scales


@pytest.mark.parametrize("op,smallest", [("dot", False), ("l2_distance", True)])
@pytest.mark.parametrize("k", [7, 100, 1000])
def test_multi_query_adversarial_row_order(rt, op, smallest, k):
    nq, n, d = 24, 300000, 128
    q, codes, scales = _ordered_case(op, nq, n, d, k)
    cands = rt.bind_q8(codes, scales)
    ids, sc, _ = _qtopk(rt, cands, op, rt.to_device(q), k, smallest=smallest)
    want_s = orc.score_q8(op, q, codes, scales)
    want_ids = orc.topk(want_s, k, smallest=smallest)
    np.testing.assert_array_equal(ids.download(), want_ids)
    np.testing.assert_array_equal(sc.download(), np.take_along_axis(want_s, want_ids, 1))
    cands.close()


@pytest.mark.parametrize("op", ["dot", "cosine", "l2_distance"])
def test_multi_query_all_ties(rt, op):
    """Identical rows: every score ties, so the lowest indices win."""
    nq, n, d, k = 16, 50000, 256, 300
    q = synth.normal_f16(5, 0, nq, d, 1.0, normalize=True)
    codes1, scale1 = synth.q8_rows(5, 1, 1, d, normalize=True)
    codes = np.repeat(codes1, n, axis=0)
    scales = np.repeat(scale1, n)
    cands = rt.bind_q8(codes, scales)
    ids, _, _ = _qtopk(rt, cands, op, rt.to_device(q), k, smallest=(op == "l2_distance"))
    want = orc.topk(orc.score_q8(op, q, codes, scales), k, smallest=(op == "l2_distance"))
    np.testing.assert_array_equal(ids.download(), want)
    np.testing.assert_array_equal(want, np.tile(np.arange(k), (nq, 1)))
    cands.close()


# ---------------------------------------------------------------------------
# q8 dot with 512 or more queries: the 512-query 16x16x64 kernel.

@pytest.mark.parametrize("smallest", [False, True])
@pytest.mark.parametrize("nq,n,d,k", [(512, 6000, 384, 50), (600, 5003, 128, 10), (1024, 4500, 256, 1),
                                      (520, 3000, 384, 300), (256, 6000, 384, 50), (300, 5003, 256, 10),
                                      (515, 3001, 128, 1500)])
def test_q8_dot_512_queries_bit_exact(rt, smallest, nq, n, d, k):
    """A full and a partial 512-query group (and 256-query groups for fewer
    than 512 queries), row counts that leave a partial last chunk; ids,
    scores and accumulators bit-exact.  515 queries with k about n/2: the
    last wave holds 3 queries, so a group of 4 slots mixes queries and empty
    slots, and the thresholds sit near 0, where an empty slot's zero scores
    would pass its neighbours' bound."""
    q, codes, scales = _q8_case(nq + n + d + k, nq, n, d, sets=1)
    cands = rt.bind_q8(codes[0], scales[0])
    ids, sc, acc = _qtopk(rt, cands, "dot", rt.to_device(q), k, smallest=smallest, with_acc=True)
    ids, sc, acc = ids.download(), sc.download(), acc.download()
    want_s, want_acc = orc.score_q8("dot", q, codes[0], scales[0], with_acc=True)
    want_ids = orc.topk(want_s, k, smallest=smallest)
    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_array_equal(sc, np.take_along_axis(want_s, want_ids, 1))
    np.testing.assert_array_equal(acc, np.take_along_axis(want_acc, want_ids, 1))
    cands.close()


@pytest.mark.parametrize("k", [7, 100])
def test_q8_dot_512_queries_adversarial_row_order(rt, k):
    """Rows ranked worst first for every query: regions fill and are
    compacted inside the 512-query kernel."""
    nq, n, d = 512, 60000, 128
    q, codes, scales = _ordered_case("dot", nq, n, d, k)
    cands = rt.bind_q8(codes, scales)
    ids, sc, _ = _qtopk(rt, cands, "dot", rt.to_device(q), k)
    want_s = orc.score_q8("dot", q, codes, scales)
    want_ids = orc.topk(want_s, k)
    np.testing.assert_array_equal(ids.download(), want_ids)
    np.testing.assert_array_equal(sc.download(), np.take_along_axis(want_s, want_ids, 1))
    cands.close()


@pytest.mark.parametrize("smallest", [False, True])
def test_q8_dot_512_queries_all_ties(rt, smallest):
    nq, n, d, k = 512, 20000, 384, 64
    q = synth.normal_f16(6, 0, nq, d, 1.0, normalize=True)
    codes1, scale1 = synth.q8_rows(6, 1, 1, d, normalize=True)
    codes = np.repeat(codes1, n, axis=0)
    scales = np.repeat(scale1, n)
    cands = rt.bind_q8(codes, scales)
    ids, _, _ = _qtopk(rt, cands, "dot", rt.to_device(q), k, smallest=smallest)
    want = orc.topk(orc.score_q8("dot", q, codes, scales), k, smallest=smallest)
    np.testing.assert_array_equal(ids.download(), want)
    np.testing.assert_array_equal(want, np.tile(np.arange(k), (nq, 1)))
    cands.close()


def test_q8_dot_512_queries_negative_scales(rt):
    """Negative row scales flip the order of a row's scores; the pre-filter
    (scale*acc against the bound) and the exact test stay consistent."""
    nq, n, d, k = 512, 3000, 128, 20
    q, codes, scales = _q8_case(77, nq, n, d, sets=1)
    scales = scales.copy()
    scales[0, ::7] *= -1.0
    cands = rt.bind_q8(codes[0], scales[0])
    ids, sc, _ = _qtopk(rt, cands, "dot", rt.to_device(q), k)
    want_s = orc.score_q8("dot", q, codes[0], scales[0])
    want_ids = orc.topk(want_s, k)
    np.testing.assert_array_equal(ids.download(), want_ids)
    np.testing.assert_array_equal(sc.download(), np.take_along_axis(want_s, want_ids, 1))
    cands.close()


# ---------------------------------------------------------------------------
# Many queries against one shared q4 matrix (the q4 matrix-core path).

def _q4_case(seed, nq, n, d, normalize=True):
    q = synth.normal_f16(200 + seed, 0, nq, d, 1.0, normalize=normalize)
    packed, s4 = synth.q4_rows(200 + seed, 1, n, d, normalize=normalize)
    return q, packed, s4


@pytest.mark.parametrize("op", ["cosine", "l2_distance", "dot"])
@pytest.mark.parametrize("d", [32, 64, 384, 512])
def test_q4_multi_query_score_matrix_bit_exact(rt, op, d):
    nq, n = 40, 3000
    q, packed, s4 = _q4_case(d, nq, n, d, normalize=(op != "l2_distance"))
    cands = rt.bind_q4(packed, s4, d)
    got = _qscore(rt, cands, op, rt.to_device(q)).download()
    np.testing.assert_array_equal(got, orc.score_q4(op, q, packed, s4, d))
    cands.close()


@pytest.mark.parametrize("op,smallest", [("cosine", False), ("l2_distance", True), ("dot", False), ("dot", True)])
@pytest.mark.parametrize("nq,n,d,k", [(8, 3000, 32, 10), (37, 5000, 128, 50), (129, 4097, 384, 100),
                                      (64, 20000, 256, 7), (16, 700, 512, 700), (9, 2000, 64, 1)])
def test_q4_multi_query_topk_bit_exact(rt, op, smallest, nq, n, d, k):
    q, packed, s4 = _q4_case(nq + n + d + k, nq, n, d, normalize=(op != "l2_distance"))
    cands = rt.bind_q4(packed, s4, d)
    ids, sc, _ = _qtopk(rt, cands, op, rt.to_device(q), k, smallest=smallest)
    want_s = orc.score_q4(op, q, packed, s4, d)
    want_ids = orc.topk(want_s, k, smallest=smallest)
    np.testing.assert_array_equal(ids.download(), want_ids)
    np.testing.assert_array_equal(sc.download(), np.take_along_axis(want_s, want_ids, 1))
    cands.close()


@pytest.mark.parametrize("k", [5, 100])
def test_q4_multi_query_adversarial_row_order(rt, k):
    """One row's nibbles repeated with block scales growing with the index
    (rounded to f16, so runs of equal scores too): every pass lets the later
    rows through, forcing region compaction and multi-round selects."""
    nq, n, d = 20, 200000, 128
    rng = np.random.default_rng(k)
    base = rng.standard_normal(d).astype(np.float32)
    q = orc.f32_to_f16((base + 0.05 * rng.standard_normal((nq, d))).reshape(nq, d).astype(np.float32))
    packed1, s1 = orc.pack_q4_blocks(base.reshape(1, -1))
    packed = np.repeat(packed1, n, axis=0)
    grow = (1.0 + np.arange(n, dtype=np.float64) / n)[:, None]
    s4 = orc.f32_to_f16((orc.f16_to_f32(s1) * grow).astype(np.float32))
    cands = rt.bind_q4(packed, s4, d)
    ids, sc, _ = _qtopk(rt, cands, "dot", rt.to_device(q), k)
    want_s = orc.score_q4("dot", q, packed, s4, d)
    want_ids = orc.topk(want_s, k)
    np.testing.assert_array_equal(ids.download(), want_ids)
    np.testing.assert_array_equal(sc.download(), np.take_along_axis(want_s, want_ids, 1))
    cands.close()


# ---------------------------------------------------------------------------
# q4 cosine / dot top-k with 256 or more queries: the int8 shadow of the q4
# matrix on the 512-query kernel, every survivor rescored with the exact q4
# score.  Results must equal the q4 contract's, bit for bit.

def _check_q4_topk(rt, cands, op, q, packed, s4, d, k, smallest=False):
    ids, sc, _ = _qtopk(rt, cands, op, rt.to_device(q), k, smallest=smallest)
    want_s = orc.score_q4(op, q, packed, s4, d)
    want_ids = orc.topk(want_s, k, smallest=smallest)
    np.testing.assert_array_equal(ids.download(), want_ids)
    np.testing.assert_array_equal(sc.download(), np.take_along_axis(want_s, want_ids, 1))
    return want_ids


@pytest.mark.parametrize("op,smallest", [("cosine", False), ("cosine", True), ("dot", False), ("dot", True)])
@pytest.mark.parametrize("nq,n,d,k", [(256, 6000, 384, 100), (300, 5003, 128, 10), (512, 4500, 256, 1),
                                      (520, 3000, 384, 300), (256, 20000, 96, 50)])
def test_q4_shadow_topk_bit_exact(rt, op, smallest, nq, n, d, k):
    """One and two wave groups per 256 queries, partial query groups and
    chunks, shadow pitches 128/256/384 (d = 96 pads to 128)."""
    q, packed, s4 = _q4_case(nq + n + d + k, nq, n, d)
    cands = rt.bind_q4(packed, s4, d)
    _check_q4_topk(rt, cands, op, q, packed, s4, d, k, smallest)
    # a second call reuses the shadow built by the first
    _check_q4_topk(rt, cands, op, q[: nq // 2 + 128], packed, s4, d, k, smallest)
    cands.close()


@pytest.mark.parametrize("op", ["cosine", "dot"])
@pytest.mark.parametrize("k", [7, 100])
def test_q4_shadow_adversarial_row_order(rt, op, k):
    """Rows ranked worst first for every query (cosine: a row turns from a
    random direction towards the queries' common direction with its index;
    dot: block scales grow with it): every pass lets the later rows through,
    so regions fill and are compacted on exact scores inside the scan."""
    nq, n, d = 256, 60000, 128
    rng = np.random.default_rng(k)
    base = rng.standard_normal(d)
    other = rng.standard_normal(d)
    q = orc.f32_to_f16((base + 0.05 * rng.standard_normal((nq, d))).astype(np.float32))
    if op == "cosine":
        w = (np.arange(n, dtype=np.float64) / n)[:, None]
        rows = (w * base[None, :] + (1.0 - w) * other[None, :]).astype(np.float32)
        packed, s4 = orc.pack_q4_blocks(rows)
    else:
        packed1, s1 = orc.pack_q4_blocks(base.astype(np.float32).reshape(1, -1))
        packed = np.repeat(packed1, n, axis=0)
        grow = (1.0 + np.arange(n, dtype=np.float64) / n)[:, None]
        s4 = orc.f32_to_f16((orc.f16_to_f32(s1) * grow).astype(np.float32))
    cands = rt.bind_q4(packed, s4, d)
    _check_q4_topk(rt, cands, op, q, packed, s4, d, k)
    cands.close()


@pytest.mark.parametrize("op,smallest", [("cosine", False), ("dot", True)])
def test_q4_shadow_all_ties_zero_rows_and_zero_query(rt, op, smallest):
    """Identical rows tie for every query (lowest indices win); all-zero
    rows and an all-zero query score 0 under the contract."""
    nq, n, d, k = 256, 20000, 384, 64
    q, _, _ = _q4_case(9, nq, 1, d)
    q = q.copy()
    q[17] = 0
    packed1, s1 = synth.q4_rows(209, 1, 1, d, normalize=True)
    packed = np.repeat(packed1, n, axis=0)
    s4 = np.repeat(s1, n, axis=0)
    packed[5::11] = 0
    s4[5::11] = 0
    cands = rt.bind_q4(packed, s4, d)
    _check_q4_topk(rt, cands, op, q, packed, s4, d, k, smallest)
    cands.close()


# ---------------------------------------------------------------------------
# After top-k: candidate ids, packed rows and scales of the selected rows
# (gather + pack_candidates of the retrieval presets), bit for bit.

@pytest.mark.parametrize("fmt,sets,d", [("q8", 1, 256), ("q8", 3, 100), ("q4", 1, 384), ("q4", 3, 64)])
def test_pack_candidates_bit_exact(rt, fmt, sets, d):
    nq, n, k = 3, 5000, 37
    rng = np.random.default_rng(d + sets)
    if fmt == "q8":
        q, codes, scales = _q8_case(d + sets, nq, n, d, sets=sets)
        codes, scales = (codes[0], scales[0]) if sets == 1 else (codes, scales)
        cands = rt.bind_q8(codes, scales)
        rows_ref, scales_ref = codes, scales[..., None]
    else:
        q = synth.normal_f16(300 + d, 0, nq, d, 1.0, normalize=True)
        packed = np.empty((sets, n, d // 2), np.uint8)
        s4 = np.empty((sets, n, d // 32), np.uint16)
        for s_ in range(sets):
            packed[s_], s4[s_] = synth.q4_rows(300 + d, 1 + s_, n, d, normalize=True)
        packed, s4 = (packed[0], s4[0]) if sets == 1 else (packed, s4)
        cands = rt.bind_q4(packed, s4, d)
        rows_ref, scales_ref = packed, s4
    cid = rng.integers(-2**62, 2**62, size=(sets, n) if sets > 1 else (n,), dtype=np.int64)
    top, _, _ = rt.score_topk(cands, "dot", rt.to_device(q), k)
    ids, rows, sc = rt.pack_candidates(cands, top, rt.to_device(cid))
    t = top.download()
    if sets == 1:
        want_ids, want_rows, want_sc = cid[t], rows_ref[t], scales_ref[t]
    else:
        qi = np.arange(nq)[:, None]
        want_ids, want_rows, want_sc = cid[qi, t], rows_ref[qi, t], scales_ref[qi, t]
    np.testing.assert_array_equal(ids.download(), want_ids)
    np.testing.assert_array_equal(rows.download(), want_rows)
    np.testing.assert_array_equal(sc.download().view(np.uint8), np.ascontiguousarray(want_sc).view(np.uint8))
    # without candidate ids: rows and scales only
    none_ids, rows2, _ = rt.pack_candidates(cands, top)
    assert none_ids is None
    np.testing.assert_array_equal(rows2.download(), want_rows)
    cands.close()


def test_pack_candidates_out_of_range_index(rt):
    nq, n, d, k = 2, 300, 128, 4
    q, codes, scales = _q8_case(7, nq, n, d, sets=1)
    cands = rt.bind_q8(codes[0], scales[0])
    top = np.array([[0, 1, 2, 3], [4, n, 5, 6]], np.int32)
    ids, rows, _ = rt.pack_candidates(cands, rt.to_device(top), rt.to_device(np.arange(n, dtype=np.int64)))
    with pytest.raises(MantaRocmError, match="gather index %d out of range" % n):
        rt.synchronize()
    got = rows.download()
    np.testing.assert_array_equal(got[1, 1], 0)  # the bad slot is zero-filled
    np.testing.assert_array_equal(got[0], codes[0][top[0]])
    cands.close()
