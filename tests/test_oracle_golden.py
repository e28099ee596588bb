"""Pin the CPU oracle to the reference's own known-answer tests.

Vectors are data transcribed from the Go tests (each entry cites its
file:line) in tests/golden/reference_known_answers.json.  The reference
checks them with assertTensorClose, 5e-4 absolute; ids are exact.
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle as orc

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))
TOL = GOLD["tol"]


def close(got, want):
    np.testing.assert_allclose(np.asarray(got, np.float64), np.asarray(want, np.float64), rtol=0, atol=TOL)


@pytest.mark.parametrize("case", GOLD["gather"], ids=lambda c: c["cite"])
def test_gather(case):
    close(orc.gather_rows(case["table"], case["idx"]), case["want"])


@pytest.mark.parametrize("case", GOLD["gather_rank1"], ids=lambda c: c["cite"])
def test_gather_rank1(case):
    table = np.asarray(case["table"], np.float32).reshape(-1, 1)
    close(orc.gather_rows(table, case["idx"]).reshape(-1), case["want"])


@pytest.mark.parametrize("case", GOLD["matmul"], ids=lambda c: c["cite"])
def test_matmul(case):
    close(orc.matmul(case["lhs"], case["rhs"]), case["want"])


@pytest.mark.parametrize("case", GOLD["normalize"], ids=lambda c: c["cite"])
def test_normalize(case):
    close(orc.normalize_rows(case["x"]), case["want"])


@pytest.mark.parametrize("case", GOLD["mean_pool_masked"], ids=lambda c: c["cite"])
def test_mean_pool_masked(case):
    close(orc.mean_pool_masked(case["x"], case["mask"]), case["want"])


@pytest.mark.parametrize("case", GOLD["mean_pool_unmasked"], ids=lambda c: c["cite"])
def test_mean_pool_all_ones_mask(case):
    x = np.asarray(case["x"], np.float32)
    close(orc.mean_pool_masked(x, np.ones(x.shape[:2], np.int32)), case["want"])


@pytest.mark.parametrize("op,fn", [("dot", orc.dot_rows), ("cosine", orc.cosine_rows),
                                   ("l2_distance", orc.l2_distance_rows)])
def test_score_rows(op, fn):
    for case in GOLD[op]:
        close(fn(case["q"], case["docs"]), case["want"])


@pytest.mark.parametrize("case", GOLD["topk"], ids=lambda c: c["cite"])
def test_topk(case):
    got = orc.topk(case["scores"], case["k"])
    np.testing.assert_array_equal(got, np.asarray(case["want"], np.int32))


def test_topk_errors_match_reference_wording():
    # tensor_ops.go:1532-1534 and :1560-1562
    with pytest.raises(orc.OracleError, match="topk limit 5 out of range for 4 scores"):
        orc.topk([1, 2, 3, 4], 5)
    with pytest.raises(orc.OracleError, match="topk limit 0 out of range for row width 3"):
        orc.topk([[1, 2, 3], [4, 5, 6]], 0)


def test_gather_out_of_range_error():
    # tensor_ops.go:804-806 wording
    with pytest.raises(orc.OracleError, match="gather index 3 out of range"):
        orc.gather_rows([[1.0], [2.0], [3.0]], [0, 3])
    with pytest.raises(orc.OracleError, match="gather index -1 out of range"):
        orc.gather_rows([[1.0], [2.0], [3.0]], [-1])


@pytest.mark.parametrize("case", GOLD["score_runtime"], ids=lambda c: c["cite"])
def test_packed_contract_on_runtime_vectors(case):
    """The packed q8 and q4 scoring contract reproduces the reference's
    runtime-level answers (5e-4) on the same tiny inputs."""
    q = orc.f32_to_f16(np.asarray(case["q"], np.float32).reshape(1, -1))
    docs = np.asarray(case["docs"], np.float32)
    codes, scales = orc.pack_q8_rows(docs)
    got8 = orc.score_q8(case["op"], q, codes, scales)[0]
    # q4 needs d % 32 == 0: zero-pad columns (zeros add nothing to any op)
    d = 32
    qp = np.zeros((1, d), np.uint16)
    qp[:, : q.shape[1]] = q
    dp = np.zeros((docs.shape[0], d), np.float32)
    dp[:, : docs.shape[1]] = docs
    packed, s4 = orc.pack_q4_blocks(dp)
    got4 = orc.score_q4(case["op"], qp, packed, s4, d)[0]
    if "want" in case:
        close(got8, case["want"])
        close(got4, case["want"])
    else:
        for got in (got8, got4):
            ids = orc.topk(got, case["topk"])
            np.testing.assert_array_equal(ids, case["want_ids"])
            close(got[ids], case["want_scores"])
