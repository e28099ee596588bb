"""GPU parity of the batched retrieval configs at their full BASELINE shapes.

The fused path (threshold passes, region compaction, select, and for the
reference scores the finish) runs on the whole candidate matrix.  C2 and C3
score with the reference's cosineRows / l2DistanceRows (the default); C4's
dot is BASELINE's quantized-query formula.  Checked per config:
* every query's ids are distinct, in range, and ordered by (score, id) in the
  requested direction (the deterministic tie-break);
* the fused ids and scores equal those of an independent device route: the
  full score matrix (`manta_rocm_score`) followed by the score-matrix top-k
  (`manta_rocm_topk`), for every query;
* for two queries, ids and scores are bit-exact with the CPU oracle scoring
  the whole matrix.
Each test moves 0.2-1.6 GB of candidates; the oracle part scores 2 queries.
"""
import numpy as np
import pytest

from manta_amd import synth
from oracle import oracle as orc

pytestmark = [pytest.mark.gpu, pytest.mark.slow]


def _check_order(ids, sc, n, smallest):
    assert ids.min() >= 0 and ids.max() < n
    for r in range(ids.shape[0]):
        assert len(np.unique(ids[r])) == ids.shape[1]
    # (score, id) order: scores monotone, equal scores by ascending id
    ds = np.diff(sc, axis=1)
    assert np.all(ds >= 0) if smallest else np.all(ds <= 0)
    tie = ds == 0
    assert np.all(np.diff(ids, axis=1)[tie] > 0)


def _check_against_matrix(rt, cands, op, qd, k, smallest, ids, sc, quantized=False):
    full = rt.score(cands, op, qd, quantized=quantized)
    mids, mvals = rt.topk(full, k, smallest=smallest)
    np.testing.assert_array_equal(ids, mids.download())
    np.testing.assert_array_equal(sc, mvals.download())
    full.free()


def test_config3_full_size(rt):
    """q8 l2_distance smallest-1000, 32 queries x 8,388,608 x 128."""
    q, codes, scales = synth.config3()
    k = 1000
    cands = rt.bind_q8(codes, scales)
    qd = rt.to_device(q)
    ids, sc, _ = rt.score_topk(cands, "l2_distance", qd, k, smallest=True)
    ids, sc = ids.download(), sc.download()
    _check_order(ids, sc, codes.shape[0], True)
    _check_against_matrix(rt, cands, "l2_distance", qd, k, True, ids, sc)
    for r in (0, q.shape[0] - 1):
        want_s = orc.ref_score_q8("l2_distance", q[r:r + 1], codes, scales)
        want_ids = orc.topk(want_s, k, smallest=True)
        np.testing.assert_array_equal(ids[r:r + 1], want_ids)
        np.testing.assert_array_equal(sc[r:r + 1], np.take_along_axis(want_s, want_ids, 1))
    cands.close()


def test_config2_full_size(rt):
    """q4 cosine top-100, 256 queries x 1,048,576 x 384 (the int8 shadow scan
    with exact q4 rescoring, then the reference finish)."""
    q, packed, scales = synth.config2()
    d, k = q.shape[1], 100
    cands = rt.bind_q4(packed, scales, d)
    qd = rt.to_device(q)
    ids, sc, _ = rt.score_topk(cands, "cosine", qd, k)
    ids, sc = ids.download(), sc.download()
    _check_order(ids, sc, packed.shape[0], False)
    _check_against_matrix(rt, cands, "cosine", qd, k, False, ids, sc)
    for r in (0, q.shape[0] - 1):
        want_s = orc.ref_score_q4("cosine", q[r:r + 1], packed, scales, d)
        want_ids = orc.topk(want_s, k)
        np.testing.assert_array_equal(ids[r:r + 1], want_ids)
        np.testing.assert_array_equal(sc[r:r + 1], np.take_along_axis(want_s, want_ids, 1))
    cands.close()


def test_config4_full_size(rt):
    """Embed 1024 queries (q8 projection), then q8 dot top-50 over
    4,194,304 x 384 with the embeddings as queries, scored with BASELINE's
    quantized-query formula.  The embeddings are checked against the oracle's
    gather -> matmul -> mean_pool -> normalize over all 1024 sequences."""
    tokens, mask, table, pcodes, cs, codes, scales = synth.config4()
    k = 50
    emb = rt.embed_pooled(rt.to_device(tokens), rt.to_device(mask), rt.to_device(table),
                          rt.to_device(pcodes), col_scale=rt.to_device(cs))
    q = emb.download()
    _, want32 = orc.embed(tokens, mask, table, proj_codes=pcodes, col_scale=cs)
    got32 = orc.f16_to_f32(q).astype(np.float64)
    w = want32.astype(np.float64)
    cos = (got32 * w).sum(1) / (np.linalg.norm(got32, axis=1) * np.linalg.norm(w, axis=1))
    assert cos.min() >= 0.9999, cos.min()
    cands = rt.bind_q8(codes, scales)
    ids, sc, _ = rt.score_topk(cands, "dot", emb, k, quantized=True)
    ids, sc = ids.download(), sc.download()
    _check_order(ids, sc, codes.shape[0], False)
    _check_against_matrix(rt, cands, "dot", emb, k, False, ids, sc, quantized=True)
    for r in (0, q.shape[0] - 1):
        want_s = orc.score_q8("dot", q[r:r + 1], codes, scales)
        want_ids = orc.topk(want_s, k)
        np.testing.assert_array_equal(ids[r:r + 1], want_ids)
        np.testing.assert_array_equal(sc[r:r + 1], np.take_along_axis(want_s, want_ids, 1))
    cands.close()
