"""GPU parity of the dense retrieval scorer (dotRetrievalVectors +
topRetrievalScores, runtime/retrieval_eval.go:586-661) with the oracle: f32
scores bit-exact, the ranking (score desc, doc ID asc) identical, with exact
ties, f16 storage, queries shorter and longer than the vectors, and k from 1
to every doc."""
import numpy as np
import pytest

from manta_amd import synth
from manta_amd._lib import MantaRocmError
from manta_amd.retrieval import DenseRetrievalIndex
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _ids(n, seed):
    rng = np.random.default_rng(seed)
    return ["doc%d" % int(x) for x in rng.permutation(n)]


@pytest.mark.parametrize("n,d,nq,k", [(20000, 384, 5, 100), (3000, 96, 3, 10), (777, 40, 2, 777), (50, 7, 3, 1)])
def test_dense_topk_matches_oracle(rt, n, d, nq, k):
    docs = synth.normal_f32(41, 0, n, d, 1.0, normalize=True)
    docs[n // 2: n // 2 + 5] = docs[3]  # exact ties, broken by id
    ids = _ids(n, 41)
    qs = synth.normal_f32(41, 1, nq, d, 1.0, normalize=True)
    qs[0] = docs[3]
    index = DenseRetrievalIndex(rt, docs, ids)
    got = index.top(qs, k)
    allscores = index.scores(qs)
    for i in range(nq):
        pos, sc = orc.top_retrieval_scores(qs[i], docs, ids, k)
        assert [g[0] for g in got[i]] == [ids[p] for p in pos]
        assert [g[1] for g in got[i]] == sc.tolist()
        np.testing.assert_array_equal(allscores[i], orc.dot_rows(qs[i], docs))


def test_f16_storage_and_mismatched_lengths(rt):
    n, d = 5000, 64
    docs16 = synth.normal_f16(42, 0, n, d, 1.0)
    docs = orc.f16_to_f32(docs16)
    ids = _ids(n, 42)
    index32 = DenseRetrievalIndex(rt, docs, ids)
    index16 = DenseRetrievalIndex(rt, docs, ids, f16=True)
    for qd in (d, d - 5, d + 9):
        q = synth.normal_f32(42, qd, 2, qd, 1.0)
        a = index32.top(q, 50)
        b = index16.top(q, 50)
        assert a == b
        for i in range(2):
            pos, sc = orc.top_retrieval_scores(q[i], docs, ids, 50)
            assert [x[0] for x in a[i]] == [ids[p] for p in pos]
            assert [x[1] for x in a[i]] == sc.tolist()


def test_every_doc_and_errors(rt):
    n, d = 300, 16
    docs = synth.normal_f32(43, 0, n, d, 1.0)
    ids = _ids(n, 43)
    index = DenseRetrievalIndex(rt, docs, ids)
    q = synth.normal_f32(43, 1, 1, d, 1.0)
    for k in (0, -1, n + 5):
        got = index.top(q, k)[0]
        pos, sc = orc.top_retrieval_scores(q[0], docs, ids, k)
        assert [x[0] for x in got] == [ids[p] for p in pos]
    with pytest.raises(MantaRocmError, match="topk limit 0 out of range"):
        rt.dense_topk(index.rows, rt.to_device(q), 0)
