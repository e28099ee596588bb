"""The oracle's topRetrievalScores restatement (runtime/retrieval_eval.go:
586-661), pinned by the reference's own retrieval-eval tests and by
independent checks: a plain sort by (score desc, id asc) over scores from a
separate f32 loop, ties broken by id bytewise, the min(len) dot, and the
"k <= 0 or k > n means every doc" rule."""
import numpy as np

from manta_amd import synth
from oracle import oracle as orc


def _normalize(v):
    v = np.asarray(v, np.float64)
    return (v / np.sqrt((v * v).sum())).astype(np.float32)


def test_bounded_top_k_known_answer():
    """retrieval_eval_test.go:40-72: docs d000..d119 scored 200-i against
    [1]; the top 100 are d000..d099 in order (recall@100 of {d000, d009,
    d099, d100} is 0.75)."""
    docs = np.array([[200 - i] for i in range(120)], np.float32)
    ids = ["d%03d" % i for i in range(120)]
    pos, sc = orc.top_retrieval_scores(np.float32([1]), docs, ids, 100)
    assert [ids[p] for p in pos] == ["d%03d" % i for i in range(100)]
    assert sc.tolist() == [float(200 - i) for i in range(100)]
    assert len({"d000", "d009", "d099", "d100"} & {ids[p] for p in pos}) == 3


def test_perfect_ranking_known_answer():
    """retrieval_eval_test.go:16-38: q1 ranks d1 first, q2 ranks d2 first."""
    docs = np.stack([_normalize([1, 0]), _normalize([0, 1]), _normalize([0.2, 0.1])])
    ids = ["d1", "d2", "d3"]
    for q, want in ((_normalize([1, 0]), "d1"), (_normalize([0, 1]), "d2")):
        pos, _ = orc.top_retrieval_scores(q, docs, ids, 100)
        assert ids[pos[0]] == want and len(pos) == 3


def _f32_dot(q, d):
    s = np.float32(0)
    for a, b in zip(q, d):
        s = np.float32(s + np.float32(a * b))
    return s


def test_matches_a_plain_sort_with_id_ties():
    rng = np.random.default_rng(3)
    n, d = 300, 12
    docs = synth.normal_f32(3, 0, n, d, 1.0)
    docs[50:60] = docs[7]  # ten exact ties with doc 7
    ids = ["doc%d" % int(x) for x in rng.permutation(n)]  # "doc10" < "doc9" bytewise
    q = synth.normal_f32(3, 1, 1, d, 1.0)[0]
    scores = [_f32_dot(q, docs[i]) for i in range(n)]
    want = sorted(range(n), key=lambda i: (-scores[i], ids[i]))
    for k in (1, 7, 20, 300, 0, -3, 1000):
        pos, sc = orc.top_retrieval_scores(q, docs, ids, k)
        kk = n if k <= 0 or k > n else k
        assert pos.tolist() == want[:kk]
        assert sc.tolist() == [float(scores[i]) for i in want[:kk]]


def test_dot_over_the_shorter_length():
    docs = np.float32([[1, 2, 3], [3, 2, 1]])
    pos, sc = orc.top_retrieval_scores(np.float32([1, 0]), docs, ["a", "b"], 2)
    assert pos.tolist() == [1, 0] and sc.tolist() == [3.0, 1.0]
    pos, sc = orc.top_retrieval_scores(np.float32([0, 0, 1, 5]), docs, ["a", "b"], 2)
    assert pos.tolist() == [0, 1] and sc.tolist() == [3.0, 1.0]


def test_planted_tie_break_by_position_fails():
    """The check has teeth: breaking ties by position instead of id gives a
    different order on this data."""
    docs = np.float32([[1], [1], [1]])
    ids = ["z", "a", "m"]
    pos, _ = orc.top_retrieval_scores(np.float32([1]), docs, ids, 3)
    assert pos.tolist() == [1, 2, 0]
    assert pos.tolist() != [0, 1, 2]
