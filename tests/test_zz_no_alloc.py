"""The allocation-free entry point (manta_rocm_score_topk_noalloc) against
manta_rocm_score_topk: ids, scores and accumulators bit-exact, on two calls
in a row with the second smaller, in a fresh runtime whose workspace the
allocation-free calls never grow; a call past the scratch limit is refused
and the next call still matches."""
import numpy as np
import pytest

from manta_amd import rocm, synth
from manta_amd._lib import Unsupported
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _case(seed, nq, n, d, sets, normalize=True):
    q = synth.normal_f16(700 + seed, 0, nq, d, 1.0, normalize=normalize)
    codes = np.empty((sets, n, d), np.int8)
    scales = np.empty((sets, n), np.float32)
    for s in range(sets):
        codes[s], scales[s] = synth.q8_rows(700 + seed, 1 + s, n, d, normalize=normalize)
    if sets == 1:
        return q, codes[0], scales[0]
    return q, codes, scales


@pytest.mark.parametrize("op,quantized,smallest", [("dot", True, False), ("cosine", False, False),
                                                   ("l2_distance", False, True), ("dot", False, False)])
def test_noalloc_matches_score_topk_on_two_calls(op, quantized, smallest):
    print("noalloc", op, quantized, smallest, flush=True)
    with rocm.Runtime(0) as rt:
        first = True
        for seed, nq, n, d, sets, k in ((1, 6, 50000, 256, 1, 40), (2, 3, 7000, 128, 3, 10)):
            q, codes, scales = _case(seed, nq, n, d, sets, normalize=(op != "l2_distance"))
            cands = rt.bind_q8(codes, scales)
            qd = rt.to_device(q)
            out = (rt.empty((nq, k), np.int32), rt.empty((nq, k), np.float32),
                   rt.empty((nq, k), np.int64) if quantized else None)
            before = rt.stats()["workspace_bytes"]
            rt.score_topk_noalloc(cands, op, qd, k, out, smallest=smallest, quantized=quantized)
            rt.synchronize()
            assert rt.stats()["workspace_bytes"] == before
            if first:
                assert before == 0  # a fresh runtime: nothing was ever allocated for scoring
            ids, sc, acc = rt.score_topk(cands, op, qd, k, smallest=smallest, quantized=quantized,
                                         with_acc=quantized)
            np.testing.assert_array_equal(out[0].download(), ids.download())
            np.testing.assert_array_equal(out[1].download(), sc.download())
            if quantized:
                np.testing.assert_array_equal(out[2].download(), acc.download())
            want = (orc.score_q8(op, q, codes, scales) if quantized else orc.ref_score_q8(op, q, codes, scales))
            np.testing.assert_array_equal(out[0].download(), orc.topk(want, k, smallest=smallest))
            cands.close()
            first = False


def test_noalloc_refuses_a_call_past_its_scratch_and_recovers():
    print("noalloc limit", flush=True)
    with rocm.Runtime(0) as rt:
        nq, n, d, k = 64, 20000, 64, 2048
        q, codes, scales = _case(3, nq, n, d, 1)
        cands = rt.bind_q8(codes, scales)
        qd = rt.to_device(q)
        out = (rt.empty((nq, k), np.int32), rt.empty((nq, k), np.float32), None)
        with pytest.raises(Unsupported, match="scratch"):
            rt.score_topk_noalloc(cands, "cosine", qd, k, out)
        small = rt.to_device(q[:2])
        out2 = (rt.empty((2, 30), np.int32), rt.empty((2, 30), np.float32), None)
        rt.score_topk_noalloc(cands, "cosine", small, 30, out2)
        ids, sc, _ = rt.score_topk(cands, "cosine", small, 30)
        np.testing.assert_array_equal(out2[0].download(), ids.download())
        np.testing.assert_array_equal(out2[1].download(), sc.download())
        cands.close()


def test_noalloc_checks_output_shapes_before_the_call():
    print("noalloc output checks", flush=True)
    with rocm.Runtime(0) as rt:
        q, codes, scales = _case(4, 3, 3000, 64, 1)
        cands = rt.bind_q8(codes, scales)
        qd = rt.to_device(q)
        for out in ((rt.empty((3, 9), np.int32), None, None),           # k too small
                    (rt.empty((2, 10), np.int32), None, None),          # too few queries
                    (rt.empty((3, 10), np.int64), None, None),          # wrong element size
                    (rt.empty((3, 10), np.int32), rt.empty((3, 10), np.float64), None),
                    (rt.empty((3, 10), np.int32), None, rt.empty((3, 10), np.int32)),
                    (None, None, None)):
            with pytest.raises(ValueError, match="score_topk_noalloc"):
                rt.score_topk_noalloc(cands, "dot", qd, 10, out, quantized=True)
        out = (rt.empty((3, 10), np.int32), None, None)
        rt.score_topk_noalloc(cands, "dot", qd, 10, out, quantized=True)
        ids, _, _ = rt.score_topk(cands, "dot", qd, 10, quantized=True)
        np.testing.assert_array_equal(out[0].download(), ids.download())
        cands.close()
