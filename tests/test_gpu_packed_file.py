"""Candidates bound from a packed container (manta_rocm_bind_packed) score
exactly as candidates bound from the same arrays and as the oracle: the
container's QCOD / QSCL bytes reach the device unchanged (bit-exact reference
scores and ids)."""
import numpy as np
import pytest

from manta_amd import mll, synth
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", ["q8", "q4"])
@pytest.mark.parametrize("op", ["dot", "cosine", "l2_distance"])
def test_bind_packed_matches_arrays_and_oracle(rt, tmp_path, dtype, op):
    n, d, nq, k = 5000, 128, 4, 25
    print("bind_packed", dtype, op, n, d, flush=True)
    x = synth.normal_f32(77, 0, n, d, 1.0, normalize=(op != "l2_distance"))
    x[123] = 0.0
    q = synth.normal_f16(78, 0, nq, d, 1.0, normalize=(op != "l2_distance"))
    codes, scales = orc.pack_q8_rows(x) if dtype == "q8" else orc.pack_q4_blocks(x)
    p = tmp_path / "cands.mll"
    mll.write_packed(p, codes, scales, ids=np.arange(n, dtype=np.int64) + 10**12)
    qd = rt.to_device(q)
    with mll.MllFile(p, verify=True) as m:
        from_file = rt.bind_packed(m)
    from_arrays = rt.bind_q8(codes, scales) if dtype == "q8" else rt.bind_q4(codes, scales, d)
    assert (from_file.n, from_file.d) == (n, d)
    got = rt.score(from_file, op, qd).download()
    np.testing.assert_array_equal(got, rt.score(from_arrays, op, qd).download())
    want = (orc.ref_score_q8(op, q, codes, scales) if dtype == "q8" else orc.ref_score_q4(op, q, codes, scales, d))
    np.testing.assert_array_equal(got, want)
    ids, sc, _ = rt.score_topk(from_file, op, qd, k, smallest=(op == "l2_distance"))
    oids = orc.topk(want, k, smallest=(op == "l2_distance"))
    np.testing.assert_array_equal(ids.download(), oids)
    from_file.close()
    from_arrays.close()
