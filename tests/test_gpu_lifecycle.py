"""Handle lifetimes across the C-ABI: candidate sets unbound after their
runtime was destroyed (the order a garbage collector may choose) free only
their handles; a runtime destroyed with sets still bound releases their
device memory."""
import numpy as np
import pytest

from manta_amd import rocm, synth

pytestmark = pytest.mark.gpu


def test_unbind_after_runtime_destroyed():
    print("lifecycle: unbind after destroy", flush=True)
    codes, scales = synth.q8_rows(41, 0, 5000, 128)
    packed, s4 = synth.q4_rows(41, 1, 3000, 128)
    rt = rocm.Runtime(0)
    a = rt.bind_q8(codes, scales)
    b = rt.bind_q4(packed, s4, 128)
    c = rt.bind_q8(codes, scales)
    c.close()  # unbound while the runtime lives
    rt.close()
    a.close()  # after the runtime: the handle alone
    b.close()
    # a new runtime works as before
    with rocm.Runtime(0) as rt2:
        d = rt2.bind_q8(codes, scales)
        q = rt2.to_device(synth.normal_f16(41, 2, 2, 128, 1.0))
        ids, _, _ = rt2.score_topk(d, "dot", q, 5, quantized=True)
        assert ids.download().shape == (2, 5)
        assert rt2.stats()["candidate_bytes"] > 0
        d.close()
        assert rt2.stats()["candidate_bytes"] == 0
