"""The C-ABI library loads on a CPU-only host and exports every entry point
include/*.h declares (no compute calls without a GPU)."""
import ctypes as C
import glob
import os
import re

import numpy as np
import pytest

from manta_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared_symbols():
    syms = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        syms |= set(re.findall(r"\b(manta_(?:rocm|mll|module|manifest)_\w+)\s*\(", text))
    return sorted(syms)


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "manta_rocm_score_topk" in syms and "manta_rocm_embed_pooled" in syms
    assert "manta_mll_open" in syms and "manta_mll_blake3" in syms
    assert len(syms) >= 35


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_python_signatures_cover_header():
    assert set(declared_symbols()) == set(_lib.SIGNATURES)


def test_abi_version_and_device_count_without_gpu():
    lib = _lib.load()
    assert lib.manta_rocm_abi_version() == 2
    n = C.c_int(-1)
    err = C.c_char_p()
    rc = lib.manta_rocm_device_count(C.byref(n), C.byref(err))
    assert rc in (0, 1)
    assert n.value >= 0


def test_pack_entry_points_are_host_only_and_match_oracle():
    import numpy as np
    from manta_amd import rocm, synth
    from oracle import oracle as orc

    x = synth.normal_f32(5, 0, 257, 96, 1.0, normalize=True)
    x[3] = 0.0
    c8, s8 = rocm.pack_q8_rows(x)
    oc8, os8 = orc.pack_q8_rows(x)
    np.testing.assert_array_equal(c8, oc8)
    np.testing.assert_array_equal(s8, os8)
    p4, s4 = rocm.pack_q4_blocks(x)
    op4, os4 = orc.pack_q4_blocks(x)
    np.testing.assert_array_equal(p4, op4)
    np.testing.assert_array_equal(s4, os4)
    with pytest.raises(_lib.MantaRocmError, match="multiple of 32"):
        rocm.pack_q4_blocks(x[:, :40])


def test_create_without_device_reports_unsupported():
    from manta_amd import rocm

    if rocm.device_count() > 0:
        pytest.skip("a device is present")
    with pytest.raises(_lib.Unsupported, match="no ROCm device"):
        rocm.Runtime(0)


def test_encoder_wrapper_validates_before_the_abi():
    """encoder_pooled hands raw device pointers to the C ABI, which cannot
    check them: the wrapper rejects mistyped or mis-shaped tokens, mask and
    token scales first (stand-ins carry only shape and dtype; no device)."""
    from types import SimpleNamespace as A

    from manta_amd import rocm

    def arr(shape, dtype):
        return A(shape=shape, dtype=np.dtype(dtype), addr=0, ptr=None)

    b, t, vocab, d, h = 2, 4, 10, 32, 64
    good = dict(tokens=arr((b, t), np.int32), mask=arr((b, t), np.int32), token_codes=arr((vocab, d), np.int8),
                token_scales=arr((vocab,), np.float32),
                weights=[(arr(s, np.int8), arr((s[1],), np.float32))
                         for s in [(d, d), (d, d), (d, d), (d, d), (d, h), (h, d)]])
    bad_cases = [
        ("tokens", arr((b, t), np.int64), "tokens must be int32"),
        ("mask", arr((b, t - 1), np.int32), "mask must be int32"),
        ("mask", arr((b, t), np.int8), "mask must be int32"),
        ("token_scales", arr((vocab - 1,), np.float32), "token scales must be f32"),
        ("token_codes", arr((vocab, d), np.uint8), "token codes must be int8"),
    ]
    for key, value, msg in bad_cases:
        kw = dict(good)
        kw[key] = value
        with pytest.raises(ValueError, match=msg):
            rocm.Runtime.encoder_pooled(None, kw["tokens"], kw["mask"], kw["token_codes"], kw["token_scales"],
                                        kw["weights"])
