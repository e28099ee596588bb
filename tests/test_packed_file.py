"""Packed candidate containers (include/manta_mll.h, manta_mll_write_packed /
manta_mll_packed_info): real int8 / nibble candidate rows on disk in the MLL
container, in place of the reference's f32-widened q4/q8 tensors
(runtime/mll_export.go:858-862, runtime/weight_file.go:304-367).  Host only.

Pins: the section bytes round-trip bit for bit against the oracle's packers
(oracle/oracle.py pack_q8_rows / pack_q4_blocks); every written container opens
under the reader whose table, STRG, HEAD and BLAKE3 digests are pinned by the
reference's example containers (tests/test_mll.py); the data sections start on
4 KiB pages; corrupted bytes and mismatched metadata fail with named errors.
"""
import os

import numpy as np
import pytest

from manta_amd import mll, synth
from manta_amd._lib import MantaRocmError
from oracle import oracle as orc

GOLD = os.path.join(os.path.dirname(__file__), "golden", "mll")


def _rows(seed, n, d):
    x = synth.normal_f32(seed, 0, n, d, 1.0, normalize=True)
    x[n // 2] = 0.0  # an all-zero row: scale 0
    return x


@pytest.mark.parametrize("dtype", ["q8", "q4"])
@pytest.mark.parametrize("with_ids", [False, True])
@pytest.mark.parametrize("n,d", [(1, 32), (300, 96), (1000, 384)])
def test_round_trip_bit_exact(tmp_path, dtype, with_ids, n, d):
    x = _rows(n + d, n, d)
    codes, scales = orc.pack_q8_rows(x) if dtype == "q8" else orc.pack_q4_blocks(x)
    ids = (np.arange(n, dtype=np.int64) * 1_000_003 - 5) if with_ids else None
    p = tmp_path / "docs.mll"
    mll.write_packed(p, codes, scales, ids=ids, name="docs")
    data = p.read_bytes()
    with mll.MllFile(data, verify=True) as m:
        tags = [s[0] for s in m.sections]
        assert tags == ["HEAD", "STRG", "QCOD", "QSCL"] + (["QIDS"] if with_ids else [])
        for tag, off, size, flags, digest in m.sections:
            assert mll.blake3(data[off:off + size]) == digest
            if tag.startswith("Q"):
                assert off % 4096 == 0 and flags == 0x10011
        name, desc, _ = m.head()
        assert name == "docs" and desc == "Manta packed candidates"
        got = m.packed()
    assert got["dtype"] == dtype and got["rows"] == n and got["dim"] == d
    np.testing.assert_array_equal(got["codes"], codes)
    np.testing.assert_array_equal(got["scales"].view(np.uint32 if dtype == "q8" else np.uint16),
                                  scales.view(np.uint32 if dtype == "q8" else np.uint16))
    if with_ids:
        np.testing.assert_array_equal(got["ids"], ids)
    else:
        assert got["ids"] is None
    # bytes on disk: 1 byte per q8 value / half a byte per q4 value, not 4
    val_bytes = n * d if dtype == "q8" else n * d // 2
    assert [s[2] for s in mll.MllFile(data).sections][2] == val_bytes


def test_manifest_read_as_authored_manifest(tmp_path):
    x = _rows(3, 64, 64)
    c, s = orc.pack_q8_rows(x)
    p = tmp_path / "a.mll"
    mll.write_packed(p, c, s)
    doc = mll.read_authored_manifest(str(p), "packed_candidates", "manta/packed-candidates/v0")
    assert doc["values"]["rows"] == (mll.I64, 64) and doc["values"]["docs_dtype"] == (mll.STRING, "q8")
    assert doc["values"]["has_ids"] == (mll.BOOL, False)


def at_rows(body):
    """Offset of the rows value (the i64 40) in a HEAD section body."""
    return body.index((40).to_bytes(8, "little"))


def test_errors(tmp_path):
    x = _rows(4, 40, 64)
    c, s = orc.pack_q8_rows(x)
    p = tmp_path / "b.mll"
    mll.write_packed(p, c, s)
    data = bytearray(p.read_bytes())
    qcod = [t for t in mll.MllFile(bytes(data)).sections if t[0] == "QCOD"][0]
    bad = bytearray(data)
    bad[qcod[1] + 17] ^= 0x40
    with pytest.raises(MantaRocmError, match="QCOD digest mismatch"):
        mll.MllFile(bytes(bad))
    # HEAD says more rows than the sections hold (opened without verification)
    head = [t for t in mll.MllFile(bytes(data)).sections if t[0] == "HEAD"][0]
    body = bytes(data[head[1]:head[1] + head[2]])
    at = body.index((40).to_bytes(8, "little"))
    bad = bytearray(data)
    bad[head[1] + at] = 41
    with mll.MllFile(bytes(bad), verify=False) as m:
        with pytest.raises(MantaRocmError, match="QCOD section is 2560 bytes, want 2624"):
            m.packed()
    # a HEAD string value naming a string id past the string table, and a
    # row count whose section sizes would wrap 64 bits (opened without
    # verification: a crafted file can carry matching digests)
    entries, at = [], 30
    for _ in range(body[28] | body[29] << 8):
        kind = body[at + 4]
        width = {1: 1, 2: 8, 3: 8, 4: 4}[kind]
        entries.append((at + 5, kind, width))
        at += 5 + width
    s_at = [e for e in entries if e[1] == 4][0][0]
    bad = bytearray(data)
    bad[head[1] + s_at:head[1] + s_at + 4] = (100000).to_bytes(4, "little")
    with mll.MllFile(bytes(bad), verify=False) as m:
        with pytest.raises(MantaRocmError, match="names string 100000"):
            m.packed()
    bad = bytearray(data)
    bad[head[1] + at_rows(body):head[1] + at_rows(body) + 8] = (2 ** 62 + 40).to_bytes(8, "little")
    with mll.MllFile(bytes(bad), verify=False) as m:
        with pytest.raises(MantaRocmError, match="bad shape"):
            m.packed()
    # a manifest of another kind
    with mll.MllFile(os.path.join(GOLD, "score_bundle.score.mll")) as m:
        with pytest.raises(MantaRocmError, match='manifest kind "score_manifest", want "packed_candidates"'):
            m.packed()
    with pytest.raises(ValueError, match="int8"):
        mll.write_packed(p, c.astype(np.int16), s)
    with pytest.raises(ValueError, match="scales shape"):
        mll.write_packed(p, c, s[:-1])
    with pytest.raises(MantaRocmError, match="bad shape"):
        mll.write_packed(p, np.zeros((4, 8), np.uint8), np.zeros((4, 0), np.uint16))
