"""Native MLL reader (include/manta_mll.h) against the reference's example
containers and the BLAKE3 specification (host only, no GPU).

Pins:
* BLAKE3: the specification's test vectors (the BLAKE3 repository's
  test_vectors.json, input byte i = i % 251): the empty input, one block,
  exactly one chunk and the first two-chunk tree.
* Container layout and digests: the five examples/*.mll files written by the
  Go runtime (copied as data under tests/golden/mll); opening them with
  digest verification reproduces all 40 stored section digests.
* HEAD / STRG decoding: the manifests' values against the reference's own
  sources -- the writer's kind, version and description constants
  (runtime/score_model.go:11,54; embedding_model.go:13,78;
  retrieval_model.go:11,55) and the entry and param names the example
  programs declare (examples/score_bundle.manta:1,5;
  examples/encoder_trainable_q8.manta:1-9,37; examples/packed_candidates.manta:1).
* HEAD f64 values (kind 3, in no example): IEEE 754 binary64 little-endian,
  bit for bit, on entries rewritten with chosen bit patterns.
* Error behaviour of readAuthoredManifestMLL
  (runtime/authored_manifest_mll.go:197-270).
"""
import os

import pytest

from manta_amd import mll
from manta_amd._lib import MantaRocmError

GOLD = os.path.join(os.path.dirname(__file__), "golden", "mll")
FILES = sorted(f for f in os.listdir(GOLD) if f.endswith(".mll"))
TAGS = ["HEAD", "STRG", "DIMS", "TYPE", "PARM", "ENTR", "TNSR", "SCHM"]


def _pattern(n):
    return bytes(i % 251 for i in range(n))


@pytest.mark.parametrize("n,want", [
    (0, "af1349b9f5f9a1a6a0404dea36dcc9499bcb25c9adc112b7cc9a93cae41f3262"),
    (1, "2d3adedff11b61f14c886e35afa036736dcd87a74d27b5c1510225d0f592e213"),
    (1024, "42214739f095a406f3fc83deb889744ac00df831c10daa55189b5d121c855af7"),
    (1025, "d00278ae47eb27b34faecf67b4fe263f82d5412916c1ffd97c8cb7fb814b8444"),
])
def test_blake3_specification_vectors(n, want):
    assert mll.blake3(_pattern(n)).hex() == want


def test_blake3_tree_is_consistent_across_chunk_counts():
    # digests of growing prefixes are all distinct and stable across calls
    # (a chunk-counter or tree-shape error shows up as a collision or a change)
    seen = {}
    for n in (1023, 2048, 2049, 3072, 4097, 8193, 16384, 31745):
        d = mll.blake3(_pattern(n))
        assert d == mll.blake3(_pattern(n))
        assert d not in seen.values()
        seen[n] = d


@pytest.mark.parametrize("name", FILES)
def test_examples_open_with_digest_verification(name):
    data = open(os.path.join(GOLD, name), "rb").read()
    with mll.MllFile(data, verify=True) as m:
        secs = m.sections
        assert [s[0] for s in secs] == TAGS
        assert m.format_word == 0x00010100
        for tag, off, size, flags, digest in secs:
            body = m.section(tag)
            assert len(body) == size and data[off:off + size] == body
            assert mll.blake3(body) == digest
        # the tensor directory starts on a 4 KiB page; the empty tables hold a zero count
        assert [s for s in secs if s[0] == "TNSR"][0][1] % 4096 == 0
        for tag in ("DIMS", "TYPE", "PARM", "ENTR", "SCHM"):
            assert m.section(tag) == b"\0\0\0\0"


def test_score_manifest_values():
    doc = mll.read_authored_manifest(os.path.join(GOLD, "score_bundle.score.mll"), "score_manifest",
                                     "manta/score-manifest/v0alpha1")
    assert doc["name"] == "score_bundle" and doc["description"] == "Manta score manifest"
    v = {k: val for k, (kind, val) in doc["values"].items()}
    assert all(kind == mll.STRING for kind, _ in doc["values"].values())
    assert v["entry"] == "score" and v["batch_entry"] == "score_batch"
    assert v["query_input"] == "query" and v["batch_query_input"] == "queries" and v["docs_input"] == "docs"
    assert v["query_dtype"] == "f16" and v["docs_dtype"] == "q4" and v["output_dtype"] == "f32"


def test_retrieval_manifest_values():
    doc = mll.read_authored_manifest(os.path.join(GOLD, "packed_candidates.retrieval.mll"),
                                     "retrieval_manifest", "manta/retrieval-manifest/v0alpha1")
    assert doc["description"] == "Manta retrieval manifest"
    v = {k: val for k, (kind, val) in doc["values"].items()}
    assert v["entry"] == "rerank_candidates_packed"
    assert v["docs_dtype"] == "q4" and v["candidate_ids_dtype"] == "i64" and v["query_dtype"] == "f16"
    assert v["candidate_ids_input"] == "candidate_ids" and v["output_name"] == "candidates"
    assert v["batch_entry"] == ""  # unset strings are stored as string 0


@pytest.mark.parametrize("name,repeats,attn", [("embed_masked_pooled.embedding.mll", 0, ""),
                                               ("encoder_trainable_q8.embedding.mll", 0, "attn_q"),
                                               ("encoder_trainable_q8x2.embedding.mll", 2, "attn_q")])
def test_embedding_manifest_values(name, repeats, attn):
    doc = mll.read_authored_manifest(os.path.join(GOLD, name), "embedding_manifest",
                                     "manta/embedding-manifest/v0alpha1")
    assert doc["description"] == "Manta embedding manifest"
    vals = doc["values"]
    assert vals["encoder_repeats"] == (mll.I64, repeats)
    assert vals["attention_query_param"] == (mll.STRING, attn)
    assert vals["pooled_entry"] == (mll.STRING, "embed_pooled")
    assert vals["batch_entry"] == (mll.STRING, "embed_pooled_batch")
    assert vals["token_embedding_param"] == (mll.STRING, "token_embedding")
    assert vals["projection_param"] == (mll.STRING, "projection")
    assert vals["attention_layernorm"][0] == mll.BOOL
    assert vals["attention_layernorm"][1] == (attn != "")
    if attn:
        assert vals["hidden_projection_param"] == (mll.STRING, "ffn_up")
        assert vals["attention_output_param"] == (mll.STRING, "attn_o")


def test_errors_follow_the_reference_reader():
    data = open(os.path.join(GOLD, "score_bundle.score.mll"), "rb").read()
    with pytest.raises(MantaRocmError, match="not an MLL manifest"):
        mll.MllFile(b"MLX\0" + data[4:])
    with pytest.raises(MantaRocmError, match="header says"):
        mll.MllFile(data[:-1])
    # one flipped byte inside the string table
    strg = [s for s in mll.MllFile(data).sections if s[0] == "STRG"][0]
    bad = bytearray(data)
    bad[strg[1] + 20] ^= 0x01
    with pytest.raises(MantaRocmError, match="STRG digest mismatch"):
        mll.MllFile(bytes(bad))
    mll.MllFile(bytes(bad), verify=False).close()  # without verification it opens
    with pytest.raises(MantaRocmError, match='manifest kind "score_manifest", want "embedding_manifest"'):
        mll.read_authored_manifest(data, "embedding_manifest")
    with pytest.raises(MantaRocmError, match="manifest version"):
        mll.read_authored_manifest(data, "score_manifest", "manta/score-manifest/v9")


# HEAD values of kind 3 (f64, authoredFloat) occur in no example container, so
# their decoding is pinned by IEEE 754 binary64 itself: an I64 entry of a
# container written here is rewritten into kind 3 holding chosen bit patterns,
# and each must decode to the double those 8 little-endian bytes are
# (struct '<d'), bit for bit.  A big-endian read, a read as an integer
# converted to double, or a narrowing through f32 fails one of them.
F64_PATTERNS = [1.0, -2.5, -0.0, 5e-324, 2.2250738585072014e-308, 1.7976931348623157e308,
                float("inf"), float("-inf"), 3.141592653589793, 1.0000000000000002, 0.1]


def _head_entries(head: bytes):
    """(offset of the kind byte, kind) of every HEAD entry: 30 header bytes
    with the entry count at 28, then key u32, kind u8 and a 1, 8, 8 or 4
    byte value (bool, i64, f64, string id)."""
    count = head[28] | head[29] << 8
    at, out = 30, []
    for _ in range(count):
        kind = head[at + 4]
        out.append((at + 4, kind))
        at += 5 + {1: 1, 2: 8, 3: 8, 4: 4}[kind]
    return out


@pytest.mark.parametrize("x", F64_PATTERNS + ["nan"])
def test_head_f64_values_decode_as_little_endian_binary64(tmp_path, x):
    import struct
    import numpy as np
    p = tmp_path / "f.mll"
    mll.write_packed(p, np.zeros((2, 32), np.int8), np.ones(2, np.float32), name="f")
    data = bytearray(open(p, "rb").read())
    with mll.MllFile(bytes(data)) as f:
        head = f.section("HEAD")
    base = bytes(data).index(head)
    ents = _head_entries(head)
    at, kind = next((a, k) for a, k in ents if k == mll.I64)
    raw = struct.pack("<Q", 0x7FF8000000000123) if x == "nan" else struct.pack("<d", x)
    data[base + at] = mll.F64
    data[base + at + 1:base + at + 9] = raw
    with mll.MllFile(bytes(data), verify=False) as f:
        _, _, entries = f.head()
    i = [a for a, _ in ents].index(at)
    name, k, got = entries[i]
    assert k == mll.F64
    assert struct.pack("<d", got) == raw
