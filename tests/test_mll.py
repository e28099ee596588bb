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
