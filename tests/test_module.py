"""The artifact codec, Validate and the serving-contract checks (CPU only).

Fixtures: tests/golden/modules/*.json are the example programs and compiler
presets lowered by the compiler's rules (make_modules.py) plus the modules
the reference's own tests build (artifact/manta/module_test.go); the
authored manifests tests/golden/mll/*.mll are the reference's example
containers.  Expected messages are the reference's (module.go:255-477,
score_model.go:276-324, retrieval_model.go:274-330, embedding_model.go:
617-847), and the manifest cases are the reference's own load tests
(score_model_test.go:39-53, retrieval_model_test.go:39-53).
"""
import copy
import glob
import json
import os
import struct

import pytest

from manta_amd import mll
from manta_amd._lib import MantaRocmError
from manta_amd.module import Module

HERE = os.path.dirname(os.path.abspath(__file__))
MODS = os.path.join(HERE, "golden", "modules")
MLLS = os.path.join(HERE, "golden", "mll")


def fixture(name):
    with open(os.path.join(MODS, name + ".json")) as f:
        return json.load(f)


def decode(obj):
    return Module.from_json(json.dumps(obj))


def decode_error(obj_or_text):
    text = obj_or_text if isinstance(obj_or_text, str) else json.dumps(obj_or_text)
    with pytest.raises(MantaRocmError) as e:
        Module.from_json(text)
    return str(e.value)


VALID = [os.path.basename(p)[:-5] for p in sorted(glob.glob(os.path.join(MODS, "*.json")))
         if not os.path.basename(p).startswith("ref_bad")]


@pytest.mark.parametrize("name", VALID)
def test_fixture_decodes_and_encodes_byte_for_byte(name):
    """The fixtures are written in MarshalIndent's layout (Go field order,
    omitempty, sorted map keys): re-encoding reproduces the file."""
    with open(os.path.join(MODS, name + ".json")) as f:
        text = f.read()
    m = Module.from_json(text)
    assert m.to_json() + "\n" == text


@pytest.mark.parametrize("name", VALID)
def test_mll_container_round_trip(name):
    m = decode(fixture(name))
    data = m.to_mll()
    assert data[:4] == b"MLL\0"
    with mll.MllFile(data) as f:
        tags = [s[0] for s in f.sections]
        assert tags == ["HEAD", "STRG", "DIMS", "TYPE", "PARM", "ENTR", "TNSR", "SCHM", "XMTA"]
        hname, desc, entries = f.head()
        assert hname == fixture(name)["name"] and desc == "Manta module artifact"
        keys = {k: v for k, _, v in entries}
        assert keys["artifact_version"] == "manta/v0alpha1"
        assert keys["entry_count"] == len(fixture(name)["entry_points"])
    back = Module.from_mll(data)
    assert json.loads(back.to_json()) == json.loads(m.to_json())


def test_reference_test_modules():
    """module_test.go: the `bad` and `bad-kernel` modules fail Validate, the
    `demo` and `packed` ones pass."""
    assert decode_error(fixture("ref_bad")) == 'step "" references unknown entrypoint "missing"'
    assert decode_error(fixture("ref_bad_kernel")) == \
        'kernel "embed_kernel" variant source is required for backend "metal"'
    decode(fixture("ref_demo"))
    decode(fixture("ref_packed"))


def mutate(fn, base="tiny_packed_candidates"):
    m = copy.deepcopy(fixture(base))
    fn(m)
    return decode_error(m)


def test_validate_messages_module_level():
    assert mutate(lambda m: m.update(name="")) == "module name is required"
    assert mutate(lambda m: m.update(version="")) == "module version is required"
    assert mutate(lambda m: m.update(version="manta/v9")) == \
        'module version "manta/v9" is not supported, want "manta/v0alpha1"'
    assert mutate(lambda m: m["requirements"].update(supported_backends=[])) == \
        "at least one supported backend is required"
    assert mutate(lambda m: m["requirements"].update(supported_backends=None)) == \
        "at least one supported backend is required"
    assert mutate(lambda m: m["requirements"].update(supported_backends=["cuda", ""])) == \
        "supported backend is required"
    assert mutate(lambda m: m["requirements"].update(supported_backends=["cuda", "cuda"])) == \
        'duplicate supported backend "cuda"'
    assert mutate(lambda m: m["requirements"].update(capabilities=[""])) == "capability name is required"
    assert mutate(lambda m: m["requirements"].update(capabilities=["a", "a"])) == 'duplicate capability "a"'


def test_validate_messages_params_entries_buffers():
    assert mutate(lambda m: m["params"][0].update(name=""), "tiny_score") == "param name is required"
    assert mutate(lambda m: m["params"][0].update(binding=""), "tiny_score") == 'param "docs" binding is required'
    assert mutate(lambda m: m["params"][0]["type"].update(kind=""), "tiny_score") == \
        'param "docs": value kind is required'
    assert mutate(lambda m: m["params"][0]["type"].update(kind="blob"), "tiny_score") == \
        'param "docs": unsupported value kind "blob"'
    assert mutate(lambda m: m["params"][0]["type"].pop("tensor"), "tiny_score") == \
        'param "docs": tensor metadata is required'
    assert mutate(lambda m: m["entry_points"][0].update(name="")) == "entrypoint name is required"
    assert mutate(lambda m: m["entry_points"][0]["inputs"][0].update(name="")) == \
        'entrypoint "rerank_candidates_packed" input name is required'
    assert mutate(lambda m: m["entry_points"][0]["inputs"][0]["type"]["tensor"].update(dtype="")) == \
        'entrypoint "rerank_candidates_packed" input "query": tensor dtype is required'
    assert mutate(lambda m: m["entry_points"][0]["outputs"][0].update(name="")) == \
        'entrypoint "rerank_candidates_packed" output name is required'
    assert mutate(lambda m: m["entry_points"][0]["outputs"][0]["type"]["candidate_pack"].update(shape=["K"])) == \
        'entrypoint "rerank_candidates_packed" output "candidates": candidate pack shape rank must be 2 or 3'
    assert mutate(lambda m: m["entry_points"][0]["outputs"][0]["type"].pop("candidate_pack")) == \
        'entrypoint "rerank_candidates_packed" output "candidates": candidate pack metadata is required'
    assert mutate(lambda m: m["buffers"][0].update(name="")) == "buffer name is required"
    assert mutate(lambda m: m["buffers"][0].update(dtype="")) == 'buffer "query" dtype is required'


def test_validate_messages_kernels():
    k = lambda m: m["kernels"][0]
    assert mutate(lambda m: k(m).update(name="")) == "kernel name is required"
    assert mutate(lambda m: k(m)["inputs"][0].update(name="")) == 'kernel "cosine" input name is required'
    assert mutate(lambda m: k(m)["outputs"][0]["type"].update(kind="")) == \
        'kernel "cosine" output "result": value kind is required'
    assert mutate(lambda m: k(m)["body"][0].update(op="")) == 'kernel "cosine" has body op with empty op name'
    assert mutate(lambda m: k(m)["variants"][1].update(backend="")) == 'kernel "cosine" variant backend is required'
    assert mutate(lambda m: k(m)["variants"][1].update(backend="cuda")) == \
        'kernel "cosine" has duplicate variant for backend "cuda"'
    assert mutate(lambda m: k(m)["variants"][1].update(entry="")) == \
        'kernel "cosine" variant entry is required for backend "metal"'
    assert mutate(lambda m: k(m).update(variants=k(m)["variants"][:4])) == \
        'kernel "cosine" is missing variant for backend "webgpu"'


def test_validate_messages_steps():
    s = lambda m, i: m["steps"][i]
    assert mutate(lambda m: s(m, 0).update(entry="")) == 'step "cosine" entry is required'
    assert mutate(lambda m: s(m, 0).update(entry="nope")) == 'step "cosine" references unknown entrypoint "nope"'
    assert mutate(lambda m: s(m, 0).update(kernel="")) == 'launch_kernel step "cosine" is missing kernel name'
    assert mutate(lambda m: s(m, 0).update(kernel="dot")) == 'step "cosine" references unknown kernel "dot"'
    assert mutate(lambda m: s(m, 1).update(inputs=[""])) == 'step "topk" has empty input name'
    # a value used before the step that produces it
    assert mutate(lambda m: s(m, 1).update(inputs=["top_docs"])) == 'step "topk" references unknown input "top_docs"'
    assert mutate(lambda m: s(m, 1).update(outputs=[""])) == 'step "topk" has empty output name'
    assert mutate(lambda m: s(m, 1).update(outputs=["unlisted"])) == \
        'step "topk" output "unlisted" is missing a declared buffer'
    assert mutate(lambda m: s(m, 6).update(outputs=["scores"])) == \
        'return step "" output "scores" is not declared on entrypoint "rerank_candidates_packed"'
    # params are known to every entry; inputs of another entry are not
    m = copy.deepcopy(fixture("packed_batch"))
    m["steps"][7]["inputs"] = ["query", "docs"]  # the batch entry's cosine
    assert decode_error(m) == 'step "cosine" references unknown input "query"'


def test_json_errors():
    assert decode_error("") == "unexpected end of JSON input"
    assert decode_error('{"name": "x"') == "unexpected end of JSON input"
    assert decode_error("x") == "invalid character 'x' looking for beginning of value"
    assert decode_error('{"name" "x"}') == "invalid character '\"' after object key"
    assert decode_error('{"name": "x",}') == "invalid character '}' looking for beginning of object key string"
    assert decode_error('{"name": "x"} 1') == "invalid character '1' after top-level value"
    assert decode_error('[1,2') == "unexpected end of JSON input"
    assert decode_error('{"name": tru}') == "invalid character '}' in literal true (expecting 'e')"
    assert decode_error('{"name": 3}') == \
        "json: cannot unmarshal number into Go struct field Module.name of type string"
    m = fixture("tiny_score")
    m["entry_points"][0]["inputs"][0]["name"] = 7
    assert decode_error(m) == \
        "json: cannot unmarshal number into Go struct field Module.entry_points.inputs.name of type string"
    m = fixture("tiny_score")
    m["kernels"][0]["hints"]["vector_width"] = 1.5
    assert decode_error(m) == \
        "json: cannot unmarshal number 1.5 into Go struct field Module.kernels.hints.vector_width of type int"
    assert decode_error("[]") == "json: cannot unmarshal array into Go value of type manta.Module"


def test_json_decoding_rules():
    """Unknown keys ignored, null leaves a field unset, keys match without
    regard to case, the last of repeated keys wins, escapes decode."""
    m = fixture("tiny_score")
    m["unknown_field"] = {"x": [1, 2]}
    m["steps"][0]["attributes"] = None
    text = json.dumps(m).replace('"binding"', '"BINDING"', 1)
    text = text.replace('"name": "tiny_score"', '"name": "first", "name": "tiny\\u005fscore"', 1)
    got = json.loads(Module.from_json(text).to_json())
    assert got["name"] == "tiny_score"
    assert got["params"][0]["binding"] == "weights/docs"
    assert "unknown_field" not in got
    # an exact key followed by a case-folded one: Unmarshal assigns both to
    # the field in document order, so the folded one (last) wins
    text = json.dumps(fixture("tiny_score")).replace('"name": "tiny_score"',
                                                     '"name": "tiny_score", "NAME": "renamed"', 1)
    assert json.loads(Module.from_json(text).to_json())["name"] == "renamed"
    text = json.dumps(fixture("tiny_score")).replace('"name": "tiny_score"',
                                                     '"NAME": "renamed", "name": "tiny_score"', 1)
    assert json.loads(Module.from_json(text).to_json())["name"] == "tiny_score"
    # Go's HTML-safe escaping on output
    m = fixture("ref_demo")
    m["kernels"][0]["variants"][0]["source"] = "a<b>&c "
    out = Module.from_json(json.dumps(m)).to_json()
    assert '"a\\u003cb\\u003e\\u0026c\\u2028"' in out
    assert json.loads(out)["kernels"][0]["variants"][0]["source"] == "a<b>&c "


def build_container(sections):
    """MLL bytes from (tag, body, flags) sections, with BLAKE3-256 digests
    (the layout include/manta_mll.h documents)."""
    at = 24 + 64 * len(sections)
    offs = []
    for tag, body, flags in sections:
        if flags & 0x10:
            at = (at + 4095) & ~4095
        offs.append(at)
        at += len(body)
    head = b"MLL\0" + struct.pack("<IQQ", 0x00010100, at, len(sections))
    for (tag, body, flags), off in zip(sections, offs):
        head += tag.encode() + struct.pack("<QQ", off, len(body)) + mll.blake3(body) + struct.pack("<IQ", flags, 0)
    out = bytearray(head)
    for (tag, body, flags), off in zip(sections, offs):
        out += b"\0" * (off - len(out)) + body
    return bytes(out)


def meta_container(meta: dict) -> bytes:
    return build_container([("XMTA", json.dumps(meta).encode(), 0x10000)])


def decode_mll_error(data):
    with pytest.raises(MantaRocmError) as e:
        Module.from_mll(data)
    return str(e.value)


def test_mll_decode_errors():
    """DecodeMLL (mll.go:291-305) and MLLMetadata.Validate (mll.go:53-88).
    The reference's example containers are manifests without an XMTA
    section: DecodeMLL refuses them with its own message."""
    for path in sorted(glob.glob(os.path.join(MLLS, "*.mll"))):
        assert decode_mll_error(path) == "mll artifact missing XMTA metadata section"
    art = fixture("tiny_score")
    good = {"version": "manta/mll/v0alpha1", "module_name": "tiny_score", "module_version": "manta/v0alpha1",
            "artifact": art}
    assert Module.from_mll(meta_container(good)).name == "tiny_score"
    assert decode_mll_error(meta_container(dict(good, version=""))) == "MLL metadata version is required"
    assert decode_mll_error(meta_container(dict(good, version="v2"))) == \
        'MLL metadata version "v2" is not supported, want "manta/mll/v0alpha1"'
    assert decode_mll_error(meta_container(dict(good, module_name=""))) == "MLL metadata module_name is required"
    assert decode_mll_error(meta_container(dict(good, module_version=""))) == \
        "MLL metadata module_version is required"
    nometa = dict(good)
    del nometa["artifact"]
    assert decode_mll_error(meta_container(nometa)) == "MLL metadata artifact must be valid JSON"
    assert decode_mll_error(meta_container(dict(good, json_files={"": {}}))) == \
        "MLL metadata json_files role is required"
    assert decode_mll_error(meta_container(dict(good, logical_tensor_dtypes={"w": ""}))) == \
        'MLL metadata logical tensor dtype for "w" is required'
    bad_art = copy.deepcopy(art)
    bad_art["name"] = ""
    assert decode_mll_error(meta_container(dict(good, artifact=bad_art))) == "module name is required"
    # digests are verified
    data = bytearray(meta_container(good))
    data[-3] ^= 1
    assert "digest mismatch" in decode_mll_error(bytes(data))


# ------------------------------------------------------- serving contracts

def test_authored_manifests_against_modules():
    """The reference's example manifests validate against the modules of the
    programs they describe, and reject the reference tests' mismatches."""
    ok = [("score_bundle", "score_bundle.score.mll"),
          ("tiny_packed_candidates", "packed_candidates.retrieval.mll"),
          ("packed_batch", "packed_candidates.retrieval.mll"),
          ("embed_masked_pooled", "embed_masked_pooled.embedding.mll")]
    for mod, man in ok:
        decode(fixture(mod)).validate_manifest(os.path.join(MLLS, man))
    bad = [("tiny_embed", "score_bundle.score.mll", 'unknown entrypoint "score"'),
           ("tiny_score", "packed_candidates.retrieval.mll", 'unknown entrypoint "rerank_candidates_packed"'),
           ("embed_masked_pooled", "encoder_trainable_q8.embedding.mll", 'missing param "attn_q"'),
           ("tiny_embed_pooled", "embed_masked_pooled.embedding.mll",
            'entrypoint "embed_pooled" does not declare input "attention_mask"'),
           ("tiny_score", "score_bundle.score.mll", 'entrypoint "score" does not declare input "docs"')]
    for mod, man, want in bad:
        with pytest.raises(MantaRocmError) as e:
            decode(fixture(mod)).validate_manifest(os.path.join(MLLS, man))
        assert str(e.value) == want


def test_score_entry_checks():
    m = decode(fixture("score_bundle"))
    m.validate_score_entry("score", "query", 1, "docs", 2, "f16", "q4", "scores", 1, "f32")
    m.validate_score_entry("score_batch", "queries", 2, "docs", 3, "f16", "q4", "result", 2, "f32")

    def err(*a):
        with pytest.raises(MantaRocmError) as e:
            m.validate_score_entry(*a)
        return str(e.value)
    assert err("nope", "query", 1, "docs", 2) == 'unknown entrypoint "nope"'
    assert err("score", "q", 1, "docs", 2) == 'entrypoint "score" does not declare input "q"'
    assert err("score", "query", 1, "docs", 2, "f32") == 'entrypoint "score" input "query" dtype = "f16", want "f32"'
    assert err("score", "query", 2, "docs", 2) == 'entrypoint "score" input "query" rank = 1, want 2'
    assert err("score", "query", 1, "docs", 2, "f16", "q8") == \
        'entrypoint "score" input "docs" dtype = "q4", want "q8"'
    assert err("score", "query", 1, "docs", 3) == 'entrypoint "score" input "docs" rank = 2, want 3'
    assert err("score", "query", 1, "docs", 2, "", "", "out") == \
        'entrypoint "score" output "scores" does not match manifest "out"'
    assert err("score", "query", 1, "docs", 2, "", "", "", 1, "f16") == \
        'entrypoint "score" output dtype = "f32", want "f16"'
    assert err("score", "query", 1, "docs", 2, "", "", "", 2) == 'entrypoint "score" output rank = 1, want 2'
    r = decode(fixture("tiny_rerank"))
    with pytest.raises(MantaRocmError) as e:
        r.validate_score_entry("rerank", "query", 1, "docs", 2)
    assert str(e.value) == 'entrypoint "rerank" does not declare input "docs"'
    p = decode(fixture("tiny_packed_candidates"))
    with pytest.raises(MantaRocmError) as e:
        p.validate_score_entry("rerank_candidates_packed", "query", 1, "docs", 2)
    assert str(e.value) == 'entrypoint "rerank_candidates_packed" output "candidates" is not a tensor'


def test_retrieval_entry_checks():
    m = decode(fixture("packed_batch"))
    m.validate_retrieval_entry("rerank_candidates_packed", "query", 1, "docs", 2, "candidate_ids", 1, "f16", "q4",
                               "i64", "candidates", 2)
    m.validate_retrieval_entry("rerank_candidates_packed_batch", "queries", 2, "docs", 3, "candidate_ids", 2,
                               "f16", "q4", "i64", "result", 3)

    def err(*a):
        with pytest.raises(MantaRocmError) as e:
            m.validate_retrieval_entry(*a)
        return str(e.value)
    assert err("rerank_candidates_packed", "query", 1, "docs", 2, "candidate_ids", 1, "", "", "i32") == \
        'entrypoint "rerank_candidates_packed" input "candidate_ids" dtype = "i64", want "i32"'
    assert err("rerank_candidates_packed", "query", 1, "docs", 2, "candidate_ids", 1, "", "", "", "", 3) == \
        'entrypoint "rerank_candidates_packed" candidate_pack rank = 2, want 3'
    c = decode(fixture("tiny_candidates"))
    with pytest.raises(MantaRocmError) as e:
        c.validate_retrieval_entry("rerank_candidates", "query", 1, "docs", 2, "candidate_ids", 1)
    assert str(e.value) == 'entrypoint "rerank_candidates" output count = 3, want 1'
    s = decode(fixture("score_bundle"))
    with pytest.raises(MantaRocmError) as e:
        s.validate_retrieval_entry("score", "query", 1, "docs", 2, "docs", 2)
    assert str(e.value) == 'entrypoint "score" output "scores" is not a candidate_pack'


def test_embedding_entry_checks():
    m = decode(fixture("embed_masked_pooled"))
    m.validate_embedding_entry("embed_pooled", "tokens", "attention_mask", 1, 1, "f16")
    m.validate_embedding_entry("embed_pooled_batch", "tokens", "attention_mask", 2, 2, "f16")
    m.validate_embedding_param("token_embedding")
    m.validate_embedding_param("")

    def err(fn, *a):
        with pytest.raises(MantaRocmError) as e:
            fn(*a)
        return str(e.value)
    assert err(m.validate_embedding_entry, "embed_pooled", "tokens", "attention_mask", 2, 1, "f16") == \
        'entrypoint "embed_pooled" input "tokens" rank = 1, want 2'
    assert err(m.validate_embedding_entry, "embed_pooled", "tokens", "attention_mask", 1, 1, "f32") == \
        'entrypoint "embed_pooled" output dtype = "f16", want "f32"'
    assert err(m.validate_embedding_param, "missing") == 'missing param "missing"'
    bad = fixture("embed_masked_pooled")
    bad["entry_points"][0]["inputs"][0]["type"]["tensor"]["dtype"] = "i64"
    bad["buffers"][0]["dtype"] = "i64"
    assert err(decode(bad).validate_embedding_entry, "embed_pooled", "tokens", "", 1, 1, "") == \
        'entrypoint "embed_pooled" input "tokens" dtype = "i64", want i32'
    three = fixture("embed_masked_pooled")
    three["params"][1]["type"]["tensor"]["shape"] = ["D", "E", "X"]
    assert err(decode(three).validate_embedding_param, "projection") == 'param "projection" rank = 3, want 2'
