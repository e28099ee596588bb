"""GPU runs of artifact entry points through the step executor
(manta_rocm_program_*), against the reference's own known answers and the
CPU oracle.

Known answers (transcribed): runtime/retrieval_test.go:14-139 (packed
candidates, single and batched), runtime/inference_test.go:215-262 and
score_model_test.go:55-130 (score tables), runtime_test.go:531-586
(tiny_rerank).  Oracle parity: ids and scores bit-exact against the
reference restatements (cosineRows / dotRows / l2DistanceRows on the
dequantized values, topKTensor), gathered rows byte-exact; embed entries
bit-exact against the same device ops called one by one, and within the
GEMM's bound of the oracle.
"""
import copy
import json
import os

import numpy as np
import pytest

from manta_amd import rocm, synth
from manta_amd._lib import MantaRocmError, Unsupported
from manta_amd.module import Docs, Module, Program
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

MODS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "modules")


def fixture(name):
    with open(os.path.join(MODS, name + ".json")) as f:
        return json.load(f)


def program(rt, name_or_obj):
    obj = fixture(name_or_obj) if isinstance(name_or_obj, str) else name_or_obj
    return Program(rt, Module.from_json(json.dumps(obj)))


def f16(x):
    return orc.f32_to_f16(np.asarray(x, np.float32))


def bind_ref_values(rt, values, bits=4):
    """A reference q4 / q8 tensor (f32 values) repacked exactly (pack_grid)."""
    v = np.asarray(values, np.float32)
    lead, d = v.shape[:-1], v.shape[-1]
    codes, scales, grid = rocm.pack_grid(v.reshape(-1, d), bits)
    assert grid > 0, "values are off every grid"
    sets = 1 if v.ndim == 2 else v.shape[0]
    n = v.shape[-2]
    cands = rt.bind_q8(codes.reshape(sets, n, d) if sets > 1 else codes, scales.reshape(sets, n) if sets > 1 else scales)
    return Docs(cands, "q4" if bits == 4 else "q8", rank=v.ndim)


def with_op(obj, op):
    """The same module with its cosine builtin replaced by `op`."""
    text = json.dumps(obj).replace('"cosine', '"' + op)
    return json.loads(text)


# ---------------------------------------------------- reference known answers

@pytest.mark.parametrize("name", ["tiny_packed_candidates", "ref_packed"])
def test_packed_candidates_known_answer(rt, name):
    """retrieval_test.go:14-69: ids 1001, 3003, scores 1 and 0.70710677,
    docs [1,0] and [1,1]."""
    p = program(rt, name)
    p.supports("rerank_candidates_packed")
    out = p.run("rerank_candidates_packed", {
        "query": f16([1, 0]),
        "docs": bind_ref_values(rt, [[1, 0], [0, 1], [1, 1]]),
        "candidate_ids": np.array([1001, 2002, 3003], np.int64),
    })
    pack = out["candidates"]
    assert pack["ids"].tolist() == [1001, 3003]
    assert pack["scores"].tolist() == [1.0, np.float32(0.70710677)]
    np.testing.assert_array_equal(pack["docs"]["values"], [[1, 0], [1, 1]])
    trace = {(k, d) for k, _, d in p.trace()}
    assert ("topk", "hip:score_topk") in trace and ("launch_kernel", "fused:topk") in trace


def test_packed_candidates_batch_known_answer(rt):
    """retrieval_test.go:71-139."""
    p = program(rt, "packed_batch")
    out = p.run("rerank_candidates_packed_batch", {
        "queries": f16([[1, 0], [0, 1]]),
        "docs": bind_ref_values(rt, [[[1, 0], [0, 1], [1, 1]], [[0, 1], [1, 0], [1, 1]]]),
        "candidate_ids": np.array([[1001, 2002, 3003], [4004, 5005, 6006]], np.int64),
    })
    pack = out["result"]
    assert pack["ids"].tolist() == [[1001, 3003], [4004, 6006]]
    np.testing.assert_array_equal(pack["docs"]["values"][:, 0], [[1, 0], [0, 1]])


def test_score_bundle_known_answer(rt):
    """inference_test.go:215-262, score_model_test.go:55-130."""
    p = program(rt, "score_bundle")
    docs = [[1, 0], [0, 1], [1, 1]]
    out = p.run("score", {"query": f16([1, 0]), "docs": bind_ref_values(rt, docs)})
    assert out["scores"].tolist() == [1.0, 0.0, np.float32(0.70710677)]
    out = p.run("score_batch", {"queries": f16([[1, 0], [0, 1]]),
                                "docs": bind_ref_values(rt, [docs, [[0, 1], [1, 0], [1, 1]]])})
    np.testing.assert_array_equal(out["result"], np.float32([[1, 0, 0.70710677], [1, 0, 0.70710677]]))


def test_rerank_known_answer(rt):
    """runtime_test.go:531-586: tiny_rerank top ids [0, 2]."""
    p = program(rt, "tiny_rerank")
    p.bind("docs", bind_ref_values(rt, [[1, 0], [0, 1], [1, 1]]))
    out = p.run("rerank", {"query": f16([1, 0])})
    assert out["top_ids"].tolist() == [0, 2]
    assert out["top_scores"].tolist() == [1.0, np.float32(0.70710677)]


# ----------------------------------------------------------- oracle parity

def _ref(op, q, docs_values):
    fn = {"dot": orc.dot_rows, "cosine": orc.cosine_rows, "l2_distance": orc.l2_distance_rows}[op]
    return fn(orc.f16_to_f32(q), docs_values)


@pytest.mark.parametrize("op", ["cosine", "dot", "l2_distance"])
def test_retrieve_parity(rt, op):
    """tiny_retrieve with q4 docs (d = 64) as a param: top ids, scores and
    the gathered rows equal the reference's on the dequantized values (the
    topk over l2 distances is largest-first, as topKTensor is)."""
    n, d = 5000, 64
    packed, s4 = synth.q4_rows(31, 0, n, d, normalize=(op == "cosine"))
    q = synth.normal_f16(31, 1, 1, d, 1.0)[0]
    p = program(rt, with_op(fixture("tiny_retrieve"), op))
    p.bind("docs", Docs(rt.bind_q4(packed, s4, d), "q4"))
    out = p.run("retrieve", {"query": q})
    ref = _ref(op, q, orc.dequant_q4(packed, s4, d))
    want = orc.topk(ref, 2)
    assert out["top_ids"].tolist() == want.tolist()
    np.testing.assert_array_equal(out["top_scores"], ref[want])
    np.testing.assert_array_equal(out["top_docs"]["codes"], packed[want])
    np.testing.assert_array_equal(out["top_docs"]["scales"], s4[want])


@pytest.mark.parametrize("op", ["cosine", "l2_distance"])
def test_batch_candidates_parity(rt, op):
    """tiny_batch_candidates: one q8 candidate set per query."""
    nq, n, d = 4, 3000, 96
    codes, scales = synth.q8_rows(32, 0, nq * n, d, normalize=False)
    codes = codes.reshape(nq, n, d)
    scales = scales.reshape(nq, n)
    qs = synth.normal_f16(32, 1, nq, d, 1.0)
    ids = (np.arange(nq * n, dtype=np.int64).reshape(nq, n) * 7 + 11)
    p = program(rt, with_op(fixture("tiny_batch_candidates"), op))
    out = p.run("rerank_candidates_batch", {"queries": qs, "docs": Docs(rt.bind_q8(codes, scales), "q4"),
                                            "candidate_ids": ids})
    ref = _ref(op, qs, orc.dequant_q8(codes, scales))
    want = orc.topk(ref, 2)
    assert out["top_candidate_ids"].tolist() == np.take_along_axis(ids, want, 1).tolist()
    np.testing.assert_array_equal(out["top_scores"], np.take_along_axis(ref, want, 1))
    for i in range(nq):
        np.testing.assert_array_equal(out["top_docs"]["codes"][i], codes[i][want[i]])


def test_full_score_matrix_and_select(rt):
    """A returned score vector is materialized (not fused); select_scores
    returns only the gathered top scores (fused)."""
    n, d = 4000, 128
    codes, scales = synth.q8_rows(33, 0, n, d, normalize=True)
    q = synth.normal_f16(33, 1, 1, d, 1.0, normalize=True)[0]
    ref = _ref("cosine", q, orc.dequant_q8(codes, scales))
    docs = Docs(rt.bind_q8(codes, scales), "q4")
    p = program(rt, "tiny_score")
    p.bind("docs", docs)
    np.testing.assert_array_equal(p.run("score", {"query": q})["scores"], ref)
    assert ("launch_kernel", "cosine", "hip:cosine") in p.trace()
    s = program(rt, "tiny_select")
    s.bind("docs", docs)
    got = s.run("select_scores", {"query": q})["top_scores"]
    np.testing.assert_array_equal(got, ref[orc.topk(ref, 2)])


def test_unfused_topk_when_scores_are_returned(rt):
    """A module that returns its scores and also ranks them: the topk runs
    over the materialized matrix (ties broken by index)."""
    obj = fixture("tiny_rerank")
    obj["entry_points"][0]["outputs"].append({"name": "scores", "type": {"kind": "tensor", "tensor": {
        "dtype": "f32", "shape": ["N"]}}})
    obj["steps"][-1]["outputs"].append("scores")
    p = program(rt, obj)
    vals = np.float32([[1, 0], [0, 1], [1, 0], [0.5, 0.5], [1, 0]])
    p.bind("docs", bind_ref_values(rt, vals))
    out = p.run("rerank", {"query": f16([1, 0])})
    assert out["top_ids"].tolist() == [0, 2]
    assert ("topk", "topk", "hip:topk") in p.trace()
    np.testing.assert_array_equal(out["scores"], orc.cosine_rows(np.float32([1, 0]), vals))


def _embed_inputs(b, t, vocab, masked):
    tokens = synth.uniform_i32(34, 0, b * t, 0, vocab).reshape(b, t)
    mask = None
    if masked:
        lens = synth.uniform_i32(34, 1, b, 1, t + 1)
        mask = (np.arange(t)[None, :] < lens[:, None]).astype(np.int32)
        mask[0] = 0  # a fully masked sequence pools to zeros
    return tokens, mask


@pytest.mark.parametrize("name,masked", [("embed_masked_pooled", True), ("tiny_embed_pooled", False)])
def test_embed_pooled_batch(rt, name, masked):
    """gather -> @matmul -> normalize -> mean_pool (the examples' order):
    bit-exact with the device ops called one by one; within the GEMM bound
    of the oracle."""
    b, t, vocab, d, e = 4, 24, 500, 64, 96
    table = synth.normal_f16(35, 0, vocab, d, 0.02)
    proj = synth.normal_f16(35, 1, d, e, 1.0 / np.sqrt(d))
    tokens, mask = _embed_inputs(b, t, vocab, masked)
    p = program(rt, name)
    p.bind("token_embedding", table)
    p.bind("projection", proj)
    inputs = {"tokens": tokens}
    if masked:
        inputs["attention_mask"] = mask
    got = p.run("embed_pooled_batch", inputs)["result"]
    assert got.dtype == np.float32 and got.shape == (b, e)
    # the same device ops, one call at a time
    hidden = rt.gather_rows_f16(rt.to_device(table), rt.to_device(tokens.reshape(-1)))
    proj_d = rt.to_device(proj)
    y = rt.matmul_f16(hidden, proj_d)
    rt.normalize_rows(y)
    y3 = rocm.DeviceArray(rt, (b, t, e), np.float32)
    call_copy = y.download().reshape(b, t, e)
    y3.upload(call_copy)
    if masked:
        direct = rt.mean_pool_masked(y3, rt.to_device(mask)).download()
    else:
        direct = rt.mean_pool(y3).download()
        # meanPoolTensor's arithmetic: f32 sum in position order / float32(t)
        acc = np.zeros((b, e), np.float32)
        for i in range(t):
            acc = (acc + call_copy[:, i]).astype(np.float32)
        np.testing.assert_array_equal(direct, (acc / np.float32(t)).astype(np.float32))
    np.testing.assert_array_equal(got, direct)
    # oracle: gather, matmul (f32 loop), normalize, pool
    x = orc.gather_rows(orc.f16_to_f32(table), tokens.reshape(-1))
    yr = orc.normalize_rows(orc.matmul(x, orc.f16_to_f32(proj)))
    yr = yr.reshape(b, t, e)
    want = orc.mean_pool_masked(yr, mask if masked else np.ones((b, t), np.int32))
    assert np.max(np.abs(got - want)) < 2e-5
    if masked:
        assert np.all(got[0] == 0)


def test_embed_single_and_user_kernel(rt):
    """embed_pooled (rank-1 tokens, unmasked mean_pool of a rank-2 value)
    and tiny_embed's declared l2_normalize kernel."""
    t, vocab, d, e = 9, 300, 64, 64
    table = synth.normal_f16(36, 0, vocab, d, 0.02)
    proj = synth.normal_f16(36, 1, d, e, 1.0 / np.sqrt(d))
    tokens = synth.uniform_i32(36, 2, t, 0, vocab)
    p = program(rt, "tiny_embed_pooled")
    p.bind("token_embedding", table)
    p.bind("projection", proj)
    got = p.run("embed_pooled", {"tokens": tokens})["result"]
    x = orc.gather_rows(orc.f16_to_f32(table), tokens)
    yr = orc.normalize_rows(orc.matmul(x, orc.f16_to_f32(proj)))
    assert np.max(np.abs(got - yr.mean(0))) < 2e-5
    k = program(rt, "tiny_embed")
    k.bind("token_embedding", table)
    k.bind("projection", proj)
    emb = k.run("embed", {"tokens": tokens})["embeddings"]
    assert emb.shape == (t, e)
    assert np.max(np.abs(emb - yr)) < 2e-5
    assert ("launch_kernel", "l2_normalize", "hip:l2_normalize") in k.trace()


# ------------------------------------------------------------------ errors

def _err(fn, *a, **kw):
    with pytest.raises(MantaRocmError) as e:
        fn(*a, **kw)
    return str(e.value)


def test_request_errors(rt):
    p = program(rt, "score_bundle")
    docs = bind_ref_values(rt, [[1, 0], [0, 1]])
    assert _err(p.run, "nope", {}) == 'unknown entrypoint "nope"'
    assert _err(p.run, "score", {"docs": docs}) == 'entrypoint "score" missing input "query"'
    assert _err(p.run, "score", {"query": f16([1, 0]), "docs": docs, "extra": f16([1])}) == \
        'entrypoint "score" does not declare input "extra"'
    assert _err(p.run, "score", {"query": f16([1, 0, 0, 0]), "docs": docs}) == \
        'input "docs": symbol "D" mismatch: expected 4, got 2'
    assert _err(p.run, "score", {"query": np.array([1, 0], np.int32), "docs": docs}) == \
        'input "query": tensor dtype "i32" does not match expected "f16"'
    assert _err(p.run, "score", {"query": f16([[1, 0]]), "docs": docs}) == \
        'input "query": tensor rank 2 does not match expected rank 1'
    r = program(rt, "tiny_rerank")
    assert _err(r.run, "rerank", {"query": f16([1, 0])}) == 'missing weight binding for param "docs"'
    r.bind("docs", bind_ref_values(rt, [[1, 0]]))
    assert _err(r.run, "rerank", {"query": f16([1, 0])}) == \
        'entrypoint "rerank" step "topk": topk limit 2 out of range for 1 scores'


def test_gather_error_reports_first_position(rt):
    """gatherTensor stops at the first bad index in position order; the
    device reports the same one whatever order its threads ran in."""
    b, t, vocab, d, e = 2, 16, 100, 64, 64
    table = synth.normal_f16(37, 0, vocab, d, 0.02)
    proj = synth.normal_f16(37, 1, d, e, 0.1)
    tokens = synth.uniform_i32(37, 2, b * t, 0, vocab).reshape(b, t)
    tokens[1, 3] = 5000
    tokens[0, 9] = -3
    tokens[1, 15] = 100
    p = program(rt, "embed_masked_pooled")
    p.bind("token_embedding", table)
    p.bind("projection", proj)
    msg = _err(p.run, "embed_pooled_batch", {"tokens": tokens, "attention_mask": np.ones((b, t), np.int32)})
    assert msg == 'entrypoint "embed_pooled_batch" step "gather": gather index -3 out of range'
    # the program runs again cleanly afterwards
    tokens[tokens >= vocab] = 1
    tokens[tokens < 0] = 2
    p.run("embed_pooled_batch", {"tokens": tokens, "attention_mask": np.ones((b, t), np.int32)})


def test_return_of_unproduced_value(rt):
    """module_test.go's demo module gathers into `x` but returns
    `embeddings`, which no step produces."""
    p = program(rt, "ref_demo")
    p.bind("token_embedding", synth.normal_f16(38, 0, 10, 4, 1.0))
    assert _err(p.run, "embed", {"tokens": np.array([1, 2], np.int32)}) == \
        'entrypoint "embed" return references unknown value "embeddings"'


def test_supports_and_unsupported_steps(rt):
    for name in ["tiny_score", "tiny_rerank", "tiny_select", "tiny_retrieve", "tiny_candidates",
                 "tiny_batch_candidates", "tiny_packed_candidates", "packed_batch", "score_bundle", "tiny_embed",
                 "tiny_embed_pooled", "embed_masked_pooled", "ref_packed", "ref_demo", "encoder_trainable_q8",
                 "encoder_trainable_q8x2"]:
        p = program(rt, name)
        for en in fixture(name)["entry_points"]:
            p.supports(en["name"])
    obj = fixture("tiny_embed")
    obj["kernels"][0]["body"][0]["op"] = "rope"
    p = program(rt, obj)
    with pytest.raises(Unsupported, match='op "rope" is not offered'):
        p.supports("embed")
    obj = fixture("tiny_embed")
    obj["steps"][1]["kind"] = "kv_read"
    p = program(rt, obj)
    with pytest.raises(Unsupported, match='kind "kv_read"'):
        p.supports("embed")


def test_program_outputs_reused_across_runs(rt):
    """Repeated runs of one entry reuse their buffers and give the same
    results; a second program on the same runtime is independent."""
    n, d = 2000, 64
    packed, s4 = synth.q4_rows(39, 0, n, d, normalize=True)
    docs = Docs(rt.bind_q4(packed, s4, d), "q4")
    p = program(rt, "tiny_packed_candidates")
    ids = np.arange(n, dtype=np.int64) + 100
    first = None
    for i in range(3):
        q = synth.normal_f16(39, 1 + (i % 2), 1, d, 1.0, normalize=True)[0]
        out = p.run("rerank_candidates_packed", {"query": q, "docs": docs, "candidate_ids": ids})["candidates"]
        ref = orc.cosine_rows(orc.f16_to_f32(q), orc.dequant_q4(packed, s4, d))
        want = orc.topk(ref, 2)
        assert out["ids"].tolist() == (want + 100).tolist()
        if i == 0:
            first = out
        if i == 2:
            assert out["ids"].tolist() == first["ids"].tolist()


def test_rebind_refreshes_prepared_weight(rt):
    """A [K, N] matmul weight is copied into the GEMM's operand when it is
    bound, as the CUDA backend's resident matmul params are uploaded once at
    Load (cuda.go:129-169): a weight changed in place keeps the bound copy
    until it is bound again, and binding it again gives the new weight's
    results (those of a program that never saw the old one)."""
    b, t, vocab, d, e = 3, 16, 200, 64, 128  # K % 32 == 0, N % 128 == 0: prepared at bind
    table = synth.normal_f16(37, 0, vocab, d, 0.02)
    p1 = synth.normal_f16(37, 1, d, e, 1.0 / 8.0)
    p2 = synth.normal_f16(37, 2, d, e, 1.0 / 8.0)
    tokens = synth.uniform_i32(37, 3, b * t, 0, vocab).reshape(b, t)

    def run(p):
        return p.run("embed_pooled_batch", {"tokens": tokens})["result"]

    def fresh(proj):
        p = program(rt, "tiny_embed_pooled")
        p.bind("token_embedding", table)
        p.bind("projection", proj)
        return run(p)

    want1, want2 = fresh(p1), fresh(p2)
    assert not np.array_equal(want1, want2)
    p = program(rt, "tiny_embed_pooled")
    p.bind("token_embedding", table)
    dev = rt.to_device(p1)
    p.bind("projection", dev)
    np.testing.assert_array_equal(run(p), want1)
    dev.upload(p2)  # changed in place, not bound again: the bound copy stays
    np.testing.assert_array_equal(run(p), want1)
    p.bind("projection", dev)
    np.testing.assert_array_equal(run(p), want2)
    # the oracle agrees with the new weight's result within the GEMM's bound
    x = orc.gather_rows(orc.f16_to_f32(table), tokens.reshape(-1))
    yr = orc.normalize_rows(orc.matmul(x, orc.f16_to_f32(p2))).reshape(b, t, e)
    assert np.max(np.abs(want2 - orc.mean_pool_masked(yr, np.ones((b, t), np.int32)))) < 2e-5


def _encoder_case(seed, b, t, vocab, d, h):
    rng = np.random.default_rng(seed)
    tokens = rng.integers(0, vocab, size=(b, t), dtype=np.int32)
    lengths = rng.integers(1, t + 1, size=b)
    mask = (np.arange(t)[None, :] < lengths[:, None]).astype(np.int32)
    table = (rng.standard_normal((vocab, d)) * 0.5).astype(np.float32)
    tcodes, tscales = orc.pack_q8_rows(table)
    ws = []
    for s in [(d, d), (d, d), (d, d), (d, d), (d, h), (h, d)]:
        w = (rng.standard_normal(s) / np.sqrt(s[0])).astype(np.float32)
        cs = (np.abs(w).max(0) / 127.0).astype(np.float32)
        cs[cs == 0] = 1.0
        ws.append((np.clip(np.round(w / cs), -127, 127).astype(np.int8), cs))
    return tokens, mask, tcodes, tscales, ws


@pytest.mark.parametrize("name,layers", [("encoder_trainable_q8", 1), ("encoder_trainable_q8x2", 2)])
def test_encoder_entries_run_step_by_step(rt, name, layers):
    """The encoder examples through the executor: gather of q8 token rows,
    dequant, q/k/v GEMMs, transpose, batched attention products, softmax,
    residual add + layernorm, gelu, normalize, masked mean pool -- every step
    on device; within the encoder's bar (cosine >= 0.9999) of the oracle."""
    from manta_amd.module import Q8Columns
    b, t, vocab, d, h = 4, 12, 60, 64, 128
    tokens, mask, tcodes, tscales, ws = _encoder_case(51 + layers, b, t, vocab, d, h)
    p = program(rt, name)
    p.bind("token_embedding", Docs(rt.bind_q8(tcodes, tscales), "q8"))
    for pname, (codes, cs) in zip(["attn_q", "attn_k", "attn_v", "attn_o", "ffn_up", "projection"], ws):
        p.bind(pname, Q8Columns(codes, cs))
    p.supports("embed_pooled_batch")
    got = p.run("embed_pooled_batch", {"tokens": tokens, "attention_mask": mask})["result"]
    table = (tcodes.astype(np.float32) * tscales[:, None]).astype(np.float32)
    wf = [(c.astype(np.float32) * s[None, :]).astype(np.float32) for c, s in ws]
    want = orc.encoder_pooled(tokens, mask, table, *wf, layers=layers)
    cos = (got * want).sum(1) / (np.linalg.norm(got, axis=1) * np.linalg.norm(want, axis=1))
    assert cos.min() >= 0.9999, cos.min()
    assert np.abs(got - want).max() < 1e-3
    # the single-sequence entry on the first sequence
    one = p.run("embed_pooled", {"tokens": tokens[0], "attention_mask": mask[0]})["result"]
    np.testing.assert_allclose(one, got[0], rtol=0, atol=1e-5)
    kinds = {k for k, _, _ in p.trace()}
    assert {"transpose", "dequant", "matmul", "launch_kernel"} <= kinds
