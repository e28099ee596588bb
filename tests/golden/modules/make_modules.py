"""Write the module (artifact) fixtures of the step-executor tests.

There is no Go toolchain here, so the reference compiler cannot build the
example programs.  This script lowers each example the way the compiler's
rules state -- restated from compiler/compiler.go (inferCallPlan 1627-1819,
lowerStmtToPlan 1542-1585, bufferForValue 2095-2116, synthesizeBuiltinKernel
2278-2300, kernelOpForCall 2249-2276, scheduleHintsForKernel 2339-2387,
emitKernelVariants 959-979, inferModuleCapabilities 259-335,
resultNameForCallable 1360-1383) -- and writes the module JSON.  The sources
are the reference's example programs (examples/*.manta) and compiler presets
(compiler.go:337-575), transcribed below as small expression trees.

One deliberate difference: each kernel variant's `source` (the generated
CUDA / Metal / ... text) is a placeholder string; the rocm executor runs
kernels by their body ops and never reads variant sources.

Run: python tests/golden/modules/make_modules.py   (rewrites the *.json here)
"""
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))
BACKENDS = ["cuda", "metal", "vulkan", "directml", "webgpu"]


def T(dtype, *shape):
    return {"kind": "tensor", "dtype": dtype, "shape": list(shape)}


def PACK(*shape):
    return {"kind": "candidate_pack", "shape": list(shape)}


def artifact_type(t):
    if t["kind"] == "candidate_pack":
        return {"kind": "candidate_pack", "candidate_pack": {"shape": t["shape"]} if t["shape"] else {}}
    tensor = {"dtype": t["dtype"]}
    if t["shape"]:
        tensor["shape"] = t["shape"]
    return {"kind": "tensor", "tensor": tensor}


# expression trees: ("id", name) | ("call", callee, [args]) | ("matmul", [a, b])
# | ("topk", arg, k) | ("bin", op, a, b)
def ID(n):
    return ("id", n)


def CALL(f, *args):
    return ("call", f, list(args))


def MATMUL(a, b):
    return ("matmul", [a, b])


def TOPK(a, k):
    return ("topk", a, k)


def ADD(a, b):
    return ("bin", "+", a, b)


BIN_NAMES = {"+": "add", "-": "sub", "*": "mul", "/": "div"}


def expr_name(e):
    """exprName (compiler.go:1471-1486)."""
    if e[0] == "id":
        return e[1]
    if e[0] == "call":
        return e[1]
    if e[0] == "matmul":
        return "matmul"
    if e[0] == "topk":
        return "topk"
    return expr_name(e[2]) + "_" + BIN_NAMES[e[1]] + "_" + expr_name(e[3])


def hints_for(name, ops):
    h = {"tile": [128], "vector_width": 4, "subgroup": False, "memory": "device_local"}
    for op in ops:
        if op == "softmax":
            h.update(tile=[64], vector_width=1, subgroup=True, memory="workgroup_local")
        elif op in ("normalize", "rmsnorm", "layernorm"):
            h.update(tile=[128], vector_width=4, subgroup=True, memory="workgroup_local")
        elif op in ("dot", "cosine", "l2_distance"):
            h.update(tile=[128], vector_width=4, subgroup=True, memory="workgroup_local")
        elif op == "mean_pool":
            h.update(tile=[64], vector_width=1, subgroup=True, memory="workgroup_local")
        elif op.startswith("binary_"):
            h.update(tile=[128], vector_width=4)
    if "norm" in name:
        h["subgroup"] = True
    return h


REDUCE_OPS = {"normalize", "rmsnorm", "layernorm", "softmax", "dot", "cosine", "l2_distance", "mean_pool"}


def make_kernel(name, inputs, output_type, ops):
    """ops: [(op, [input names], output, attributes)]; a return of the last
    output."""
    hints = hints_for(name, [o[0] for o in ops])
    body = []
    for op, ins, out, attrs in ops:
        o = {"kind": "reduce" if op in REDUCE_OPS else "pointwise", "name": out, "op": op, "inputs": ins,
             "outputs": [out]}
        if attrs:
            o["attributes"] = dict(sorted(attrs.items()))
        body.append(o)
    body.append({"kind": "return", "op": "return", "outputs": [ops[-1][2]]})
    tile = lambda v: "[" + ",".join(str(x) for x in v) + "]"
    meta = {"tile": tile(hints["tile"]), "tile_2d": "[]", "vector_width": str(hints["vector_width"]),
            "subgroup": "true" if hints["subgroup"] else "false", "subgroup_2d": "[]", "halo": "[]",
            "memory": hints["memory"]}
    # MarshalIndent's field order: tile, vector_width, subgroup, memory
    ahints = {"tile": hints["tile"], "vector_width": hints["vector_width"]}
    if hints["subgroup"]:
        ahints["subgroup"] = True
    ahints["memory"] = hints["memory"]
    return {
        "name": name,
        "inputs": [{"name": n, "type": artifact_type(t)} for n, t in inputs],
        "outputs": [{"name": "result", "type": artifact_type(output_type)}],
        "hints": ahints,
        "body": body,
        "variants": [{"backend": b, "entry": "%s_%s" % (name, b),
                      "source": "// %s variant source: not reproduced in this fixture" % b,
                      "meta": dict(sorted(meta.items()))} for b in BACKENDS],  # Go writes map keys sorted
    }


class Lowering:
    def __init__(self, name, ndecls):
        self.name = name
        self.ndecls = ndecls
        self.params = []
        self.entries = []
        self.buffers = []
        self.kernels = []
        self.steps = []
        self.user_kernels = {}
        self.env_global = {}

    def param(self, name, t, binding, trainable=False):
        self.params.append((name, t, binding, trainable))
        self.env_global[name] = t

    def kernel(self, name, inputs, result_type, ops):
        # a declared kernel: its body lowered with output "result"
        k = make_kernel(name, inputs, result_type, [o + ({},) for o in ops])
        self.kernels.append(k)
        self.user_kernels[name] = result_type

    def buffer(self, name, t, is_input=False):
        if any(b["name"] == name for b in self.buffers):
            return
        if t["kind"] == "candidate_pack":
            b = {"name": name, "dtype": "candidate_pack", "shape": t["shape"], "storage_class": "host_visible"}
        else:
            b = {"name": name, "dtype": t["dtype"], "shape": t["shape"],
                 "storage_class": "host_visible" if is_input else "device_local"}
        if not b["shape"]:
            del b["shape"]
        self.buffers.append(b)

    def add_kernel(self, k):
        if not any(x["name"] == k["name"] for x in self.kernels):
            self.kernels.append(k)

    def type_of(self, expr, env):
        """inferExprType (compiler.go:1821-...): no steps, no buffers."""
        return self.plan(expr, "", env, [], dry=True)

    def plan(self, expr, out, env, steps, dry=False):
        """inferExprPlan / inferCallPlan: appends the steps, returns the type."""
        kind = expr[0]
        if kind == "id":
            t = env[expr[1]]
            if out and out != expr[1] and not dry:
                steps.append({"kind": "alias", "name": out, "inputs": [expr[1]], "outputs": [out]})
                self.buffer(out, t)
            return t
        if kind == "bin":
            t = self.type_of(expr[2], env)
            if out and not dry:
                name = "binary_" + BIN_NAMES[expr[1]]
                steps.append({"kind": "launch_kernel", "name": name, "kernel": name,
                              "inputs": [expr_name(expr[2]), expr_name(expr[3])], "outputs": [out]})
                self.buffer(out, t)
                ins = [("lhs", self.type_of(expr[2], env)), ("rhs", self.type_of(expr[3], env))]
                self.add_kernel(make_kernel(name, ins, t, [(name, ["lhs", "rhs"], "result", {"operator": expr[1]})]))
            return t
        if kind == "topk":
            at = self.type_of(expr[1], env)
            arg = self.arg(expr[1], out, "topk", 0, env, steps, dry)
            k = expr[2]
            t = T("i32", str(k)) if len(at["shape"]) == 1 else T("i32", at["shape"][0], str(k))
            if not dry:
                steps.append({"kind": "topk", "name": "topk", "inputs": [arg], "outputs": [out] if out else [],
                              "attributes": {"k": str(k)}})
                if out:
                    self.buffer(out, t)
            return t
        callee = expr[1] if kind == "call" else "matmul"
        args = expr[2] if kind == "call" else expr[1]
        types = [self.type_of(a, env) for a in args]
        names = [self.arg(a, out, callee, i, env, steps, dry) for i, a in enumerate(args)]
        step = {"kind": "launch_kernel", "name": callee, "kernel": callee, "inputs": names,
                "outputs": [out] if out else []}
        kernel = None
        if kind == "matmul":
            l, r = types
            shape = []
            if len(l["shape"]) == 2 and len(r["shape"]) == 2:
                shape = [l["shape"][0], r["shape"][1]]
            if len(l["shape"]) == 3 and len(r["shape"]) == 2:
                shape = [l["shape"][0], l["shape"][1], r["shape"][1]]
            if len(l["shape"]) == 3 and len(r["shape"]) == 3:
                shape = [l["shape"][0], l["shape"][1], r["shape"][2]]
            t = T(l["dtype"], *shape)
            step = {"kind": "matmul", "name": "matmul", "inputs": names, "outputs": step["outputs"]}
        elif callee == "transpose":
            x = types[0]
            shape = []
            if len(x["shape"]) == 2:
                shape = [x["shape"][1], x["shape"][0]]
            if len(x["shape"]) == 3:
                shape = [x["shape"][0], x["shape"][2], x["shape"][1]]
            t = T(x["dtype"], *shape)
            step = {"kind": "transpose", "name": "transpose", "inputs": names, "outputs": step["outputs"]}
        elif callee == "gather":
            tb, ix = types
            shape = []
            if len(tb["shape"]) == 1 and len(ix["shape"]) == 1:
                shape = [ix["shape"][0]]
            if len(tb["shape"]) == 2 and len(ix["shape"]) == 1:
                shape = [ix["shape"][0], tb["shape"][1]]
            if len(tb["shape"]) == 2 and len(ix["shape"]) == 2:
                if tb["shape"][0] == ix["shape"][0]:
                    shape = [ix["shape"][0], ix["shape"][1]]
                else:
                    shape = [ix["shape"][0], ix["shape"][1], tb["shape"][1]]
            if len(tb["shape"]) == 3 and len(ix["shape"]) == 2:
                shape = [ix["shape"][0], ix["shape"][1], tb["shape"][2]]
            t = T(tb["dtype"], *shape)
            step = {"kind": "gather", "name": "gather", "inputs": names, "outputs": step["outputs"]}
        elif callee == "pack_candidates":
            ids, sc, docs = types
            shape = []
            if len(ids["shape"]) == 1 and len(sc["shape"]) == 1 and len(docs["shape"]) == 2:
                shape = list(docs["shape"])
            if len(ids["shape"]) == 2 and len(sc["shape"]) == 2 and len(docs["shape"]) == 3:
                shape = list(docs["shape"])
            t = PACK(*shape)
            step = {"kind": "pack_candidates", "name": "pack_candidates", "inputs": names,
                    "outputs": step["outputs"]}
        elif callee == "dequant":
            t = T("f16", *types[0]["shape"])
            step = {"kind": "dequant", "name": "dequant", "inputs": names, "outputs": step["outputs"]}
        elif callee == "mean_pool":
            x = types[0]
            shape = []
            if len(x["shape"]) == 2:
                shape = [x["shape"][1]]
            if len(x["shape"]) == 3:
                shape = [x["shape"][0], x["shape"][2]]
            t = T(x["dtype"], *shape)
            kernel = self.builtin(callee, args, types, t)
        elif callee in ("dot", "cosine", "l2_distance"):
            q, d = types
            shape = []
            if len(d["shape"]) == 2:
                shape = [d["shape"][0]]
            if len(q["shape"]) == 2 and len(d["shape"]) == 3:
                shape = [q["shape"][0], d["shape"][1]]
            t = T("f32", *shape)
            kernel = self.builtin(callee, args, types, t)
        else:
            t = types[0]
            if callee not in self.user_kernels:
                kernel = self.builtin(callee, args, types, t)
        if dry:
            return t
        steps.append(step)
        if kernel:
            self.add_kernel(kernel)
        if out:
            self.buffer(out, t)
        for s in steps:
            if not s["outputs"]:
                del s["outputs"]
        return t

    def builtin(self, callee, args, types, out_type):
        names = [expr_name(a) for a in args]
        attrs = {"axis": "-1"} if callee == "softmax" else {}
        return make_kernel(callee, list(zip(names, types)), out_type, [(callee, names, "result", attrs)])

    def arg(self, expr, out, callee, index, env, steps, dry=False):
        """materializeCallArg (compiler.go:2069-2093)."""
        if expr[0] == "id":
            return expr[1]
        name = "%s_arg%d_%s" % (out or callee, index, expr_name(expr))
        if not dry:
            env[name] = self.plan(expr, name, env, steps)
        return name

    def pipeline(self, name, inputs, results, body):
        env = dict(self.env_global)
        for n, t in inputs:
            env[n] = t
            self.buffer(n, t, is_input=True)
        self.entries.append({"name": name, "kind": "pipeline",
                             "inputs": [{"name": n, "type": artifact_type(t)} for n, t in inputs],
                             "outputs": [{"name": n, "type": artifact_type(t)} for n, t in results]})
        for stmt in body:
            steps = []
            if stmt[0] == "let":
                t = self.plan(stmt[2], stmt[1], env, steps)
                env[stmt[1]] = t
                self.buffer(stmt[1], t)
            else:  # return
                outs = []
                for (rname, _), expr in zip(results, stmt[1]):
                    t = self.plan(expr, rname, env, steps)
                    env[rname] = t
                    self.buffer(rname, t)
                    outs.append(rname)
                steps.append({"kind": "return", "outputs": outs})
            for s in steps:
                s["entry"] = name
            self.steps.extend(steps)

    def capabilities(self):
        caps = []

        def add(c):
            if c not in caps:
                caps.append(c)
        for p in self.params:
            if p[1]["kind"] == "candidate_pack":
                add("candidate_pack")
        for e in self.entries:
            for b in e["inputs"] + e["outputs"]:
                if b["type"]["kind"] == "candidate_pack":
                    add("candidate_pack")
        for b in self.buffers:
            if b["dtype"] == "candidate_pack":
                add("candidate_pack")
        for k in self.kernels:
            for op in k["body"]:
                if op["op"] == "mean_pool" and len(op.get("inputs", [])) > 1:
                    add("masked_mean_pool")
        for s in self.steps:
            if s["kind"] == "pack_candidates":
                add("candidate_pack")
        return caps

    def module(self):
        steps = []
        for s in self.steps:
            o = {"entry": s["entry"], "kind": s["kind"]}
            for key in ("name", "kernel", "inputs", "outputs", "attributes"):
                if s.get(key):
                    o[key] = s[key]
            steps.append(o)
        m = {"version": "manta/v0alpha1", "name": self.name}
        if self.params:
            m["params"] = []
            for n, t, binding, trainable in self.params:
                p = {"name": n, "type": artifact_type(t), "binding": binding}
                if trainable:
                    p["trainable"] = True
                m["params"].append(p)
        m["entry_points"] = self.entries
        req = {"supported_backends": list(BACKENDS)}
        caps = self.capabilities()
        if caps:
            req["capabilities"] = caps
        m["requirements"] = req
        m["buffers"] = self.buffers
        if self.kernels:
            m["kernels"] = self.kernels
        m["steps"] = steps
        m["metadata"] = {"source_decls": self.ndecls}
        return m


def score_like(name, ndecls, entry, result_name, body_kind):
    lw = Lowering(name, ndecls)
    lw.param("docs", T("q4", "N", "D"), "weights/docs")
    q = [("query", T("f16", "D"))]
    if body_kind == "score":
        lw.pipeline(entry, q, [(result_name, T("f32", "N"))], [("return", [CALL("cosine", ID("query"), ID("docs"))])])
    elif body_kind == "rerank":
        lw.pipeline(entry, q, [("top_ids", T("i32", "2")), ("top_scores", T("f32", "2"))], [
            ("let", "scores", CALL("cosine", ID("query"), ID("docs"))),
            ("let", "top_ids", TOPK(ID("scores"), 2)),
            ("let", "top_scores", CALL("gather", ID("scores"), ID("top_ids"))),
            ("return", [ID("top_ids"), ID("top_scores")])])
    elif body_kind == "select":
        lw.pipeline(entry, q, [(result_name, T("f32", "2"))], [
            ("let", "scores", CALL("cosine", ID("query"), ID("docs"))),
            ("let", "ids", TOPK(ID("scores"), 2)),
            ("return", [CALL("gather", ID("scores"), ID("ids"))])])
    elif body_kind == "retrieve":
        lw.pipeline(entry, q, [("top_ids", T("i32", "2")), ("top_scores", T("f32", "2")),
                               ("top_docs", T("q4", "2", "D"))], [
            ("let", "scores", CALL("cosine", ID("query"), ID("docs"))),
            ("let", "top_ids", TOPK(ID("scores"), 2)),
            ("let", "top_scores", CALL("gather", ID("scores"), ID("top_ids"))),
            ("let", "top_docs", CALL("gather", ID("docs"), ID("top_ids"))),
            ("return", [ID("top_ids"), ID("top_scores"), ID("top_docs")])])
    return lw.module()


def candidates_body(q, scores_op="cosine"):
    return [
        ("let", "scores", CALL(scores_op, ID(q), ID("docs"))),
        ("let", "top_indices", TOPK(ID("scores"), 2)),
        ("let", "top_candidate_ids", CALL("gather", ID("candidate_ids"), ID("top_indices"))),
        ("let", "top_scores", CALL("gather", ID("scores"), ID("top_indices"))),
        ("let", "top_docs", CALL("gather", ID("docs"), ID("top_indices"))),
    ]


def modules():
    out = {}
    # compiler presets (compiler.go:485-575) and examples/*.manta
    out["tiny_score"] = score_like("tiny_score", 2, "score", "scores", "score")
    out["tiny_rerank"] = score_like("tiny_rerank", 2, "rerank", None, "rerank")
    out["tiny_select"] = score_like("tiny_select", 2, "select_scores", "top_scores", "select")
    out["tiny_retrieve"] = score_like("tiny_retrieve", 2, "retrieve", None, "retrieve")

    lw = Lowering("tiny_candidates", 1)
    lw.pipeline("rerank_candidates", [("query", T("f16", "D")), ("docs", T("q4", "N", "D")),
                                      ("candidate_ids", T("i64", "N"))],
                [("top_candidate_ids", T("i64", "2")), ("top_scores", T("f32", "2")), ("top_docs", T("q4", "2", "D"))],
                candidates_body("query") + [("return", [ID("top_candidate_ids"), ID("top_scores"), ID("top_docs")])])
    out["tiny_candidates"] = lw.module()

    lw = Lowering("tiny_batch_candidates", 1)
    lw.pipeline("rerank_candidates_batch", [("queries", T("f16", "Q", "D")), ("docs", T("q4", "Q", "N", "D")),
                                            ("candidate_ids", T("i64", "Q", "N"))],
                [("top_candidate_ids", T("i64", "Q", "2")), ("top_scores", T("f32", "Q", "2")),
                 ("top_docs", T("q4", "Q", "2", "D"))],
                candidates_body("queries") + [("return", [ID("top_candidate_ids"), ID("top_scores"), ID("top_docs")])])
    out["tiny_batch_candidates"] = lw.module()

    lw = Lowering("tiny_packed_candidates", 1)
    lw.pipeline("rerank_candidates_packed", [("query", T("f16", "D")), ("docs", T("q4", "N", "D")),
                                             ("candidate_ids", T("i64", "N"))],
                [("candidates", PACK("2", "D"))],
                candidates_body("query") + [
                    ("return", [CALL("pack_candidates", ID("top_candidate_ids"), ID("top_scores"), ID("top_docs"))])])
    out["tiny_packed_candidates"] = lw.module()

    # runtime/retrieval_model_test.go:96-113: both retrieval entries in one module
    lw = Lowering("packed_batch", 2)
    lw.pipeline("rerank_candidates_packed", [("query", T("f16", "D")), ("docs", T("q4", "N", "D")),
                                             ("candidate_ids", T("i64", "N"))],
                [("candidates", PACK("2", "D"))],
                candidates_body("query") + [
                    ("return", [CALL("pack_candidates", ID("top_candidate_ids"), ID("top_scores"), ID("top_docs"))])])
    lw.pipeline("rerank_candidates_packed_batch", [("queries", T("f16", "Q", "D")), ("docs", T("q4", "Q", "N", "D")),
                                                   ("candidate_ids", T("i64", "Q", "N"))],
                [("result", PACK("Q", "2", "D"))],
                candidates_body("queries") + [
                    ("return", [CALL("pack_candidates", ID("top_candidate_ids"), ID("top_scores"), ID("top_docs"))])])
    out["packed_batch"] = lw.module()

    # examples/score_bundle.manta
    lw = Lowering("score_bundle", 2)
    lw.pipeline("score", [("query", T("f16", "D")), ("docs", T("q4", "N", "D"))], [("scores", T("f32", "N"))],
                [("return", [CALL("cosine", ID("query"), ID("docs"))])])
    lw.pipeline("score_batch", [("queries", T("f16", "Q", "D")), ("docs", T("q4", "Q", "N", "D"))],
                [("result", T("f32", "Q", "N"))], [("return", [CALL("cosine", ID("queries"), ID("docs"))])])
    out["score_bundle"] = lw.module()

    # compiler.go:339-353 (tiny_embed, examples/embed.manta)
    lw = Lowering("tiny_embed", 4)
    lw.param("token_embedding", T("f16", "V", "D"), "weights/token_embedding")
    lw.param("projection", T("f16", "D", "E"), "weights/projection")
    lw.kernel("l2_normalize", [("x", T("f16", "T", "E"))], T("f16", "T", "E"), [("normalize", ["x"], "result")])
    lw.pipeline("embed", [("tokens", T("i32", "T"))], [("embeddings", T("f16", "T", "E"))], [
        ("let", "hidden", CALL("gather", ID("token_embedding"), ID("tokens"))),
        ("let", "projected", MATMUL(ID("hidden"), ID("projection"))),
        ("return", [CALL("l2_normalize", ID("projected"))])])
    out["tiny_embed"] = lw.module()

    # examples/embed_pooled.manta and embed_masked_pooled.manta
    for name, masked in (("tiny_embed_pooled", False), ("embed_masked_pooled", True)):
        lw = Lowering(name, 4)
        lw.param("token_embedding", T("f16", "V", "D"), "weights/token_embedding")
        lw.param("projection", T("f16", "D", "E"), "weights/projection")
        single = [("tokens", T("i32", "T"))] + ([("attention_mask", T("i32", "T"))] if masked else [])
        batch = [("tokens", T("i32", "B", "T"))] + ([("attention_mask", T("i32", "B", "T"))] if masked else [])
        pool = (lambda x: CALL("mean_pool", ID(x), ID("attention_mask"))) if masked else (
            lambda x: CALL("mean_pool", ID(x)))
        lw.pipeline("embed_pooled", single, [("result", T("f16", "E"))], [
            ("let", "hidden", CALL("gather", ID("token_embedding"), ID("tokens"))),
            ("let", "projected", MATMUL(ID("hidden"), ID("projection"))),
            ("let", "normalized", CALL("normalize", ID("projected"))),
            ("return", [pool("normalized")])])
        lw.pipeline("embed_pooled_batch", batch, [("result", T("f16", "B", "E"))], [
            ("let", "batch_hidden", CALL("gather", ID("token_embedding"), ID("tokens"))),
            ("let", "batch_projected", MATMUL(ID("batch_hidden"), ID("projection"))),
            ("let", "batch_normalized", CALL("normalize", ID("batch_projected"))),
            ("return", [pool("batch_normalized")])])
        out[name] = lw.module()

    # examples/encoder_trainable_q8.manta and encoder_trainable_q8x2.manta
    for name, layers in (("encoder_trainable_q8", 1), ("encoder_trainable_q8x2", 2)):
        lw = Lowering(name, 9)
        shapes = {"token_embedding": ("V", "D"), "attn_q": ("D", "D"), "attn_k": ("D", "D"), "attn_v": ("D", "D"),
                  "attn_o": ("D", "D"), "ffn_up": ("D", "H"), "projection": ("H", "D")}
        for pname, shp in shapes.items():
            lw.param(pname, T("q8", *shp), "weights/" + pname, trainable=True)
        for entry, single in (("embed_pooled", True), ("embed_pooled_batch", False)):
            lead = ("T",) if single else ("B", "T")
            body = [("let", "hidden_q", CALL("gather", ID("token_embedding"), ID("tokens"))),
                    ("let", "hidden", CALL("dequant", ID("hidden_q"))),
                    ("let", "wq_f", CALL("dequant", ID("attn_q"))),
                    ("let", "wk_f", CALL("dequant", ID("attn_k"))),
                    ("let", "wv_f", CALL("dequant", ID("attn_v"))),
                    ("let", "wo_f", CALL("dequant", ID("attn_o"))),
                    ("let", "ffn_up_f", CALL("dequant", ID("ffn_up"))),
                    ("let", "projection_f", CALL("dequant", ID("projection")))]
            x = "hidden"
            for layer in range(1, layers + 1):
                sfx = "" if layers == 1 else str(layer)
                v = lambda n: n + sfx
                body += [("let", v("q"), MATMUL(ID(x), ID("wq_f"))),
                         ("let", v("k"), MATMUL(ID(x), ID("wk_f"))),
                         ("let", v("v"), MATMUL(ID(x), ID("wv_f"))),
                         ("let", v("kt"), CALL("transpose", ID(v("k")))),
                         ("let", v("scores"), MATMUL(ID(v("q")), ID(v("kt")))),
                         ("let", v("probs"), CALL("softmax", ID(v("scores")))),
                         ("let", v("mixed"), MATMUL(ID(v("probs")), ID(v("v")))),
                         ("let", v("attended"), MATMUL(ID(v("mixed")), ID("wo_f"))),
                         ("let", v("attn_hidden"), CALL("layernorm", ADD(ID(v("attended")), ID(x)))),
                         ("let", v("ffn_hidden"), MATMUL(ID(v("attn_hidden")), ID("ffn_up_f"))),
                         ("let", v("activated"), CALL("gelu", ID(v("ffn_hidden")))),
                         ("let", v("projected"), MATMUL(ID(v("activated")), ID("projection_f"))),
                         ("let", v("encoded"), CALL("layernorm", ADD(ID(v("projected")), ID(v("attn_hidden")))))]
                x = v("encoded")
            body += [("let", "normalized", CALL("normalize", ID(x))),
                     ("return", [CALL("mean_pool", ID("normalized"), ID("attention_mask"))])]
            lw.pipeline(entry, [("tokens", T("i32", *lead)), ("attention_mask", T("i32", *lead))],
                        [("result", T("f16", *(("D",) if single else ("B", "D"))))], body)
        out[name] = lw.module()
    return out


def tensor_binding(name, dtype, *shape):
    return {"name": name, "type": artifact_type(T(dtype, *shape))}


def reference_test_modules():
    """The modules the reference's own tests build (artifact/manta/
    module_test.go), transcribed as data: `demo` (10-88, valid), `bad`
    (177-199, a step naming an unknown entry point), `bad-kernel` (201-243,
    a variant without source) and `packed` (245-300, a valid candidate-pack
    entry point)."""
    out = {}
    tensor_bindings = lambda *bs: [tensor_binding(*b) for b in bs]
    out["ref_demo"] = {
        "version": "manta/v0alpha1", "name": "demo",
        "params": [{"name": "token_embedding", "type": artifact_type(T("f16", "V", "D")),
                    "binding": "weights/token_embedding"}],
        "entry_points": [{"name": "embed", "kind": "pipeline",
                          "inputs": tensor_bindings(("tokens", "i32", "T")),
                          "outputs": tensor_bindings(("embeddings", "f16", "T", "D"))}],
        "requirements": {"supported_backends": ["cuda", "metal"]},
        "buffers": [{"name": "x", "dtype": "f16", "shape": ["N", "D"], "storage_class": "device_local"}],
        "kernels": [{
            "name": "rmsnorm",
            "inputs": tensor_bindings(("x", "f16", "T", "D")),
            "outputs": tensor_bindings(("y", "f16", "T", "D")),
            "hints": {"tile": [128], "vector_width": 4, "subgroup": True, "memory": "device_local"},
            "body": [{"kind": "pointwise", "name": "normalize", "op": "normalize", "inputs": ["x"], "outputs": ["y"]},
                     {"kind": "return", "op": "return", "outputs": ["y"]}],
            "variants": [{"backend": "cuda", "entry": "rmsnorm_cuda",
                          "source": "extern \"C\" __global__ void rmsnorm_cuda() {}"},
                         {"backend": "metal", "entry": "rmsnorm_metal", "source": "kernel void rmsnorm_metal() {}"}],
        }],
        "steps": [{"entry": "embed", "kind": "gather", "name": "embed_lookup", "inputs": ["token_embedding", "tokens"],
                   "outputs": ["x"]},
                  {"entry": "embed", "kind": "return", "outputs": ["embeddings"]}],
    }
    embed_entry = [{"name": "embed", "kind": "pipeline", "inputs": tensor_bindings(("tokens", "i32", "T")),
                    "outputs": tensor_bindings(("embeddings", "f16", "T", "D"))}]
    out["ref_bad"] = {
        "version": "manta/v0alpha1", "name": "bad", "entry_points": embed_entry,
        "requirements": {"supported_backends": list(BACKENDS)},
        "buffers": [{"name": "x", "dtype": "f16", "shape": ["T", "D"]}],
        "steps": [{"entry": "missing", "kind": "gather", "inputs": ["tokens"], "outputs": ["x"]}],
    }
    out["ref_bad_kernel"] = {
        "version": "manta/v0alpha1", "name": "bad-kernel", "entry_points": embed_entry,
        "requirements": {"supported_backends": list(BACKENDS)},
        "buffers": [{"name": "embeddings", "dtype": "f16", "shape": ["T", "D"]}],
        "kernels": [{
            "name": "embed_kernel",
            "inputs": tensor_bindings(("x", "f16", "T", "D")),
            "outputs": tensor_bindings(("result", "f16", "T", "D")),
            "hints": {},
            "body": [{"kind": "pointwise", "op": "identity", "inputs": ["x"], "outputs": ["result"]},
                     {"kind": "return", "op": "return", "outputs": ["result"]}],
            "variants": [{"backend": "cuda", "entry": "embed_kernel_cuda",
                          "source": "extern \"C\" __global__ void embed_kernel_cuda() {}"},
                         {"backend": "metal", "entry": "embed_kernel_metal"}],
        }],
        "steps": [{"entry": "embed", "kind": "launch_kernel", "name": "embed_kernel", "kernel": "embed_kernel",
                   "inputs": ["tokens"], "outputs": ["embeddings"]},
                  {"entry": "embed", "kind": "return", "outputs": ["embeddings"]}],
    }
    out["ref_packed"] = {
        "version": "manta/v0alpha1", "name": "packed",
        "entry_points": [{"name": "rerank_candidates_packed", "kind": "pipeline",
                          "inputs": tensor_bindings(("query", "f16", "D"), ("docs", "q4", "N", "D"),
                                                    ("candidate_ids", "i64", "N")),
                          "outputs": [{"name": "candidates", "type": artifact_type(PACK("K", "D"))}]}],
        "requirements": {"supported_backends": ["cuda", "metal"]},
        "buffers": [{"name": "scores", "dtype": "f32", "shape": ["N"]},
                    {"name": "top_indices", "dtype": "i32", "shape": ["K"]},
                    {"name": "top_candidate_ids", "dtype": "i64", "shape": ["K"]},
                    {"name": "top_scores", "dtype": "f32", "shape": ["K"]},
                    {"name": "top_docs", "dtype": "q4", "shape": ["K", "D"]},
                    {"name": "candidates", "dtype": "candidate_pack", "shape": ["K", "D"]}],
        "kernels": [{
            "name": "cosine",
            "inputs": tensor_bindings(("query", "f16", "D"), ("docs", "q4", "N", "D")),
            "outputs": tensor_bindings(("scores", "f32", "N")),
            "hints": {},
            "body": [{"kind": "builtin", "op": "cosine", "inputs": ["query", "docs"], "outputs": ["scores"]},
                     {"kind": "return", "op": "return", "outputs": ["scores"]}],
            "variants": [{"backend": "cuda", "entry": "cosine_cuda",
                          "source": "extern \"C\" __global__ void cosine_cuda() {}"},
                         {"backend": "metal", "entry": "cosine_metal", "source": "kernel void cosine_metal() {}"}],
        }],
        "steps": [
            {"entry": "rerank_candidates_packed", "kind": "launch_kernel", "name": "cosine", "kernel": "cosine",
             "inputs": ["query", "docs"], "outputs": ["scores"]},
            {"entry": "rerank_candidates_packed", "kind": "topk", "name": "topk", "inputs": ["scores"],
             "outputs": ["top_indices"], "attributes": {"k": "2"}},
            {"entry": "rerank_candidates_packed", "kind": "gather", "name": "gather_ids",
             "inputs": ["candidate_ids", "top_indices"], "outputs": ["top_candidate_ids"]},
            {"entry": "rerank_candidates_packed", "kind": "gather", "name": "gather_scores",
             "inputs": ["scores", "top_indices"], "outputs": ["top_scores"]},
            {"entry": "rerank_candidates_packed", "kind": "gather", "name": "gather_docs",
             "inputs": ["docs", "top_indices"], "outputs": ["top_docs"]},
            {"entry": "rerank_candidates_packed", "kind": "pack_candidates", "name": "pack_candidates",
             "inputs": ["top_candidate_ids", "top_scores", "top_docs"], "outputs": ["candidates"]},
            {"entry": "rerank_candidates_packed", "kind": "return", "outputs": ["candidates"]}],
    }
    return out


def main():
    mods = modules()
    mods.update(reference_test_modules())
    for name, m in mods.items():
        with open(os.path.join(HERE, name + ".json"), "w") as f:
            json.dump(m, f, indent=2)
            f.write("\n")


if __name__ == "__main__":
    main()
