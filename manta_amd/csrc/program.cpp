// program.cpp -- the artifact step executor on the MI355X.
//
// Runs an entry point's plan steps (artifact/manta/module.go:199-207) the
// way backend.ExecuteSymbolic does (runtime/backend/symbolic.go:14-163):
// request inputs checked and their shapes bound, params materialized
// eagerly, steps in module order with their inputs looked up by name, the
// return step's values collected -- with the reference's error wording at
// every stage.  Each step runs on device through this library:
//
//   alias            the value itself (no copy)
//   gather           kernels_exec gather_elems for dense tables (every
//                    table-rank x index-rank case of gatherTensor), the
//                    candidate pack kernel for rows of bound q8 / q4
//                    candidates (docs gathered by top-k indices)
//   pack_candidates  ids, scores and gathered rows as one candidate_pack
//   matmul           the f16 MFMA GEMM for f16 / q8 operands, the f32 MFMA
//                    GEMM for f32 ones, batched products per sequence
//                    (f32 out)
//   topk             the device top-k over an f32 score matrix
//   dequant          the value relabelled f16, as the reference's clone
//   transpose        the last two axes swapped (kernels_exec transpose)
//   launch_kernel    the kernel's body ops in order (executeKernel,
//                    tensor_ops.go:476-516): dot / cosine / l2_distance on
//                    bound candidates with the reference's arithmetic,
//                    normalize / rmsnorm, mean_pool (masked or not),
//                    softmax and layernorm over rows, gelu, and the
//                    element-wise binary_add / _sub / _mul / _div
//   return           the entry's outputs
//
// A score kernel whose only consumers are one topk step and gathers of the
// scores by that topk's indices is not materialized: the topk step runs the
// fused score + top-k (manta_rocm_score_topk, whose scores are the
// reference's bit for bit) and the gathers take its top scores.  Steps and
// ops outside this set (kv_cache, image ops, ...) return
// MANTA_ROCM_UNSUPPORTED (manta_rocm_program_supports names the first such
// step): the Go backend runs such entries through ExecuteSymbolic with
// per-kernel dispatch instead.
//
// Values live in device memory owned by the program: one buffer per
// allocation site of an entry, reused (and grown) by later runs of the same
// entry, so a steady-state run allocates nothing.  Gathers record their
// out-of-range indices in one device word per step; the run synchronizes
// once at the end and reports the first failing step with its index.
#include <hip/hip_runtime.h>

#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "manta_module.h"
#include "manta_rocm.h"
#include "module_internal.hpp"
#include "runtime_internal.hpp"

using manta_mod::EntryPoint;
using manta_mod::Kernel;
using manta_mod::KernelOp;
using manta_mod::Module;
using manta_mod::Step;
using manta_mod::ValueType;

namespace {

constexpr int VK_DEFERRED = 100;  // a score folded into the following topk

int dtype_code(const std::string& s) {
    if (s == "f32") return MANTA_DT_F32;
    if (s == "f16") return MANTA_DT_F16;
    if (s == "i32") return MANTA_DT_I32;
    if (s == "i64") return MANTA_DT_I64;
    if (s == "q8") return MANTA_DT_Q8;
    if (s == "q4") return MANTA_DT_Q4;
    return 0;
}

const char* dtype_name(int c) {
    switch (c) {
        case MANTA_DT_F32: return "f32";
        case MANTA_DT_F16: return "f16";
        case MANTA_DT_I32: return "i32";
        case MANTA_DT_I64: return "i64";
        case MANTA_DT_Q8: return "q8";
        case MANTA_DT_Q4: return "q4";
        default: return "";
    }
}

int elem_bytes(int storage) {
    switch (storage) {
        case MANTA_DT_F16: return 2;
        case MANTA_DT_F32:
        case MANTA_DT_I32: return 4;
        case MANTA_DT_I64: return 8;
        default: return 0;
    }
}

std::string q(const std::string& s) { return "\"" + s + "\""; }

std::string fmt(const char* f, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    return buf;
}

// Go's %v of an []int shape: "[3 2]".
std::string go_shape(const std::vector<int64_t>& s) {
    std::string o = "[";
    for (size_t i = 0; i < s.size(); i++) o += (i ? " " : "") + std::to_string(s[i]);
    return o + "]";
}

struct Val {
    int kind = MANTA_VALUE_TENSOR;
    std::string dtype;  // the artifact's dtype string
    int storage = 0;    // a q8 TENSOR holds int8 codes and an f32 scale per column in `scales`
    std::vector<int64_t> shape;
    void* data = nullptr;
    void* scales = nullptr;
    void* ids = nullptr;
    void* scores = nullptr;
    int ids_storage = 0;
    const MantaRocmCandidates* cands = nullptr;
    int rows_format = 0;  // MANTA_ROCM_Q8_ROWS / Q4_BLOCKS for rows and packs
    // a bound [K, N] matmul weight prepared at bind time
    // (manta_rocm_prepare_projection): f16 [N][K], owned by the program
    void* prep = nullptr;
    int prep_kind = -1;
    // deferred score: op and the names of its query and docs values
    int op = -1;
    std::string qname, dname;

    int64_t elems() const {
        int64_t n = 1;
        for (int64_t x : shape) n *= x;
        return n;
    }
    bool tensor_like() const {
        return kind == MANTA_VALUE_TENSOR || kind == MANTA_VALUE_CANDIDATES || kind == MANTA_VALUE_ROWS ||
               kind == VK_DEFERRED;
    }
};

struct TraceStep {
    std::string kind, name, dispatch;
};

struct DevBuf {
    void* p = nullptr;
    size_t cap = 0;
};

struct EntryPlan {
    std::vector<int> steps;           // module step indices of this entry
    std::map<int, int> fused_topk;    // score launch step -> its topk step
    std::set<int> fused_gathers;      // gathers served by a fused top-k
    std::vector<DevBuf> pool;         // per allocation site
    DevBuf errs;                      // one gather error word per step
};

}  // namespace

struct MantaRocmProgram {
    MantaRocm* rt = nullptr;
    Module m;
    std::map<std::string, Val> weights;
    std::map<std::string, EntryPlan> plans;
    std::vector<TraceStep> trace;
};

namespace {

int set_err(char** err, int code, const std::string& msg) {
    if (err) {
        *err = (char*)malloc(msg.size() + 1);
        if (*err) memcpy(*err, msg.c_str(), msg.size() + 1);
    }
    return code;
}

bool is_score_op(const std::string& op) { return op == "dot" || op == "cosine" || op == "l2_distance"; }
int score_op_code(const std::string& op) {
    return op == "dot" ? MANTA_ROCM_DOT : op == "cosine" ? MANTA_ROCM_COSINE : MANTA_ROCM_L2_DISTANCE;
}

// The kernel's single computing op when its body is that op and a return
// of its output (what synthesizeBuiltinKernel emits, compiler.go:2278-2300).
const KernelOp* single_op(const Kernel& k) {
    const KernelOp* op = nullptr;
    for (const auto& o : k.body) {
        if (o.kind == "return") continue;
        if (op) return nullptr;
        op = &o;
    }
    if (!op || op->outputs.size() != 1) return nullptr;
    for (const auto& o : k.body)
        if (o.kind == "return" && !(o.outputs.size() == 1 && o.outputs[0] == op->outputs[0])) return nullptr;
    return op;
}

// resolveStepOutputType (symbolic.go:298-318).
ValueType resolve_type(const Module& m, const EntryPoint& en, const Step& s, size_t i,
                       const std::map<std::string, Val>* env) {
    if (i < s.outputs.size()) {
        const std::string& name = s.outputs[i];
        for (const auto& o : en.outputs)
            if (o.name == name) return o.type;
        if (const manta_mod::Buffer* b = manta_mod::find_buffer(m, name)) {
            ValueType t;
            if (b->dtype == "kv_cache") {
                t.kind = "kv_cache";
            } else if (b->dtype == "candidate_pack") {
                t.kind = "candidate_pack";
                t.has_pack = true;
                t.pack_shape = b->shape;
            } else {
                t.kind = "tensor";
                t.has_tensor = true;
                t.dtype = b->dtype;
                t.shape = b->shape;
            }
            return t;
        }
    }
    if (s.kind == "launch_kernel")
        if (const Kernel* k = manta_mod::find_kernel(m, s.kernel))
            if (i < k->outputs.size()) return k->outputs[i].type;
    if (env && !s.inputs.empty()) {
        auto it = env->find(s.inputs[0]);
        if (it != env->end()) {
            ValueType t;
            t.kind = "tensor";
            t.has_tensor = true;
            t.dtype = it->second.dtype;
            for (int64_t x : it->second.shape) t.shape.push_back(std::to_string(x));
            return t;
        }
    }
    ValueType t;
    t.kind = "tensor";
    t.has_tensor = true;
    t.dtype = "f32";
    return t;
}

// bindShape (tensor.go:491-516).
bool bind_shape(const std::vector<std::string>& symbols, const std::vector<int64_t>& actual,
                std::map<std::string, int64_t>* bindings, std::string* e) {
    if (symbols.empty()) return true;
    if (symbols.size() != actual.size())
        return *e = fmt("rank mismatch: expected %d dims, got %d", (int)symbols.size(), (int)actual.size()), false;
    for (size_t i = 0; i < symbols.size(); i++) {
        const std::string& sym = symbols[i];
        if (sym.empty()) continue;
        char* end = nullptr;
        const long long lit = strtoll(sym.c_str(), &end, 10);
        if (end && *end == 0 && end != sym.c_str()) {
            if (lit != actual[i])
                return *e = fmt("dimension %d mismatch: expected %lld, got %lld", (int)i, lit,
                                (long long)actual[i]),
                       false;
            continue;
        }
        auto it = bindings->find(sym);
        if (it != bindings->end()) {
            if (it->second != actual[i])
                return *e = fmt("symbol %s mismatch: expected %lld, got %lld", q(sym).c_str(), (long long)it->second,
                                (long long)actual[i]),
                       false;
            continue;
        }
        (*bindings)[sym] = actual[i];
    }
    return true;
}

// validateTensorType + concretizeValueType for a value handed in by the
// caller (tensor.go:385-403, 446-489).
bool check_value(const ValueType& t, const Val& v, std::map<std::string, int64_t>* bindings, std::string* e,
                 bool* unsupported) {
    if (t.kind == "tensor") {
        if (v.kind != MANTA_VALUE_TENSOR && v.kind != MANTA_VALUE_CANDIDATES)
            return *e = "expected tensor value, got a candidate pack", false;
        if (!t.has_tensor) return *e = "expected tensor type metadata", false;
        if (!t.dtype.empty() && v.dtype != t.dtype && !(t.dtype == "f16" && v.dtype == "f32"))
            return *e = "tensor dtype " + q(v.dtype) + " does not match expected " + q(t.dtype), false;
        if (!t.shape.empty() && t.shape.size() != v.shape.size())
            return *e = fmt("tensor rank %d does not match expected rank %d", (int)v.shape.size(), (int)t.shape.size()),
                   false;
        return bind_shape(t.shape, v.shape, bindings, e);
    }
    *unsupported = true;
    *e = "value kind " + q(t.kind) + " is not offered by the rocm executor";
    return false;
}

// A value handed in through the C-ABI.
bool import_value(const MantaRocmValue& in, Val* v, std::string* e) {
    *v = Val();
    v->kind = in.kind;
    v->dtype = dtype_name(in.dtype);
    if (v->dtype.empty()) return *e = fmt("unknown dtype code %d", in.dtype), false;
    if (in.rank < 0 || in.rank > 4) return *e = fmt("bad rank %d", in.rank), false;
    for (int i = 0; i < in.rank; i++) {
        if (in.shape[i] < 0) return *e = "negative dimension", false;
        v->shape.push_back(in.shape[i]);
    }
    if (in.kind == MANTA_VALUE_TENSOR) {
        v->storage = in.storage ? in.storage : in.dtype;
        if (v->storage == MANTA_DT_Q8) {
            // int8 codes with an f32 scale per column (a per-tensor grid is
            // one scale repeated)
            if (v->shape.empty()) return *e = "a q8 tensor needs a shape", false;
            if (!in.scales) return *e = "a q8 tensor needs its per-column scales", false;
            v->scales = in.scales;
        } else if (!elem_bytes(v->storage)) {
            return *e = "tensor storage must be f32, f16, i32, i64 or q8", false;
        }
        if (!in.data && v->elems() > 0) return *e = "nil tensor data", false;
        v->data = in.data;
        return true;
    }
    if (in.kind == MANTA_VALUE_CANDIDATES) {
        if (!in.candidates) return *e = "nil candidates", false;
        int format = 0;
        int64_t sets = 0, n = 0, d = 0;
        manta_rocm_candidates_info(in.candidates, &format, &sets, &n, &d);
        const bool ok = (in.rank == 2 && sets == 1 && in.shape[0] == n && in.shape[1] == d) ||
                        (in.rank == 3 && in.shape[0] == sets && in.shape[1] == n && in.shape[2] == d);
        if (!ok)
            return *e = fmt("candidates shape %s does not match the bound [%lld %lld %lld]", go_shape(v->shape).c_str(),
                            (long long)sets, (long long)n, (long long)d),
                   false;
        v->cands = in.candidates;
        v->storage = format == MANTA_ROCM_Q8_ROWS ? MANTA_DT_Q8 : MANTA_DT_Q4;
        return true;
    }
    return *e = fmt("values of kind %d cannot be passed in", in.kind), false;
}

struct Run {
    MantaRocmProgram* p;
    EntryPlan* plan;
    const EntryPoint* en;
    hipStream_t s;
    std::map<std::string, Val> env;
    std::map<std::string, int64_t> bindings;
    std::map<std::string, Val> fused;  // score value name -> its fused top scores
    size_t cursor = 0;
    int step_pos = 0;  // position of the running step in the entry's plan
    int code = MANTA_ROCM_OK;
    std::string err;

    bool fail(const std::string& e, int c = MANTA_ROCM_ERROR) {
        err = e;
        code = c;
        return false;
    }
    bool unsupported(const std::string& e) { return fail(e, MANTA_ROCM_UNSUPPORTED); }
    bool hip(hipError_t e, const char* what) {
        if (e == hipSuccess) return true;
        return fail(fmt("%s: %s", what, hipGetErrorString(e)));
    }
    bool abi(int rc, char* e) {
        if (rc == MANTA_ROCM_OK) return true;
        std::string msg = e ? e : "device call failed";
        free(e);
        return fail(msg, rc);
    }
    // Device memory for the next allocation site of this run.
    void* alloc(size_t bytes) {
        bytes = bytes ? (bytes + 255) & ~(size_t)255 : 256;
        if (cursor >= plan->pool.size()) plan->pool.emplace_back();
        DevBuf& b = plan->pool[cursor++];
        if (b.cap < bytes) {
            if (b.p) (void)hipFree(b.p);
            b.p = nullptr;
            b.cap = 0;
            if (hipMalloc(&b.p, bytes) != hipSuccess) {
                b.p = nullptr;
                return nullptr;
            }
            b.cap = bytes;
        }
        return b.p;
    }
    unsigned long long* err_slot() { return (unsigned long long*)plan->errs.p + step_pos; }
    bool tensor(const std::string& name, Val** out) {
        auto it = env.find(name);
        if (it == env.end() || !it->second.tensor_like()) return fail(name + " is not a tensor");
        *out = &it->second;
        return true;
    }
    // The f32 values of a value: itself when it is held in f32 and `copy` is
    // false, else a new f32 buffer (f16 widened, q8 dequantized to the
    // f32 products code * scale the reference's tensors hold).
    bool f32_of(const Val& in, Val* out, const char* what, bool copy) {
        const bool dense = in.kind == MANTA_VALUE_TENSOR;
        const bool rows_q8 = in.kind == MANTA_VALUE_ROWS && in.storage == MANTA_DT_Q8;
        if (!(dense && (in.storage == MANTA_DT_F32 || in.storage == MANTA_DT_F16 || in.storage == MANTA_DT_Q8)) &&
            !rows_q8)
            return unsupported(std::string(what) + " of a " + dtype_name(in.storage) +
                               " value is not offered by the rocm executor");
        if (dense && in.storage == MANTA_DT_F32 && !copy) {
            *out = in;
            return true;
        }
        *out = in;
        out->kind = MANTA_VALUE_TENSOR;
        out->storage = MANTA_DT_F32;
        out->scales = nullptr;
        out->data = alloc((size_t)in.elems() * 4);
        if (!out->data) return fail("out of device memory");
        if (in.storage == MANTA_DT_F16)
            return hip(manta::launch_widen_f16((const uint16_t*)in.data, (float*)out->data, in.elems(), s), what);
        if (in.storage == MANTA_DT_Q8) {
            const int64_t cols = in.shape.back();
            return hip(manta::launch_dequant_q8((const int8_t*)in.data, (const float*)in.scales,
                                                cols ? in.elems() / cols : 0, cols, dense ? 1 : 0, (float*)out->data,
                                                s),
                       what);
        }
        return hip(hipMemcpyAsync(out->data, in.data, (size_t)in.elems() * 4, hipMemcpyDeviceToDevice, s), what);
    }
    bool as_f32(const Val& in, Val* out, const char* what) { return f32_of(in, out, what, true); }
};

// ------------------------------------------------------------ kernel ops

// scoreLayout (tensor_ops.go:1499-1521) for a query tensor and bound docs.
bool score_layout(Run& r, const Val& qv, const Val& dv, int64_t* nq) {
    if (dv.kind != MANTA_VALUE_CANDIDATES)
        return r.unsupported("scores over " + dv.dtype + " docs held densely are not offered by the rocm executor");
    if (qv.shape.size() == 1 && dv.shape.size() == 2) {
        if (qv.shape[0] != dv.shape[1])
            return r.fail("score mismatch " + go_shape(qv.shape) + " x " + go_shape(dv.shape));
        *nq = 1;
    } else if (qv.shape.size() == 2 && dv.shape.size() == 3) {
        if (qv.shape[0] != dv.shape[0] || qv.shape[1] != dv.shape[2])
            return r.fail("score mismatch " + go_shape(qv.shape) + " x " + go_shape(dv.shape));
        *nq = qv.shape[0];
    } else {
        return r.fail("score expects query/docs as [D] x [N,D] or [Q,D] x [Q,N,D]");
    }
    if (qv.kind != MANTA_VALUE_TENSOR || qv.storage != MANTA_DT_F16)
        return r.unsupported("score queries computed in f32 are not offered by the rocm executor");
    return true;
}

// The full score matrix of a score op (dotRows / cosineRows /
// l2DistanceRows with the reference's arithmetic).
bool run_score(Run& r, int op, const Val& qv, const Val& dv, Val* out) {
    int64_t nq = 0;
    if (!score_layout(r, qv, dv, &nq)) return false;
    const int64_t n = dv.shape[dv.shape.size() - 2];
    *out = Val();
    out->dtype = "f32";
    out->storage = MANTA_DT_F32;
    out->shape = qv.shape.size() == 1 ? std::vector<int64_t>{n} : std::vector<int64_t>{nq, n};
    out->data = r.alloc((size_t)(nq * n) * 4);
    if (!out->data) return r.fail("out of device memory");
    char* e = nullptr;
    return r.abi(manta_rocm_score(r.p->rt, dv.cands, op, (const uint16_t*)qv.data, nq, (float*)out->data, &e), e);
}

bool run_normalize(Run& r, const Val& in, Val* out) {
    if (!r.as_f32(in, out, "normalize")) return false;
    // normalizeRows normalizes rank-2 and rank-3 values only
    if (in.shape.size() != 2 && in.shape.size() != 3) return true;
    const int64_t cols = in.shape.back();
    const int64_t rows = cols ? in.elems() / cols : 0;
    char* e = nullptr;
    return r.abi(manta_rocm_normalize_rows(r.p->rt, (float*)out->data, rows, cols, &e), e);
}

bool run_mean_pool(Run& r, const Val& in, const Val* mask, Val* out) {
    if (mask && (mask->kind != MANTA_VALUE_TENSOR || mask->storage != MANTA_DT_I32))
        return r.fail("mean_pool mask dtype " + q(mask->dtype) + " is not supported");
    if (in.shape.size() != 2 && in.shape.size() != 3)
        return r.fail("mean_pool expects rank-2 or rank-3 tensor input");
    Val x;
    if (!r.f32_of(in, &x, "mean_pool", false)) return false;
    const bool r3 = in.shape.size() == 3;
    const int64_t B = r3 ? in.shape[0] : 1, T = in.shape[r3 ? 1 : 0], C = in.shape.back();
    *out = Val();
    out->dtype = in.dtype;
    out->storage = MANTA_DT_F32;
    out->shape = r3 ? std::vector<int64_t>{B, C} : std::vector<int64_t>{C};
    out->data = r.alloc((size_t)(B * C) * 4);
    if (!out->data) return r.fail("out of device memory");
    if (!mask) {
        if (T == 0) return r.hip(hipMemsetAsync(out->data, 0, (size_t)(B * C) * 4, r.s), "mean_pool");
        char* e = nullptr;
        return r.abi(manta_rocm_mean_pool(r.p->rt, (const float*)x.data, B, T, C, (float*)out->data, &e), e);
    }
    const bool shape_ok = r3 ? (mask->shape.size() == 2 && mask->shape[0] == B && mask->shape[1] == T)
                             : (mask->shape.size() == 1 && mask->shape[0] == T);
    if (!shape_ok)
        return r.fail("mean_pool mask shape " + go_shape(mask->shape) + " does not match input " + go_shape(in.shape));
    if (T == 0) return r.hip(hipMemsetAsync(out->data, 0, (size_t)(B * C) * 4, r.s), "mean_pool");
    char* e = nullptr;
    return r.abi(manta_rocm_mean_pool_masked(r.p->rt, (const float*)x.data, (const int32_t*)mask->data, B, T, C,
                                             (float*)out->data, &e),
                 e);
}

// softmaxRows / layerNormRows / geluTensor (tensor_ops.go:1140-1168,
// 1303-1344): rank-2 and rank-3 values row by row (softmax and layernorm
// leave other ranks unchanged, as the reference does); the encoder's
// kernels, whose reductions run in tree order.
bool run_rowwise(Run& r, const std::string& op, const Val& in, Val* out) {
    const int64_t n = in.elems();
    const bool rowwise = in.shape.size() == 2 || in.shape.size() == 3;
    const int64_t cols = rowwise ? in.shape.back() : 0, rows = cols ? n / cols : 0;
    if (cols > 0x7FFFFFFF) return r.unsupported(op + " rows wider than 2^31");
    if (op == "layernorm" && rowwise) {
        // out of place: the f32 source, a new output
        Val src;
        if (!r.f32_of(in, &src, "layernorm", false)) return false;
        *out = src;
        out->data = r.alloc((size_t)n * 4);
        if (!out->data) return r.fail("out of device memory");
        return r.hip(manta::launch_enc_add_layernorm((const float*)src.data, nullptr, (float*)out->data, rows,
                                                     (int)cols, r.s),
                     "layernorm");
    }
    if (!r.as_f32(in, out, op.c_str())) return false;  // a copy the in-place kernels own
    if (op == "gelu") return r.hip(manta::launch_enc_gelu((float*)out->data, n, r.s), "gelu");
    if (op == "softmax" && rowwise)
        return r.hip(manta::launch_enc_softmax_rows((float*)out->data, rows, (int)cols, r.s), "softmax");
    return true;
}

// binaryTensorOp (tensor_ops.go:724-742): equal shapes, f32 elementwise.
bool run_binary(Run& r, const std::string& op, const Val& a, const Val& b, Val* out) {
    if (a.shape != b.shape) return r.fail("shape mismatch " + go_shape(a.shape) + " vs " + go_shape(b.shape));
    Val x, y;
    if (!r.f32_of(a, &x, op.c_str(), false) || !r.f32_of(b, &y, op.c_str(), false)) return false;
    *out = a;
    out->kind = MANTA_VALUE_TENSOR;
    out->storage = MANTA_DT_F32;
    out->scales = nullptr;
    out->data = r.alloc((size_t)a.elems() * 4);
    if (!out->data) return r.fail("out of device memory");
    const int code = op == "binary_add" ? 0 : op == "binary_sub" ? 1 : op == "binary_mul" ? 2 : 3;
    return r.hip(manta::launch_binary_f32(code, (const float*)x.data, (const float*)y.data, (float*)out->data,
                                          a.elems(), r.s),
                 op.c_str());
}

// executeKernel (tensor_ops.go:476-516) over the supported ops.
bool run_kernel(Run& r, const Kernel& k, const std::vector<Val*>& args, std::vector<Val>* results) {
    std::map<std::string, Val> locals;
    for (size_t i = 0; i < k.inputs.size(); i++) {
        if (i >= args.size()) return r.fail("kernel " + q(k.name) + " missing input " + q(k.inputs[i].name));
        locals[k.inputs[i].name] = *args[i];
    }
    std::vector<std::string> returns;
    for (const auto& op : k.body) {
        if (op.kind == "return") {
            returns = op.outputs;
            continue;
        }
        auto arg = [&](size_t i, Val** v) -> bool {
            if (i >= op.inputs.size()) return r.fail(fmt("missing input %d", (int)i));
            auto it = locals.find(op.inputs[i]);
            if (it == locals.end()) return r.fail("unknown local " + q(op.inputs[i]));
            *v = &it->second;
            return true;
        };
        Val out;
        bool ok = true;
        Val *a = nullptr, *b = nullptr;
        if (op.op == "normalize" || op.op == "rmsnorm") {
            ok = arg(0, &a) && run_normalize(r, *a, &out);
        } else if (op.op == "mean_pool") {
            ok = arg(0, &a) && (op.inputs.size() > 1 ? arg(1, &b) : true) && run_mean_pool(r, *a, b, &out);
        } else if (is_score_op(op.op)) {
            ok = arg(0, &a) && arg(1, &b) && run_score(r, score_op_code(op.op), *a, *b, &out);
        } else if (op.op == "softmax" || op.op == "layernorm" || op.op == "gelu") {
            ok = arg(0, &a) && run_rowwise(r, op.op, *a, &out);
        } else if (op.op == "binary_add" || op.op == "binary_sub" || op.op == "binary_mul" || op.op == "binary_div") {
            ok = arg(0, &a) && arg(1, &b) && run_binary(r, op.op, *a, *b, &out);
        } else {
            return r.unsupported("kernel " + q(k.name) + " op " + q(op.op) + " is not offered by the rocm executor");
        }
        if (!ok) {
            if (r.code == MANTA_ROCM_ERROR) r.err = "kernel " + q(k.name) + " op " + q(op.op) + ": " + r.err;
            return false;
        }
        if (!op.outputs.empty()) locals[op.outputs[0]] = out;
    }
    if (returns.empty())
        for (const auto& o : k.outputs) returns.push_back(o.name);
    for (const auto& name : returns) {
        auto it = locals.find(name);
        if (it == locals.end()) return r.fail("missing kernel return value " + q(name));
        results->push_back(it->second);
    }
    return true;
}

// ----------------------------------------------------------------- steps

bool step_gather(Run& r, const Module& m, const Step& s, Val* out) {
    if (s.inputs.size() != 2 || s.outputs.size() != 1)
        return r.fail("gather step " + q(s.name) + " expects 2 inputs and 1 output");
    Val *table = nullptr, *idx = nullptr;
    if (!r.tensor(s.inputs[0], &table) || !r.tensor(s.inputs[1], &idx)) return false;
    if (table->kind == VK_DEFERRED || idx->kind == VK_DEFERRED)
        return r.fail("a score folded into its top-k has no matrix to gather from");
    if (idx->shape.size() != 1 && idx->shape.size() != 2) return r.fail("gather expects indices rank 1 or 2");
    if (idx->kind != MANTA_VALUE_TENSOR || idx->storage != MANTA_DT_I32 || idx->elems() == 0)
        return r.fail("gather expects i32 indices");
    const ValueType want = resolve_type(m, *r.en, s, 0, &r.env);
    const size_t want_rank = want.has_tensor ? want.shape.size() : 0;
    const size_t tr = table->shape.size(), ir = idx->shape.size();
    // the case analysis of gatherTensor: rows per batch, columns per row,
    // batch stride (elements) and the output shape
    int64_t rows = 0, cols = 1, bstride = 0, B = 1, K = idx->elems();
    std::vector<int64_t> oshape;
    bool per_batch = false;
    if (tr == 1 && ir == 1) {
        rows = table->elems();
        oshape = {K};
    } else if (tr == 2 && ir == 1) {
        rows = table->shape[0];
        cols = table->shape[1];
        oshape = {K, cols};
    } else if (tr == 2 && ir == 2) {
        if (want_rank == 3 || table->shape[0] != idx->shape[0]) {
            rows = table->shape[0];
            cols = table->shape[1];
            oshape = {idx->shape[0], idx->shape[1], cols};
        } else {
            B = table->shape[0];
            rows = table->shape[1];
            K = idx->shape[1];
            bstride = rows;
            per_batch = true;
            oshape = {B, K};
        }
    } else if (tr == 3 && ir == 2) {
        if (idx->shape[0] != table->shape[0])
            return r.fail("gather batch mismatch " + go_shape(table->shape) + " x " + go_shape(idx->shape));
        B = table->shape[0];
        rows = table->shape[1];
        cols = table->shape[2];
        K = idx->shape[1];
        bstride = rows * cols;
        per_batch = true;
        oshape = {B, K, cols};
    } else {
        return r.fail("gather expects table rank 1, 2, or 3 with compatible indices");
    }
    *out = Val();
    out->dtype = table->dtype;
    out->shape = oshape;
    if (table->kind == MANTA_VALUE_CANDIDATES) {
        // rows of bound q8 / q4 candidates: the candidate pack kernel
        if (cols == 1 || (per_batch && tr == 2))
            return r.unsupported("gathering single values of " + table->dtype +
                                 " candidates is not offered by the rocm executor");
        int format = 0;
        int64_t sets = 0, n = 0, d = 0;
        manta_rocm_candidates_info(table->cands, &format, &sets, &n, &d);
        const int64_t nq = tr == 3 ? B : (ir == 2 ? idx->shape[0] : 1);
        const int64_t kk = ir == 2 ? idx->shape[1] : idx->shape[0];
        const int64_t row_bytes = format == MANTA_ROCM_Q8_ROWS ? d : d / 2;
        const int64_t scale_bytes = format == MANTA_ROCM_Q8_ROWS ? 4 : (d / 32) * 2;
        out->kind = MANTA_VALUE_ROWS;
        out->storage = table->storage;
        out->rows_format = format;
        out->data = r.alloc((size_t)(nq * kk * row_bytes));
        out->scales = r.alloc((size_t)(nq * kk * scale_bytes));
        if (!out->data || !out->scales) return r.fail("out of device memory");
        char* e = nullptr;
        return r.abi(manta_rt::pack_candidates_into(r.p->rt, table->cands, (const int32_t*)idx->data, nq, kk, nullptr,
                                                    nullptr, out->data, out->scales, r.err_slot(), &e),
                     e);
    }
    if (table->kind != MANTA_VALUE_TENSOR)
        return r.unsupported("gathering from " + table->dtype + " rows is not offered by the rocm executor");
    const int es = elem_bytes(table->storage);
    out->storage = table->storage;
    out->data = r.alloc((size_t)(B * K * cols * es));
    if (!out->data) return r.fail("out of device memory");
    if (!per_batch) {
        // row gathers: every index picks from the whole table
        K = idx->elems();
        B = 1;
    }
    return r.hip(manta::launch_gather_elems(table->data, es, rows, cols, bstride, (const int32_t*)idx->data, B, K,
                                            out->data, r.err_slot(), r.s),
                 "gather");
}

bool topk_limit(Run& r, const Step& s, int64_t* k) {
    auto it = s.attributes.find("k");
    if (it == s.attributes.end() || it->second.empty())
        return r.fail("topk step " + q(s.name) + " is missing limit attribute");
    char* end = nullptr;
    errno = 0;
    const long long v = strtoll(it->second.c_str(), &end, 10);
    if (errno || !end || *end || end == it->second.c_str() || v <= 0)
        return r.fail("topk step " + q(s.name) + " has invalid limit " + q(it->second));
    *k = v;
    return true;
}

bool topk_range(Run& r, const std::vector<int64_t>& shape, int64_t k) {
    if (shape.size() == 1) {
        if (k > shape[0]) return r.fail(fmt("topk limit %lld out of range for %lld scores", (long long)k,
                                            (long long)shape[0]));
    } else if (shape.size() == 2) {
        if (k > shape[1]) return r.fail(fmt("topk limit %lld out of range for row width %lld", (long long)k,
                                            (long long)shape[1]));
    } else {
        return r.fail("topk expects rank-1 or rank-2 scores");
    }
    return true;
}

bool step_topk(Run& r, const Step& s, Val* out, std::string* dispatch) {
    if (s.inputs.size() != 1 || s.outputs.size() != 1)
        return r.fail("topk step " + q(s.name) + " expects 1 input and 1 output");
    Val* in = nullptr;
    if (!r.tensor(s.inputs[0], &in)) return false;
    int64_t k = 0;
    if (!topk_limit(r, s, &k)) return false;
    if (!topk_range(r, in->shape, k)) return false;
    const int64_t rows = in->shape.size() == 2 ? in->shape[0] : 1, cols = in->shape.back();
    *out = Val();
    out->dtype = "i32";
    out->storage = MANTA_DT_I32;
    out->shape = in->shape.size() == 2 ? std::vector<int64_t>{rows, k} : std::vector<int64_t>{k};
    out->data = r.alloc((size_t)(rows * k) * 4);
    if (!out->data) return r.fail("out of device memory");
    if (in->kind == VK_DEFERRED) {
        // the fused score + top-k; its top scores serve the gathers
        Val& qv = r.env[in->qname];
        Val& dv = r.env[in->dname];
        Val sc;
        sc.dtype = "f32";
        sc.storage = MANTA_DT_F32;
        sc.shape = out->shape;
        sc.data = r.alloc((size_t)(rows * k) * 4);
        if (!sc.data) return r.fail("out of device memory");
        char* e = nullptr;
        const int rc = manta_rocm_score_topk(r.p->rt, dv.cands, in->op, MANTA_ROCM_LARGEST,
                                             (const uint16_t*)qv.data, rows, k, (int32_t*)out->data,
                                             (float*)sc.data, nullptr, &e);
        if (rc == MANTA_ROCM_OK) {
            r.fused[s.inputs[0]] = sc;
            *dispatch = "hip:score_topk";
            return true;
        }
        if (rc != MANTA_ROCM_UNSUPPORTED) return r.abi(rc, e);
        free(e);
        // beyond the fused path's limits: materialize the scores
        Val full;
        if (!run_score(r, in->op, qv, dv, &full)) return false;
        r.env[s.inputs[0]] = full;
        in = &r.env[s.inputs[0]];
    }
    if (in->kind != MANTA_VALUE_TENSOR || in->storage != MANTA_DT_F32)
        return r.unsupported("topk over " + in->dtype + " values is not offered by the rocm executor");
    char* e = nullptr;
    *dispatch = "hip:topk";
    return r.abi(manta_rocm_topk(r.p->rt, (const float*)in->data, rows, cols, k, MANTA_ROCM_LARGEST,
                                 (int32_t*)out->data, nullptr, &e),
                 e);
}

// transposeTensor (tensor_ops.go:1064-1112): the last two dimensions.
bool step_transpose(Run& r, const Step& s, Val* out) {
    if (s.inputs.size() != 1 || s.outputs.size() != 1)
        return r.fail("transpose step " + q(s.name) + " expects 1 input and 1 output");
    Val* in = nullptr;
    if (!r.tensor(s.inputs[0], &in)) return false;
    if (in->kind == VK_DEFERRED) return r.fail("a score folded into its top-k has no matrix to transpose");
    if (in->shape.size() != 2 && in->shape.size() != 3) return r.fail("transpose expects rank-2 or rank-3 tensor input");
    Val src;
    if (in->kind != MANTA_VALUE_TENSOR || in->storage == MANTA_DT_Q8) {
        if (!r.f32_of(*in, &src, "transpose", false)) return false;
    } else {
        src = *in;
    }
    const bool r3 = src.shape.size() == 3;
    const int64_t B = r3 ? src.shape[0] : 1, R = src.shape[r3 ? 1 : 0], C = src.shape.back();
    *out = src;
    out->shape = r3 ? std::vector<int64_t>{B, C, R} : std::vector<int64_t>{C, R};
    const int es = elem_bytes(src.storage);
    out->data = r.alloc((size_t)(B * R * C * es));
    if (!out->data) return r.fail("out of device memory");
    return r.hip(manta::launch_transpose(src.data, es, B, R, C, out->data, r.s), "transpose");
}

// matmulTensor (tensor_ops.go:981-1062): [M,K] x [K,N], [B,M,K] x [K,N] and
// [B,M,K] x [B,K,N].  f16 x f16 (or q8 columns) runs on the f16 matrix
// cores; an operand the pipeline holds in f32 runs on the f32 ones (the
// encoder's GEMM; q8 weights are dequantized while staging).
bool step_matmul(Run& r, const Step& s, Val* out) {
    if (s.inputs.size() != 2 || s.outputs.size() != 1)
        return r.fail("matmul step " + q(s.name) + " expects 2 inputs and 1 output");
    Val *lhs = nullptr, *rhs = nullptr;
    if (!r.tensor(s.inputs[0], &lhs) || !r.tensor(s.inputs[1], &rhs)) return false;
    if (lhs->kind == VK_DEFERRED || rhs->kind == VK_DEFERRED)
        return r.fail("a score folded into its top-k has no matrix to multiply");
    const size_t lr = lhs->shape.size(), rr = rhs->shape.size();
    if ((lr != 2 && lr != 3) || (rr != 2 && rr != 3)) return r.fail("matmul expects rank-2 or rank-3 tensor inputs");
    if (lr == 2 && rr != 2) return r.fail("matmul rank-2 lhs requires rank-2 rhs");
    const int64_t K = lhs->shape.back();
    const int64_t N = rhs->shape.back();
    if (rr == 2 && rhs->shape[0] != K)
        return r.fail("matmul mismatch " + go_shape(lhs->shape) + " x " + go_shape(rhs->shape));
    if (rr == 3 && (rhs->shape[0] != lhs->shape[0] || rhs->shape[1] != K))
        return r.fail("matmul mismatch " + go_shape(lhs->shape) + " x " + go_shape(rhs->shape));
    const int64_t M = lhs->elems() / (K ? K : 1);
    *out = Val();
    out->dtype = lhs->dtype;
    out->storage = MANTA_DT_F32;
    out->shape = lhs->shape;
    out->shape.back() = N;
    out->data = r.alloc((size_t)(M * N) * 4);
    if (!out->data) return r.fail("out of device memory");
    const bool lhs_f16 = lhs->kind == MANTA_VALUE_TENSOR && lhs->storage == MANTA_DT_F16;
    const bool rhs_q8 = rhs->kind == MANTA_VALUE_TENSOR && rhs->storage == MANTA_DT_Q8 && rr == 2;
    const bool rhs_f16 = rhs->kind == MANTA_VALUE_TENSOR && rhs->storage == MANTA_DT_F16 && rr == 2;
    if (lhs_f16 && (rhs_f16 || rhs_q8)) {
        char* e = nullptr;
        const bool prep = rhs->prep != nullptr;
        const int rc = manta_rocm_matmul_f16(
            r.p->rt, (const uint16_t*)lhs->data, M, K, prep ? rhs->prep : rhs->data,
            prep ? rhs->prep_kind : (rhs_q8 ? MANTA_ROCM_PROJ_Q8_COL : MANTA_ROCM_PROJ_F16),
            rhs_q8 ? (const float*)rhs->scales : nullptr, N, (float*)out->data, &e);
        if (rc != MANTA_ROCM_UNSUPPORTED) return r.abi(rc, e);
        free(e);  // a shape the f16 GEMM does not take: the f32 path below
    }
    if (M > 0x7FFFFFFF || N > 0x7FFFFFFF || K > 0x7FFFFFFF || (M + 63) / 64 > 65535)
        return r.unsupported("matmul shape beyond the device path");
    Val a;
    if (!r.f32_of(*lhs, &a, "matmul", false)) return false;
    if (rhs_q8)
        return r.hip(manta::launch_enc_gemm(1, (const float*)a.data, 0, rhs->data, (const float*)rhs->scales, 0,
                                            (float*)out->data, 0, (int)M, (int)N, (int)K, 1, r.s),
                     "matmul");
    Val b;
    if (!r.f32_of(*rhs, &b, "matmul", false)) return false;
    if (rr == 2)
        return r.hip(manta::launch_enc_gemm(0, (const float*)a.data, 0, b.data, nullptr, 0, (float*)out->data, 0,
                                            (int)M, (int)N, (int)K, 1, r.s),
                     "matmul");
    const int64_t B = lhs->shape[0], Mb = lhs->shape[1];
    if (B > 65535 || (Mb + 63) / 64 > 65535) return r.unsupported("batched matmul shape beyond the device path");
    return r.hip(manta::launch_enc_gemm(0, (const float*)a.data, Mb * K, b.data, nullptr, K * N, (float*)out->data,
                                        Mb * N, (int)Mb, (int)N, (int)K, (int)B, r.s),
                 "matmul");
}

// Finds the fused score + top-k pairs of an entry (see the file comment).
void plan_fusion(const Module& m, const EntryPoint& en, EntryPlan* plan) {
    const std::vector<int>& st = plan->steps;
    for (size_t a = 0; a < st.size(); a++) {
        const Step& s = m.steps[st[a]];
        if (s.kind != "launch_kernel" || s.outputs.size() != 1) continue;
        const Kernel* k = manta_mod::find_kernel(m, s.kernel);
        if (!k) continue;
        const KernelOp* op = single_op(*k);
        if (!op || !is_score_op(op->op)) continue;
        const std::string& sv = s.outputs[0];
        int topk = -1;
        std::vector<int> gathers;
        bool ok = true;
        for (size_t b = a + 1; b < st.size() && ok; b++) {
            const Step& u = m.steps[st[b]];
            bool uses = false;
            for (const auto& in : u.inputs) uses |= in == sv;
            for (const auto& o : u.outputs)
                if (o == sv && u.kind != "return") ok = false;  // the name is redefined
            if (u.kind == "return")
                for (const auto& o : u.outputs) ok &= o != sv;
            if (!uses || !ok) continue;
            if (u.kind == "topk" && topk < 0 && u.inputs.size() == 1 && u.outputs.size() == 1) {
                topk = (int)b;
            } else if (u.kind == "gather" && topk >= 0 && u.inputs.size() == 2 && u.inputs[0] == sv &&
                       u.inputs[1] == m.steps[st[topk]].outputs[0] && u.outputs.size() == 1 &&
                       resolve_type(m, en, u, 0, nullptr).shape.size() != 3) {
                // the element gather of each row's top scores (a declared
                // rank-3 output would make gatherTensor copy rows instead)
                gathers.push_back((int)b);
            } else {
                ok = false;
            }
        }
        if (!ok || topk < 0) continue;
        plan->fused_topk[(int)a] = topk;
        for (int g : gathers) plan->fused_gathers.insert(g);
    }
}

bool run_entry(Run& r) {
    MantaRocmProgram* p = r.p;
    const Module& m = p->m;
    const EntryPlan& plan = *r.plan;
    p->trace.clear();
    for (size_t i = 0; i < plan.steps.size(); i++) {
        r.step_pos = (int)i;
        const Step& s = m.steps[plan.steps[i]];
        for (const auto& in : s.inputs)
            if (!r.env.count(in))
                return r.fail("entrypoint " + q(r.en->name) + " step " + q(s.name) + " missing runtime input " + q(in));
        std::vector<Val> values;
        std::string dispatch;
        bool ok = true;
        if (s.kind == "alias") {
            if (s.inputs.size() != 1 || s.outputs.size() != 1) {
                ok = r.fail("alias step " + q(s.name) + " expects 1 input and 1 output");
            } else {
                values.push_back(r.env[s.inputs[0]]);
                dispatch = "alias";
            }
        } else if (s.kind == "gather") {
            Val out;
            if (plan.fused_gathers.count((int)i) && r.env[s.inputs[0]].kind == VK_DEFERRED &&
                r.fused.count(s.inputs[0])) {
                values.push_back(r.fused[s.inputs[0]]);
                dispatch = "fused:topk";
            } else {
                ok = step_gather(r, m, s, &out);
                values.push_back(out);
                dispatch = "hip:gather";
            }
        } else if (s.kind == "pack_candidates") {
            if (s.inputs.size() != 3 || s.outputs.size() != 1) {
                ok = r.fail("pack_candidates step " + q(s.name) + " expects 3 inputs and 1 output");
            } else {
                Val *ids = nullptr, *sc = nullptr, *docs = nullptr;
                ok = r.tensor(s.inputs[0], &ids) && r.tensor(s.inputs[1], &sc) && r.tensor(s.inputs[2], &docs);
                if (ok && (docs->kind != MANTA_VALUE_ROWS || ids->kind != MANTA_VALUE_TENSOR ||
                           sc->kind != MANTA_VALUE_TENSOR))
                    ok = r.unsupported("pack_candidates of dense docs is not offered by the rocm executor");
                if (ok) {
                    Val pk = *docs;
                    pk.kind = MANTA_VALUE_CANDIDATE_PACK;
                    pk.ids = ids->data;
                    pk.ids_storage = ids->storage;
                    pk.scores = sc->data;
                    values.push_back(pk);
                    dispatch = "pack";
                }
            }
        } else if (s.kind == "matmul") {
            Val out;
            ok = step_matmul(r, s, &out);
            values.push_back(out);
            dispatch = "hip:matmul";
        } else if (s.kind == "topk") {
            Val out;
            ok = step_topk(r, s, &out, &dispatch);
            values.push_back(out);
        } else if (s.kind == "dequant") {
            if (s.inputs.size() != 1 || s.outputs.size() != 1) {
                ok = r.fail("dequant step " + q(s.name) + " expects 1 input and 1 output");
            } else {
                // the reference relabels a clone f16 (tensor_ops.go:416-428):
                // dense values pass as they are (a q8 tensor stays codes +
                // column scales until a step needs its f32 values), gathered
                // q8 rows become their f32 products
                Val* in = nullptr;
                ok = r.tensor(s.inputs[0], &in);
                Val v;
                if (ok && in->kind == MANTA_VALUE_TENSOR) {
                    v = *in;
                    dispatch = "alias";
                } else if (ok && in->kind == MANTA_VALUE_ROWS && in->storage == MANTA_DT_Q8) {
                    ok = r.f32_of(*in, &v, "dequant", false);
                    dispatch = "hip:dequant";
                } else if (ok) {
                    ok = r.unsupported("dequant of " + in->dtype + " values is not offered by the rocm executor");
                }
                if (ok) {
                    v.dtype = "f16";
                    values.push_back(v);
                }
            }
        } else if (s.kind == "launch_kernel") {
            const Kernel* k = manta_mod::find_kernel(m, s.kernel);
            if (!k) {
                ok = r.fail("entrypoint " + q(r.en->name) + " step " + q(s.name) + " references unknown kernel " +
                            q(s.kernel));
            } else {
                std::vector<Val*> args;
                for (const auto& in : s.inputs) {
                    Val* v = nullptr;
                    if (!r.tensor(in, &v)) {
                        ok = false;
                        break;
                    }
                    args.push_back(v);
                }
                auto fz = plan.fused_topk.find((int)i);
                if (ok && fz != plan.fused_topk.end()) {
                    // deferred to the topk step; the layout is checked now, as
                    // the reference scores here
                    const KernelOp* op = single_op(*k);
                    Val *qv = nullptr, *dv = nullptr;
                    std::map<std::string, Val*> loc;
                    for (size_t j = 0; j < k->inputs.size() && j < args.size(); j++) loc[k->inputs[j].name] = args[j];
                    if (op->inputs.size() < 2 || !loc.count(op->inputs[0]) || !loc.count(op->inputs[1])) {
                        ok = r.fail("kernel " + q(k->name) + " op " + q(op->op) + ": malformed score op");
                    } else {
                        qv = loc[op->inputs[0]];
                        dv = loc[op->inputs[1]];
                        int64_t nq = 0;
                        ok = score_layout(r, *qv, *dv, &nq);
                        if (!ok && r.code == MANTA_ROCM_ERROR)
                            r.err = "kernel " + q(k->name) + " op " + q(op->op) + ": " + r.err;
                    }
                    if (ok) {
                        Val d;
                        d.kind = VK_DEFERRED;
                        d.dtype = "f32";
                        d.storage = MANTA_DT_F32;
                        const int64_t n = dv->shape[dv->shape.size() - 2];
                        d.shape = qv->shape.size() == 1 ? std::vector<int64_t>{n}
                                                        : std::vector<int64_t>{qv->shape[0], n};
                        d.op = score_op_code(op->op);
                        // the deferred score reads its operands at the topk step
                        d.qname = "\x01q" + s.outputs[0];
                        d.dname = "\x01d" + s.outputs[0];
                        r.env[d.qname] = *qv;
                        r.env[d.dname] = *dv;
                        values.push_back(d);
                        dispatch = "fused:" + m.steps[plan.steps[fz->second]].name;
                    }
                } else if (ok) {
                    ok = run_kernel(r, *k, args, &values);
                    dispatch = "hip:" + k->name;
                }
            }
        } else if (s.kind == "transpose") {
            Val out;
            ok = step_transpose(r, s, &out);
            values.push_back(out);
            dispatch = "hip:transpose";
        } else if (s.kind == "return") {
            dispatch = "return";
        } else if (s.kind == "kv_read" || s.kind == "kv_write" || s.kind == "conv2d" ||
                   s.kind == "conv2d_transpose" || s.kind == "gdn" || s.kind == "igdn" ||
                   s.kind == "turboquant_encode" || s.kind == "turboquant_decode" ||
                   s.kind == "cross_entropy_factorized" || s.kind == "mse_loss" || s.kind == "ms_ssim_loss" ||
                   s.kind == "scalar_add" || s.kind == "rate_distortion_loss") {
            ok = r.unsupported("step kind " + q(s.kind) + " is not offered by the rocm executor");
        } else {
            dispatch = "none";  // executeStep's default: no values
        }
        if (!ok) {
            if (r.code == MANTA_ROCM_ERROR)
                r.err = "entrypoint " + q(r.en->name) + " step " + q(s.name) + ": " + r.err;
            return false;
        }
        p->trace.push_back({s.kind, s.name, dispatch});
        if (s.kind == "return") continue;
        if (values.size() < s.outputs.size())
            return r.fail("entrypoint " + q(r.en->name) + " step " + q(s.name) + ": " +
                          fmt("step produced %d values for %d outputs", (int)values.size(), (int)s.outputs.size()));
        for (size_t j = 0; j < s.outputs.size(); j++) {
            Val v = values[j];
            // makeTensorValue: the artifact's type for the output
            const ValueType t = resolve_type(m, *r.en, s, j, nullptr);
            if (v.kind != MANTA_VALUE_CANDIDATE_PACK && t.has_tensor && !t.dtype.empty()) v.dtype = t.dtype;
            r.env[s.outputs[j]] = v;
        }
    }
    return true;
}

}  // namespace

// ------------------------------------------------------------------ C ABI

extern "C" {

int manta_rocm_program_load(MantaRocm* rt, const MantaModule* mod, MantaRocmProgram** out, char** err) {
    if (!out) return set_err(err, MANTA_ROCM_ERROR, "nil output handle");
    *out = nullptr;
    if (!rt) return set_err(err, MANTA_ROCM_ERROR, "nil rocm runtime");
    if (!mod) return set_err(err, MANTA_ROCM_ERROR, "nil module");
    std::string e;
    if (!manta_mod::validate(mod->m, &e)) return set_err(err, MANTA_ROCM_ERROR, e);
    bool supported = false;
    for (const auto& b : mod->m.supported_backends) supported |= b == "rocm" || b == "cuda";
    if (!supported) return set_err(err, MANTA_ROCM_UNSUPPORTED, "rocm: unsupported backend");
    auto* p = new MantaRocmProgram();
    p->rt = rt;
    p->m = mod->m;
    for (const auto& en : p->m.entry_points) {
        if (p->plans.count(en.name)) continue;
        EntryPlan& plan = p->plans[en.name];
        for (size_t i = 0; i < p->m.steps.size(); i++)
            if (p->m.steps[i].entry == en.name) plan.steps.push_back((int)i);
        plan_fusion(p->m, en, &plan);
    }
    *out = p;
    return MANTA_ROCM_OK;
}

void manta_rocm_program_destroy(MantaRocmProgram* p) {
    if (!p) return;
    for (auto& kv : p->weights)
        if (kv.second.prep) (void)hipFree(kv.second.prep);
    for (auto& kv : p->plans) {
        for (auto& b : kv.second.pool)
            if (b.p) (void)hipFree(b.p);
        if (kv.second.errs.p) (void)hipFree(kv.second.errs.p);
    }
    delete p;
}

int manta_rocm_program_bind(MantaRocmProgram* p, const MantaRocmValue* value, char** err) {
    if (!p) return set_err(err, MANTA_ROCM_ERROR, "nil program");
    if (!value || !value->name) return set_err(err, MANTA_ROCM_ERROR, "nil value");
    const manta_mod::Param* param = manta_mod::find_param(p->m, value->name);
    if (!param) return set_err(err, MANTA_ROCM_ERROR, "unknown param " + q(value->name));
    Val v;
    std::string e;
    if (!import_value(*value, &v, &e)) return set_err(err, MANTA_ROCM_ERROR, "param " + q(value->name) + ": " + e);
    // an f16 or q8-column [K, N] weight the pipelined f16 GEMM takes is
    // transposed once here, not on every matmul step
    if (v.kind == MANTA_VALUE_TENSOR && v.shape.size() == 2 &&
        (v.storage == MANTA_DT_F16 || v.storage == MANTA_DT_Q8) && v.shape[0] % 32 == 0 && v.shape[1] % 128 == 0 &&
        v.shape[1] <= 4096) {
        void* prep = nullptr;
        if (hipMalloc(&prep, (size_t)(v.shape[0] * v.shape[1]) * 2) == hipSuccess) {
            int kind = -1;
            char* pe = nullptr;
            const int rc = manta_rocm_prepare_projection(
                p->rt, v.data, v.storage == MANTA_DT_Q8 ? MANTA_ROCM_PROJ_Q8_COL : MANTA_ROCM_PROJ_F16, v.shape[0],
                v.shape[1], (uint16_t*)prep, &kind, &pe);
            free(pe);
            if (rc == MANTA_ROCM_OK) {
                v.prep = prep;
                v.prep_kind = kind;
            } else {
                (void)hipFree(prep);
            }
        } else {
            (void)hipGetLastError();  // no room: matmul steps transpose per call
        }
    }
    auto old = p->weights.find(value->name);
    if (old != p->weights.end() && old->second.prep) {
        // the previous binding's copy may still be read by queued work
        (void)hipStreamSynchronize((hipStream_t)manta_rt::runtime_stream(p->rt));
        (void)hipFree(old->second.prep);
    }
    p->weights[value->name] = v;
    return MANTA_ROCM_OK;
}

int manta_rocm_program_supports(const MantaRocmProgram* p, const char* entry, char** err) {
    if (!p) return set_err(err, MANTA_ROCM_ERROR, "nil program");
    const std::string name = entry ? entry : "";
    const EntryPoint* en = manta_mod::find_entry(p->m, name);
    if (!en) return set_err(err, MANTA_ROCM_ERROR, "unknown entrypoint " + q(name));
    static const std::set<std::string> steps = {"alias", "gather", "pack_candidates", "matmul", "topk",
                                                "dequant", "transpose", "launch_kernel", "return"};
    static const std::set<std::string> ops = {"normalize", "rmsnorm", "mean_pool", "dot", "cosine", "l2_distance",
                                              "softmax", "layernorm", "gelu", "binary_add", "binary_sub",
                                              "binary_mul", "binary_div"};
    for (const auto& s : p->m.steps) {
        if (s.entry != name) continue;
        if (!steps.count(s.kind))
            return set_err(err, MANTA_ROCM_UNSUPPORTED,
                           "step " + q(s.name) + " of kind " + q(s.kind) + " is not offered by the rocm executor");
        if (s.kind != "launch_kernel") continue;
        const Kernel* k = manta_mod::find_kernel(p->m, s.kernel);
        if (!k) continue;
        for (const auto& op : k->body)
            if (op.kind != "return" && !ops.count(op.op))
                return set_err(err, MANTA_ROCM_UNSUPPORTED,
                               "kernel " + q(k->name) + " op " + q(op.op) + " is not offered by the rocm executor");
    }
    for (const auto& in : en->inputs)
        if (in.type.kind != "tensor")
            return set_err(err, MANTA_ROCM_UNSUPPORTED,
                           "input " + q(in.name) + " of kind " + q(in.type.kind) + " is not offered by the rocm executor");
    return MANTA_ROCM_OK;
}

int manta_rocm_program_run(MantaRocmProgram* p, const char* entry, const MantaRocmValue* inputs, int64_t n_inputs,
                           MantaRocmValue* outputs, int64_t max_outputs, int64_t* n_outputs, char** err) {
    if (!p) return set_err(err, MANTA_ROCM_ERROR, "nil program");
    if (n_outputs) *n_outputs = 0;
    if (n_inputs < 0 || (n_inputs > 0 && !inputs)) return set_err(err, MANTA_ROCM_ERROR, "nil inputs");
    if (hipSetDevice(manta_rt::runtime_device(p->rt)) != hipSuccess)
        return set_err(err, MANTA_ROCM_ERROR, "hipSetDevice failed");
    const Module& m = p->m;
    const std::string name = entry ? entry : "";
    const EntryPoint* en = manta_mod::find_entry(m, name);
    if (!en) return set_err(err, MANTA_ROCM_ERROR, "unknown entrypoint " + q(name));
    // validateRequestInputs (symbolic.go:265-277)
    for (const auto& in : en->inputs) {
        bool given = false;
        for (int64_t i = 0; i < n_inputs; i++) given |= inputs[i].name && in.name == inputs[i].name;
        if (!given) return set_err(err, MANTA_ROCM_ERROR, "entrypoint " + q(name) + " missing input " + q(in.name));
    }
    for (int64_t i = 0; i < n_inputs; i++) {
        bool declared = false;
        for (const auto& in : en->inputs) declared |= inputs[i].name && in.name == inputs[i].name;
        if (!declared)
            return set_err(err, MANTA_ROCM_ERROR,
                           "entrypoint " + q(name) + " does not declare input " + q(inputs[i].name ? inputs[i].name : ""));
    }
    Run r;
    r.p = p;
    r.plan = &p->plans[en->name];
    r.en = en;
    r.s = (hipStream_t)manta_rt::runtime_stream(p->rt);
    std::string e;
    bool unsupported = false;
    // params, eagerly (shouldEagerMaterializeParam for device-resident weights)
    for (const auto& param : m.params) {
        auto it = p->weights.find(param.name);
        if (it == p->weights.end())
            return set_err(err, MANTA_ROCM_ERROR, "missing weight binding for param " + q(param.name));
        if (!check_value(param.type, it->second, &r.bindings, &e, &unsupported))
            return set_err(err, unsupported ? MANTA_ROCM_UNSUPPORTED : MANTA_ROCM_ERROR,
                           "param " + q(param.name) + ": " + e);
        Val v = it->second;
        v.dtype = param.type.dtype.empty() ? v.dtype : param.type.dtype;
        r.env[param.name] = v;
    }
    for (const auto& in : en->inputs) {
        const MantaRocmValue* given = nullptr;
        for (int64_t i = 0; i < n_inputs; i++)
            if (inputs[i].name && in.name == inputs[i].name) given = &inputs[i];
        Val v;
        if (!import_value(*given, &v, &e)) return set_err(err, MANTA_ROCM_ERROR, "input " + q(in.name) + ": " + e);
        if (!check_value(in.type, v, &r.bindings, &e, &unsupported))
            return set_err(err, unsupported ? MANTA_ROCM_UNSUPPORTED : MANTA_ROCM_ERROR, "input " + q(in.name) + ": " + e);
        r.env[in.name] = v;
    }
    if (r.plan->steps.empty()) return set_err(err, MANTA_ROCM_ERROR, "entrypoint " + q(name) + " has no plan steps");
    // one gather error word per step, cleared
    const size_t ebytes = r.plan->steps.size() * sizeof(unsigned long long);
    if (r.plan->errs.cap < ebytes) {
        if (r.plan->errs.p) (void)hipFree(r.plan->errs.p);
        r.plan->errs.p = nullptr;
        r.plan->errs.cap = 0;
        if (hipMalloc(&r.plan->errs.p, ebytes) != hipSuccess) return set_err(err, MANTA_ROCM_ERROR, "out of device memory");
        r.plan->errs.cap = ebytes;
    }
    if (hipMemsetAsync(r.plan->errs.p, 0, ebytes, r.s) != hipSuccess)
        return set_err(err, MANTA_ROCM_ERROR, "hipMemsetAsync failed");
    const bool ok = run_entry(r);
    // drain the stream whatever happened: buffers may be reused next run
    const hipError_t se = hipStreamSynchronize(r.s);
    if (!ok) return set_err(err, r.code, r.err);
    if (se != hipSuccess) return set_err(err, MANTA_ROCM_ERROR, std::string("run: ") + hipGetErrorString(se));
    std::vector<unsigned long long> words(r.plan->steps.size());
    if (hipMemcpy(words.data(), r.plan->errs.p, ebytes, hipMemcpyDeviceToHost) != hipSuccess)
        return set_err(err, MANTA_ROCM_ERROR, "reading gather errors failed");
    for (size_t i = 0; i < words.size(); i++)
        if (words[i])
            return set_err(err, MANTA_ROCM_ERROR,
                           "entrypoint " + q(name) + " step " + q(m.steps[r.plan->steps[i]].name) + ": " +
                               fmt("gather index %d out of range", manta_rt::gather_error_index(words[i])));
    // the return step's values, in the entry's declaration order
    std::map<std::string, Val> result;
    for (int si : r.plan->steps) {
        const Step& s = m.steps[si];
        if (s.kind != "return") continue;
        for (const auto& o : s.outputs) {
            auto it = r.env.find(o);
            if (it == r.env.end())
                return set_err(err, MANTA_ROCM_ERROR, "entrypoint " + q(name) + " return references unknown value " + q(o));
            result[o] = it->second;
        }
    }
    if (result.empty()) return set_err(err, MANTA_ROCM_ERROR, "entrypoint " + q(name) + " produced no outputs");
    int64_t n = 0;
    for (const auto& o : en->outputs) {
        auto it = result.find(o.name);
        if (it == result.end()) continue;
        if (n >= max_outputs) return set_err(err, MANTA_ROCM_ERROR, "output array too small");
        const Val& v = it->second;
        MantaRocmValue& out = outputs[n++];
        memset(&out, 0, sizeof out);
        out.name = o.name.c_str();
        out.kind = v.kind == VK_DEFERRED ? MANTA_VALUE_TENSOR : v.kind;
        out.dtype = dtype_code(v.dtype);
        out.storage = v.storage;
        out.rank = (int)v.shape.size();
        for (int i = 0; i < out.rank && i < 4; i++) out.shape[i] = v.shape[i];
        out.data = v.data;
        out.scales = v.scales;
        out.ids = v.ids;
        out.scores = v.scores;
        out.ids_dtype = v.ids_storage;
        out.candidates = v.cands;
    }
    if (n_outputs) *n_outputs = n;
    return MANTA_ROCM_OK;
}

int64_t manta_rocm_program_trace_count(const MantaRocmProgram* p) { return p ? (int64_t)p->trace.size() : 0; }

int manta_rocm_program_trace_step(const MantaRocmProgram* p, int64_t index, const char** kind, const char** name,
                                  const char** dispatch) {
    if (!p || index < 0 || index >= (int64_t)p->trace.size()) return MANTA_ROCM_ERROR;
    const TraceStep& t = p->trace[(size_t)index];
    if (kind) *kind = t.kind.c_str();
    if (name) *name = t.name.c_str();
    if (dispatch) *dispatch = t.dispatch.c_str();
    return MANTA_ROCM_OK;
}

}  // extern "C"
