// module.cpp -- the Manta artifact (module) codec and checks, host only.
//
//   * decode: JSON -> Module with json.Unmarshal's field rules (JSON names
//     from the struct tags of artifact/manta/module.go:85-207, unknown keys
//     ignored, null leaves a field unset, case-insensitive key match) and
//     its type-error wording, then Module.Validate (module.go:255-424)
//     restated check for check with the same messages;
//   * encode: Validate, then MarshalIndent(m, "", "  ") field order and
//     omitempty rules (module.go:486-492);
//   * containers: the XMTA section of an MLL container holds MLLMetadata
//     JSON whose "artifact" member is the module (mll.go:15-88, 291-305);
//     manta_module_encode_mll writes such a container;
//   * serving contracts: validateScoreEntry / validateRetrievalEntry /
//     validateEmbeddingEntry / validateEmbeddingParam (score_model.go:
//     276-324, retrieval_model.go:274-330, embedding_model.go:734-800) and
//     the manifests' normalized() defaults + ValidateModule.
#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <set>
#include <string>
#include <vector>

#include "manta_mll.h"
#include "manta_module.h"
#include "manta_rocm.h"
#include "mll_internal.hpp"
#include "module_internal.hpp"

using mjson::Kind;
using mjson::Value;

namespace {

int set_err(char** err, int code, const std::string& msg) {
    if (err) {
        *err = (char*)malloc(msg.size() + 1);
        if (*err) memcpy(*err, msg.c_str(), msg.size() + 1);
    }
    return code;
}

// Go's %q for the strings that occur here.
std::string q(const std::string& s) {
    std::string o = "\"";
    for (unsigned char c : s) {
        if (c == '"' || c == '\\') {
            o.push_back('\\');
            o.push_back((char)c);
        } else if (c == '\n') {
            o += "\\n";
        } else if (c == '\t') {
            o += "\\t";
        } else if (c == '\r') {
            o += "\\r";
        } else if (c < 0x20 || c == 0x7f) {
            char b[8];
            snprintf(b, sizeof b, "\\x%02x", c);
            o += b;
        } else {
            o.push_back((char)c);
        }
    }
    return o + "\"";
}

std::string fmt(const char* f, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    return buf;
}

// ------------------------------------------------------------------ decoding

struct Dec {
    std::string root;  // Go type of the decoded value, e.g. "Module"
    std::string err;

    bool type_error(const Value& v, const std::string& path, const char* go_type) {
        if (!err.empty()) return false;
        std::string what = v.kind_name();
        if (v.kind == Kind::Number && std::string(go_type) == "int") what = "number " + v.text;
        err = "json: cannot unmarshal " + what + " into Go struct field " + root + "." + path + " of type " +
              go_type;
        return false;
    }
    bool str(const Value* v, const std::string& path, std::string* out) {
        if (!v || v->kind == Kind::Null) return true;
        if (v->kind != Kind::String) return type_error(*v, path, "string");
        *out = v->text;
        return true;
    }
    bool boolean(const Value* v, const std::string& path, bool* out) {
        if (!v || v->kind == Kind::Null) return true;
        if (v->kind != Kind::Bool) return type_error(*v, path, "bool");
        *out = v->b;
        return true;
    }
    bool integer(const Value* v, const std::string& path, long long* out) {
        if (!v || v->kind == Kind::Null) return true;
        if (v->kind != Kind::Number || v->text.find_first_of(".eE") != std::string::npos)
            return type_error(*v, path, "int");
        errno = 0;
        char* end = nullptr;
        const long long x = strtoll(v->text.c_str(), &end, 10);
        if (errno != 0) return type_error(*v, path, "int");
        *out = x;
        return true;
    }
    bool strs(const Value* v, const std::string& path, std::vector<std::string>* out, bool* was_null = nullptr) {
        if (!v || v->kind == Kind::Null) {
            if (v) out->clear();
            return true;
        }
        if (v->kind != Kind::Array) return type_error(*v, path, "[]string");
        out->clear();
        if (was_null) *was_null = false;
        for (const auto& it : v->items) {
            std::string s;
            if (!str(&it, path, &s)) return false;
            out->push_back(s);
        }
        return true;
    }
    bool ints(const Value* v, const std::string& path, std::vector<long long>* out) {
        if (!v || v->kind == Kind::Null) {
            if (v) out->clear();
            return true;
        }
        if (v->kind != Kind::Array) return type_error(*v, path, "[]int");
        out->clear();
        for (const auto& it : v->items) {
            long long x = 0;
            if (!integer(&it, path, &x)) return false;
            out->push_back(x);
        }
        return true;
    }
    bool strmap(const Value* v, const std::string& path, manta_mod::StrMap* out) {
        if (!v || v->kind == Kind::Null) {
            if (v) out->clear();
            return true;
        }
        if (v->kind != Kind::Object) return type_error(*v, path, "map[string]string");
        for (const auto& kv : v->members) {
            std::string s;
            if (!str(&kv.second, path + "." + kv.first, &s)) return false;
            (*out)[kv.first] = s;
        }
        return true;
    }
    // An object-valued field: null/absent -> skip (false `present`).
    bool object(const Value* v, const std::string& path, const char* go_type, bool* present) {
        *present = false;
        if (!v || v->kind == Kind::Null) return true;
        if (v->kind != Kind::Object) return type_error(*v, path, go_type);
        *present = true;
        return true;
    }
    bool array(const Value* v, const std::string& path, const char* go_type, bool* present) {
        *present = false;
        if (!v || v->kind == Kind::Null) return true;
        if (v->kind != Kind::Array) return type_error(*v, path, go_type);
        *present = true;
        return true;
    }

    bool value_type(const Value* v, const std::string& path, manta_mod::ValueType* t) {
        bool present = false;
        if (!object(v, path, "manta.ValueType", &present)) return false;
        if (!present) return true;
        if (!str(v->get("kind"), path + ".kind", &t->kind)) return false;
        const Value* tv = v->get("tensor");
        if (!object(tv, path + ".tensor", "manta.TensorType", &present)) return false;
        if (present) {
            t->has_tensor = true;
            if (!str(tv->get("dtype"), path + ".tensor.dtype", &t->dtype)) return false;
            if (!strs(tv->get("shape"), path + ".tensor.shape", &t->shape)) return false;
        }
        const Value* pv = v->get("candidate_pack");
        if (!object(pv, path + ".candidate_pack", "manta.CandidatePackType", &present)) return false;
        if (present) {
            t->has_pack = true;
            if (!strs(pv->get("shape"), path + ".candidate_pack.shape", &t->pack_shape)) return false;
        }
        return true;
    }
    bool bindings(const Value* v, const std::string& path, std::vector<manta_mod::ValueBinding>* out) {
        bool present = false;
        if (!array(v, path, "[]manta.ValueBinding", &present)) return false;
        if (!v) return true;
        out->clear();
        if (!present) return true;
        for (const auto& it : v->items) {
            bool p2 = false;
            if (!object(&it, path, "manta.ValueBinding", &p2)) return false;
            manta_mod::ValueBinding b;
            if (p2) {
                if (!str(it.get("name"), path + ".name", &b.name)) return false;
                if (!value_type(it.get("type"), path + ".type", &b.type)) return false;
            }
            out->push_back(b);
        }
        return true;
    }
};

const char* kVersion = "manta/v0alpha1";
const char* kMLLMetadataVersion = "manta/mll/v0alpha1";

}  // namespace

namespace manta_mod {

bool decode_value(const Value& v, Module* m, std::string* err) {
    *m = Module();
    Dec d;
    d.root = "Module";
    if (v.kind == Kind::Null) return true;
    if (v.kind != Kind::Object) {
        *err = std::string("json: cannot unmarshal ") + v.kind_name() + " into Go value of type manta.Module";
        return false;
    }
    bool present = false;
    auto done = [&]() {
        *err = d.err;
        return false;
    };
    if (!d.str(v.get("version"), "version", &m->version)) return done();
    if (!d.str(v.get("name"), "name", &m->name)) return done();
    const Value* pv = v.get("params");
    if (!d.array(pv, "params", "[]manta.Param", &present)) return done();
    if (present)
        for (const auto& it : pv->items) {
            bool p2 = false;
            if (!d.object(&it, "params", "manta.Param", &p2)) return done();
            Param p;
            if (p2) {
                if (!d.str(it.get("name"), "params.name", &p.name)) return done();
                if (!d.value_type(it.get("type"), "params.type", &p.type)) return done();
                if (!d.str(it.get("binding"), "params.binding", &p.binding)) return done();
                if (!d.boolean(it.get("trainable"), "params.trainable", &p.trainable)) return done();
            }
            m->params.push_back(p);
        }
    const Value* ev = v.get("entry_points");
    if (!d.array(ev, "entry_points", "[]manta.EntryPoint", &present)) return done();
    if (present) {
        m->entry_points_null = false;
        for (const auto& it : ev->items) {
            bool p2 = false;
            if (!d.object(&it, "entry_points", "manta.EntryPoint", &p2)) return done();
            EntryPoint e;
            if (p2) {
                if (!d.str(it.get("name"), "entry_points.name", &e.name)) return done();
                if (!d.str(it.get("kind"), "entry_points.kind", &e.kind)) return done();
                if (!d.bindings(it.get("inputs"), "entry_points.inputs", &e.inputs)) return done();
                if (!d.bindings(it.get("outputs"), "entry_points.outputs", &e.outputs)) return done();
            }
            m->entry_points.push_back(e);
        }
    }
    const Value* rv = v.get("requirements");
    if (!d.object(rv, "requirements", "manta.Requirements", &present)) return done();
    if (present) {
        const Value* sb = rv->get("supported_backends");
        bool was_null = true;
        if (!d.strs(sb, "requirements.supported_backends", &m->supported_backends, &was_null)) return done();
        m->supported_backends_null = was_null;
        if (!d.strs(rv->get("capabilities"), "requirements.capabilities", &m->capabilities)) return done();
    }
    const Value* bv = v.get("buffers");
    if (!d.array(bv, "buffers", "[]manta.Buffer", &present)) return done();
    if (present)
        for (const auto& it : bv->items) {
            bool p2 = false;
            if (!d.object(&it, "buffers", "manta.Buffer", &p2)) return done();
            Buffer b;
            if (p2) {
                if (!d.str(it.get("name"), "buffers.name", &b.name)) return done();
                if (!d.str(it.get("dtype"), "buffers.dtype", &b.dtype)) return done();
                if (!d.strs(it.get("shape"), "buffers.shape", &b.shape)) return done();
                if (!d.str(it.get("storage_class"), "buffers.storage_class", &b.storage_class)) return done();
            }
            m->buffers.push_back(b);
        }
    const Value* kv = v.get("kernels");
    if (!d.array(kv, "kernels", "[]manta.Kernel", &present)) return done();
    if (present)
        for (const auto& it : kv->items) {
            bool p2 = false;
            if (!d.object(&it, "kernels", "manta.Kernel", &p2)) return done();
            Kernel k;
            if (p2) {
                if (!d.str(it.get("name"), "kernels.name", &k.name)) return done();
                if (!d.bindings(it.get("inputs"), "kernels.inputs", &k.inputs)) return done();
                if (!d.bindings(it.get("outputs"), "kernels.outputs", &k.outputs)) return done();
                const Value* hv = it.get("hints");
                bool p3 = false;
                if (!d.object(hv, "kernels.hints", "manta.ScheduleHints", &p3)) return done();
                if (p3) {
                    Hints& h = k.hints;
                    if (!d.ints(hv->get("tile"), "kernels.hints.tile", &h.tile)) return done();
                    if (!d.ints(hv->get("tile_2d"), "kernels.hints.tile_2d", &h.tile_2d)) return done();
                    if (!d.integer(hv->get("vector_width"), "kernels.hints.vector_width", &h.vector_width))
                        return done();
                    if (!d.boolean(hv->get("subgroup"), "kernels.hints.subgroup", &h.subgroup)) return done();
                    if (!d.ints(hv->get("subgroup_2d"), "kernels.hints.subgroup_2d", &h.subgroup_2d)) return done();
                    if (!d.ints(hv->get("halo"), "kernels.hints.halo", &h.halo)) return done();
                    if (!d.str(hv->get("memory"), "kernels.hints.memory", &h.memory)) return done();
                }
                const Value* body = it.get("body");
                if (!d.array(body, "kernels.body", "[]manta.KernelOp", &p3)) return done();
                if (p3)
                    for (const auto& ot : body->items) {
                        bool p4 = false;
                        if (!d.object(&ot, "kernels.body", "manta.KernelOp", &p4)) return done();
                        KernelOp op;
                        if (p4) {
                            if (!d.str(ot.get("kind"), "kernels.body.kind", &op.kind)) return done();
                            if (!d.str(ot.get("name"), "kernels.body.name", &op.name)) return done();
                            if (!d.str(ot.get("op"), "kernels.body.op", &op.op)) return done();
                            if (!d.strs(ot.get("inputs"), "kernels.body.inputs", &op.inputs)) return done();
                            if (!d.strs(ot.get("outputs"), "kernels.body.outputs", &op.outputs)) return done();
                            if (!d.strmap(ot.get("attributes"), "kernels.body.attributes", &op.attributes))
                                return done();
                        }
                        k.body.push_back(op);
                    }
                const Value* vars = it.get("variants");
                if (!d.array(vars, "kernels.variants", "[]manta.KernelVariant", &p3)) return done();
                if (p3)
                    for (const auto& vt : vars->items) {
                        bool p4 = false;
                        if (!d.object(&vt, "kernels.variants", "manta.KernelVariant", &p4)) return done();
                        KernelVariant kvar;
                        if (p4) {
                            if (!d.str(vt.get("backend"), "kernels.variants.backend", &kvar.backend)) return done();
                            if (!d.str(vt.get("entry"), "kernels.variants.entry", &kvar.entry)) return done();
                            if (!d.str(vt.get("source"), "kernels.variants.source", &kvar.source)) return done();
                            if (!d.strmap(vt.get("meta"), "kernels.variants.meta", &kvar.meta)) return done();
                        }
                        k.variants.push_back(kvar);
                    }
            }
            m->kernels.push_back(k);
        }
    const Value* sv = v.get("steps");
    if (!d.array(sv, "steps", "[]manta.Step", &present)) return done();
    if (present)
        for (const auto& it : sv->items) {
            bool p2 = false;
            if (!d.object(&it, "steps", "manta.Step", &p2)) return done();
            Step s;
            if (p2) {
                if (!d.str(it.get("entry"), "steps.entry", &s.entry)) return done();
                if (!d.str(it.get("kind"), "steps.kind", &s.kind)) return done();
                if (!d.str(it.get("name"), "steps.name", &s.name)) return done();
                if (!d.str(it.get("kernel"), "steps.kernel", &s.kernel)) return done();
                if (!d.strs(it.get("inputs"), "steps.inputs", &s.inputs)) return done();
                if (!d.strs(it.get("outputs"), "steps.outputs", &s.outputs)) return done();
                if (!d.strmap(it.get("attributes"), "steps.attributes", &s.attributes)) return done();
            }
            m->steps.push_back(s);
        }
    const Value* md = v.get("metadata");
    if (md && md->kind != Kind::Null) {
        if (md->kind != Kind::Object) {
            d.type_error(*md, "metadata", "map[string]interface {}");
            return done();
        }
        m->metadata = *md;
    }
    return true;
}

namespace {

// validateValueType (module.go:451-477)
bool validate_value_type(const ValueType& v, std::string* e) {
    if (v.kind == "tensor") {
        if (!v.has_tensor) return *e = "tensor metadata is required", false;
        if (v.dtype.empty()) return *e = "tensor dtype is required", false;
        return true;
    }
    if (v.kind == "kv_cache") return true;
    if (v.kind == "candidate_pack") {
        if (!v.has_pack) return *e = "candidate pack metadata is required", false;
        if (v.pack_shape.size() != 2 && v.pack_shape.size() != 3)
            return *e = "candidate pack shape rank must be 2 or 3", false;
        return true;
    }
    if (v.kind.empty()) return *e = "value kind is required", false;
    *e = "unsupported value kind " + q(v.kind);
    return false;
}

}  // namespace

bool validate(const Module& m, std::string* err) {
    std::string e;
    if (m.name.empty()) return *err = "module name is required", false;
    if (m.version.empty()) return *err = "module version is required", false;
    if (m.version != kVersion)
        return *err = "module version " + q(m.version) + " is not supported, want " + q(kVersion), false;
    if (m.supported_backends.empty()) return *err = "at least one supported backend is required", false;
    std::set<std::string> seen;
    for (const auto& kind : m.supported_backends) {
        if (kind.empty()) return *err = "supported backend is required", false;
        if (!seen.insert(kind).second) return *err = "duplicate supported backend " + q(kind), false;
    }
    seen.clear();
    for (const auto& cap : m.capabilities) {
        if (cap.empty()) return *err = "capability name is required", false;
        if (!seen.insert(cap).second) return *err = "duplicate capability " + q(cap), false;
    }
    for (const auto& p : m.params) {
        if (p.name.empty()) return *err = "param name is required", false;
        if (p.binding.empty()) return *err = "param " + q(p.name) + " binding is required", false;
        if (!validate_value_type(p.type, &e)) return *err = "param " + q(p.name) + ": " + e, false;
    }
    for (const auto& en : m.entry_points) {
        if (en.name.empty()) return *err = "entrypoint name is required", false;
        for (const auto& in : en.inputs) {
            if (in.name.empty()) return *err = "entrypoint " + q(en.name) + " input name is required", false;
            if (!validate_value_type(in.type, &e))
                return *err = "entrypoint " + q(en.name) + " input " + q(in.name) + ": " + e, false;
        }
        for (const auto& out : en.outputs) {
            if (out.name.empty()) return *err = "entrypoint " + q(en.name) + " output name is required", false;
            if (!validate_value_type(out.type, &e))
                return *err = "entrypoint " + q(en.name) + " output " + q(out.name) + ": " + e, false;
        }
    }
    for (const auto& b : m.buffers) {
        if (b.name.empty()) return *err = "buffer name is required", false;
        if (b.dtype.empty()) return *err = "buffer " + q(b.name) + " dtype is required", false;
    }
    for (const auto& k : m.kernels) {
        if (k.name.empty()) return *err = "kernel name is required", false;
        for (const auto& in : k.inputs) {
            if (in.name.empty()) return *err = "kernel " + q(k.name) + " input name is required", false;
            if (!validate_value_type(in.type, &e))
                return *err = "kernel " + q(k.name) + " input " + q(in.name) + ": " + e, false;
        }
        for (const auto& out : k.outputs) {
            if (out.name.empty()) return *err = "kernel " + q(k.name) + " output name is required", false;
            if (!validate_value_type(out.type, &e))
                return *err = "kernel " + q(k.name) + " output " + q(out.name) + ": " + e, false;
        }
        for (const auto& op : k.body)
            if (op.op.empty()) return *err = "kernel " + q(k.name) + " has body op with empty op name", false;
        // validateKernelVariants (module.go:426-449)
        std::set<std::string> vs;
        for (const auto& v : k.variants) {
            if (v.backend.empty()) return *err = "kernel " + q(k.name) + " variant backend is required", false;
            if (!vs.insert(v.backend).second)
                return *err = "kernel " + q(k.name) + " has duplicate variant for backend " + q(v.backend), false;
            if (v.entry.empty())
                return *err = "kernel " + q(k.name) + " variant entry is required for backend " + q(v.backend), false;
            if (v.source.empty())
                return *err = "kernel " + q(k.name) + " variant source is required for backend " + q(v.backend),
                       false;
        }
        for (const auto& b : m.supported_backends)
            if (!vs.count(b)) return *err = "kernel " + q(k.name) + " is missing variant for backend " + q(b), false;
    }
    // known values per entry: params, the entry's inputs, then step outputs
    std::map<std::string, std::set<std::string>> known;
    for (const auto& en : m.entry_points) {
        std::set<std::string>& k = known[en.name];
        k.clear();  // a repeated entry name: the last declaration's inputs
        for (const auto& p : m.params) k.insert(p.name);
        for (const auto& in : en.inputs) k.insert(in.name);
    }
    for (const auto& s : m.steps) {
        if (s.entry.empty()) return *err = "step " + q(s.name) + " entry is required", false;
        const EntryPoint* en = nullptr;
        for (const auto& cand : m.entry_points)
            if (cand.name == s.entry) en = &cand;  // the last one with the name
        if (!en) return *err = "step " + q(s.name) + " references unknown entrypoint " + q(s.entry), false;
        if (s.kind == "launch_kernel") {
            if (s.kernel.empty()) return *err = "launch_kernel step " + q(s.name) + " is missing kernel name", false;
            if (!find_kernel(m, s.kernel))
                return *err = "step " + q(s.name) + " references unknown kernel " + q(s.kernel), false;
        }
        std::set<std::string>& k = known[s.entry];
        for (const auto& in : s.inputs) {
            if (in.empty()) return *err = "step " + q(s.name) + " has empty input name", false;
            if (!k.count(in)) return *err = "step " + q(s.name) + " references unknown input " + q(in), false;
        }
        for (const auto& out : s.outputs) {
            if (out.empty()) return *err = "step " + q(s.name) + " has empty output name", false;
            if (s.kind == "return") {
                bool declared = false;
                for (const auto& o : en->outputs) declared |= o.name == out;
                if (!declared)
                    return *err = "return step " + q(s.name) + " output " + q(out) + " is not declared on entrypoint " +
                                  q(s.entry),
                           false;
                continue;
            }
            if (!find_buffer(m, out))
                return *err = "step " + q(s.name) + " output " + q(out) + " is missing a declared buffer", false;
            k.insert(out);
        }
    }
    return true;
}

bool decode_json(const char* p, size_t n, Module* m, std::string* err) {
    Value v;
    mjson::Parser parser(p, n);
    if (!parser.parse(&v, err)) return false;
    if (!decode_value(v, m, err)) return false;
    return validate(*m, err);
}

// -------------------------------------------------------------- encoding

namespace {

void put_strs(mjson::Writer* w, const std::vector<std::string>& v) {
    w->begin_array();
    for (const auto& s : v) w->str(s);
    w->end_array();
}
void put_ints(mjson::Writer* w, const std::vector<long long>& v) {
    w->begin_array();
    for (long long x : v) w->num(x);
    w->end_array();
}
void put_map(mjson::Writer* w, const StrMap& m) {
    w->begin_object();
    for (const auto& kv : m) {  // std::map: sorted keys, as Go writes maps
        w->key(kv.first.c_str());
        w->str(kv.second);
    }
    w->end_object();
}
void put_type(mjson::Writer* w, const ValueType& t) {
    w->begin_object();
    w->key("kind");
    w->str(t.kind);
    if (t.has_tensor) {
        w->key("tensor");
        w->begin_object();
        w->key("dtype");
        w->str(t.dtype);
        if (!t.shape.empty()) {
            w->key("shape");
            put_strs(w, t.shape);
        }
        w->end_object();
    }
    if (t.has_pack) {
        w->key("candidate_pack");
        w->begin_object();
        if (!t.pack_shape.empty()) {
            w->key("shape");
            put_strs(w, t.pack_shape);
        }
        w->end_object();
    }
    w->end_object();
}
void put_bindings(mjson::Writer* w, const char* key, const std::vector<ValueBinding>& v) {
    if (v.empty()) return;
    w->key(key);
    w->begin_array();
    for (const auto& b : v) {
        w->begin_object();
        w->key("name");
        w->str(b.name);
        w->key("type");
        put_type(w, b.type);
        w->end_object();
    }
    w->end_array();
}

}  // namespace

bool encode_json(const Module& m, std::string* out, std::string* err) {
    if (!validate(m, err)) return false;
    mjson::Writer w;
    w.begin_object();
    w.key("version");
    w.str(m.version);
    w.key("name");
    w.str(m.name);
    if (!m.params.empty()) {
        w.key("params");
        w.begin_array();
        for (const auto& p : m.params) {
            w.begin_object();
            w.key("name");
            w.str(p.name);
            w.key("type");
            put_type(&w, p.type);
            w.key("binding");
            w.str(p.binding);
            if (p.trainable) {
                w.key("trainable");
                w.boolean(true);
            }
            w.end_object();
        }
        w.end_array();
    }
    w.key("entry_points");
    if (m.entry_points_null && m.entry_points.empty()) {
        w.null();
    } else {
        w.begin_array();
        for (const auto& e : m.entry_points) {
            w.begin_object();
            w.key("name");
            w.str(e.name);
            w.key("kind");
            w.str(e.kind);
            put_bindings(&w, "inputs", e.inputs);
            put_bindings(&w, "outputs", e.outputs);
            w.end_object();
        }
        w.end_array();
    }
    w.key("requirements");
    w.begin_object();
    w.key("supported_backends");
    if (m.supported_backends_null && m.supported_backends.empty()) w.null();
    else put_strs(&w, m.supported_backends);
    if (!m.capabilities.empty()) {
        w.key("capabilities");
        put_strs(&w, m.capabilities);
    }
    w.end_object();
    if (!m.buffers.empty()) {
        w.key("buffers");
        w.begin_array();
        for (const auto& b : m.buffers) {
            w.begin_object();
            w.key("name");
            w.str(b.name);
            w.key("dtype");
            w.str(b.dtype);
            if (!b.shape.empty()) {
                w.key("shape");
                put_strs(&w, b.shape);
            }
            if (!b.storage_class.empty()) {
                w.key("storage_class");
                w.str(b.storage_class);
            }
            w.end_object();
        }
        w.end_array();
    }
    if (!m.kernels.empty()) {
        w.key("kernels");
        w.begin_array();
        for (const auto& k : m.kernels) {
            w.begin_object();
            w.key("name");
            w.str(k.name);
            put_bindings(&w, "inputs", k.inputs);
            put_bindings(&w, "outputs", k.outputs);
            w.key("hints");  // a struct: omitempty does not apply
            w.begin_object();
            const Hints& h = k.hints;
            if (!h.tile.empty()) {
                w.key("tile");
                put_ints(&w, h.tile);
            }
            if (!h.tile_2d.empty()) {
                w.key("tile_2d");
                put_ints(&w, h.tile_2d);
            }
            if (h.vector_width) {
                w.key("vector_width");
                w.num(h.vector_width);
            }
            if (h.subgroup) {
                w.key("subgroup");
                w.boolean(true);
            }
            if (!h.subgroup_2d.empty()) {
                w.key("subgroup_2d");
                put_ints(&w, h.subgroup_2d);
            }
            if (!h.halo.empty()) {
                w.key("halo");
                put_ints(&w, h.halo);
            }
            if (!h.memory.empty()) {
                w.key("memory");
                w.str(h.memory);
            }
            w.end_object();
            if (!k.body.empty()) {
                w.key("body");
                w.begin_array();
                for (const auto& op : k.body) {
                    w.begin_object();
                    w.key("kind");
                    w.str(op.kind);
                    if (!op.name.empty()) {
                        w.key("name");
                        w.str(op.name);
                    }
                    w.key("op");
                    w.str(op.op);
                    if (!op.inputs.empty()) {
                        w.key("inputs");
                        put_strs(&w, op.inputs);
                    }
                    if (!op.outputs.empty()) {
                        w.key("outputs");
                        put_strs(&w, op.outputs);
                    }
                    if (!op.attributes.empty()) {
                        w.key("attributes");
                        put_map(&w, op.attributes);
                    }
                    w.end_object();
                }
                w.end_array();
            }
            if (!k.variants.empty()) {
                w.key("variants");
                w.begin_array();
                for (const auto& v : k.variants) {
                    w.begin_object();
                    w.key("backend");
                    w.str(v.backend);
                    w.key("entry");
                    w.str(v.entry);
                    if (!v.source.empty()) {
                        w.key("source");
                        w.str(v.source);
                    }
                    if (!v.meta.empty()) {
                        w.key("meta");
                        put_map(&w, v.meta);
                    }
                    w.end_object();
                }
                w.end_array();
            }
            w.end_object();
        }
        w.end_array();
    }
    if (!m.steps.empty()) {
        w.key("steps");
        w.begin_array();
        for (const auto& s : m.steps) {
            w.begin_object();
            if (!s.entry.empty()) {
                w.key("entry");
                w.str(s.entry);
            }
            w.key("kind");
            w.str(s.kind);
            if (!s.name.empty()) {
                w.key("name");
                w.str(s.name);
            }
            if (!s.kernel.empty()) {
                w.key("kernel");
                w.str(s.kernel);
            }
            if (!s.inputs.empty()) {
                w.key("inputs");
                put_strs(&w, s.inputs);
            }
            if (!s.outputs.empty()) {
                w.key("outputs");
                put_strs(&w, s.outputs);
            }
            if (!s.attributes.empty()) {
                w.key("attributes");
                put_map(&w, s.attributes);
            }
            w.end_object();
        }
        w.end_array();
    }
    if (m.metadata.kind == Kind::Object && !m.metadata.members.empty()) {
        w.key("metadata");
        mjson::write_value(&w, m.metadata);
    }
    w.end_object();
    *out = w.out;
    return true;
}

const EntryPoint* find_entry(const Module& m, const std::string& name) {
    for (const auto& e : m.entry_points)
        if (e.name == name) return &e;
    return nullptr;
}
const Kernel* find_kernel(const Module& m, const std::string& name) {
    for (const auto& k : m.kernels)
        if (k.name == name) return &k;
    return nullptr;
}
const Buffer* find_buffer(const Module& m, const std::string& name) {
    for (const auto& b : m.buffers)
        if (b.name == name) return &b;
    return nullptr;
}
const Param* find_param(const Module& m, const std::string& name) {
    for (const auto& p : m.params)
        if (p.name == name) return &p;
    return nullptr;
}

}  // namespace manta_mod

// ------------------------------------------------------- serving contracts

namespace {

using manta_mod::EntryPoint;
using manta_mod::Module;
using manta_mod::ValueBinding;

// findEntryPoint / requireEntryInput (embedding_model.go:816-847)
bool find_entry_point(const Module& m, const std::string& name, const EntryPoint** out, std::string* e) {
    for (const auto& en : m.entry_points)
        if (en.name == name) {
            *out = &en;
            return true;
        }
    *e = "unknown entrypoint " + q(name);
    return false;
}
bool require_input(const EntryPoint& en, const std::string& name, const ValueBinding** out, std::string* e) {
    for (const auto& in : en.inputs)
        if (in.name == name) {
            *out = &in;
            return true;
        }
    *e = "entrypoint " + q(en.name) + " does not declare input " + q(name);
    return false;
}
bool is_tensor(const ValueBinding& b) { return b.type.kind == "tensor" && b.type.has_tensor; }

// The tensor-input checks shared by the three validators.
bool check_tensor_input(const EntryPoint& en, const std::string& input, const std::string& dtype, int rank,
                        std::string* e) {
    const ValueBinding* b = nullptr;
    if (!require_input(en, input, &b, e)) return false;
    if (!is_tensor(*b)) return *e = "entrypoint " + q(en.name) + " input " + q(input) + " is not a tensor", false;
    if (!dtype.empty() && b->type.dtype != dtype)
        return *e = "entrypoint " + q(en.name) + " input " + q(input) + " dtype = " + q(b->type.dtype) + ", want " +
                    q(dtype),
               false;
    if ((int)b->type.shape.size() != rank)
        return *e = fmt("entrypoint %s input %s rank = %d, want %d", q(en.name).c_str(), q(input).c_str(),
                        (int)b->type.shape.size(), rank),
               false;
    return true;
}

bool validate_score_entry(const Module& m, const std::string& entry, const std::string& query_input, int query_rank,
                          const std::string& docs_input, int docs_rank, const std::string& query_dtype,
                          const std::string& docs_dtype, const std::string& output_name, int output_rank,
                          const std::string& output_dtype, std::string* e) {
    const EntryPoint* en = nullptr;
    if (!find_entry_point(m, entry, &en, e)) return false;
    if (!check_tensor_input(*en, query_input, query_dtype, query_rank, e)) return false;
    if (!check_tensor_input(*en, docs_input, docs_dtype, docs_rank, e)) return false;
    if (en->outputs.size() != 1)
        return *e = fmt("entrypoint %s output count = %d, want 1", q(entry).c_str(), (int)en->outputs.size()), false;
    const ValueBinding& out = en->outputs[0];
    if (!output_name.empty() && out.name != output_name)
        return *e = "entrypoint " + q(entry) + " output " + q(out.name) + " does not match manifest " + q(output_name),
               false;
    if (!is_tensor(out)) return *e = "entrypoint " + q(entry) + " output " + q(out.name) + " is not a tensor", false;
    if (!output_dtype.empty() && out.type.dtype != output_dtype)
        return *e = "entrypoint " + q(entry) + " output dtype = " + q(out.type.dtype) + ", want " + q(output_dtype),
               false;
    if ((int)out.type.shape.size() != output_rank)
        return *e = fmt("entrypoint %s output rank = %d, want %d", q(entry).c_str(), (int)out.type.shape.size(),
                        output_rank),
               false;
    return true;
}

bool validate_retrieval_entry(const Module& m, const std::string& entry, const std::string& query_input,
                              int query_rank, const std::string& docs_input, int docs_rank,
                              const std::string& ids_input, int ids_rank, const std::string& query_dtype,
                              const std::string& docs_dtype, const std::string& ids_dtype,
                              const std::string& output_name, int output_rank, std::string* e) {
    const EntryPoint* en = nullptr;
    if (!find_entry_point(m, entry, &en, e)) return false;
    if (!check_tensor_input(*en, query_input, query_dtype, query_rank, e)) return false;
    if (!check_tensor_input(*en, docs_input, docs_dtype, docs_rank, e)) return false;
    if (!check_tensor_input(*en, ids_input, ids_dtype, ids_rank, e)) return false;
    if (en->outputs.size() != 1)
        return *e = fmt("entrypoint %s output count = %d, want 1", q(entry).c_str(), (int)en->outputs.size()), false;
    const ValueBinding& out = en->outputs[0];
    if (!output_name.empty() && out.name != output_name)
        return *e = "entrypoint " + q(entry) + " output " + q(out.name) + " does not match manifest " + q(output_name),
               false;
    if (out.type.kind != "candidate_pack" || !out.type.has_pack)
        return *e = "entrypoint " + q(entry) + " output " + q(out.name) + " is not a candidate_pack", false;
    if ((int)out.type.pack_shape.size() != output_rank)
        return *e = fmt("entrypoint %s candidate_pack rank = %d, want %d", q(entry).c_str(),
                        (int)out.type.pack_shape.size(), output_rank),
               false;
    return true;
}

bool validate_embedding_entry(const Module& m, const std::string& entry, const std::string& token_input,
                              const std::string& mask_input, int token_rank, int output_rank,
                              const std::string& output_dtype, std::string* e) {
    const EntryPoint* en = nullptr;
    if (!find_entry_point(m, entry, &en, e)) return false;
    if (!check_tensor_input(*en, token_input, "i32", token_rank, e)) {
        // the embedding check names the dtype unquoted ("want i32")
        const ValueBinding* b = nullptr;
        std::string ignore;
        if (require_input(*en, token_input, &b, &ignore) && is_tensor(*b) && b->type.dtype != "i32")
            *e = "entrypoint " + q(entry) + " input " + q(token_input) + " dtype = " + q(b->type.dtype) + ", want i32";
        return false;
    }
    if (!mask_input.empty() && !check_tensor_input(*en, mask_input, "i32", token_rank, e)) {
        const ValueBinding* b = nullptr;
        std::string ignore;
        if (require_input(*en, mask_input, &b, &ignore) && is_tensor(*b) && b->type.dtype != "i32")
            *e = "entrypoint " + q(entry) + " input " + q(mask_input) + " dtype = " + q(b->type.dtype) + ", want i32";
        return false;
    }
    if (en->outputs.size() != 1)
        return *e = fmt("entrypoint %s output count = %d, want 1", q(entry).c_str(), (int)en->outputs.size()), false;
    const ValueBinding& out = en->outputs[0];
    if (!is_tensor(out)) return *e = "entrypoint " + q(entry) + " output " + q(out.name) + " is not a tensor", false;
    if (!output_dtype.empty() && out.type.dtype != output_dtype)
        return *e = "entrypoint " + q(entry) + " output dtype = " + q(out.type.dtype) + ", want " + q(output_dtype),
               false;
    if ((int)out.type.shape.size() != output_rank)
        return *e = fmt("entrypoint %s output rank = %d, want %d", q(entry).c_str(), (int)out.type.shape.size(),
                        output_rank),
               false;
    return true;
}

bool validate_embedding_param(const Module& m, const std::string& name, std::string* e) {
    if (name.empty()) return true;
    for (const auto& p : m.params)
        if (p.name == name) {
            if (p.type.kind != "tensor" || !p.type.has_tensor) return *e = "param " + q(name) + " is not a tensor", false;
            if (p.type.shape.size() != 2)
                return *e = fmt("param %s rank = %d, want 2", q(name).c_str(), (int)p.type.shape.size()), false;
            return true;
        }
    *e = "missing param " + q(name);
    return false;
}

// ------------------------------------------------ authored manifest values

// authoredManifestDoc's typed accessors (authored_manifest_mll.go:278-309).
struct Doc {
    const MantaMll* c;
    const char* key_kind_err(const char* key, int kind, const char* want, std::string* e) {
        *e = "manifest key " + q(key) + " kind = " + std::to_string(kind) + ", want " + want;
        return nullptr;
    }
    bool find(const char* key, int* kind, int64_t* i64, uint32_t* str) {
        uint32_t nm = 0, ds = 0;
        int n = 0;
        if (manta_mll_head(c, &nm, &ds, &n, nullptr) != 0) return false;
        bool found = false;
        for (int i = 0; i < n; i++) {
            uint32_t k = 0, s = 0;
            int kd = 0;
            int64_t v = 0;
            double f = 0;
            if (manta_mll_head_entry(c, i, &k, &kd, &v, &f, &s, nullptr) != 0) continue;
            const char* ks = manta_mll_string(c, k);
            if (ks && strcmp(ks, key) == 0) {  // the last entry with the key wins
                *kind = kd;
                *i64 = v;
                *str = s;
                found = true;
            }
        }
        return found;
    }
    bool str(const char* key, std::string* out, std::string* e) {
        int kind = 0;
        int64_t v = 0;
        uint32_t s = 0;
        if (!find(key, &kind, &v, &s)) return true;
        if (kind != MANTA_MLL_STRING) return key_kind_err(key, kind, "string", e), false;
        const char* t = manta_mll_string(c, s);
        *out = t ? t : "";
        return true;
    }
    bool boolean(const char* key, bool* out, std::string* e) {
        int kind = 0;
        int64_t v = 0;
        uint32_t s = 0;
        if (!find(key, &kind, &v, &s)) return true;
        if (kind != MANTA_MLL_BOOL) return key_kind_err(key, kind, "bool", e), false;
        *out = v != 0;
        return true;
    }
    bool integer(const char* key, int64_t* out, std::string* e) {
        int kind = 0;
        int64_t v = 0;
        uint32_t s = 0;
        if (!find(key, &kind, &v, &s)) return true;
        if (kind != MANTA_MLL_I64) return key_kind_err(key, kind, "int", e), false;
        *out = v;
        return true;
    }
};

// readAuthoredManifestMLL's kind / version checks (authored_manifest_mll.go:
// 238-265).
bool check_manifest_kind(Doc& d, const char* kind, const char* version, std::string* e) {
    const char* keys[2] = {"manifest_kind", "manifest_version"};
    const char* want[2] = {kind, version};
    for (int i = 0; i < 2; i++) {
        int kd = 0;
        int64_t v = 0;
        uint32_t s = 0;
        if (!d.find(keys[i], &kd, &v, &s)) return *e = std::string("manifest missing ") + q(keys[i]), false;
        if (kd != MANTA_MLL_STRING) return d.key_kind_err(keys[i], kd, "string", e), false;
        const char* got = manta_mll_string(d.c, s);
        if (!got || strcmp(got, want[i]) != 0)
            return *e = std::string("manifest ") + (i == 0 ? "kind " : "version ") + q(got ? got : "") + ", want " +
                        q(want[i]),
                   false;
    }
    return true;
}

#define DOC_STR(key, field) \
    if (!d.str(key, &field, e)) return false
#define DOC_BOOL(key, field) \
    if (!d.boolean(key, &field, e)) return false

// ScoreManifest: scoreManifestFromDoc + normalized + ValidateModule
// (score_model.go:116-153, 212-251).
bool validate_score_manifest(Doc& d, const Module& m, std::string* e) {
    std::string entry, batch_entry, query_input, batch_query_input, docs_input, output_name, batch_output_name,
        query_dtype, docs_dtype, output_dtype;
    DOC_STR("entry", entry);
    DOC_STR("batch_entry", batch_entry);
    DOC_STR("query_input", query_input);
    DOC_STR("batch_query_input", batch_query_input);
    DOC_STR("docs_input", docs_input);
    DOC_STR("output_name", output_name);
    DOC_STR("batch_output_name", batch_output_name);
    DOC_STR("query_dtype", query_dtype);
    DOC_STR("docs_dtype", docs_dtype);
    DOC_STR("output_dtype", output_dtype);
    if (entry.empty()) entry = "score";
    if (query_input.empty()) query_input = "query";
    if (batch_query_input.empty()) batch_query_input = "queries";
    if (docs_input.empty()) docs_input = "docs";
    if (query_dtype.empty()) query_dtype = "f16";
    if (docs_dtype.empty()) docs_dtype = "q4";
    if (output_dtype.empty()) output_dtype = "f32";
    if (!validate_score_entry(m, entry, query_input, 1, docs_input, 2, query_dtype, docs_dtype, output_name, 1,
                              output_dtype, e))
        return false;
    if (!batch_entry.empty() && !validate_score_entry(m, batch_entry, batch_query_input, 2, docs_input, 3, query_dtype,
                                                      docs_dtype, batch_output_name, 2, output_dtype, e))
        return false;
    return true;
}

// RetrievalManifest (retrieval_model.go:118-158, 217-259).
bool validate_retrieval_manifest(Doc& d, const Module& m, std::string* e) {
    std::string entry, batch_entry, query_input, batch_query_input, docs_input, ids_input, output_name,
        batch_output_name, query_dtype, docs_dtype, ids_dtype;
    DOC_STR("entry", entry);
    DOC_STR("batch_entry", batch_entry);
    DOC_STR("query_input", query_input);
    DOC_STR("batch_query_input", batch_query_input);
    DOC_STR("docs_input", docs_input);
    DOC_STR("candidate_ids_input", ids_input);
    DOC_STR("output_name", output_name);
    DOC_STR("batch_output_name", batch_output_name);
    DOC_STR("query_dtype", query_dtype);
    DOC_STR("docs_dtype", docs_dtype);
    DOC_STR("candidate_ids_dtype", ids_dtype);
    if (entry.empty()) entry = "rerank_candidates_packed";
    if (query_input.empty()) query_input = "query";
    if (batch_query_input.empty()) batch_query_input = "queries";
    if (docs_input.empty()) docs_input = "docs";
    if (ids_input.empty()) ids_input = "candidate_ids";
    if (query_dtype.empty()) query_dtype = "f16";
    if (docs_dtype.empty()) docs_dtype = "q4";
    if (ids_dtype.empty()) ids_dtype = "i64";
    if (!validate_retrieval_entry(m, entry, query_input, 1, docs_input, 2, ids_input, 1, query_dtype, docs_dtype,
                                  ids_dtype, output_name, 2, e))
        return false;
    if (!batch_entry.empty() &&
        !validate_retrieval_entry(m, batch_entry, batch_query_input, 2, docs_input, 3, ids_input, 2, query_dtype,
                                  docs_dtype, ids_dtype, batch_output_name, 3, e))
        return false;
    return true;
}

// EmbeddingManifest (embedding_model.go:154-260, 617-673, 801-815).
bool validate_embedding_manifest(Doc& d, const Module& m, std::string* e) {
    std::string pooled_entry, batch_entry, token_input, mask_input, output_dtype, token_param, aq, ak, av, ao,
        hidden_param, projection_param, output_name;
    bool attn_residual = false, attn_ln = false, ffn_residual = false, ffn_ln = false;
    int64_t repeats = 0;
    DOC_STR("pooled_entry", pooled_entry);
    DOC_STR("batch_entry", batch_entry);
    if (!d.integer("encoder_repeats", &repeats, e)) return false;
    DOC_STR("token_input", token_input);
    DOC_STR("mask_input", mask_input);
    DOC_STR("output_name", output_name);
    DOC_STR("output_dtype", output_dtype);
    DOC_STR("token_embedding_param", token_param);
    DOC_STR("attention_query_param", aq);
    DOC_STR("attention_key_param", ak);
    DOC_STR("attention_value_param", av);
    DOC_STR("attention_output_param", ao);
    DOC_BOOL("attention_residual", attn_residual);
    DOC_BOOL("attention_layernorm", attn_ln);
    DOC_STR("hidden_projection_param", hidden_param);
    DOC_BOOL("ffn_residual", ffn_residual);
    DOC_BOOL("ffn_layernorm", ffn_ln);
    DOC_STR("projection_param", projection_param);
    if (pooled_entry.empty()) pooled_entry = "embed_pooled";
    if (batch_entry.empty()) batch_entry = "embed_pooled_batch";
    if (token_input.empty()) token_input = "tokens";
    if (output_dtype.empty()) output_dtype = "f16";
    if (token_param.empty()) token_param = "token_embedding";
    if (projection_param.empty()) projection_param = "projection";
    if ((attn_residual || attn_ln) && aq.empty())
        return *e = "attention residual/layernorm requires attention params", false;
    if ((ffn_residual || ffn_ln) && hidden_param.empty())
        return *e = "ffn residual/layernorm requires hidden_projection_param", false;
    if (!validate_embedding_entry(m, pooled_entry, token_input, mask_input, 1, 1, output_dtype, e)) return false;
    if (!validate_embedding_entry(m, batch_entry, token_input, mask_input, 2, 2, output_dtype, e)) return false;
    if (!validate_embedding_param(m, token_param, e)) return false;
    // validateAttentionParams: all four or none
    const std::string names[4] = {aq, ak, av, ao};
    int set = 0;
    for (const auto& n : names) set += !n.empty();
    if (set != 0) {
        if (set != 4) return *e = "attention params must declare query, key, value, and output together", false;
        for (const auto& n : names)
            if (!validate_embedding_param(m, n, e)) return false;
    }
    if (!hidden_param.empty() && !validate_embedding_param(m, hidden_param, e)) return false;
    return validate_embedding_param(m, projection_param, e);
}

}  // namespace

// ------------------------------------------------------------------ C ABI

extern "C" {

int manta_module_decode_json(const char* json, size_t len, MantaModule** out, char** err) {
    if (!out) return set_err(err, MANTA_ROCM_ERROR, "nil output handle");
    *out = nullptr;
    if (!json && len) return set_err(err, MANTA_ROCM_ERROR, "nil JSON input");
    auto* m = new MantaModule();
    std::string e;
    if (!manta_mod::decode_json(json ? json : "", len, &m->m, &e)) {
        delete m;
        return set_err(err, MANTA_ROCM_ERROR, e);
    }
    *out = m;
    return MANTA_ROCM_OK;
}

int manta_module_decode_mll(const MantaMll* container, MantaModule** out, char** err) {
    if (!out) return set_err(err, MANTA_ROCM_ERROR, "nil output handle");
    *out = nullptr;
    if (!container) return set_err(err, MANTA_ROCM_ERROR, "nil MLL container");
    uint64_t n = 0;
    const uint8_t* p = manta_mll::section_body(container, "XMTA", &n);
    if (!p) return set_err(err, MANTA_ROCM_ERROR, "mll artifact missing XMTA metadata section");
    // DecodeMLLMetadata: Unmarshal into MLLMetadata, then its Validate
    Value meta;
    std::string e;
    mjson::Parser parser((const char*)p, (size_t)n);
    if (!parser.parse(&meta, &e)) return set_err(err, MANTA_ROCM_ERROR, e);
    if (meta.kind != Kind::Object && meta.kind != Kind::Null)
        return set_err(err, MANTA_ROCM_ERROR,
                       std::string("json: cannot unmarshal ") + meta.kind_name() +
                           " into Go value of type manta.MLLMetadata");
    Dec d;
    d.root = "MLLMetadata";
    std::string version, module_name, module_version;
    if (meta.kind == Kind::Object) {
        if (!d.str(meta.get("version"), "version", &version) ||
            !d.str(meta.get("module_name"), "module_name", &module_name) ||
            !d.str(meta.get("module_version"), "module_version", &module_version))
            return set_err(err, MANTA_ROCM_ERROR, d.err);
    }
    const Value* art = meta.kind == Kind::Object ? meta.get("artifact") : nullptr;
    if (version.empty()) return set_err(err, MANTA_ROCM_ERROR, "MLL metadata version is required");
    if (version != kMLLMetadataVersion)
        return set_err(err, MANTA_ROCM_ERROR,
                       "MLL metadata version " + q(version) + " is not supported, want " + q(kMLLMetadataVersion));
    if (module_name.empty()) return set_err(err, MANTA_ROCM_ERROR, "MLL metadata module_name is required");
    if (module_version.empty()) return set_err(err, MANTA_ROCM_ERROR, "MLL metadata module_version is required");
    if (!art) return set_err(err, MANTA_ROCM_ERROR, "MLL metadata artifact must be valid JSON");
    const Value* files = meta.get("json_files");
    if (files && files->kind == Kind::Object)
        for (const auto& kv : files->members)
            if (kv.first.empty()) return set_err(err, MANTA_ROCM_ERROR, "MLL metadata json_files role is required");
    const Value* dts = meta.get("logical_tensor_dtypes");
    if (dts && dts->kind == Kind::Object)
        for (const auto& kv : dts->members) {
            if (kv.first.empty())
                return set_err(err, MANTA_ROCM_ERROR, "MLL metadata logical tensor name is required");
            if (kv.second.kind == Kind::String && kv.second.text.empty())
                return set_err(err, MANTA_ROCM_ERROR,
                               "MLL metadata logical tensor dtype for " + q(kv.first) + " is required");
        }
    // DecodeJSON(meta.Artifact)
    auto* m = new MantaModule();
    if (!manta_mod::decode_value(*art, &m->m, &e) || !manta_mod::validate(m->m, &e)) {
        delete m;
        return set_err(err, MANTA_ROCM_ERROR, e);
    }
    *out = m;
    return MANTA_ROCM_OK;
}

void manta_module_free(MantaModule* m) { delete m; }

int manta_module_validate(const MantaModule* m, char** err) {
    if (!m) return set_err(err, MANTA_ROCM_ERROR, "nil module");
    std::string e;
    if (!manta_mod::validate(m->m, &e)) return set_err(err, MANTA_ROCM_ERROR, e);
    return MANTA_ROCM_OK;
}

int manta_module_encode_json(const MantaModule* m, char** out, size_t* len, char** err) {
    if (!m) return set_err(err, MANTA_ROCM_ERROR, "nil module");
    if (!out) return set_err(err, MANTA_ROCM_ERROR, "nil output");
    std::string s, e;
    if (!manta_mod::encode_json(m->m, &s, &e)) return set_err(err, MANTA_ROCM_ERROR, e);
    *out = (char*)malloc(s.size() + 1);
    if (!*out) return set_err(err, MANTA_ROCM_ERROR, "out of host memory");
    memcpy(*out, s.c_str(), s.size() + 1);
    if (len) *len = s.size();
    return MANTA_ROCM_OK;
}

int manta_module_encode_mll(const MantaModule* m, void** out, size_t* len, char** err) {
    if (!m) return set_err(err, MANTA_ROCM_ERROR, "nil module");
    if (!out || !len) return set_err(err, MANTA_ROCM_ERROR, "nil output");
    std::string art, e;
    if (!manta_mod::encode_json(m->m, &art, &e)) return set_err(err, MANTA_ROCM_ERROR, e);
    // MLLMetadata: json.Marshal (compact); the artifact is the indented
    // module text with surrounding space trimmed, embedded as raw JSON
    std::string meta = "{\"version\":";
    mjson::put_string(&meta, kMLLMetadataVersion);
    meta += ",\"module_name\":";
    mjson::put_string(&meta, m->m.name);
    meta += ",\"module_version\":";
    mjson::put_string(&meta, m->m.version);
    meta += ",\"artifact\":" + art + "}";
    std::string backends, caps;
    for (size_t i = 0; i < m->m.supported_backends.size(); i++)
        backends += (i ? "," : "") + m->m.supported_backends[i];
    for (size_t i = 0; i < m->m.capabilities.size(); i++) caps += (i ? "," : "") + m->m.capabilities[i];
    std::vector<manta_mll::HeadEntry> entries = {
        {"artifact_version", MANTA_MLL_STRING, 0, 0.0, m->m.version},
        {"supported_backends", MANTA_MLL_STRING, 0, 0.0, backends},
        {"capabilities", MANTA_MLL_STRING, 0, 0.0, caps},
        {"param_count", MANTA_MLL_I64, (int64_t)m->m.params.size(), 0.0, ""},
        {"entry_count", MANTA_MLL_I64, (int64_t)m->m.entry_points.size(), 0.0, ""},
        {"kernel_count", MANTA_MLL_I64, (int64_t)m->m.kernels.size(), 0.0, ""},
    };
    std::vector<uint8_t> head, strg;
    manta_mll::build_head(m->m.name, "Manta module artifact", entries, &head, &strg);
    static const uint8_t empty_table[4] = {0, 0, 0, 0};
    static const uint8_t empty_tensors[64] = {0};
    // the typed DIMS / TYPE / PARM / ENTR / TNSR / SCHM tables are written
    // empty: the module travels whole in XMTA, which is what DecodeMLL reads
    std::vector<manta_mll::SectionRef> secs = {
        {"HEAD", head.data(), head.size(), 0x10001u, 0},
        {"STRG", strg.data(), strg.size(), 0x10001u, 0},
        {"DIMS", empty_table, 4, 0x10001u, 0},
        {"TYPE", empty_table, 4, 0x10000u, 0},
        {"PARM", empty_table, 4, 0x10001u, 0},
        {"ENTR", empty_table, 4, 0x10001u, 0},
        {"TNSR", empty_tensors, 64, 0x10011u, 0},
        {"SCHM", empty_table, 4, 0x10000u, 0},
        {"XMTA", (const uint8_t*)meta.data(), meta.size(), 0x10000u, 0},
    };
    const std::vector<uint8_t> bytes = manta_mll::build_container(&secs);
    *out = malloc(bytes.size());
    if (!*out) return set_err(err, MANTA_ROCM_ERROR, "out of host memory");
    memcpy(*out, bytes.data(), bytes.size());
    *len = bytes.size();
    return MANTA_ROCM_OK;
}

void manta_module_free_buffer(void* p) { free(p); }

const char* manta_module_name(const MantaModule* m) { return m ? m->m.name.c_str() : nullptr; }

int manta_module_validate_score_entry(const MantaModule* m, const char* entry, const char* query_input,
                                      int query_rank, const char* docs_input, int docs_rank, const char* query_dtype,
                                      const char* docs_dtype, const char* output_name, int output_rank,
                                      const char* output_dtype, char** err) {
    if (!m) return set_err(err, MANTA_ROCM_ERROR, "nil module");
    auto s = [](const char* x) { return std::string(x ? x : ""); };
    std::string e;
    if (!validate_score_entry(m->m, s(entry), s(query_input), query_rank, s(docs_input), docs_rank, s(query_dtype),
                              s(docs_dtype), s(output_name), output_rank, s(output_dtype), &e))
        return set_err(err, MANTA_ROCM_ERROR, e);
    return MANTA_ROCM_OK;
}

int manta_module_validate_retrieval_entry(const MantaModule* m, const char* entry, const char* query_input,
                                          int query_rank, const char* docs_input, int docs_rank,
                                          const char* ids_input, int ids_rank, const char* query_dtype,
                                          const char* docs_dtype, const char* ids_dtype, const char* output_name,
                                          int output_rank, char** err) {
    if (!m) return set_err(err, MANTA_ROCM_ERROR, "nil module");
    auto s = [](const char* x) { return std::string(x ? x : ""); };
    std::string e;
    if (!validate_retrieval_entry(m->m, s(entry), s(query_input), query_rank, s(docs_input), docs_rank, s(ids_input),
                                  ids_rank, s(query_dtype), s(docs_dtype), s(ids_dtype), s(output_name), output_rank,
                                  &e))
        return set_err(err, MANTA_ROCM_ERROR, e);
    return MANTA_ROCM_OK;
}

int manta_module_validate_embedding_entry(const MantaModule* m, const char* entry, const char* token_input,
                                          const char* mask_input, int token_rank, int output_rank,
                                          const char* output_dtype, char** err) {
    if (!m) return set_err(err, MANTA_ROCM_ERROR, "nil module");
    auto s = [](const char* x) { return std::string(x ? x : ""); };
    std::string e;
    if (!validate_embedding_entry(m->m, s(entry), s(token_input), s(mask_input), token_rank, output_rank,
                                  s(output_dtype), &e))
        return set_err(err, MANTA_ROCM_ERROR, e);
    return MANTA_ROCM_OK;
}

int manta_module_validate_embedding_param(const MantaModule* m, const char* name, char** err) {
    if (!m) return set_err(err, MANTA_ROCM_ERROR, "nil module");
    std::string e;
    if (!validate_embedding_param(m->m, name ? name : "", &e)) return set_err(err, MANTA_ROCM_ERROR, e);
    return MANTA_ROCM_OK;
}

int manta_manifest_validate_module(const MantaMll* manifest, const MantaModule* m, char** err) {
    if (!m) return set_err(err, MANTA_ROCM_ERROR, "nil module");
    if (!manifest) return set_err(err, MANTA_ROCM_ERROR, "nil manifest");
    char* herr = nullptr;
    uint32_t nm = 0, ds = 0;
    int n = 0;
    if (manta_mll_head(manifest, &nm, &ds, &n, &herr) != 0) {
        std::string e = herr ? herr : "manifest has no HEAD section";
        free(herr);
        return set_err(err, MANTA_ROCM_ERROR, e);
    }
    Doc d{manifest};
    std::string kind, e;
    if (!d.str("manifest_kind", &kind, &e)) return set_err(err, MANTA_ROCM_ERROR, e);
    bool ok;
    if (kind == "score_manifest") {
        ok = check_manifest_kind(d, "score_manifest", "manta/score-manifest/v0alpha1", &e) &&
             validate_score_manifest(d, m->m, &e);
    } else if (kind == "retrieval_manifest") {
        ok = check_manifest_kind(d, "retrieval_manifest", "manta/retrieval-manifest/v0alpha1", &e) &&
             validate_retrieval_manifest(d, m->m, &e);
    } else if (kind == "embedding_manifest") {
        ok = check_manifest_kind(d, "embedding_manifest", "manta/embedding-manifest/v0alpha1", &e) &&
             validate_embedding_manifest(d, m->m, &e);
    } else {
        return set_err(err, MANTA_ROCM_UNSUPPORTED, "manifest kind " + q(kind) + " has no serving contract here");
    }
    if (!ok) return set_err(err, MANTA_ROCM_ERROR, e);
    return MANTA_ROCM_OK;
}

}  // extern "C"
