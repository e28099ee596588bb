// module_internal.hpp -- the artifact schema (artifact/manta/module.go:8-207)
// as plain C++ values, shared by the codec (module.cpp) and the step
// executor (program.cpp).
#pragma once

#include <map>
#include <string>
#include <vector>

#include "json.hpp"

namespace manta_mod {

// ValueType (module.go:91-96) with its tensor / candidate_pack payloads.
struct ValueType {
    std::string kind;  // "tensor", "kv_cache", "candidate_pack"
    bool has_tensor = false;
    std::string dtype;               // tensor.dtype
    std::vector<std::string> shape;  // tensor.shape
    bool has_pack = false;
    std::vector<std::string> pack_shape;  // candidate_pack.shape
};

struct Param {
    std::string name;
    ValueType type;
    std::string binding;
    bool trainable = false;
};

struct ValueBinding {
    std::string name;
    ValueType type;
};

struct EntryPoint {
    std::string name;
    std::string kind;
    std::vector<ValueBinding> inputs, outputs;
};

struct Buffer {
    std::string name, dtype;
    std::vector<std::string> shape;
    std::string storage_class;
};

struct Hints {
    std::vector<long long> tile, tile_2d;
    long long vector_width = 0;
    bool subgroup = false;
    std::vector<long long> subgroup_2d, halo;
    std::string memory;
};

using StrMap = std::map<std::string, std::string>;

struct KernelVariant {
    std::string backend, entry, source;
    StrMap meta;
};

struct KernelOp {
    std::string kind, name, op;
    std::vector<std::string> inputs, outputs;
    StrMap attributes;
};

struct Kernel {
    std::string name;
    std::vector<ValueBinding> inputs, outputs;
    Hints hints;
    std::vector<KernelOp> body;
    std::vector<KernelVariant> variants;
};

struct Step {
    std::string entry, kind, name, kernel;
    std::vector<std::string> inputs, outputs;
    StrMap attributes;
};

struct Module {
    std::string version, name;
    std::vector<Param> params;
    std::vector<EntryPoint> entry_points;
    bool entry_points_null = true;  // Go nil slice (encodes as null)
    std::vector<std::string> supported_backends;
    bool supported_backends_null = true;
    std::vector<std::string> capabilities;
    std::vector<Buffer> buffers;
    std::vector<Kernel> kernels;
    std::vector<Step> steps;
    mjson::Value metadata;  // Object (possibly empty) or Null
};

// DecodeJSON (module.go:494-505): parse, then Validate.
bool decode_json(const char* p, size_t n, Module* out, std::string* err);
// Unmarshal only (no validation), from a parsed value.
bool decode_value(const mjson::Value& v, Module* out, std::string* err);
// Module.Validate (module.go:255-424).
bool validate(const Module& m, std::string* err);
// EncodeJSON (module.go:486-492): Validate, then MarshalIndent(m, "", "  ").
bool encode_json(const Module& m, std::string* out, std::string* err);

const EntryPoint* find_entry(const Module& m, const std::string& name);
const Kernel* find_kernel(const Module& m, const std::string& name);
const Buffer* find_buffer(const Module& m, const std::string& name);
const Param* find_param(const Module& m, const std::string& name);

}  // namespace manta_mod

struct MantaModule {
    manta_mod::Module m;
};
