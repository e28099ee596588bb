// mll_internal.hpp -- container-building pieces shared by the packed
// candidate writer (mll.cpp) and the module artifact writer (module.cpp).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

struct MantaMll;

namespace manta_mll {

// One section to write: tag, body (not copied), flags (bit 0 required,
// bit 4 page aligned, schema version in bits 16+).  build_table fills `off`.
struct SectionRef {
    char tag[5];
    const uint8_t* p;
    uint64_t n;
    uint32_t flags;
    uint64_t off;
};

// The 24-byte header and 64-byte section table (BLAKE3-256 digest of each
// body) for `secs`, laid out in order after the table, page-aligned sections
// at multiples of 4096.  Sets each section's offset; returns the header and
// table bytes and the total file size.
std::vector<uint8_t> build_table(std::vector<SectionRef>* secs, uint64_t* total);

// The whole container in memory.
std::vector<uint8_t> build_container(std::vector<SectionRef>* secs);

// HEAD metadata entry to encode (kind: MANTA_MLL_BOOL / I64 / F64 / STRING).
struct HeadEntry {
    std::string key;
    int kind;
    int64_t i64;
    double f64;
    std::string str;
};

// STRG and HEAD section bodies for a container named `name`: the string
// table interns "" (id 0), then every string in order of first use.
void build_head(const std::string& name, const std::string& description, const std::vector<HeadEntry>& entries,
                std::vector<uint8_t>* head, std::vector<uint8_t>* strg);

void put32(std::vector<uint8_t>& b, uint32_t v);
void put64(std::vector<uint8_t>& b, uint64_t v);

// Raw section body of an opened container (nullptr when absent).
const uint8_t* section_body(const MantaMll* m, const char* tag, uint64_t* size);

}  // namespace manta_mll
