// mll.cpp -- native reader of Manta's MLL containers (host only): section
// table with BLAKE3-256 digest verification, string table, HEAD metadata.
// The layout is documented in include/manta_mll.h.
#include "manta_mll.h"

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "manta_rocm.h"
#include "mll_internal.hpp"

namespace {

int mll_fail(char** err, const char* fmt, ...) {
    if (err) {
        char buf[256];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof(buf), fmt, ap);
        va_end(ap);
        const size_t n = strlen(buf) + 1;
        *err = (char*)malloc(n);
        if (*err) memcpy(*err, buf, n);
    }
    return MANTA_ROCM_ERROR;
}

uint32_t rd32(const uint8_t* p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24; }
uint64_t rd64(const uint8_t* p) { return (uint64_t)rd32(p) | (uint64_t)rd32(p + 4) << 32; }

// ---------------------------------------------------------------- BLAKE3
// The hash function of the BLAKE3 specification (O'Connor, Aumasson, Neves,
// Wilcox-O'Hearn, 2020): 1024-byte chunks of 64-byte blocks compressed with
// the 7-round function below, chunk chaining values merged pairwise in a
// left-complete binary tree, 32-byte root output.  Unkeyed mode only.
constexpr uint32_t kIV[8] = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                             0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};
constexpr int kPerm[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};
enum : uint32_t { CHUNK_START = 1, CHUNK_END = 2, PARENT = 4, ROOT = 8 };

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

inline void g(uint32_t* s, int a, int b, int c, int d, uint32_t mx, uint32_t my) {
    s[a] = s[a] + s[b] + mx;
    s[d] = rotr(s[d] ^ s[a], 16);
    s[c] = s[c] + s[d];
    s[b] = rotr(s[b] ^ s[c], 12);
    s[a] = s[a] + s[b] + my;
    s[d] = rotr(s[d] ^ s[a], 8);
    s[c] = s[c] + s[d];
    s[b] = rotr(s[b] ^ s[c], 7);
}

// out[0..8) = the first 8 words of the compression output (chaining value)
void compress(const uint32_t cv[8], const uint32_t block[16], uint64_t counter, uint32_t len, uint32_t flags,
              uint32_t out[8]) {
    uint32_t s[16] = {cv[0], cv[1], cv[2], cv[3], cv[4], cv[5], cv[6], cv[7],
                      kIV[0], kIV[1], kIV[2], kIV[3], (uint32_t)counter, (uint32_t)(counter >> 32), len, flags};
    uint32_t m[16], t[16];
    memcpy(m, block, sizeof(m));
    for (int r = 0; r < 7; r++) {
        g(s, 0, 4, 8, 12, m[0], m[1]);
        g(s, 1, 5, 9, 13, m[2], m[3]);
        g(s, 2, 6, 10, 14, m[4], m[5]);
        g(s, 3, 7, 11, 15, m[6], m[7]);
        g(s, 0, 5, 10, 15, m[8], m[9]);
        g(s, 1, 6, 11, 12, m[10], m[11]);
        g(s, 2, 7, 8, 13, m[12], m[13]);
        g(s, 3, 4, 9, 14, m[14], m[15]);
        for (int i = 0; i < 16; i++) t[i] = m[kPerm[i]];
        memcpy(m, t, sizeof(m));
    }
    for (int i = 0; i < 8; i++) out[i] = s[i] ^ s[i + 8];
}

void load_block(const uint8_t* p, size_t n, uint32_t w[16]) {
    uint8_t b[64] = {0};
    memcpy(b, p, n);
    for (int i = 0; i < 16; i++) w[i] = rd32(b + 4 * i);
}

// Chaining value of chunk `index` (bytes p[0..n), n <= 1024); root = the
// input is this one chunk, so its last block carries ROOT.
void chunk_cv(const uint8_t* p, size_t n, uint64_t index, bool root, uint32_t out[8]) {
    uint32_t cv[8];
    memcpy(cv, kIV, sizeof(cv));
    const size_t blocks = n == 0 ? 1 : (n + 63) / 64;
    for (size_t b = 0; b < blocks; b++) {
        const size_t len = b + 1 < blocks ? 64 : n - 64 * b;
        uint32_t w[16];
        load_block(p + 64 * b, len, w);
        uint32_t flags = (b == 0 ? CHUNK_START : 0) | (b + 1 == blocks ? CHUNK_END : 0);
        if (root && b + 1 == blocks) flags |= ROOT;
        compress(cv, w, index, (uint32_t)len, flags, cv);
    }
    memcpy(out, cv, sizeof(cv));
}

// Chaining value of chunks [lo, hi) of the input: the left subtree holds the
// largest power of two of chunks that leaves at least one on the right.
void subtree_cv(const uint8_t* p, size_t n, uint64_t lo, uint64_t hi, bool root, uint32_t out[8]) {
    if (hi - lo == 1) {
        const size_t off = (size_t)lo * 1024;
        chunk_cv(p + off, n - off < 1024 ? n - off : 1024, lo, root, out);
        return;
    }
    uint64_t left = 1;
    while (left * 2 < hi - lo) left *= 2;
    uint32_t w[16];
    subtree_cv(p, n, lo, lo + left, false, w);
    subtree_cv(p, n, lo + left, hi, false, w + 8);
    compress(kIV, w, 0, 64, PARENT | (root ? ROOT : 0), out);
}

void blake3(const uint8_t* p, size_t n, uint8_t digest[32]) {
    const uint64_t chunks = n == 0 ? 1 : (n + 1023) / 1024;
    uint32_t h[8];
    subtree_cv(p, n, 0, chunks, true, h);
    for (int i = 0; i < 8; i++)
        for (int j = 0; j < 4; j++) digest[4 * i + j] = (uint8_t)(h[i] >> (8 * j));
}

}  // namespace

struct MantaMll {
    std::vector<uint8_t> bytes;
    uint32_t format_word = 0;
    struct Section {
        char tag[5];
        uint64_t offset, size;
        uint32_t flags;
        uint8_t digest[32];
    };
    std::vector<Section> sections;
    bool strings_ok = false;
    std::vector<std::string> strings;  // id 0 = ""
    std::string strg_error;
    struct Entry {
        uint32_t key;
        int kind;
        int64_t i64;
        double f64;
        uint32_t str;
    };
    bool head_present = false;
    std::string head_error;
    uint32_t name = 0, description = 0;
    std::vector<Entry> entries;
};

namespace {

const MantaMll::Section* find_section(const MantaMll* m, const char* tag) {
    for (const auto& s : m->sections)
        if (strncmp(s.tag, tag, 4) == 0) return &s;
    return nullptr;
}

void parse_strings(MantaMll* m, const uint8_t* p, uint64_t n) {
    if (n < 8) {
        m->strg_error = "malformed STRG section: no count";
        return;
    }
    const uint64_t count = rd64(p);
    if (count == 0 || count > n) {
        m->strg_error = "malformed STRG section: count " + std::to_string(count);
        return;
    }
    m->strings.assign(1, std::string());
    uint64_t at = 8;
    for (uint64_t i = 1; i < count; i++) {
        if (at + 4 > n) {
            m->strg_error = "malformed STRG section: string " + std::to_string(i) + " past the end";
            return;
        }
        const uint32_t len = rd32(p + at);
        if (at + 4 + len > n) {
            m->strg_error = "malformed STRG section: string " + std::to_string(i) + " past the end";
            return;
        }
        m->strings.emplace_back((const char*)p + at + 4, len);
        at += 4 + (uint64_t)len;
    }
    if (at != n) {
        m->strg_error = "malformed STRG section: " + std::to_string(n - at) + " trailing bytes";
        return;
    }
    m->strings_ok = true;
}

void parse_head(MantaMll* m, const uint8_t* p, uint64_t n) {
    m->head_present = true;
    if (n < 30) {
        m->head_error = "malformed HEAD section: " + std::to_string(n) + " bytes";
        return;
    }
    m->name = rd32(p);
    m->description = rd32(p + 4);
    const uint32_t count = (uint32_t)p[28] | (uint32_t)p[29] << 8;
    uint64_t at = 30;
    for (uint32_t i = 0; i < count; i++) {
        if (at + 5 > n) {
            m->head_error = "malformed HEAD section: entry " + std::to_string(i) + " past the end";
            return;
        }
        MantaMll::Entry e{rd32(p + at), p[at + 4], 0, 0.0, 0};
        at += 5;
        const uint64_t width = e.kind == MANTA_MLL_BOOL ? 1 : (e.kind == MANTA_MLL_STRING ? 4 : 8);
        if (e.kind < MANTA_MLL_BOOL || e.kind > MANTA_MLL_STRING) {
            m->head_error = "malformed HEAD section: entry " + std::to_string(i) + " kind " + std::to_string(e.kind);
            return;
        }
        if (at + width > n) {
            m->head_error = "malformed HEAD section: entry " + std::to_string(i) + " past the end";
            return;
        }
        if (e.kind == MANTA_MLL_BOOL) e.i64 = p[at] != 0;
        if (e.kind == MANTA_MLL_I64) e.i64 = (int64_t)rd64(p + at);
        if (e.kind == MANTA_MLL_F64) {
            const uint64_t bits = rd64(p + at);
            memcpy(&e.f64, &bits, 8);
        }
        if (e.kind == MANTA_MLL_STRING) e.str = rd32(p + at);
        if (e.key >= m->strings.size() || (e.kind == MANTA_MLL_STRING && e.str >= m->strings.size())) {
            m->head_error = "malformed HEAD section: entry " + std::to_string(i) + " names string " +
                            std::to_string(e.key >= m->strings.size() ? e.key : e.str) + " of " +
                            std::to_string(m->strings.size());
            return;
        }
        at += width;
        m->entries.push_back(e);
    }
    if (at != n) m->head_error = "malformed HEAD section: " + std::to_string(n - at) + " trailing bytes";
}


// ------------------------------------------------ packed candidate containers

const char kPackedKind[] = "packed_candidates";
const char kPackedVersion[] = "manta/packed-candidates/v0";

using manta_mll::put32;
using manta_mll::put64;

// Expected byte sizes of the code and scale sections of `rows` rows of `dim`
// values: q8 = int8 codes + one f32 scale per row, q4 = two values per byte
// + one f16 scale per 32-value block.
// (rows < 2^31 and dim < 2^32, so no product overflows.)
void packed_sizes(int dtype, uint64_t rows, uint64_t dim, uint64_t* codes, uint64_t* scales) {
    if (dtype == MANTA_ROCM_Q8_ROWS) {
        *codes = rows * dim;
        *scales = rows * 4;
    } else {
        *codes = rows * (dim / 2);
        *scales = rows * (dim / 32) * 2;
    }
}

const MantaMll::Entry* head_value(const MantaMll* m, const char* key) {
    for (const auto& e : m->entries)
        if (e.key < m->strings.size() && m->strings[e.key] == key) return &e;
    return nullptr;
}

}  // namespace

// ------------------------------------------------------ container building

namespace manta_mll {

void put32(std::vector<uint8_t>& b, uint32_t v) {
    for (int i = 0; i < 4; i++) b.push_back((uint8_t)(v >> (8 * i)));
}
void put64(std::vector<uint8_t>& b, uint64_t v) {
    for (int i = 0; i < 8; i++) b.push_back((uint8_t)(v >> (8 * i)));
}

std::vector<uint8_t> build_table(std::vector<SectionRef>* secs, uint64_t* total) {
    uint64_t at = 24 + 64 * (uint64_t)secs->size();
    for (auto& s : *secs) {
        if (s.flags & 0x10u) at = (at + 4095) & ~(uint64_t)4095;
        s.off = at;
        at += s.n;
    }
    *total = at;
    std::vector<uint8_t> top;
    top.insert(top.end(), {'M', 'L', 'L', 0});
    put32(top, 0x00010100u);
    put64(top, at);
    put64(top, secs->size());
    for (const auto& s : *secs) {
        top.insert(top.end(), s.tag, s.tag + 4);
        put64(top, s.off);
        put64(top, s.n);
        uint8_t d[32];
        blake3(s.p, (size_t)s.n, d);
        top.insert(top.end(), d, d + 32);
        put32(top, s.flags);
        put64(top, 0);
    }
    return top;
}

std::vector<uint8_t> build_container(std::vector<SectionRef>* secs) {
    uint64_t total = 0;
    std::vector<uint8_t> out = build_table(secs, &total);
    out.resize((size_t)total, 0);
    for (const auto& s : *secs)
        if (s.n) memcpy(out.data() + s.off, s.p, (size_t)s.n);
    return out;
}

void build_head(const std::string& name, const std::string& description, const std::vector<HeadEntry>& entries,
                std::vector<uint8_t>* head, std::vector<uint8_t>* strg) {
    std::vector<std::string> strs(1);
    auto intern = [&](const std::string& x) -> uint32_t {
        for (size_t i = 0; i < strs.size(); i++)
            if (strs[i] == x) return (uint32_t)i;
        strs.push_back(x);
        return (uint32_t)(strs.size() - 1);
    };
    head->clear();
    put32(*head, intern(name));
    put32(*head, intern(description));
    head->resize(head->size() + 20, 0);
    head->push_back((uint8_t)(entries.size() & 0xFF));
    head->push_back((uint8_t)(entries.size() >> 8));
    for (const auto& e : entries) {
        put32(*head, intern(e.key));
        head->push_back((uint8_t)e.kind);
        if (e.kind == MANTA_MLL_BOOL) head->push_back(e.i64 ? 1 : 0);
        if (e.kind == MANTA_MLL_I64) put64(*head, (uint64_t)e.i64);
        if (e.kind == MANTA_MLL_F64) {
            uint64_t bits;
            memcpy(&bits, &e.f64, 8);
            put64(*head, bits);
        }
        if (e.kind == MANTA_MLL_STRING) put32(*head, intern(e.str));
    }
    strg->clear();
    put64(*strg, strs.size());
    for (size_t i = 1; i < strs.size(); i++) {
        put32(*strg, (uint32_t)strs[i].size());
        strg->insert(strg->end(), strs[i].begin(), strs[i].end());
    }
}

const uint8_t* section_body(const MantaMll* m, const char* tag, uint64_t* size) {
    const MantaMll::Section* s = find_section(m, tag);
    if (!s) return nullptr;
    *size = s->size;
    return m->bytes.data() + s->offset;
}

}  // namespace manta_mll

extern "C" {

void manta_mll_blake3(const void* data, size_t size, uint8_t out[32]) {
    blake3((const uint8_t*)data, size, out);
}

int manta_mll_open(const void* data, size_t size, int verify, MantaMll** out, char** err) {
    if (!out) return mll_fail(err, "nil output handle");
    *out = nullptr;
    const uint8_t* p = (const uint8_t*)data;
    if (!p || size < 4 || memcmp(p, "MLL\0", 4) != 0) return mll_fail(err, "not an MLL manifest");
    if (size < 24) return mll_fail(err, "MLL header truncated: %zu bytes", size);
    const uint64_t declared = rd64(p + 8), count = rd64(p + 16);
    if (declared != size)
        return mll_fail(err, "MLL file size %llu, header says %llu", (unsigned long long)size,
                        (unsigned long long)declared);
    if (count > (size - 24) / 64) return mll_fail(err, "MLL section table of %llu entries past the end",
                                                  (unsigned long long)count);
    MantaMll* m = new MantaMll();
    m->bytes.assign(p, p + size);
    m->format_word = rd32(p + 4);
    const uint64_t body = 24 + 64 * count;
    for (uint64_t i = 0; i < count; i++) {
        const uint8_t* e = p + 24 + 64 * i;
        MantaMll::Section s;
        memcpy(s.tag, e, 4);
        s.tag[4] = 0;
        s.offset = rd64(e + 4);
        s.size = rd64(e + 12);
        memcpy(s.digest, e + 20, 32);
        s.flags = rd32(e + 52);
        if (s.offset < body || s.offset > size || s.size > size - s.offset) {
            manta_mll_close(m);
            return mll_fail(err, "MLL section %s [%llu, +%llu) outside the file", s.tag,
                            (unsigned long long)s.offset, (unsigned long long)s.size);
        }
        if (verify) {
            uint8_t d[32];
            blake3(p + s.offset, (size_t)s.size, d);
            if (memcmp(d, s.digest, 32) != 0) {
                manta_mll_close(m);
                return mll_fail(err, "MLL section %s digest mismatch", s.tag);
            }
        }
        m->sections.push_back(s);
    }
    if (const auto* s = find_section(m, "STRG")) parse_strings(m, m->bytes.data() + s->offset, s->size);
    if (const auto* s = find_section(m, "HEAD")) parse_head(m, m->bytes.data() + s->offset, s->size);
    *out = m;
    return MANTA_ROCM_OK;
}

void manta_mll_close(MantaMll* m) { delete m; }

uint32_t manta_mll_format_word(const MantaMll* m) { return m ? m->format_word : 0; }

int manta_mll_section_count(const MantaMll* m) { return m ? (int)m->sections.size() : 0; }

int manta_mll_section_info(const MantaMll* m, int index, char tag[5], uint64_t* offset, uint64_t* size,
                           uint32_t* flags, uint8_t digest[32], char** err) {
    if (!m) return mll_fail(err, "nil MLL handle");
    if (index < 0 || index >= (int)m->sections.size()) return mll_fail(err, "section index %d out of range", index);
    const auto& s = m->sections[(size_t)index];
    if (tag) memcpy(tag, s.tag, 5);
    if (offset) *offset = s.offset;
    if (size) *size = s.size;
    if (flags) *flags = s.flags;
    if (digest) memcpy(digest, s.digest, 32);
    return MANTA_ROCM_OK;
}

int manta_mll_section(const MantaMll* m, const char* tag, const void** data, uint64_t* size, char** err) {
    if (!m || !tag) return mll_fail(err, "nil MLL handle or tag");
    const auto* s = find_section(m, tag);
    if (!s) return mll_fail(err, "manifest missing %.4s section", tag);
    if (data) *data = m->bytes.data() + s->offset;
    if (size) *size = s->size;
    return MANTA_ROCM_OK;
}

int manta_mll_string_count(const MantaMll* m) { return m && m->strings_ok ? (int)m->strings.size() : 0; }

const char* manta_mll_string(const MantaMll* m, uint32_t id) {
    if (!m || !m->strings_ok || id >= m->strings.size()) return "";
    return m->strings[id].c_str();
}

int manta_mll_head(const MantaMll* m, uint32_t* name, uint32_t* description, int* entries, char** err) {
    if (!m) return mll_fail(err, "nil MLL handle");
    if (!find_section(m, "HEAD")) return mll_fail(err, "manifest missing HEAD section");
    if (!find_section(m, "STRG")) return mll_fail(err, "manifest missing STRG section");
    if (!m->head_error.empty()) return mll_fail(err, "%s", m->head_error.c_str());
    if (!m->strings_ok) return mll_fail(err, "%s", m->strg_error.c_str());
    if (name) *name = m->name;
    if (description) *description = m->description;
    if (entries) *entries = (int)m->entries.size();
    return MANTA_ROCM_OK;
}

int manta_mll_head_entry(const MantaMll* m, int index, uint32_t* key, int* kind, int64_t* i64, double* f64,
                         uint32_t* str, char** err) {
    int rc = manta_mll_head(m, nullptr, nullptr, nullptr, err);
    if (rc) return rc;
    if (index < 0 || index >= (int)m->entries.size()) return mll_fail(err, "HEAD entry %d out of range", index);
    const auto& e = m->entries[(size_t)index];
    if (key) *key = e.key;
    if (kind) *kind = e.kind;
    if (i64) *i64 = e.i64;
    if (f64) *f64 = e.f64;
    if (str) *str = e.str;
    return MANTA_ROCM_OK;
}

int manta_mll_write_packed(const char* path, const char* name, int dtype, uint64_t rows, uint32_t dim,
                           const void* codes, const void* scales, const int64_t* ids, char** err) {
    if (!path) return mll_fail(err, "nil path");
    if (dtype != MANTA_ROCM_Q8_ROWS && dtype != MANTA_ROCM_Q4_BLOCKS)
        return mll_fail(err, "packed candidates: dtype %d is neither q8 (8) nor q4 (4)", dtype);
    if (rows == 0 || dim == 0 || (dtype == MANTA_ROCM_Q4_BLOCKS && dim % 32 != 0))
        return mll_fail(err, "packed candidates: bad shape [%llu,%u]", (unsigned long long)rows, dim);
    if (!codes || !scales) return mll_fail(err, "packed candidates: nil codes or scales");
    uint64_t ncode = 0, nscale = 0;
    packed_sizes(dtype, rows, dim, &ncode, &nscale);
    // string table: 1 name, 2 description, then keys and string values
    const char* strs[] = {name ? name : "", "Manta packed candidates", "manifest_kind", kPackedKind,
                          "manifest_version", kPackedVersion, "docs_dtype",
                          dtype == MANTA_ROCM_Q8_ROWS ? "q8" : "q4", "rows", "dim", "has_ids"};
    const int nstr = (int)(sizeof(strs) / sizeof(strs[0]));
    std::vector<uint8_t> strg;
    put64(strg, (uint64_t)nstr + 1);
    for (int i = 0; i < nstr; i++) {
        const uint32_t len = (uint32_t)strlen(strs[i]);
        put32(strg, len);
        strg.insert(strg.end(), strs[i], strs[i] + len);
    }
    std::vector<uint8_t> head;
    put32(head, 1);
    put32(head, 2);
    head.resize(head.size() + 20, 0);
    head.push_back(6);
    head.push_back(0);
    for (uint32_t k = 3; k <= 7; k += 2) {  // three string-valued entries
        put32(head, k);
        head.push_back(MANTA_MLL_STRING);
        put32(head, k + 1);
    }
    put32(head, 9);
    head.push_back(MANTA_MLL_I64);
    put64(head, rows);
    put32(head, 10);
    head.push_back(MANTA_MLL_I64);
    put64(head, dim);
    put32(head, 11);
    head.push_back(MANTA_MLL_BOOL);
    head.push_back(ids ? 1 : 0);

    // flags: bit 0 required, bit 4 page aligned, schema version in bits 16+
    std::vector<manta_mll::SectionRef> secs = {{"HEAD", head.data(), head.size(), 0x10001u, 0},
                                               {"STRG", strg.data(), strg.size(), 0x10001u, 0},
                                               {"QCOD", (const uint8_t*)codes, ncode, 0x10011u, 0},
                                               {"QSCL", (const uint8_t*)scales, nscale, 0x10011u, 0}};
    if (ids) secs.push_back({"QIDS", (const uint8_t*)ids, rows * 8, 0x10011u, 0});
    uint64_t total = 0;
    const std::vector<uint8_t> top = manta_mll::build_table(&secs, &total);
    FILE* f = fopen(path, "wb");
    if (!f) return mll_fail(err, "packed candidates: cannot create %s", path);
    bool ok = fwrite(top.data(), 1, top.size(), f) == top.size();
    uint64_t pos = top.size();
    static const uint8_t zeros[4096] = {0};
    for (const auto& s : secs) {
        if (!ok) break;
        ok = fwrite(zeros, 1, (size_t)(s.off - pos), f) == (size_t)(s.off - pos) &&
             fwrite(s.p, 1, (size_t)s.n, f) == (size_t)s.n;
        pos = s.off + s.n;
    }
    if (fclose(f) != 0) ok = false;
    if (!ok) return mll_fail(err, "packed candidates: short write to %s", path);
    return MANTA_ROCM_OK;
}

int manta_mll_packed_info(const MantaMll* m, int* dtype, uint64_t* rows, uint32_t* dim, const void** codes,
                          const void** scales, const int64_t** ids, char** err) {
    int rc = manta_mll_head(m, nullptr, nullptr, nullptr, err);
    if (rc) return rc;
    const MantaMll::Entry* kind = head_value(m, "manifest_kind");
    const MantaMll::Entry* version = head_value(m, "manifest_version");
    if (!kind || kind->kind != MANTA_MLL_STRING || m->strings[kind->str] != kPackedKind)
        return mll_fail(err, "manifest kind \"%s\", want \"%s\"",
                        kind && kind->kind == MANTA_MLL_STRING ? manta_mll_string(m, kind->str) : "",
                        kPackedKind);
    if (!version || version->kind != MANTA_MLL_STRING || m->strings[version->str] != kPackedVersion)
        return mll_fail(err, "manifest version \"%s\", want \"%s\"",
                        version && version->kind == MANTA_MLL_STRING ? manta_mll_string(m, version->str) : "",
                        kPackedVersion);
    const MantaMll::Entry* dt = head_value(m, "docs_dtype");
    const MantaMll::Entry* nr = head_value(m, "rows");
    const MantaMll::Entry* nd = head_value(m, "dim");
    const MantaMll::Entry* hi = head_value(m, "has_ids");
    if (!dt || dt->kind != MANTA_MLL_STRING || !nr || nr->kind != MANTA_MLL_I64 || !nd ||
        nd->kind != MANTA_MLL_I64 || !hi || hi->kind != MANTA_MLL_BOOL)
        return mll_fail(err, "packed candidates: docs_dtype, rows, dim or has_ids missing or mistyped");
    const std::string& dts = m->strings[dt->str];
    const int t = dts == "q8" ? MANTA_ROCM_Q8_ROWS : (dts == "q4" ? MANTA_ROCM_Q4_BLOCKS : 0);
    if (!t) return mll_fail(err, "packed candidates: docs_dtype \"%s\" is neither q8 nor q4", dts.c_str());
    // rows index with int32 ids and every section size must fit 64 bits
    if (nr->i64 <= 0 || nr->i64 >= (1ll << 31) || nd->i64 <= 0 || nd->i64 > 0xFFFFFFFFll ||
        (t == MANTA_ROCM_Q4_BLOCKS && nd->i64 % 32))
        return mll_fail(err, "packed candidates: bad shape [%lld,%lld]", (long long)nr->i64, (long long)nd->i64);
    uint64_t want[3] = {0, 0, (uint64_t)nr->i64 * 8};
    packed_sizes(t, (uint64_t)nr->i64, (uint64_t)nd->i64, &want[0], &want[1]);
    const char* tags[3] = {"QCOD", "QSCL", "QIDS"};
    const void* ptr[3] = {nullptr, nullptr, nullptr};
    for (int i = 0; i < (hi->i64 ? 3 : 2); i++) {
        const MantaMll::Section* s = find_section(m, tags[i]);
        if (!s) return mll_fail(err, "manifest missing %s section", tags[i]);
        if (s->size != want[i])
            return mll_fail(err, "packed candidates: %s section is %llu bytes, want %llu", tags[i],
                            (unsigned long long)s->size, (unsigned long long)want[i]);
        ptr[i] = m->bytes.data() + s->offset;
    }
    if (dtype) *dtype = t;
    if (rows) *rows = (uint64_t)nr->i64;
    if (dim) *dim = (uint32_t)nd->i64;
    if (codes) *codes = ptr[0];
    if (scales) *scales = ptr[1];
    if (ids) *ids = (const int64_t*)ptr[2];
    return MANTA_ROCM_OK;
}

}  // extern "C"
