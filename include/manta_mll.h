/* manta_mll.h -- native reader of Manta's MLL containers (host code, no GPU).
 *
 * Lets a C, C++ or Python host open the same `.mll` files the Go runtime
 * writes -- the authored manifests (`*.score.mll`, `*.embedding.mll`,
 * `*.retrieval.mll`, ...) and the section table of any container -- without
 * the Go toolchain.  The container codec is the external Go module
 * github.com/odvcencio/mll v0.0.1 (go.mod:6), which the reference does not
 * vendor; its layout is restated here from the reference's call sites
 * (artifact/manta/mll.go:90-96, runtime/authored_manifest_mll.go:47-270) and
 * from the bytes of the reference's example containers (the .mll files in
 * examples/), all
 * of whose section digests this reader reproduces:
 *
 *   header   "MLL\0", u32 format word, u64 file size, u64 section count
 *   table    per section 64 bytes: tag[4], u64 offset, u64 size,
 *            BLAKE3-256 digest of the section's bytes [32], u32 flags,
 *            8 reserved bytes
 *   STRG     u64 count, then strings 1..count-1 as u32 length + UTF-8 bytes
 *            (id 0 is the empty string)
 *   HEAD     u32 name id, u32 description id, 20 reserved bytes, u16 entry
 *            count, entries of u32 key id, u8 kind, value: kind 1 bool (1
 *            byte), 2 i64 (8), 3 f64 (8), 4 string id (u32)
 *
 * All integers little-endian.  Functions return MANTA_ROCM_OK (0) or an
 * error code with a malloc'd message in *err (free with
 * manta_rocm_free_error), as the rest of the library. */
#ifndef MANTA_MLL_H
#define MANTA_MLL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct MantaMll MantaMll;

/* HEAD metadata value kinds (mll.HeadValueBool/I64/F64/String). */
enum { MANTA_MLL_BOOL = 1, MANTA_MLL_I64 = 2, MANTA_MLL_F64 = 3, MANTA_MLL_STRING = 4 };

/* Parse a container from memory (the bytes are copied).  verify != 0 checks
 * every section's BLAKE3-256 digest, as mll.ReadBytes(data,
 * mll.WithDigestVerification()) does for manifests
 * (authored_manifest_mll.go:205).  A buffer that does not start with the
 * magic fails with "not an MLL manifest" (mantaartifact.IsMLLBytes,
 * mll.go:94-96; authored_manifest_mll.go:202-204). */
int manta_mll_open(const void* data, size_t size, int verify, MantaMll** out, char** err);
void manta_mll_close(MantaMll* m);

/* The u32 after the magic (0x00010100 in every example container). */
uint32_t manta_mll_format_word(const MantaMll* m);

/* Section table (reader.Section(tag), authored_manifest_mll.go:212-219). */
int manta_mll_section_count(const MantaMll* m);
int manta_mll_section_info(const MantaMll* m, int index, char tag[5], uint64_t* offset, uint64_t* size,
                           uint32_t* flags, uint8_t digest[32], char** err);
/* Bytes of the first section with this 4-character tag; returns
 * MANTA_ROCM_ERROR with "missing <tag> section" if there is none. */
int manta_mll_section(const MantaMll* m, const char* tag, const void** data, uint64_t* size, char** err);

/* String table (mll.ReadStringTable + strg.At): count includes id 0 (""). */
int manta_mll_string_count(const MantaMll* m);
/* NUL-terminated string of id (owned by the handle; "" for id 0 or an id
 * out of range, as strg.At). */
const char* manta_mll_string(const MantaMll* m, uint32_t id);

/* HEAD section (mll.ReadHeadSection): name and description string ids and
 * the metadata entries. */
int manta_mll_head(const MantaMll* m, uint32_t* name, uint32_t* description, int* entries, char** err);
int manta_mll_head_entry(const MantaMll* m, int index, uint32_t* key, int* kind, int64_t* i64, double* f64,
                         uint32_t* str, char** err);

/* BLAKE3-256 of a byte string (the section digest). */
void manta_mll_blake3(const void* data, size_t size, uint8_t out[32]);

/* ---- packed candidate containers ----------------------------------------
 * Real int8 / nibble candidate rows on disk, in place of the f32-widened q4/q8
 * tensors the reference stores (runtime/mll_export.go:858-862, decoded back to
 * f32 by decodeTensorEntry, runtime/weight_file.go:304-367).  The container is
 * the MLL layout above; HEAD holds manifest_kind "packed_candidates",
 * manifest_version "manta/packed-candidates/v0", docs_dtype "q8"|"q4" and
 * rows / dim (i64) / has_ids (bool); the data sections start on 4 KiB pages
 * (flag bit 4, as the reference's TNSR section) and hold raw little-endian
 * arrays:
 *   QCOD  q8: int8 codes [rows][dim]; q4: packed nibbles [rows][dim/2]
 *         (value 2j in the low nibble, 2j+1 in the high one, 4-bit two's
 *         complement)
 *   QSCL  q8: f32 scale per row; q4: f16 scale per 32-value block [rows][dim/32]
 *   QIDS  optional i64 candidate ids [rows]
 * These are the layouts manta_rocm_pack_q8_rows / manta_rocm_pack_q4_blocks
 * produce and manta_rocm_bind_q8_rows / manta_rocm_bind_q4_blocks take, so a
 * container binds to the device without conversion.  No reference
 * counterpart: the format is this library's own (the reference's TNSR tensor
 * entries come from the unvendored codec and hold f32 for q4/q8). */

/* Write a container.  dtype: MANTA_ROCM_Q8_ROWS (8) or MANTA_ROCM_Q4_BLOCKS (4);
 * ids may be NULL. */
int manta_mll_write_packed(const char* path, const char* name, int dtype, uint64_t rows, uint32_t dim,
                           const void* codes, const void* scales, const int64_t* ids, char** err);

/* Check an opened container's metadata and section sizes and return pointers
 * into its bytes (owned by the handle); *ids is NULL without a QIDS section. */
int manta_mll_packed_info(const MantaMll* m, int* dtype, uint64_t* rows, uint32_t* dim, const void** codes,
                          const void** scales, const int64_t** ids, char** err);

#ifdef __cplusplus
}
#endif

#endif /* MANTA_MLL_H */
