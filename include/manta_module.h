/*
 * manta_module.h -- Manta artifacts (modules) and their step executor on
 * the MI355X: the C-ABI a non-Go host (or the Go rocm backend) uses to
 * decode an artifact, check it against a serving manifest, and run its
 * entry points on device.
 *
 * Reference interfaces replaced (odvcencio/manta):
 *   manta_module_decode_json   <- mantaartifact.DecodeJSON (artifact/manta/module.go:494-505)
 *   manta_module_decode_mll    <- mantaartifact.DecodeMLL  (artifact/manta/mll.go:291-305)
 *   manta_module_encode_json   <- mantaartifact.EncodeJSON (module.go:486-492)
 *   manta_module_encode_mll    <- the XMTA / HEAD / STRG part of mantaartifact.EncodeMLL
 *                                 (mll.go:94-289); not a full replacement (see the function)
 *   manta_module_validate      <- (*Module).Validate       (module.go:255-424)
 *   manta_module_validate_*    <- validateScoreEntry (runtime/score_model.go:276-324),
 *                                 validateRetrievalEntry (runtime/retrieval_model.go:274-330),
 *                                 validateEmbeddingEntry / validateEmbeddingParam
 *                                 (runtime/embedding_model.go:734-800)
 *   manta_manifest_validate_module <- {Score,Retrieval,Embedding}Manifest.ValidateModule after
 *                                 normalized() (score_model.go:212-251, retrieval_model.go:217-259,
 *                                 embedding_model.go:617-673) for an authored .mll manifest
 *   manta_rocm_program_*       <- Backend.Load + Executor.Run driving backend.ExecuteSymbolic
 *                                 (runtime/backend/symbolic.go:14-163, tensor_ops.go:13-474)
 *
 * Error convention as manta_rocm.h: int status (MANTA_ROCM_OK / _ERROR /
 * _UNSUPPORTED), message in *err (free with manta_rocm_free_error).
 */
#ifndef MANTA_MODULE_H
#define MANTA_MODULE_H

#include <stddef.h>
#include <stdint.h>

#include "manta_mll.h"
#include "manta_rocm.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct MantaModule MantaModule;

/* ---- artifact codec ----------------------------------------------------- */

/* Parse module JSON (json.Unmarshal field rules and error wording), then
 * Validate. */
int manta_module_decode_json(const char* json, size_t len, MantaModule** out, char** err);
/* The module held in an opened container's XMTA section: MLLMetadata JSON
 * (version "manta/mll/v0alpha1", module_name, module_version, artifact)
 * checked like MLLMetadata.Validate (mll.go:53-88), then the artifact
 * decoded like manta_module_decode_json.  Open the container with digest
 * verification (manta_mll_open verify=1) as DecodeMLL does. */
int manta_module_decode_mll(const MantaMll* container, MantaModule** out, char** err);
void manta_module_free(MantaModule* m);
int manta_module_validate(const MantaModule* m, char** err);
const char* manta_module_name(const MantaModule* m);
/* Validate, then the module as MarshalIndent(m, "", "  ") text; *out is
 * malloc'd (free with manta_module_free_buffer). */
int manta_module_encode_json(const MantaModule* m, char** out, size_t* len, char** err);
/* A container holding the module: HEAD (name, description "Manta module
 * artifact", artifact_version, supported_backends, capabilities, param /
 * entry / kernel counts), STRG, and XMTA with the MLLMetadata JSON -- what
 * DecodeMLL reads, so a container written here decodes to the same module
 * there and here.  It differs from EncodeMLL's output: the typed DIMS /
 * TYPE / PARM / ENTR / TNSR / SCHM tables are written empty and the BUFF /
 * KRNL sections are left out (their layout belongs to the unvendored mll
 * codec and no reference container carries them filled), so a tool that
 * reads the typed tables sees none.  *out is malloc'd
 * (manta_module_free_buffer). */
int manta_module_encode_mll(const MantaModule* m, void** out, size_t* len, char** err);
void manta_module_free_buffer(void* p);

/* ---- serving contracts ------------------------------------------------- */

/* Empty strings mean "not checked", as the reference's empty manifest
 * fields do (after the manifests' own defaults). */
int manta_module_validate_score_entry(const MantaModule* m, const char* entry, const char* query_input,
                                      int query_rank, const char* docs_input, int docs_rank, const char* query_dtype,
                                      const char* docs_dtype, const char* output_name, int output_rank,
                                      const char* output_dtype, char** err);
int manta_module_validate_retrieval_entry(const MantaModule* m, const char* entry, const char* query_input,
                                          int query_rank, const char* docs_input, int docs_rank,
                                          const char* ids_input, int ids_rank, const char* query_dtype,
                                          const char* docs_dtype, const char* ids_dtype, const char* output_name,
                                          int output_rank, char** err);
int manta_module_validate_embedding_entry(const MantaModule* m, const char* entry, const char* token_input,
                                          const char* mask_input, int token_rank, int output_rank,
                                          const char* output_dtype, char** err);
int manta_module_validate_embedding_param(const MantaModule* m, const char* name, char** err);
/* An authored manifest container (score_manifest, retrieval_manifest or
 * embedding_manifest HEAD metadata, as the *.score.mll / *.retrieval.mll /
 * *.embedding.mll files carry) checked against a module: the manifest's
 * kind and version, its values read with the typed accessors' wording, the
 * normalized() defaults, then ValidateModule. */
int manta_manifest_validate_module(const MantaMll* manifest, const MantaModule* m, char** err);

/* ---- runtime values ------------------------------------------------------ */

/* Element types: the artifact's dtype strings f32, f16, i32, i64, q8, q4. */
enum {
    MANTA_DT_F32 = 1,
    MANTA_DT_F16 = 2, /* IEEE binary16 bits */
    MANTA_DT_I32 = 3,
    MANTA_DT_I64 = 4,
    MANTA_DT_Q8 = 5,
    MANTA_DT_Q4 = 6
};

/* Value kinds. */
enum {
    /* dense tensor: `data` holds prod(shape) elements of type `storage`;
     * storage MANTA_DT_Q8: int8 codes with an f32 scale per column (last
     * dimension) in `scales` -- a q8 weight matrix, whose values are the
     * f32 products code * scale (a reference per-tensor grid repacks
     * exactly, one scale repeated) */
    MANTA_VALUE_TENSOR = 0,
    /* a q8 / q4 tensor [n, d] or [sets, n, d] bound on device
     * (manta_rocm_bind_q8_rows / _q4_blocks / _packed): `candidates` */
    MANTA_VALUE_CANDIDATES = 1,
    /* packed rows gathered from candidates, shape [k, d] or [q, k, d]:
     * `data` rows (storage MANTA_DT_Q8: d int8 codes per row; MANTA_DT_Q4:
     * d/2 nibble bytes), `scales` (q8: one f32 per row; q4: d/32 f16) */
    MANTA_VALUE_ROWS = 2,
    /* a candidate_pack (tensor.go:27-31): ids [..., k] in `ids` (ids_dtype),
     * f32 scores [..., k] in `scores`, docs as MANTA_VALUE_ROWS in
     * data/scales with shape = the docs' shape */
    MANTA_VALUE_CANDIDATE_PACK = 3
};

typedef struct MantaRocmValue {
    const char* name;
    int kind;
    int dtype;   /* the artifact's element type (MANTA_DT_*) */
    int storage; /* layout of `data`: a value the artifact types f16 but that is
                  * computed in f32 (a matmul, normalize or mean_pool result) is
                  * returned in f32, as the reference's Tensor carries f16 values
                  * in F32 (tensor.go:11-19) */
    int rank;
    int64_t shape[4];
    void* data;
    void* scales;
    void* ids;
    void* scores;
    int ids_dtype;
    const MantaRocmCandidates* candidates;
} MantaRocmValue;

/* ---- step executor ----------------------------------------------------- */

typedef struct MantaRocmProgram MantaRocmProgram;

/* Backend.Load: the module must list "rocm" or "cuda" among its supported
 * backends (artifacts built for the CUDA backend run unchanged; kernel
 * variant sources are not used: every kernel is run by its body ops).  The
 * program copies the module. */
int manta_rocm_program_load(MantaRocm* rt, const MantaModule* m, MantaRocmProgram** out, char** err);
void manta_rocm_program_destroy(MantaRocmProgram* p);
/* Bind a param's weight (WeightBinding): a device tensor or bound candidates
 * named after the param; the caller keeps the memory alive.  Steps read the
 * bound memory on every run, except matmul: an f16 or q8 [K, N] weight with
 * K % 32 == 0 and N % 128 == 0 is copied once, here, into the transposed f16
 * operand the pipelined GEMM reads (owned by the program), as the CUDA
 * backend uploads its resident matmul params once at Load
 * (bindResidentMatMulParams, runtime/backends/cuda/cuda.go:129-169).  A
 * weight changed in place after bind must therefore be bound again: binding
 * the same name replaces the copy. */
int manta_rocm_program_bind(MantaRocmProgram* p, const MantaRocmValue* value, char** err);
/* MANTA_ROCM_OK when every step of `entry` runs on device, else
 * MANTA_ROCM_UNSUPPORTED naming the first step that does not (the caller
 * then runs that entry through its host path). */
int manta_rocm_program_supports(const MantaRocmProgram* p, const char* entry, char** err);
/* Run an entry point (ExecuteSymbolic): inputs are device values named
 * after the entry's inputs; the entry's outputs are written to outputs[0 ..
 * *n_outputs) in declaration order.  Output memory belongs to the program
 * and stays valid until the next run of the same entry or destroy.  Score
 * kernels use the reference's arithmetic (manta_rocm_score without
 * MANTA_ROCM_QUANTIZED_QUERY).  A score whose only consumers are one topk
 * and gathers by that topk's indices is computed with
 * manta_rocm_score_topk: the score matrix is never written.  Synchronous. */
int manta_rocm_program_run(MantaRocmProgram* p, const char* entry, const MantaRocmValue* inputs, int64_t n_inputs,
                           MantaRocmValue* outputs, int64_t max_outputs, int64_t* n_outputs, char** err);
/* The last run's trace (TraceStep, backend.go): step kind, name, and how it
 * ran ("hip:<kernel family>", "alias", "fused:<step>" for a score folded
 * into the following topk, "return"). */
int64_t manta_rocm_program_trace_count(const MantaRocmProgram* p);
int manta_rocm_program_trace_step(const MantaRocmProgram* p, int64_t index, const char** kind, const char** name,
                                  const char** dispatch);

#ifdef __cplusplus
}
#endif

#endif /* MANTA_MODULE_H */
