// runtime_internal.hpp -- entry points shared between runtime.cpp and the
// allocation-free entry point (noalloc.hip); internal to libmanta_rocm.so.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "manta_rocm.h"

namespace manta_rt {

// Device memory a call carves its buffers from instead of the runtime's
// workspace: [base, base + bytes), `used` bytes taken so far, and the
// last-workgroup tickets (zero between calls) the streaming scans need.
struct Scratch {
    char* base = nullptr;
    size_t bytes = 0;
    size_t used = 0;
    uint32_t* tickets = nullptr;
};

// manta_rocm_score_topk; with sc the call allocates nothing (streaming scans
// only, every buffer from sc, no timing events).
int score_topk_impl(MantaRocm* rt, const MantaRocmCandidates* c, int op, int order, const uint16_t* q, int64_t nq,
                    int64_t k, int32_t* out_ids, float* out_scores, int64_t* out_acc, Scratch* sc, char** err);

int runtime_device(const MantaRocm* rt);

// The stream a runtime launches on (hipStream_t).
void* runtime_stream(const MantaRocm* rt);

// manta_rocm_pack_candidates recording an out-of-range index in err_word
// (a device word the caller owns and clears) instead of the runtime's
// deferred error.
int pack_candidates_into(MantaRocm* rt, const MantaRocmCandidates* c, const int32_t* top, int64_t nq, int64_t k,
                         const int64_t* candidate_ids, int64_t* out_ids, void* out_rows, void* out_scales,
                         unsigned long long* err_word, char** err);

// The index a gather error word holds (report_gather_error's encoding).
inline int gather_error_index(unsigned long long w) { return (int)(uint32_t)(~w & 0xFFFFFFFFull); }

// noalloc.hip: look up the device address of the allocation-free path's
// scratch array on `device` (which must be current); its usable bytes.
void noalloc_init(int device);
size_t noalloc_scratch_bytes();

}  // namespace manta_rt
