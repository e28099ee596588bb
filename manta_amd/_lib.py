"""ctypes bindings of libmanta_rocm.so (include/manta_rocm.h).

The library is loaded from this package directory only.  There is no
fallback: if it is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmanta_rocm.so")
SYNTH_PATH = os.path.join(HERE, "libmanta_synth.so")

OK, ERROR, UNSUPPORTED = 0, 1, 2
DOT, COSINE, L2_DISTANCE = 0, 1, 2
QUANTIZED_QUERY = 0x100
LARGEST, SMALLEST = 0, 1
Q8_ROWS, Q4_BLOCKS = 8, 4
PROJ_F16, PROJ_Q8_COL, PROJ_F16_T, PROJ_Q8_COL_T = 0, 1, 2, 3
DENSE_F32, DENSE_F16 = 32, 16

OPS = {"dot": DOT, "cosine": COSINE, "l2_distance": L2_DISTANCE}

# Every exported symbol of include/manta_rocm.h, include/manta_mll.h and
# include/manta_module.h:
# name -> (restype, argtypes).
_p = C.c_void_p
_i64 = C.c_int64
_err = C.POINTER(C.c_char_p)


class Stats(C.Structure):
    _fields_ = [
        ("kernel_launches", C.c_uint64),
        ("bytes_uploaded", C.c_uint64),
        ("bytes_downloaded", C.c_uint64),
        ("workspace_bytes", C.c_uint64),
        ("candidate_bytes", C.c_uint64),
    ]


class EncoderWeights(C.Structure):
    """MantaRocmEncoderWeights: device pointers of the encoder's q8 weights."""
    _fields_ = [
        ("token_codes", C.c_void_p),
        ("token_scales", C.c_void_p),
        ("codes", C.c_void_p * 6),
        ("col_scales", C.c_void_p * 6),
    ]


class Value(C.Structure):
    """MantaRocmValue (include/manta_module.h)."""
    _fields_ = [
        ("name", C.c_char_p),
        ("kind", C.c_int),
        ("dtype", C.c_int),
        ("storage", C.c_int),
        ("rank", C.c_int),
        ("shape", C.c_int64 * 4),
        ("data", C.c_void_p),
        ("scales", C.c_void_p),
        ("ids", C.c_void_p),
        ("scores", C.c_void_p),
        ("ids_dtype", C.c_int),
        ("candidates", C.c_void_p),
    ]


SIGNATURES = {
    "manta_rocm_abi_version": (C.c_int, []),
    "manta_rocm_device_count": (C.c_int, [C.POINTER(C.c_int), _err]),
    "manta_rocm_create": (C.c_int, [C.c_int, C.POINTER(_p), _err]),
    "manta_rocm_destroy": (None, [_p]),
    "manta_rocm_free_error": (None, [_p]),
    "manta_rocm_set_stream": (C.c_int, [_p, _p, _err]),
    "manta_rocm_synchronize": (C.c_int, [_p, _err]),
    "manta_rocm_malloc": (C.c_int, [_p, C.POINTER(_p), C.c_size_t, _err]),
    "manta_rocm_free": (C.c_int, [_p, _p, _err]),
    "manta_rocm_upload": (C.c_int, [_p, _p, _p, C.c_size_t, _err]),
    "manta_rocm_download": (C.c_int, [_p, _p, _p, C.c_size_t, _err]),
    "manta_rocm_stats": (C.c_int, [_p, C.POINTER(Stats)]),
    "manta_rocm_set_timing": (C.c_int, [_p, C.c_int, _err]),
    "manta_rocm_timing": (
        C.c_int,
        [_p, C.c_char_p, C.POINTER(C.c_uint64), C.POINTER(C.c_double), C.c_int, _err],
    ),
    "manta_rocm_span": (C.c_int, [_p, C.c_int, C.POINTER(C.c_double), _err]),
    "manta_rocm_encoder_pooled_layers": (
        C.c_int, [_p, _p, _p, _i64, _i64, C.POINTER(EncoderWeights), _i64, _i64, _i64, _i64, _p, _err]),
    "manta_rocm_encoder_pooled": (
        C.c_int, [_p, _p, _p, _i64, _i64, C.POINTER(EncoderWeights), _i64, _i64, _i64, _p, _err]),
    # include/manta_mll.h (host only)
    "manta_mll_open": (C.c_int, [_p, C.c_size_t, C.c_int, C.POINTER(_p), _err]),
    "manta_mll_close": (None, [_p]),
    "manta_mll_format_word": (C.c_uint32, [_p]),
    "manta_mll_section_count": (C.c_int, [_p]),
    "manta_mll_section_info": (
        C.c_int,
        [_p, C.c_int, C.c_char_p, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), C.POINTER(C.c_uint32), _p, _err],
    ),
    "manta_mll_section": (C.c_int, [_p, C.c_char_p, C.POINTER(_p), C.POINTER(C.c_uint64), _err]),
    "manta_mll_string_count": (C.c_int, [_p]),
    "manta_mll_string": (C.c_char_p, [_p, C.c_uint32]),
    "manta_mll_head": (
        C.c_int, [_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.POINTER(C.c_int), _err]),
    "manta_mll_head_entry": (
        C.c_int,
        [_p, C.c_int, C.POINTER(C.c_uint32), C.POINTER(C.c_int), C.POINTER(C.c_int64), C.POINTER(C.c_double),
         C.POINTER(C.c_uint32), _err],
    ),
    "manta_mll_blake3": (None, [_p, C.c_size_t, _p]),
    "manta_mll_write_packed": (
        C.c_int, [C.c_char_p, C.c_char_p, C.c_int, C.c_uint64, C.c_uint32, _p, _p, _p, _err]),
    "manta_mll_packed_info": (
        C.c_int, [_p, C.POINTER(C.c_int), C.POINTER(C.c_uint64), C.POINTER(C.c_uint32), C.POINTER(_p),
                  C.POINTER(_p), C.POINTER(_p), _err]),
    "manta_rocm_pack_q8_rows": (C.c_int, [_p, _i64, _i64, _p, _p, _err]),
    "manta_rocm_pack_q4_blocks": (C.c_int, [_p, _i64, _i64, _p, _p, _err]),
    "manta_rocm_pack_grid": (C.c_int, [_p, _i64, _i64, C.c_int, _p, _p, C.POINTER(C.c_int), _err]),
    "manta_rocm_bind_q8_rows": (C.c_int, [_p, _p, _p, _i64, _i64, _i64, C.POINTER(_p), _err]),
    "manta_rocm_bind_q4_blocks": (C.c_int, [_p, _p, _p, _i64, _i64, _i64, C.POINTER(_p), _err]),
    "manta_rocm_bind_packed": (C.c_int, [_p, _p, C.POINTER(_p), _err]),
    "manta_rocm_unbind": (None, [_p]),
    "manta_rocm_candidates_info": (
        C.c_int,
        [_p, C.POINTER(C.c_int), C.POINTER(_i64), C.POINTER(_i64), C.POINTER(_i64)],
    ),
    "manta_rocm_score": (C.c_int, [_p, _p, C.c_int, _p, _i64, _p, _err]),
    "manta_rocm_score_topk": (
        C.c_int,
        [_p, _p, C.c_int, C.c_int, _p, _i64, _i64, _p, _p, _p, _err],
    ),
    "manta_rocm_score_topk_noalloc": (
        C.c_int,
        [_p, _p, C.c_int, C.c_int, _p, _i64, _i64, _p, _p, _p, _err],
    ),
    "manta_rocm_topk": (C.c_int, [_p, _p, _i64, _i64, _i64, C.c_int, _p, _p, _err]),
    "manta_rocm_gather_rows_f16": (C.c_int, [_p, _p, _i64, _i64, _p, _i64, _p, _err]),
    "manta_rocm_pack_candidates": (C.c_int, [_p, _p, _p, _i64, _i64, _p, _p, _p, _p, _err]),
    "manta_rocm_matmul_f16": (C.c_int, [_p, _p, _i64, _i64, _p, C.c_int, _p, _i64, _p, _err]),
    "manta_rocm_mean_pool_masked": (C.c_int, [_p, _p, _p, _i64, _i64, _i64, _p, _err]),
    "manta_rocm_normalize_rows": (C.c_int, [_p, _p, _i64, _i64, _err]),
    "manta_rocm_mean_pool": (C.c_int, [_p, _p, _i64, _i64, _i64, _p, _err]),
    "manta_rocm_dense_scores": (C.c_int, [_p, _p, C.c_int, _i64, _i64, _p, _i64, _i64, _p, _err]),
    "manta_rocm_dense_topk": (C.c_int, [_p, _p, C.c_int, _i64, _i64, _p, _i64, _i64, _i64, _p, _p, _err]),
    # include/manta_module.h
    "manta_module_decode_json": (C.c_int, [C.c_char_p, C.c_size_t, C.POINTER(_p), _err]),
    "manta_module_decode_mll": (C.c_int, [_p, C.POINTER(_p), _err]),
    "manta_module_free": (None, [_p]),
    "manta_module_validate": (C.c_int, [_p, _err]),
    "manta_module_name": (C.c_char_p, [_p]),
    "manta_module_encode_json": (C.c_int, [_p, C.POINTER(_p), C.POINTER(C.c_size_t), _err]),
    "manta_module_encode_mll": (C.c_int, [_p, C.POINTER(_p), C.POINTER(C.c_size_t), _err]),
    "manta_module_free_buffer": (None, [_p]),
    "manta_module_validate_score_entry": (
        C.c_int, [_p, C.c_char_p, C.c_char_p, C.c_int, C.c_char_p, C.c_int, C.c_char_p, C.c_char_p, C.c_char_p,
                  C.c_int, C.c_char_p, _err]),
    "manta_module_validate_retrieval_entry": (
        C.c_int, [_p, C.c_char_p, C.c_char_p, C.c_int, C.c_char_p, C.c_int, C.c_char_p, C.c_int, C.c_char_p,
                  C.c_char_p, C.c_char_p, C.c_char_p, C.c_int, _err]),
    "manta_module_validate_embedding_entry": (
        C.c_int, [_p, C.c_char_p, C.c_char_p, C.c_char_p, C.c_int, C.c_int, C.c_char_p, _err]),
    "manta_module_validate_embedding_param": (C.c_int, [_p, C.c_char_p, _err]),
    "manta_manifest_validate_module": (C.c_int, [_p, _p, _err]),
    "manta_rocm_program_load": (C.c_int, [_p, _p, C.POINTER(_p), _err]),
    "manta_rocm_program_destroy": (None, [_p]),
    "manta_rocm_program_bind": (C.c_int, [_p, C.POINTER(Value), _err]),
    "manta_rocm_program_supports": (C.c_int, [_p, C.c_char_p, _err]),
    "manta_rocm_program_run": (
        C.c_int, [_p, C.c_char_p, C.POINTER(Value), _i64, C.POINTER(Value), _i64, C.POINTER(_i64), _err]),
    "manta_rocm_program_trace_count": (_i64, [_p]),
    "manta_rocm_program_trace_step": (
        C.c_int, [_p, _i64, C.POINTER(C.c_char_p), C.POINTER(C.c_char_p), C.POINTER(C.c_char_p)]),
    "manta_rocm_embed_pooled": (
        C.c_int,
        [_p, _p, _p, _i64, _i64, _p, _i64, _i64, _p, C.c_int, _p, _i64, _p, _err],
    ),
    "manta_rocm_prepare_projection": (C.c_int, [_p, _p, C.c_int, _i64, _i64, _p, C.POINTER(C.c_int), _err]),
}


class MantaRocmError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class Unsupported(MantaRocmError):
    """The device path does not take this shape (host fallback territory)."""


_LIB = None


def load() -> C.CDLL:
    """Load libmanta_rocm.so from the package directory; raise if absent."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            "libmanta_rocm.so is not built (%s); run `python -m manta_amd.build`" % LIB_PATH
        )
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def call(name: str, *args) -> None:
    """Call an error-returning entry point; raise with the library's message."""
    lib = load()
    err = C.c_char_p()
    rc = getattr(lib, name)(*args, C.byref(err))
    if rc != OK:
        msg = err.value.decode() if err.value else "%s failed (%d)" % (name, rc)
        if err.value:
            lib.manta_rocm_free_error(C.cast(err, C.c_void_p))
        if rc == UNSUPPORTED:
            raise Unsupported(rc, msg)
        raise MantaRocmError(rc, msg)
