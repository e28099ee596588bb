"""Deterministic synthetic workloads of the five BASELINE configurations.

Thin ctypes layer over libmanta_synth.so (csrc/synth.cpp): counter-based
SplitMix64 streams keyed by (seed, tensor id), Box-Muller normals, rows
generated in f64, optionally L2-normalized, narrowed to f32 and rounded to
f16 or packed with the library's q8/q4 packers.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from ._lib import SYNTH_PATH

_S = None


def _lib() -> C.CDLL:
    global _S
    if _S is None:
        if not os.path.exists(SYNTH_PATH):
            raise RuntimeError("libmanta_synth.so is not built; run `python -m manta_amd.build`")
        lib = C.CDLL(SYNTH_PATH)
        u64, i64, i32, dbl, p = C.c_uint64, C.c_int64, C.c_int32, C.c_double, C.c_void_p
        lib.manta_synth_normal_rows_f32.argtypes = [u64, u64, i64, i64, dbl, C.c_int, p]
        lib.manta_synth_normal_rows_f16.argtypes = [u64, u64, i64, i64, dbl, C.c_int, p]
        lib.manta_synth_q8_rows.argtypes = [u64, u64, i64, i64, C.c_int, p, p]
        lib.manta_synth_q4_rows.argtypes = [u64, u64, i64, i64, C.c_int, p, p]
        lib.manta_synth_uniform_i32.argtypes = [u64, u64, i64, i32, i32, p]
        lib.manta_synth_uniform_i8.argtypes = [u64, u64, i64, i32, i32, p]
        for f in ("manta_synth_normal_rows_f32", "manta_synth_normal_rows_f16", "manta_synth_q8_rows",
                  "manta_synth_q4_rows", "manta_synth_uniform_i32", "manta_synth_uniform_i8"):
            getattr(lib, f).restype = None
        _S = lib
    return _S


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def normal_f32(seed, tensor, n, d, sigma=1.0, normalize=False) -> np.ndarray:
    out = np.empty((n, d), np.float32)
    _lib().manta_synth_normal_rows_f32(seed, tensor, n, d, sigma, int(normalize), _p(out))
    return out


def normal_f16(seed, tensor, n, d, sigma=1.0, normalize=False) -> np.ndarray:
    """f16 bit patterns (uint16) of N(0, sigma) rows."""
    out = np.empty((n, d), np.uint16)
    _lib().manta_synth_normal_rows_f16(seed, tensor, n, d, sigma, int(normalize), _p(out))
    return out


def q8_rows(seed, tensor, n, d, normalize=False):
    codes = np.empty((n, d), np.int8)
    scales = np.empty((n,), np.float32)
    _lib().manta_synth_q8_rows(seed, tensor, n, d, int(normalize), _p(codes), _p(scales))
    return codes, scales


def q4_rows(seed, tensor, n, d, normalize=False):
    packed = np.empty((n, d // 2), np.uint8)
    scales = np.empty((n, d // 32), np.uint16)
    _lib().manta_synth_q4_rows(seed, tensor, n, d, int(normalize), _p(packed), _p(scales))
    return packed, scales


def uniform_i32(seed, tensor, n, lo, hi) -> np.ndarray:
    out = np.empty((n,), np.int32)
    _lib().manta_synth_uniform_i32(seed, tensor, n, lo, hi, _p(out))
    return out


def uniform_i8(seed, tensor, n, lo, hi) -> np.ndarray:
    out = np.empty((n,), np.int8)
    _lib().manta_synth_uniform_i8(seed, tensor, n, lo, hi, _p(out))
    return out


# ---------------------------------------------------------------- configs
# Tensor ids per config are part of the workload definition.

def config0(n=65536, d=256, sets=1, set_offset=0):
    """q8 dot + top-10 (seed 0).  sets > 1 gives independent candidate
    matrices (tensor ids 1+set_offset+s) and one query per set."""
    queries = normal_f16(0, 0, sets, d, 1.0, normalize=True)
    codes = np.empty((sets, n, d), np.int8)
    scales = np.empty((sets, n), np.float32)
    for s in range(sets):
        codes[s], scales[s] = q8_rows(0, 1 + set_offset + s, n, d, normalize=True)
    return queries, codes, scales


def config1(b=64, t=128, vocab=32000, d=384, e=384):
    """Embed pipeline f16 (seed 1)."""
    tokens = uniform_i32(1, 0, b * t, 0, vocab).reshape(b, t)
    lengths = uniform_i32(1, 1, b, 16, 129)
    mask = (np.arange(t)[None, :] < lengths[:, None]).astype(np.int32)
    table = normal_f16(1, 2, vocab, d, 0.02)
    proj = normal_f16(1, 3, d, e, 1.0 / np.sqrt(d))
    return tokens, mask, table, proj


def config2(nq=256, n=1048576, d=384):
    """Batched q4 cosine + top-100 (seed 2)."""
    queries = normal_f16(2, 0, nq, d, 1.0, normalize=True)
    packed, scales = q4_rows(2, 1, n, d, normalize=True)
    return queries, packed, scales


def config3(nq=32, n=8388608, d=128):
    """q8 l2 rerank, smallest-1000 (seed 3); rows unnormalized N(0,1)."""
    queries = normal_f16(3, 0, nq, d, 1.0)
    codes, scales = q8_rows(3, 1, n, d, normalize=False)
    return queries, codes, scales


def config4(nq=1024, t=64, vocab=32000, d=384, n=4194304):
    """Embed (q8 projection) then q8 dot top-50 (seed 4)."""
    tokens = uniform_i32(4, 0, nq * t, 0, vocab).reshape(nq, t)
    mask = np.ones((nq, t), np.int32)
    table = normal_f16(4, 1, vocab, d, 0.02)
    proj_codes = uniform_i8(4, 2, d * d, -127, 127).reshape(d, d)
    col_scale = np.full((d,), 1.0 / (127.0 * np.sqrt(d)), np.float32)
    codes, scales = q8_rows(4, 3, n, d, normalize=True) if n else (None, None)
    return tokens, mask, table, proj_codes, col_scale, codes, scales
