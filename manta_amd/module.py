"""Manta artifacts and their step executor (include/manta_module.h).

`Module` decodes, validates and encodes an artifact (DecodeJSON / DecodeMLL /
EncodeJSON / Validate, artifact/manta/module.go and mll.go) and checks it
against the serving contracts (validateScoreEntry / validateRetrievalEntry /
validateEmbeddingEntry, and the authored manifests' ValidateModule).
`Program` runs an entry point's plan steps on the device (ExecuteSymbolic,
runtime/backend/symbolic.go:14-163): inputs are numpy arrays (uploaded) or
bound candidates, outputs come back as numpy.  All of it is the native
library; this module only packs arguments and unpacks results.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Dict, Optional, Union

import numpy as np

from . import _lib
from ._lib import call, load
from .rocm import Candidates, DeviceArray, Runtime

TENSOR, CANDIDATES, ROWS, CANDIDATE_PACK = 0, 1, 2, 3
F32, F16, I32, I64, Q8, Q4 = 1, 2, 3, 4, 5, 6
DTYPE_NAMES = {F32: "f32", F16: "f16", I32: "i32", I64: "i64", Q8: "q8", Q4: "q4"}
DTYPE_CODES = {v: k for k, v in DTYPE_NAMES.items()}
_NP = {F32: np.float32, F16: np.uint16, I32: np.int32, I64: np.int64}


def _take_buffer(ptr: C.c_void_p, n: int) -> bytes:
    data = C.string_at(ptr, n)
    load().manta_module_free_buffer(ptr)
    return data


class Module:
    """A decoded, validated artifact (MantaModule*)."""

    def __init__(self, handle: C.c_void_p):
        self.handle = handle

    @classmethod
    def from_json(cls, text: Union[str, bytes]) -> "Module":
        data = text.encode() if isinstance(text, str) else bytes(text)
        h = C.c_void_p()
        call("manta_module_decode_json", data, len(data), C.byref(h))
        return cls(h)

    @classmethod
    def from_mll(cls, data: Union[bytes, str, os.PathLike], verify: bool = True) -> "Module":
        from .mll import MllFile
        with MllFile(data, verify=verify) as f:
            h = C.c_void_p()
            call("manta_module_decode_mll", f._h, C.byref(h))
        return cls(h)

    def close(self) -> None:
        if self.handle is not None and self.handle.value:
            load().manta_module_free(self.handle)
        self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def name(self) -> str:
        return load().manta_module_name(self.handle).decode()

    def validate(self) -> None:
        call("manta_module_validate", self.handle)

    def to_json(self) -> str:
        out, n = C.c_void_p(), C.c_size_t()
        call("manta_module_encode_json", self.handle, C.byref(out), C.byref(n))
        return _take_buffer(out, n.value).decode()

    def to_mll(self) -> bytes:
        out, n = C.c_void_p(), C.c_size_t()
        call("manta_module_encode_mll", self.handle, C.byref(out), C.byref(n))
        return _take_buffer(out, n.value)

    # serving contracts
    def validate_score_entry(self, entry, query_input, query_rank, docs_input, docs_rank, query_dtype="",
                             docs_dtype="", output_name="", output_rank=1, output_dtype="") -> None:
        e = lambda s: (s or "").encode()
        call("manta_module_validate_score_entry", self.handle, e(entry), e(query_input), query_rank,
             e(docs_input), docs_rank, e(query_dtype), e(docs_dtype), e(output_name), output_rank, e(output_dtype))

    def validate_retrieval_entry(self, entry, query_input, query_rank, docs_input, docs_rank, ids_input, ids_rank,
                                 query_dtype="", docs_dtype="", ids_dtype="", output_name="", output_rank=2) -> None:
        e = lambda s: (s or "").encode()
        call("manta_module_validate_retrieval_entry", self.handle, e(entry), e(query_input), query_rank,
             e(docs_input), docs_rank, e(ids_input), ids_rank, e(query_dtype), e(docs_dtype), e(ids_dtype),
             e(output_name), output_rank)

    def validate_embedding_entry(self, entry, token_input, mask_input, token_rank, output_rank,
                                 output_dtype="") -> None:
        e = lambda s: (s or "").encode()
        call("manta_module_validate_embedding_entry", self.handle, e(entry), e(token_input), e(mask_input),
             token_rank, output_rank, e(output_dtype))

    def validate_embedding_param(self, name: str) -> None:
        call("manta_module_validate_embedding_param", self.handle, (name or "").encode())

    def validate_manifest(self, manifest: Union[bytes, str, os.PathLike]) -> None:
        """An authored *.score.mll / *.retrieval.mll / *.embedding.mll
        manifest's ValidateModule against this module."""
        from .mll import MllFile
        with MllFile(manifest, verify=True) as f:
            call("manta_manifest_validate_module", f._h, self.handle)


class Docs:
    """Bound candidates as a q8 / q4 artifact value ([n, d] or [sets, n, d])."""

    def __init__(self, cands: Candidates, dtype: str = "q4", rank: Optional[int] = None):
        self.cands = cands
        self.dtype = dtype
        self.rank = rank if rank is not None else (2 if cands.sets == 1 else 3)

    @property
    def shape(self):
        return (self.cands.n, self.cands.d) if self.rank == 2 else (self.cands.sets, self.cands.n, self.cands.d)


class Q8Columns:
    """A q8 matrix value: int8 codes [k, n] with an f32 scale per column (a
    reference per-tensor grid is one scale repeated); uploaded on first use."""

    def __init__(self, codes: np.ndarray, col_scales: np.ndarray, dtype: str = "q8"):
        self.codes = np.ascontiguousarray(codes, dtype=np.int8)
        self.scales = np.ascontiguousarray(col_scales, dtype=np.float32)
        if self.codes.ndim < 1 or self.scales.shape != (self.codes.shape[-1],):
            raise ValueError("q8 columns: codes [..., n] and n scales expected")
        self.dtype = dtype


class Program:
    """An artifact loaded on a runtime (MantaRocmProgram*)."""

    def __init__(self, rt: Runtime, module: Module):
        self.rt = rt
        self.module = module
        h = C.c_void_p()
        call("manta_rocm_program_load", rt.handle, module.handle, C.byref(h))
        self.handle = h
        self._keep = {}  # device arrays and names the program refers to

    def close(self) -> None:
        if self.handle is not None and self.handle.value:
            load().manta_rocm_program_destroy(self.handle)
        self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _value(self, name: str, v, keep: list, dtype: Optional[str] = None) -> _lib.Value:
        val = _lib.Value()
        bname = name.encode()
        keep.append(bname)
        val.name = bname
        if isinstance(v, Docs):
            val.kind = CANDIDATES
            val.dtype = DTYPE_CODES[v.dtype]
            val.rank = v.rank
            for i, s in enumerate(v.shape):
                val.shape[i] = s
            val.candidates = v.cands.handle.value
            keep.append(v)
            return val
        if isinstance(v, Q8Columns):
            codes, scales = self.rt.to_device(v.codes), self.rt.to_device(v.scales)
            keep.extend([codes, scales])
            val.kind = TENSOR
            val.storage = Q8
            val.dtype = DTYPE_CODES[v.dtype]
            val.rank = v.codes.ndim
            for i, s in enumerate(v.codes.shape):
                val.shape[i] = s
            val.data = codes.addr
            val.scales = scales.addr
            return val
        if isinstance(v, DeviceArray):
            dev, arr_dtype, shape = v, v.dtype, v.shape
        else:
            arr = np.asarray(v)
            if arr.dtype == np.float16:
                arr = arr.view(np.uint16)
            dev = self.rt.to_device(np.ascontiguousarray(arr))
            arr_dtype, shape = arr.dtype, arr.shape
        storage = {np.dtype(np.float32): F32, np.dtype(np.uint16): F16, np.dtype(np.int32): I32,
                   np.dtype(np.int64): I64}.get(np.dtype(arr_dtype))
        if storage is None:
            raise ValueError("value %r: unsupported array dtype %s" % (name, arr_dtype))
        keep.append(dev)
        val.kind = TENSOR
        val.storage = storage
        val.dtype = DTYPE_CODES[dtype] if dtype else storage
        val.rank = len(shape)
        if val.rank > 4:
            raise ValueError("value %r: rank %d > 4" % (name, val.rank))
        for i, s in enumerate(shape):
            val.shape[i] = s
        val.data = dev.addr
        return val

    def bind(self, name: str, value, dtype: Optional[str] = None) -> None:
        """Bind a param's weight: a numpy array (uploaded; uint16 / float16
        arrays are f16), a DeviceArray, or Docs."""
        keep = []
        val = self._value(name, value, keep, dtype)
        call("manta_rocm_program_bind", self.handle, C.byref(val))
        self._keep[("param", name)] = keep

    def supports(self, entry: str) -> None:
        call("manta_rocm_program_supports", self.handle, entry.encode())

    def run(self, entry: str, inputs: Dict[str, object], dtypes: Optional[Dict[str, str]] = None) -> dict:
        """Run an entry; returns {output name: value}: numpy arrays for
        tensors, dicts for gathered rows ({"codes", "scales", "format",
        "values"}) and candidate packs ({"ids", "scores", "docs"})."""
        keep = []
        dtypes = dtypes or {}
        arr = (_lib.Value * max(1, len(inputs)))()
        for i, (name, v) in enumerate(inputs.items()):
            arr[i] = self._value(name, v, keep, dtypes.get(name))
        outs = (_lib.Value * 16)()
        n = C.c_int64()
        call("manta_rocm_program_run", self.handle, entry.encode(), arr, len(inputs), outs, 16, C.byref(n))
        return {outs[i].name.decode(): self._fetch(outs[i]) for i in range(n.value)}

    def trace(self) -> list:
        lib = load()
        out = []
        for i in range(lib.manta_rocm_program_trace_count(self.handle)):
            k, nm, d = C.c_char_p(), C.c_char_p(), C.c_char_p()
            lib.manta_rocm_program_trace_step(self.handle, i, C.byref(k), C.byref(nm), C.byref(d))
            out.append((k.value.decode(), (nm.value or b"").decode(), d.value.decode()))
        return out

    # ------------------------------------------------------------ results
    def _download(self, ptr: int, nbytes: int, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if nbytes:
            call("manta_rocm_download", self.rt.handle, out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr),
                 C.c_size_t(nbytes))
        return out

    def _rows(self, v: _lib.Value, shape) -> dict:
        d = shape[-1]
        nrows = int(np.prod(shape[:-1], dtype=np.int64))
        if v.storage == Q8:
            codes = self._download(v.data, nrows * d, np.int8, tuple(shape[:-1]) + (d,))
            scales = self._download(v.scales, nrows * 4, np.float32, tuple(shape[:-1]))
            values = codes.astype(np.float32) * scales[..., None].astype(np.float32)
            fmt = "q8"
        else:
            codes = self._download(v.data, nrows * (d // 2), np.uint8, tuple(shape[:-1]) + (d // 2,))
            scales = self._download(v.scales, nrows * (d // 32) * 2, np.uint16, tuple(shape[:-1]) + (d // 32,))
            lo = (codes & 0xF).astype(np.int8)
            hi = (codes >> 4).astype(np.int8)
            nib = np.empty(tuple(shape[:-1]) + (d,), np.int8)
            nib[..., 0::2] = np.where(lo >= 8, lo - 16, lo)
            nib[..., 1::2] = np.where(hi >= 8, hi - 16, hi)
            sc = scales.view(np.float16).astype(np.float32)
            values = (nib.astype(np.float64) * np.repeat(sc.astype(np.float64), 32, axis=-1)).astype(np.float32)
            fmt = "q4"
        return {"format": fmt, "dtype": DTYPE_NAMES.get(v.dtype, ""), "codes": codes, "scales": scales,
                "values": values}

    def _fetch(self, v: _lib.Value):
        shape = tuple(v.shape[i] for i in range(v.rank))
        if v.kind == TENSOR:
            dt = _NP[v.storage]
            n = int(np.prod(shape, dtype=np.int64))
            return self._download(v.data, n * np.dtype(dt).itemsize, dt, shape)
        if v.kind == ROWS:
            return self._rows(v, shape)
        if v.kind == CANDIDATE_PACK:
            lead = shape[:-1]
            n = int(np.prod(lead, dtype=np.int64))
            ids_dt = _NP.get(v.ids_dtype, np.int64)
            return {"ids": self._download(v.ids, n * np.dtype(ids_dt).itemsize, ids_dt, lead),
                    "scores": self._download(v.scores, n * 4, np.float32, lead),
                    "docs": self._rows(v, shape)}
        raise ValueError("unexpected output kind %d" % v.kind)
