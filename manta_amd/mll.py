"""Python view of the native MLL reader (include/manta_mll.h).

`MllFile` exposes a container's section table (with BLAKE3-256 digest
verification), string table and HEAD metadata; `read_authored_manifest`
follows the Go runtime's readAuthoredManifestMLL
(runtime/authored_manifest_mll.go:197-270): magic check, digest-verified
read, HEAD and STRG required, metadata keyed by string (empty keys skipped),
manifest_kind / manifest_version checked against the expected values.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Union

import numpy as np

from . import _lib
from ._lib import MantaRocmError, call, load

BOOL, I64, F64, STRING = 1, 2, 3, 4


def blake3(data: bytes) -> bytes:
    """BLAKE3-256 digest (the section digest of the container)."""
    out = C.create_string_buffer(32)
    buf = C.create_string_buffer(bytes(data), len(data)) if data else None
    load().manta_mll_blake3(C.cast(buf, C.c_void_p) if buf else None, len(data), C.cast(out, C.c_void_p))
    return out.raw


class MllFile:
    """An opened container.  data: bytes, or a path to read."""

    def __init__(self, data: Union[bytes, str, os.PathLike], verify: bool = True):
        if not isinstance(data, (bytes, bytearray)):
            with open(data, "rb") as f:
                data = f.read()
        self._buf = C.create_string_buffer(bytes(data), len(data))
        self._h = C.c_void_p()
        call("manta_mll_open", C.cast(self._buf, C.c_void_p), len(data), 1 if verify else 0, C.byref(self._h))

    def close(self) -> None:
        if self._h:
            load().manta_mll_close(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def format_word(self) -> int:
        return load().manta_mll_format_word(self._h)

    @property
    def sections(self) -> list:
        """[(tag, offset, size, flags, digest bytes)] in table order."""
        out = []
        for i in range(load().manta_mll_section_count(self._h)):
            tag = C.create_string_buffer(5)
            off, size, flags = C.c_uint64(), C.c_uint64(), C.c_uint32()
            dig = C.create_string_buffer(32)
            call("manta_mll_section_info", self._h, i, tag, C.byref(off), C.byref(size), C.byref(flags),
                 C.cast(dig, C.c_void_p))
            out.append((tag.value.decode(), off.value, size.value, flags.value, dig.raw))
        return out

    def section(self, tag: str) -> bytes:
        ptr, size = C.c_void_p(), C.c_uint64()
        call("manta_mll_section", self._h, tag.encode(), C.byref(ptr), C.byref(size))
        return C.string_at(ptr, size.value) if size.value else b""

    @property
    def strings(self) -> list:
        n = load().manta_mll_string_count(self._h)
        return [load().manta_mll_string(self._h, i).decode() for i in range(n)]

    def string(self, sid: int) -> str:
        return load().manta_mll_string(self._h, sid).decode()

    def head(self):
        """(name, description, [(key, kind, value)]) of the HEAD section."""
        name, desc, n = C.c_uint32(), C.c_uint32(), C.c_int()
        call("manta_mll_head", self._h, C.byref(name), C.byref(desc), C.byref(n))
        entries = []
        for i in range(n.value):
            key, kind = C.c_uint32(), C.c_int()
            i64, f64, sid = C.c_int64(), C.c_double(), C.c_uint32()
            call("manta_mll_head_entry", self._h, i, C.byref(key), C.byref(kind), C.byref(i64), C.byref(f64),
                 C.byref(sid))
            k = kind.value
            value = (bool(i64.value) if k == BOOL else i64.value if k == I64 else f64.value if k == F64
                     else self.string(sid.value))
            entries.append((self.string(key.value), k, value))
        return self.string(name.value), self.string(desc.value), entries

    def packed(self) -> dict:
        """Contents of a packed candidate container (manta_mll_packed_info):
        {"dtype": "q8"|"q4", "rows", "dim", "codes", "scales", "ids"} with
        numpy copies of the sections (ids None without a QIDS section)."""
        t, rows, dim = C.c_int(), C.c_uint64(), C.c_uint32()
        pc, ps, pi = C.c_void_p(), C.c_void_p(), C.c_void_p()
        call("manta_mll_packed_info", self._h, C.byref(t), C.byref(rows), C.byref(dim), C.byref(pc),
             C.byref(ps), C.byref(pi))
        n, d = rows.value, dim.value
        if t.value == _lib.Q8_ROWS:
            codes = np.frombuffer(C.string_at(pc, n * d), np.int8).reshape(n, d)
            scales = np.frombuffer(C.string_at(ps, n * 4), np.float32).copy()
        else:
            codes = np.frombuffer(C.string_at(pc, n * d // 2), np.uint8).reshape(n, d // 2)
            scales = np.frombuffer(C.string_at(ps, n * (d // 32) * 2), np.uint16).reshape(n, d // 32)
        ids = np.frombuffer(C.string_at(pi, n * 8), np.int64) if pi.value else None
        return {"dtype": "q8" if t.value == _lib.Q8_ROWS else "q4", "rows": n, "dim": d, "codes": codes,
                "scales": scales, "ids": ids}


def write_packed(path: Union[str, os.PathLike], codes: np.ndarray, scales: np.ndarray,
                 ids: Optional[np.ndarray] = None, name: str = "") -> None:
    """Write a packed candidate container.  q8: codes int8 [n,d], scales f32 [n];
    q4: codes uint8 [n,d/2] (packed nibbles), scales f16 bits uint16 [n,d/32]."""
    if codes.dtype == np.int8:
        t, (n, d) = _lib.Q8_ROWS, codes.shape
        scales = np.ascontiguousarray(scales, np.float32)
        if scales.shape != (n,):
            raise ValueError("q8 scales shape %s, want (%d,)" % (scales.shape, n))
    elif codes.dtype == np.uint8:
        t, (n, half) = _lib.Q4_BLOCKS, codes.shape
        d = 2 * half
        scales = np.ascontiguousarray(scales, np.uint16)
        if scales.shape != (n, d // 32):
            raise ValueError("q4 scales shape %s, want (%d, %d)" % (scales.shape, n, d // 32))
    else:
        raise ValueError("codes must be int8 (q8) or uint8 packed nibbles (q4), got %s" % codes.dtype)
    codes = np.ascontiguousarray(codes)
    if ids is not None:
        ids = np.ascontiguousarray(ids, np.int64)
        if ids.shape != (n,):
            raise ValueError("ids shape %s, want (%d,)" % (ids.shape, n))
    call("manta_mll_write_packed", os.fsencode(path), name.encode(), t, n, d, codes.ctypes.data_as(C.c_void_p),
         scales.ctypes.data_as(C.c_void_p), ids.ctypes.data_as(C.c_void_p) if ids is not None else None)


def read_authored_manifest(data: Union[bytes, str, os.PathLike], expected_kind: str = "",
                           expected_version: str = "") -> dict:
    """{"name", "description", "values": {key: (kind, value)}} of an authored
    manifest, with readAuthoredManifestMLL's checks and error wording."""
    with MllFile(data, verify=True) as m:
        name, desc, entries = m.head()
        values = {}
        for key, kind, value in entries:
            if key == "":
                continue
            values[key] = (kind, value)
    for key, want in (("manifest_kind", expected_kind), ("manifest_version", expected_version)):
        if not want:
            continue
        if key not in values:
            raise MantaRocmError(_lib.ERROR, 'manifest missing "%s"' % key)
        kind, got = values[key]
        if kind != STRING:
            raise MantaRocmError(_lib.ERROR, 'manifest key "%s" kind = %d, want string' % (key, kind))
        if got != want:
            what = "kind" if key == "manifest_kind" else "version"
            raise MantaRocmError(_lib.ERROR, 'manifest %s "%s", want "%s"' % (what, got, want))
    return {"name": name, "description": desc, "values": values}
