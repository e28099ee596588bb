"""Python face of the rocm backend (ctypes over libmanta_rocm.so).

Mirrors the operator surface the reference's Go backend offers for the
retrieval hot path (runtime/backend/tensor_ops.go: dotRows, cosineRows,
l2DistanceRows, topKTensor, gatherTensor, matmulTensor,
meanPoolMaskedTensor, normalizeRows) over packed q8/q4 candidates held in
device memory.  All compute runs in the HIP library; this module only moves
buffers and checks shapes.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional

import numpy as np

from . import _lib
from ._lib import call, load

DTYPES = {np.dtype(np.float32), np.dtype(np.uint16), np.dtype(np.int8), np.dtype(np.uint8),
          np.dtype(np.int32), np.dtype(np.int64)}


def device_count() -> int:
    n = C.c_int(0)
    call("manta_rocm_device_count", C.byref(n))
    return n.value


class PreparedProjection:
    """A projection in the MFMA kernels' layout: data is f16 [e, d]; kind is
    PROJ_F16_T or PROJ_Q8_COL_T (the latter still takes its column scales)."""

    def __init__(self, data: "DeviceArray", kind: int, d: int, e: int):
        self.data, self.kind, self.d, self.e = data, kind, d, e


class DeviceArray:
    """A device allocation with a numpy dtype and shape."""

    def __init__(self, rt: "Runtime", shape, dtype):
        self.rt = rt
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        ptr = C.c_void_p()
        call("manta_rocm_malloc", rt.handle, C.byref(ptr), C.c_size_t(max(self.nbytes, 1)))
        self.ptr = ptr

    @property
    def addr(self) -> int:
        return int(self.ptr.value or 0)

    def upload(self, host: np.ndarray) -> "DeviceArray":
        host = np.ascontiguousarray(host, dtype=self.dtype)
        if host.nbytes != self.nbytes:
            raise ValueError("upload size mismatch: %d vs %d" % (host.nbytes, self.nbytes))
        call("manta_rocm_upload", self.rt.handle, self.ptr, host.ctypes.data_as(C.c_void_p),
             C.c_size_t(self.nbytes))
        return self

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        call("manta_rocm_download", self.rt.handle, out.ctypes.data_as(C.c_void_p), self.ptr,
             C.c_size_t(self.nbytes))
        return out

    def free(self) -> None:
        if self.ptr is not None and self.ptr.value:
            call("manta_rocm_free", self.rt.handle, self.ptr)
        self.ptr = C.c_void_p()

    def __del__(self):  # best effort; explicit free() is preferred
        try:
            if self.ptr is not None and self.ptr.value and self.rt.handle:
                self.free()
        except Exception:
            pass


class Candidates:
    """Device-resident packed candidate matrix ([sets, n, d])."""

    def __init__(self, rt: "Runtime", handle: C.c_void_p, fmt: int, sets: int, n: int, d: int):
        self.rt, self.handle, self.format = rt, handle, fmt
        self.sets, self.n, self.d = sets, n, d

    def close(self) -> None:
        if self.handle is not None and self.handle.value:
            load().manta_rocm_unbind(self.handle)
        self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _ptr(a: Optional[DeviceArray]):
    return a.ptr if a is not None else None


class Runtime:
    """One HIP device + stream (MantaRocm*)."""

    def __init__(self, device: int = 0):
        load()
        h = C.c_void_p()
        call("manta_rocm_create", C.c_int(device), C.byref(h))
        self.handle = h

    def close(self) -> None:
        if self.handle is not None and self.handle.value:
            load().manta_rocm_destroy(self.handle)
        self.handle = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ------------------------------------------------------------ memory
    def empty(self, shape, dtype) -> DeviceArray:
        return DeviceArray(self, shape, dtype)

    def to_device(self, host: np.ndarray, dtype=None) -> DeviceArray:
        host = np.ascontiguousarray(host, dtype=dtype or host.dtype)
        return DeviceArray(self, host.shape, host.dtype).upload(host)

    def synchronize(self) -> None:
        call("manta_rocm_synchronize", self.handle)

    def set_stream(self, stream_ptr: int) -> None:
        call("manta_rocm_set_stream", self.handle, C.c_void_p(stream_ptr))

    def set_timing(self, on: bool) -> None:
        call("manta_rocm_set_timing", self.handle, C.c_int(1 if on else 0))

    def timing(self, name=None, reset=False):
        """(launch count, summed device ms) of one kernel family."""
        cnt = C.c_uint64()
        ms = C.c_double()
        call("manta_rocm_timing", self.handle, name.encode() if name else None, C.byref(cnt),
             C.byref(ms), C.c_int(1 if reset else 0))
        return cnt.value, ms.value

    def span(self, end: bool) -> float:
        """Start (end=False) or stop (end=True) a span timer on the runtime's
        stream; stopping waits and returns the span's device milliseconds."""
        ms = C.c_double()
        call("manta_rocm_span", self.handle, C.c_int(1 if end else 0), C.byref(ms))
        return ms.value

    def stats(self) -> dict:
        s = _lib.Stats()
        load().manta_rocm_stats(self.handle, C.byref(s))
        return {f: getattr(s, f) for f, _ in _lib.Stats._fields_}

    # ------------------------------------------------------------ binding
    def bind_q8(self, codes: np.ndarray, scales: np.ndarray) -> Candidates:
        """codes int8 [n,d] or [sets,n,d]; scales f32 [n] or [sets,n]."""
        codes = np.ascontiguousarray(codes, dtype=np.int8)
        scales = np.ascontiguousarray(scales, dtype=np.float32)
        if codes.ndim == 2:
            codes = codes[None]
            scales = scales.reshape(1, -1)
        sets, n, d = codes.shape
        if scales.shape != (sets, n):
            raise ValueError("q8 scales shape %s does not match codes %s" % (scales.shape, codes.shape))
        h = C.c_void_p()
        call("manta_rocm_bind_q8_rows", self.handle, codes.ctypes.data_as(C.c_void_p),
             scales.ctypes.data_as(C.c_void_p), C.c_int64(sets), C.c_int64(n), C.c_int64(d),
             C.byref(h))
        return Candidates(self, h, _lib.Q8_ROWS, sets, n, d)

    def bind_q4(self, packed: np.ndarray, scales: np.ndarray, d: int) -> Candidates:
        """packed uint8 [n,d/2] or [sets,n,d/2]; scales f16 bits [n,d/32] or [sets,...]."""
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype=np.uint16)
        if packed.ndim == 2:
            packed = packed[None]
            scales = scales[None]
        sets, n, half = packed.shape
        if half * 2 != d or scales.shape != (sets, n, d // 32):
            raise ValueError("q4 shapes do not match d=%d" % d)
        h = C.c_void_p()
        call("manta_rocm_bind_q4_blocks", self.handle, packed.ctypes.data_as(C.c_void_p),
             scales.ctypes.data_as(C.c_void_p), C.c_int64(sets), C.c_int64(n), C.c_int64(d),
             C.byref(h))
        return Candidates(self, h, _lib.Q4_BLOCKS, sets, n, d)

    def bind_packed(self, container) -> Candidates:
        """Bind the candidates of a packed container (an opened mll.MllFile)
        straight from its QCOD / QSCL bytes."""
        h = C.c_void_p()
        call("manta_rocm_bind_packed", self.handle, container._h, C.byref(h))
        fmt, sets, n, d = C.c_int(), C.c_int64(), C.c_int64(), C.c_int64()
        load().manta_rocm_candidates_info(h, C.byref(fmt), C.byref(sets), C.byref(n), C.byref(d))
        return Candidates(self, h, fmt.value, sets.value, n.value, d.value)

    # ------------------------------------------------------------ scoring
    @staticmethod
    def _query_rows(cands: Candidates, queries: DeviceArray) -> int:
        """Rows of a query array: f16 values (float16, or uint16 f16 bits),
        [d] or [nq, d].  The C ABI reads the buffer as f16 bits, so any other
        dtype would be misread."""
        if np.dtype(queries.dtype) not in (np.dtype(np.float16), np.dtype(np.uint16)):
            raise TypeError("queries must be float16 or uint16 f16 bits (got %s)" % np.dtype(queries.dtype))
        if queries.shape[-1] != cands.d or len(queries.shape) not in (1, 2):
            raise ValueError("queries must be [d] or [nq, d] with d=%d (got %s)" % (cands.d, tuple(queries.shape)))
        return queries.shape[0] if len(queries.shape) == 2 else 1

    @staticmethod
    def _op(op: str, quantized: bool) -> int:
        if op not in _lib.OPS:
            raise ValueError("unknown score op %r (dot, cosine, l2_distance)" % (op,))
        return _lib.OPS[op] | (_lib.QUANTIZED_QUERY if quantized else 0)

    def score(self, cands: Candidates, op: str, queries: DeviceArray,
              out: Optional[DeviceArray] = None, quantized: bool = False) -> DeviceArray:
        """Score matrix [nq, n].  Default: the reference's dotRows /
        cosineRows / l2DistanceRows on the dequantized candidates, bit for
        bit; quantized=True: the quantized-query scores."""
        nq = self._query_rows(cands, queries)
        if out is None:
            out = self.empty((nq, cands.n), np.float32)
        call("manta_rocm_score", self.handle, cands.handle, C.c_int(self._op(op, quantized)), queries.ptr,
             C.c_int64(nq), out.ptr)
        return out

    def score_topk(self, cands: Candidates, op: str, queries: DeviceArray, k: int,
                   smallest: bool = False, with_scores: bool = True, with_acc: bool = False,
                   out=None, quantized: bool = False):
        """(ids [nq, k] int32, scores [nq, k] f32 or None, accumulators
        [nq, k] int64 or None); topKTensor's order.  Reference scores by
        default, quantized-query scores with quantized=True (which the
        integer accumulators need)."""
        nq = self._query_rows(cands, queries)
        if out is None:
            ids = self.empty((nq, k), np.int32)
            sc = self.empty((nq, k), np.float32) if with_scores else None
            acc = self.empty((nq, k), np.int64) if with_acc else None
        else:
            ids, sc, acc = out
        call("manta_rocm_score_topk", self.handle, cands.handle, C.c_int(self._op(op, quantized)),
             C.c_int(_lib.SMALLEST if smallest else _lib.LARGEST), queries.ptr, C.c_int64(nq),
             C.c_int64(k), ids.ptr, _ptr(sc), _ptr(acc))
        return ids, sc, acc

    def score_topk_noalloc(self, cands: Candidates, op: str, queries: DeviceArray, k: int, out,
                           smallest: bool = False, quantized: bool = False):
        """score_topk through the allocation-free entry point into the given
        (ids, scores or None, accumulators or None) device arrays."""
        nq = self._query_rows(cands, queries)
        ids, sc, acc = out
        # the kernels write nq x k entries through these pointers: a buffer
        # of another shape or element size would be written out of bounds
        for name, arr, dt, need in (("ids", ids, np.int32, True), ("scores", sc, np.float32, False),
                                    ("acc", acc, np.int64, False)):
            if arr is None:
                if need:
                    raise ValueError("score_topk_noalloc: ids output is required")
                continue
            if tuple(arr.shape) != (nq, k) or np.dtype(arr.dtype) != np.dtype(dt):
                raise ValueError("score_topk_noalloc: %s must be (%d, %d) %s, got %s %s"
                                 % (name, nq, k, np.dtype(dt).name, tuple(arr.shape), np.dtype(arr.dtype).name))
        call("manta_rocm_score_topk_noalloc", self.handle, cands.handle, C.c_int(self._op(op, quantized)),
             C.c_int(_lib.SMALLEST if smallest else _lib.LARGEST), queries.ptr, C.c_int64(nq), C.c_int64(k),
             ids.ptr, _ptr(sc), _ptr(acc))
        return ids, sc, acc

    def pack_candidates(self, cands: Candidates, top: DeviceArray,
                        candidate_ids: Optional[DeviceArray] = None):
        """Candidate ids (int64, when given), packed rows and row scales of
        the top-k rows: (ids or None, rows [nq, k, row_bytes] int8 (q8) or
        uint8 nibble pairs (q4), scales [nq, k, s] f32 (q8) or f16 bits (q4))."""
        nq, k = top.shape
        q8 = cands.format == _lib.Q8_ROWS
        row_bytes = cands.d if q8 else cands.d // 2
        rows = self.empty((nq, k, row_bytes), np.int8 if q8 else np.uint8)
        scales = self.empty((nq, k, 1), np.float32) if q8 else self.empty((nq, k, cands.d // 32), np.uint16)
        ids = self.empty((nq, k), np.int64) if candidate_ids is not None else None
        call("manta_rocm_pack_candidates", self.handle, cands.handle, top.ptr, C.c_int64(nq), C.c_int64(k),
             _ptr(candidate_ids), _ptr(ids), rows.ptr, scales.ptr)
        return ids, rows, scales

    def topk(self, scores: DeviceArray, k: int, smallest: bool = False):
        rows, cols = (1, scores.shape[0]) if len(scores.shape) == 1 else scores.shape
        ids = self.empty((rows, k), np.int32)
        vals = self.empty((rows, k), np.float32)
        call("manta_rocm_topk", self.handle, scores.ptr, C.c_int64(rows), C.c_int64(cols),
             C.c_int64(k), C.c_int(_lib.SMALLEST if smallest else _lib.LARGEST), ids.ptr, vals.ptr)
        return ids, vals

    # ------------------------------------------------------------ embed
    def gather_rows_f16(self, table: DeviceArray, idx: DeviceArray) -> DeviceArray:
        vocab, d = table.shape
        nidx = int(np.prod(idx.shape))
        out = self.empty((nidx, d), np.uint16)
        call("manta_rocm_gather_rows_f16", self.handle, table.ptr, C.c_int64(vocab), C.c_int64(d),
             idx.ptr, C.c_int64(nidx), out.ptr)
        return out

    def prepare_projection(self, proj: DeviceArray) -> "PreparedProjection":
        """A [d, e] f16 or int8 projection in the MFMA kernels' layout (f16
        [e, d]), for embed_pooled / matmul_f16 without a per-call transpose."""
        d, e = proj.shape
        kind = _lib.PROJ_Q8_COL if proj.dtype == np.int8 else _lib.PROJ_F16
        out = self.empty((e, d), np.uint16)
        k = C.c_int()
        call("manta_rocm_prepare_projection", self.handle, proj.ptr, C.c_int(kind), C.c_int64(d), C.c_int64(e),
             out.ptr, C.byref(k))
        return PreparedProjection(out, k.value, d, e)

    @staticmethod
    def _proj(rhs) -> tuple:
        """(pointer, kind, k, n) of a [k, n] projection or a prepared one."""
        if isinstance(rhs, PreparedProjection):
            return rhs.data.ptr, rhs.kind, rhs.d, rhs.e
        k, n = rhs.shape
        return rhs.ptr, (_lib.PROJ_Q8_COL if rhs.dtype == np.int8 else _lib.PROJ_F16), k, n

    def matmul_f16(self, lhs: DeviceArray, rhs, col_scale: Optional[DeviceArray] = None
                   ) -> DeviceArray:
        m, k = lhs.shape
        ptr, kind, k2, n = self._proj(rhs)
        if k2 != k:
            raise ValueError("matmul mismatch %s x [%d,%d]" % (lhs.shape, k2, n))
        out = self.empty((m, n), np.float32)
        call("manta_rocm_matmul_f16", self.handle, lhs.ptr, C.c_int64(m), C.c_int64(k), ptr,
             C.c_int(kind), _ptr(col_scale), C.c_int64(n), out.ptr)
        return out

    def mean_pool_masked(self, x: DeviceArray, mask: DeviceArray) -> DeviceArray:
        b, t, c = x.shape
        out = self.empty((b, c), np.float32)
        call("manta_rocm_mean_pool_masked", self.handle, x.ptr, mask.ptr, C.c_int64(b),
             C.c_int64(t), C.c_int64(c), out.ptr)
        return out

    # ------------------------------------------------------ dense vectors
    @staticmethod
    def _dense_kind(rows: DeviceArray) -> int:
        if rows.dtype == np.float32:
            return _lib.DENSE_F32
        if rows.dtype == np.uint16:
            return _lib.DENSE_F16
        raise ValueError("dense rows must be f32 or f16 bits (uint16), not %s" % rows.dtype)

    def dense_scores(self, rows: DeviceArray, queries: DeviceArray) -> DeviceArray:
        """dotRetrievalVectors of f32 queries [nq, qd] against rows [n, d]."""
        if queries.dtype != np.float32:
            raise ValueError("queries must be f32")
        n, d = rows.shape
        nq, qd = queries.shape if len(queries.shape) == 2 else (1, queries.shape[0])
        out = self.empty((nq, n), np.float32)
        call("manta_rocm_dense_scores", self.handle, rows.ptr, self._dense_kind(rows), C.c_int64(n), C.c_int64(d),
             queries.ptr, C.c_int64(nq), C.c_int64(qd), out.ptr)
        return out

    def dense_topk(self, rows: DeviceArray, queries: DeviceArray, k: int):
        """The k best rows per query, (score desc, row asc): (ids, scores)."""
        if queries.dtype != np.float32:
            raise ValueError("queries must be f32")
        n, d = rows.shape
        nq, qd = queries.shape if len(queries.shape) == 2 else (1, queries.shape[0])
        ids = self.empty((nq, max(k, 1)), np.int32)
        scores = self.empty((nq, max(k, 1)), np.float32)
        call("manta_rocm_dense_topk", self.handle, rows.ptr, self._dense_kind(rows), C.c_int64(n), C.c_int64(d),
             queries.ptr, C.c_int64(nq), C.c_int64(qd), C.c_int64(k), ids.ptr, scores.ptr)
        return ids, scores

    def mean_pool(self, x: DeviceArray) -> DeviceArray:
        """meanPoolTensor: f32 [b, t, c] -> [b, c] (sum / float32(t))."""
        b, t, c = x.shape
        out = self.empty((b, c), np.float32)
        call("manta_rocm_mean_pool", self.handle, x.ptr, C.c_int64(b), C.c_int64(t), C.c_int64(c), out.ptr)
        return out

    def normalize_rows(self, x: DeviceArray) -> DeviceArray:
        rows, cols = x.shape[0] if len(x.shape) == 2 else x.shape[0] * x.shape[1], x.shape[-1]
        call("manta_rocm_normalize_rows", self.handle, x.ptr, C.c_int64(rows), C.c_int64(cols))
        return x

    def embed_pooled(self, tokens: DeviceArray, mask: DeviceArray, table: DeviceArray,
                     proj, col_scale: Optional[DeviceArray] = None,
                     out: Optional[DeviceArray] = None) -> DeviceArray:
        """proj: [d, e] f16 or int8 device array, or prepare_projection's result."""
        b, t = tokens.shape
        vocab, d = table.shape
        ptr, kind, d2, e = self._proj(proj)
        if d2 != d:
            raise ValueError("matmul mismatch [%d,%d,%d] x [%d,%d]" % (b, t, d, d2, e))
        if out is None:
            out = self.empty((b, e), np.uint16)
        call("manta_rocm_embed_pooled", self.handle, tokens.ptr, mask.ptr, C.c_int64(b),
             C.c_int64(t), table.ptr, C.c_int64(vocab), C.c_int64(d), ptr, C.c_int(kind),
             _ptr(col_scale), C.c_int64(e), out.ptr)
        return out


    # ------------------------------------------------------------ encoder
    def encoder_pooled(self, tokens: DeviceArray, mask: DeviceArray, token_codes: DeviceArray,
                       token_scales: DeviceArray, weights, out: Optional[DeviceArray] = None,
                       layers: int = 1) -> DeviceArray:
        """The encoder's embed_pooled_batch: f16 [b, d].  weights: six (int8
        [k, n] codes, f32 [n] column scales) device pairs in the order
        attn_q, attn_k, attn_v, attn_o, ffn_up, projection; `layers` blocks
        with those weights (encoder_trainable_q8x2: 2)."""
        if len(tokens.shape) != 2 or np.dtype(tokens.dtype) != np.dtype(np.int32):
            raise ValueError("encoder tokens must be int32 [b, t] (got %s %s)" % (tokens.dtype, tokens.shape))
        if tuple(mask.shape) != tuple(tokens.shape) or np.dtype(mask.dtype) != np.dtype(np.int32):
            raise ValueError("encoder mask must be int32 %s (got %s %s)" % (tokens.shape, mask.dtype, mask.shape))
        b, t = tokens.shape
        if len(token_codes.shape) != 2 or np.dtype(token_codes.dtype) != np.dtype(np.int8):
            raise ValueError("encoder token codes must be int8 [vocab, d]")
        vocab, d = token_codes.shape
        if tuple(token_scales.shape) != (vocab,) or np.dtype(token_scales.dtype) != np.dtype(np.float32):
            raise ValueError("encoder token scales must be f32 [%d] (got %s %s)" % (vocab, token_scales.dtype,
                                                                                   token_scales.shape))
        if len(weights) != 6:
            raise ValueError("encoder weights: six (codes, scales) pairs")
        h = weights[4][0].shape[1]
        shapes = [(d, d), (d, d), (d, d), (d, d), (d, h), (h, d)]
        for (codes, scales), want in zip(weights, shapes):
            if tuple(codes.shape) != want or tuple(scales.shape) != (want[1],):
                raise ValueError("encoder weight shape %s / %s, want %s" % (codes.shape, scales.shape, want))
            if np.dtype(codes.dtype) != np.dtype(np.int8) or np.dtype(scales.dtype) != np.dtype(np.float32):
                raise ValueError("encoder weights must be int8 codes with f32 column scales")
        w = _lib.EncoderWeights()
        w.token_codes, w.token_scales = token_codes.addr, token_scales.addr
        for i, (codes, scales) in enumerate(weights):
            w.codes[i], w.col_scales[i] = codes.addr, scales.addr
        if out is None:
            out = self.empty((b, d), np.uint16)
        call("manta_rocm_encoder_pooled_layers", self.handle, tokens.ptr, mask.ptr, C.c_int64(b), C.c_int64(t),
             C.byref(w), C.c_int64(vocab), C.c_int64(d), C.c_int64(h), C.c_int64(layers), out.ptr)
        return out


def pack_q8_rows(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, d = x.shape
    codes = np.empty((n, d), np.int8)
    scales = np.empty((n,), np.float32)
    call("manta_rocm_pack_q8_rows", x.ctypes.data_as(C.c_void_p), C.c_int64(n), C.c_int64(d),
         codes.ctypes.data_as(C.c_void_p), scales.ctypes.data_as(C.c_void_p))
    return codes, scales


def pack_q4_blocks(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, d = x.shape
    packed = np.empty((n, d // 2), np.uint8)
    scales = np.empty((n, d // 32), np.uint16)
    call("manta_rocm_pack_q4_blocks", x.ctypes.data_as(C.c_void_p), C.c_int64(n), C.c_int64(d),
         packed.ctypes.data_as(C.c_void_p), scales.ctypes.data_as(C.c_void_p))
    return packed, scales


GRID_NONE, GRID_ROWS, GRID_TENSOR = 0, 1, 2


def pack_grid(x: np.ndarray, bits: int):
    """Exact q8-row repack of the f32 values of a reference q8 / q4 tensor:
    (codes int8 [n, d], scales f32 [n], grid) with grid 2 for one
    per-tensor grid (fakeQuantizeDataInPlace), 1 for a grid per row, 0 when
    the rows had to be re-quantized (lossy)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, d = x.shape
    codes = np.empty((n, d), np.int8)
    scales = np.empty((n,), np.float32)
    grid = C.c_int(-1)
    call("manta_rocm_pack_grid", x.ctypes.data_as(C.c_void_p), C.c_int64(n), C.c_int64(d), C.c_int(bits),
         codes.ctypes.data_as(C.c_void_p), scales.ctypes.data_as(C.c_void_p), C.byref(grid))
    return codes, scales, grid.value
