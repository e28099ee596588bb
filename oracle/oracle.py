"""numpy face of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the manta_amd package.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

DOT, COSINE, L2, DOT16 = 0, 1, 2, 3
OPS = {"dot": DOT, "cosine": COSINE, "l2_distance": L2, "dot16": DOT16}

_L = None


def build() -> str:
    subprocess.run(["make", "-B", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _L
    if _L is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        p, i64, ci = C.c_void_p, C.c_int64, C.c_int
        sig = {
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
            "orc_f16_to_f32_array": (None, [p, i64, p]),
            "orc_f32_to_f16_array": (None, [p, i64, p]),
            "orc_dot_rows": (None, [p, p, i64, i64, i64, ci, p]),
            "orc_cosine_rows": (None, [p, p, i64, i64, i64, ci, p]),
            "orc_l2_distance_rows": (None, [p, p, i64, i64, i64, ci, p]),
            "orc_topk": (ci, [p, i64, i64, i64, ci, p, C.c_char_p, ci]),
            "orc_gather_rows": (ci, [p, i64, i64, p, i64, p, C.c_char_p, ci]),
            "orc_matmul": (None, [p, p, i64, i64, i64, p]),
            "orc_mean_pool_masked": (None, [p, p, i64, i64, i64, p]),
            "orc_normalize_rows": (None, [p, i64, i64]),
            "orc_embed": (ci, [p, p, i64, i64, p, i64, i64, p, p, p, i64, p, p, C.c_char_p, ci]),
            "orc_pack_q8_rows": (None, [p, i64, i64, p, p]),
            "orc_pack_q4_blocks": (None, [p, i64, i64, p, p]),
            "orc_q8_row_consts": (None, [p, p, i64, i64, p, p]),
            "orc_q4_row_consts": (None, [p, p, i64, i64, p, p]),
            "orc_query_e8": (None, [p, i64, p, p]),
            "orc_query_e16": (None, [p, i64, p, p, p, p]),
            "orc_score_q8": (None, [ci, p, i64, p, p, p, p, i64, i64, i64, p, p]),
            "orc_score_q4": (None, [ci, p, i64, p, p, p, p, i64, i64, i64, p]),
            "orc_dequant_q8": (None, [p, p, i64, i64, p]),
            "orc_dequant_q4": (None, [p, p, i64, i64, p]),
            "orc_ref_score_q8": (None, [ci, p, i64, p, p, i64, i64, i64, p]),
            "orc_ref_score_q4": (None, [ci, p, i64, p, p, i64, i64, i64, p]),
            "orc_fake_quantize": (None, [p, i64, ci]),
            "orc_fair_q8_topk": (None, [ci, p, i64, p, p, p, p, i64, i64, i64, ci, ci, p, p]),
            "orc_fair_q4_topk": (None, [ci, p, i64, p, p, p, p, i64, i64, i64, ci, ci, p, p]),
            "orc_fair_embed": (None, [p, p, i64, i64, p, i64, i64, p, p, p, i64, ci, p]),
            "orc_layernorm_rows": (None, [p, i64, i64]),
            "orc_softmax_rows": (None, [p, i64, i64]),
            "orc_gelu": (None, [p, i64]),
            "orc_encoder_pooled": (ci, [p, p, i64, i64, p, i64, i64, p, p, p, p, p, p, i64, p, C.c_char_p, ci]),
            "orc_top_retrieval_scores": (i64, [p, i64, p, i64, i64, p, i64, p, p]),
            "orc_encoder_pooled_layers": (
                ci, [p, p, i64, i64, p, i64, i64, p, p, p, p, p, p, i64, i64, p, C.c_char_p, ci]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _L = L
    return _L


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


class OracleError(ValueError):
    pass


# ------------------------------------------------------------------ f16
def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_array(_p(h), h.size, _p(out))
    return out


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_array(_p(x), x.size, _p(out))
    return out


# ------------------------------------------------ reference restatements
def _score_f32(fn, q, docs):
    q = _c(q, np.float32)
    docs = _c(docs, np.float32)
    if q.ndim == 1 and docs.ndim == 2:
        nq, rows, cols, per = 1, docs.shape[0], docs.shape[1], 0
        shape = (rows,)
    elif q.ndim == 2 and docs.ndim == 3:
        nq, rows, cols, per = q.shape[0], docs.shape[1], docs.shape[2], 1
        shape = (nq, rows)
    elif q.ndim == 2 and docs.ndim == 2:
        nq, rows, cols, per = q.shape[0], docs.shape[0], docs.shape[1], 0
        shape = (nq, rows)
    else:
        raise OracleError("score expects query/docs as [D] x [N,D] or [Q,D] x [Q,N,D]")
    if q.shape[-1] != cols:
        raise OracleError("score mismatch %s x %s" % (q.shape, docs.shape))
    out = np.empty(shape, np.float32)
    fn(_p(q), _p(docs), nq, rows, cols, per, _p(out))
    return out


def dot_rows(q, docs):
    return _score_f32(lib().orc_dot_rows, q, docs)


def cosine_rows(q, docs):
    return _score_f32(lib().orc_cosine_rows, q, docs)


def l2_distance_rows(q, docs):
    return _score_f32(lib().orc_l2_distance_rows, q, docs)


def topk(scores, k, smallest=False):
    s = _c(scores, np.float32)
    rank1 = s.ndim == 1
    s2 = s.reshape(1, -1) if rank1 else s
    out = np.empty((s2.shape[0], max(int(k), 0)), np.int32)
    msg = C.create_string_buffer(256)
    rc = lib().orc_topk(_p(s2), s2.shape[0], s2.shape[1], int(k), 0 if smallest else 1,
                        _p(out) if k > 0 else None, msg, 256)
    if rc:
        raise OracleError(msg.value.decode())
    return out[0] if rank1 else out


def gather_rows(table, idx):
    table = _c(table, np.float32)
    idx = _c(idx, np.int32)
    out = np.empty((idx.size, table.shape[1]), np.float32)
    msg = C.create_string_buffer(256)
    rc = lib().orc_gather_rows(_p(table), table.shape[0], table.shape[1], _p(idx), idx.size,
                               _p(out), msg, 256)
    if rc:
        raise OracleError(msg.value.decode())
    return out.reshape(idx.shape + (table.shape[1],))


def matmul(lhs, rhs):
    lhs = _c(lhs, np.float32)
    rhs = _c(rhs, np.float32)
    lead = lhs.shape[:-1]
    m = int(np.prod(lead))
    k, n = rhs.shape
    out = np.empty((m, n), np.float32)
    lib().orc_matmul(_p(lhs), _p(rhs), m, k, n, _p(out))
    return out.reshape(lead + (n,))


def mean_pool_masked(x, mask):
    x = _c(x, np.float32)
    mask = _c(mask, np.int32)
    b, t, c = x.shape
    out = np.empty((b, c), np.float32)
    lib().orc_mean_pool_masked(_p(x), _p(mask), b, t, c, _p(out))
    return out


def normalize_rows(x):
    x = np.array(x, dtype=np.float32, copy=True, order="C")
    lib().orc_normalize_rows(_p(x), int(np.prod(x.shape[:-1])), x.shape[-1])
    return x


def embed(tokens, mask, table_f16, proj_f16=None, proj_codes=None, col_scale=None):
    tokens = _c(tokens, np.int32)
    mask = _c(mask, np.int32)
    table = _c(table_f16, np.uint16)
    b, t = tokens.shape
    vocab, d = table.shape
    if proj_codes is not None:
        proj_codes = _c(proj_codes, np.int8)
        col_scale = _c(col_scale, np.float32)
        e = proj_codes.shape[1]
    else:
        proj_f16 = _c(proj_f16, np.uint16)
        e = proj_f16.shape[1]
    out16 = np.empty((b, e), np.uint16)
    out32 = np.empty((b, e), np.float32)
    msg = C.create_string_buffer(256)
    rc = lib().orc_embed(_p(tokens), _p(mask), b, t, _p(table), vocab, d, _p(proj_f16),
                         _p(proj_codes), _p(col_scale), e, _p(out16), _p(out32), msg, 256)
    if rc:
        raise OracleError(msg.value.decode())
    return out16, out32


# ------------------------------------------------------------ encoder
def layernorm_rows(x):
    x = np.array(x, dtype=np.float32, order="C", copy=True)
    lib().orc_layernorm_rows(_p(x), int(np.prod(x.shape[:-1])), x.shape[-1])
    return x


def softmax_rows(x):
    x = np.array(x, dtype=np.float32, order="C", copy=True)
    lib().orc_softmax_rows(_p(x), int(np.prod(x.shape[:-1])), x.shape[-1])
    return x


def gelu(x):
    x = np.array(x, dtype=np.float32, order="C", copy=True)
    lib().orc_gelu(_p(x), x.size)
    return x


def encoder_pooled(tokens, mask, table, wq, wk, wv, wo, wup, wproj, layers=1):
    """f32 [b, d] of the encoder pipeline over dequantized f32 weights (the
    block applied `layers` times with shared weights)."""
    tokens = _c(tokens, np.int32)
    mask = _c(mask, np.int32)
    table = _c(table, np.float32)
    ws = [_c(w, np.float32) for w in (wq, wk, wv, wo, wup, wproj)]
    b, t = tokens.shape
    vocab, d = table.shape
    h = ws[4].shape[1]
    out = np.empty((b, d), np.float32)
    msg = C.create_string_buffer(256)
    rc = lib().orc_encoder_pooled_layers(_p(tokens), _p(mask), b, t, _p(table), vocab, d, *[_p(w) for w in ws], h,
                                         int(layers), _p(out), msg, 256)
    if rc:
        raise OracleError(msg.value.decode())
    return out


# ------------------------------------------------ packed scoring contract
def pack_q8_rows(x):
    x = _c(x, np.float32)
    n, d = x.shape
    codes = np.empty((n, d), np.int8)
    scales = np.empty((n,), np.float32)
    lib().orc_pack_q8_rows(_p(x), n, d, _p(codes), _p(scales))
    return codes, scales


def pack_q4_blocks(x):
    x = _c(x, np.float32)
    n, d = x.shape
    packed = np.empty((n, d // 2), np.uint8)
    scales = np.empty((n, d // 32), np.uint16)
    lib().orc_pack_q4_blocks(_p(x), n, d, _p(packed), _p(scales))
    return packed, scales


def q8_row_consts(codes, scales):
    codes = _c(codes, np.int8)
    scales = _c(scales, np.float32)
    d = codes.shape[-1]
    n = codes.size // d
    dn = np.empty((n,), np.float32)
    dd = np.empty((n,), np.float32)
    lib().orc_q8_row_consts(_p(codes), _p(scales), n, d, _p(dn), _p(dd))
    return dn, dd


def q4_row_consts(packed, scales, d):
    packed = _c(packed, np.uint8)
    scales = _c(scales, np.uint16)
    n = packed.size // (d // 2)
    dn = np.empty((n,), np.float32)
    dd = np.empty((n,), np.float32)
    lib().orc_q4_row_consts(_p(packed), _p(scales), n, d, _p(dn), _p(dd))
    return dn, dd


def query_e8(q):
    q = _c(q, np.uint16)
    codes = np.empty(q.shape, np.int8)
    qmax = C.c_float()
    lib().orc_query_e8(_p(q), q.size, _p(codes), C.byref(qmax))
    return codes, np.float32(qmax.value)


def query_e16(q):
    q = _c(q, np.uint16)
    codes = np.empty(q.shape, np.int16)
    qs, qn, qq = C.c_float(), C.c_float(), C.c_float()
    lib().orc_query_e16(_p(q), q.size, _p(codes), C.byref(qs), C.byref(qn), C.byref(qq))
    return codes, np.float32(qs.value), np.float32(qn.value), np.float32(qq.value)


def score_q8(op, queries, codes, scales, with_acc=False):
    """queries f16 bits [nq,d]; codes [n,d] (shared) or [nq,n,d]."""
    queries = _c(queries, np.uint16)
    codes = _c(codes, np.int8)
    scales = _c(scales, np.float32)
    nq, d = queries.shape
    if codes.ndim == 2:
        sets, (n, _) = 1, codes.shape
    else:
        sets, n, _ = codes.shape
    dn, dd = q8_row_consts(codes, scales)
    out = np.empty((nq, n), np.float32)
    acc = np.empty((nq, n), np.int64) if with_acc else None
    lib().orc_score_q8(OPS[op], _p(queries), nq, _p(codes), _p(scales), _p(dn), _p(dd), sets, n,
                       d, _p(out), _p(acc))
    return (out, acc) if with_acc else out


def score_q4(op, queries, packed, scales, d):
    queries = _c(queries, np.uint16)
    packed = _c(packed, np.uint8)
    scales = _c(scales, np.uint16)
    nq = queries.shape[0]
    if packed.ndim == 2:
        sets, n = 1, packed.shape[0]
    else:
        sets, n = packed.shape[0], packed.shape[1]
    dn, dd = q4_row_consts(packed, scales, d)
    out = np.empty((nq, n), np.float32)
    lib().orc_score_q4(OPS[op], _p(queries), nq, _p(packed), _p(scales), _p(dn), _p(dd), sets, n,
                       d, _p(out))
    return out


# ------------------------------------- reference scores of packed candidates
def dequant_q8(codes, scales):
    """The f32 values a reference q8 tensor holds: code*scale (f32)."""
    codes = _c(codes, np.int8)
    scales = _c(scales, np.float32)
    d = codes.shape[-1]
    n = codes.size // d
    out = np.empty(codes.shape, np.float32)
    lib().orc_dequant_q8(_p(codes), _p(scales), n, d, _p(out))
    return out


def dequant_q4(packed, scales, d):
    """The f32 values of a q4 tensor: nibble code times its block's f16 scale."""
    packed = _c(packed, np.uint8)
    scales = _c(scales, np.uint16)
    n = packed.size // (d // 2)
    out = np.empty(packed.shape[:-1] + (d,), np.float32)
    lib().orc_dequant_q4(_p(packed), _p(scales), n, d, _p(out))
    return out


def ref_score_q8(op, queries, codes, scales):
    """dotRows / cosineRows / l2DistanceRows of f16 queries [nq, d] against
    the dequantized rows of q8 candidates [n, d] (shared) or [nq, n, d]."""
    queries = _c(queries, np.uint16)
    codes = _c(codes, np.int8)
    scales = _c(scales, np.float32)
    nq, d = queries.shape
    sets, n = (1, codes.shape[0]) if codes.ndim == 2 else codes.shape[:2]
    out = np.empty((nq, n), np.float32)
    lib().orc_ref_score_q8(OPS[op], _p(queries), nq, _p(codes), _p(scales), sets, n, d, _p(out))
    return out


def ref_score_q4(op, queries, packed, scales, d):
    queries = _c(queries, np.uint16)
    packed = _c(packed, np.uint8)
    scales = _c(scales, np.uint16)
    nq = queries.shape[0]
    sets, n = (1, packed.shape[0]) if packed.ndim == 2 else packed.shape[:2]
    out = np.empty((nq, n), np.float32)
    lib().orc_ref_score_q4(OPS[op], _p(queries), nq, _p(packed), _p(scales), sets, n, d, _p(out))
    return out


def fake_quantize(x, bits):
    """fakeQuantizeDataInPlace on a copy of x (one grid for the whole array)."""
    x = np.array(x, dtype=np.float32, order="C", copy=True)
    lib().orc_fake_quantize(_p(x), x.size, int(bits))
    return x


# --------------------------------------------- bench.py's fair CPU baseline
def fair_q8_topk(op, queries, codes, scales, k, smallest=False, threads=None):
    """Quantized-query q8 top-k on all cores (fair_cpu.c)."""
    queries = _c(queries, np.uint16)
    codes = _c(codes, np.int8)
    scales = _c(scales, np.float32)
    nq, d = queries.shape
    n = codes.shape[0]
    dn, dd = q8_row_consts(codes, scales) if op != "dot" else (None, None)
    ids = np.empty((nq, k), np.int32)
    vals = np.empty((nq, k), np.float32)
    lib().orc_fair_q8_topk(OPS[op], _p(queries), nq, _p(codes), _p(scales), _p(dn), _p(dd), n, d, k,
                           1 if smallest else 0, int(threads or os.cpu_count() or 1), _p(ids), _p(vals))
    return ids, vals


def fair_q4_topk(op, queries, packed, scales, d, k, smallest=False, threads=None):
    queries = _c(queries, np.uint16)
    packed = _c(packed, np.uint8)
    scales = _c(scales, np.uint16)
    nq = queries.shape[0]
    n = packed.shape[0]
    dn, dd = q4_row_consts(packed, scales, d)
    ids = np.empty((nq, k), np.int32)
    vals = np.empty((nq, k), np.float32)
    lib().orc_fair_q4_topk(OPS[op], _p(queries), nq, _p(packed), _p(scales), _p(dn), _p(dd), n, d, k,
                           1 if smallest else 0, int(threads or os.cpu_count() or 1), _p(ids), _p(vals))
    return ids, vals


def fair_embed(tokens, mask, table_f16, proj_f16=None, proj_codes=None, col_scale=None, threads=None):
    tokens = _c(tokens, np.int32)
    mask = _c(mask, np.int32)
    table = _c(table_f16, np.uint16)
    b, t = tokens.shape
    vocab, d = table.shape
    if proj_codes is not None:
        proj_codes = _c(proj_codes, np.int8)
        col_scale = _c(col_scale, np.float32)
        e = proj_codes.shape[1]
    else:
        proj_f16 = _c(proj_f16, np.uint16)
        e = proj_f16.shape[1]
    out = np.empty((b, e), np.float32)
    lib().orc_fair_embed(_p(tokens), _p(mask), b, t, _p(table), vocab, d, _p(proj_f16), _p(proj_codes),
                         _p(col_scale), e, int(threads or os.cpu_count() or 1), _p(out))
    return out


def top_retrieval_scores(query, docs, ids, top_k):
    """topRetrievalScores (retrieval_eval.go:586-623) for one query:
    (positions of the chosen docs, their f32 scores) in rank order."""
    q = _c(query, np.float32)
    d = _c(docs, np.float32)
    n = d.shape[0]
    arr = (C.c_char_p * max(n, 1))(*[x.encode() if isinstance(x, str) else x for x in ids])
    pos = np.empty(max(n, 1), np.int64)
    sc = np.empty(max(n, 1), np.float32)
    cnt = lib().orc_top_retrieval_scores(_p(q), q.shape[-1], _p(d), n, d.shape[1], C.cast(arr, C.c_void_p),
                                         int(top_k), _p(pos), _p(sc))
    return pos[:cnt], sc[:cnt]
