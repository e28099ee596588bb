"""GPU parity of the embed pipeline (gather -> @matmul -> masked mean_pool ->
normalize) against the CPU oracle's restatement of the reference host ops.

Bars: gather, mean_pool and normalize are bit-exact (same order of
operations as the reference); matmul runs on f16 MFMA with f32 accumulation
in a different summation order, so |gpu - ref| <= 3e-5 * sum_k |a_ik b_kj|
+ 1e-7; embeddings (f16 out) have cosine >= 0.9999 per row against the f32
oracle and stay within 2 f16 ulps.
"""
import numpy as np
import pytest

from manta_amd import synth
from manta_amd._lib import MantaRocmError
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _matmul_bound(a, b):
    return 3e-5 * (np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))) + 1e-7


def _cos_rows(x, y):
    x = x.astype(np.float64)
    y = y.astype(np.float64)
    return (x * y).sum(1) / (np.linalg.norm(x, axis=1) * np.linalg.norm(y, axis=1))


def test_gather_rows_bit_exact_and_errors(rt):
    table = synth.normal_f16(11, 0, 1000, 384, 0.02)
    idx = synth.uniform_i32(11, 1, 777, 0, 1000)
    out = rt.gather_rows_f16(rt.to_device(table), rt.to_device(idx)).download()
    np.testing.assert_array_equal(out, table[idx])
    bad = idx.copy()
    bad[5] = 1000
    res = rt.gather_rows_f16(rt.to_device(table), rt.to_device(bad))
    with pytest.raises(MantaRocmError, match="gather index 1000 out of range"):
        rt.synchronize()
    # the error is reported once, then cleared
    rt.synchronize()
    res.free()


@pytest.mark.parametrize("m,k,n", [(64, 384, 384), (100, 384, 200), (8192, 384, 384), (3, 64, 130),
                                   (100, 64, 384), (33, 768, 384)])
def test_matmul_f16(rt, m, k, n):
    a = synth.normal_f16(12, 0, m, k, 0.02)
    b = synth.normal_f16(12, 1, k, n, 1.0 / np.sqrt(k))
    got = rt.matmul_f16(rt.to_device(a), rt.to_device(b)).download()
    af, bf = orc.f16_to_f32(a), orc.f16_to_f32(b)
    want = orc.matmul(af, bf)
    assert np.all(np.abs(got - want) <= _matmul_bound(af, bf))


def test_matmul_q8_projection(rt):
    m, k, n = 256, 384, 384
    a = synth.normal_f16(13, 0, m, k, 0.02)
    codes = synth.uniform_i8(13, 1, k * n, -127, 127).reshape(k, n)
    cs = (np.arange(n, dtype=np.float32) + 1.0) / (127.0 * np.sqrt(k) * n)
    got = rt.matmul_f16(rt.to_device(a), rt.to_device(codes), rt.to_device(cs.astype(np.float32))).download()
    af = orc.f16_to_f32(a)
    w = codes.astype(np.float32) * cs[None, :].astype(np.float32)
    want = orc.matmul(af, w)
    assert np.all(np.abs(got - want) <= _matmul_bound(af, w))


def test_mean_pool_masked_bit_exact(rt):
    b, t, c = 9, 37, 96
    x = synth.normal_f32(14, 0, b * t, c).reshape(b, t, c)
    lengths = synth.uniform_i32(14, 1, b, 0, t + 1)
    lengths[0] = 0  # a fully masked sequence pools to zeros
    mask = (np.arange(t)[None, :] < lengths[:, None]).astype(np.int32)
    got = rt.mean_pool_masked(rt.to_device(x), rt.to_device(mask)).download()
    np.testing.assert_array_equal(got, orc.mean_pool_masked(x, mask))
    assert np.all(got[0] == 0)


@pytest.mark.parametrize("rows,cols", [(70, 384), (1000, 17), (33, 1), (5, 20000), (65, 511)])
def test_normalize_rows_bit_exact(rt, rows, cols):
    """Both launch shapes: rows staged in LDS (pitch cols + 1), and one
    thread per row when a row does not fit."""
    x = synth.normal_f32(15, 0, rows, cols)
    x[3] = 0.0  # zero row stays unchanged
    d = rt.to_device(x)
    rt.normalize_rows(d)
    got = d.download()
    np.testing.assert_array_equal(got, orc.normalize_rows(x))
    assert np.all(got[3] == 0)


def test_embed_config1_full_shape(rt):
    tokens, mask, table, proj = synth.config1()
    got = rt.embed_pooled(rt.to_device(tokens), rt.to_device(mask), rt.to_device(table),
                          rt.to_device(proj)).download()
    want16, want32 = orc.embed(tokens, mask, table, proj_f16=proj)
    g = orc.f16_to_f32(got)
    assert _cos_rows(g, want32).min() >= 0.9999
    # within 2 f16 ulps of the rounded oracle output
    ulp = np.spacing(np.abs(orc.f16_to_f32(want16)).astype(np.float16)).astype(np.float32)
    assert np.all(np.abs(g - orc.f16_to_f32(want16)) <= 2 * ulp + 1e-7)


def test_embed_config4_q8_projection_slice(rt):
    tokens, mask, table, pcodes, cs, _, _ = synth.config4(nq=96, n=0)
    got = rt.embed_pooled(rt.to_device(tokens), rt.to_device(mask), rt.to_device(table),
                          rt.to_device(pcodes), rt.to_device(cs)).download()
    _, want32 = orc.embed(tokens, mask, table, proj_codes=pcodes, col_scale=cs)
    assert _cos_rows(orc.f16_to_f32(got), want32).min() >= 0.9999


@pytest.mark.parametrize("d,e", [(64, 96), (384, 384), (128, 384)])
def test_embed_ragged_and_empty_sequences(rt, d, e):
    """Lengths 0 .. T with T = 100 (not a multiple of the 32- and 64-row
    tiles); e = 384 with an f16 projection takes the single-pass kernel."""
    b, t, v = 7, 100, 500
    tokens = synth.uniform_i32(16, 0, b * t, 0, v).reshape(b, t)
    lengths = np.array([0, 1, 63, 64, 65, 99, 100], np.int32)
    mask = (np.arange(t)[None, :] < lengths[:, None]).astype(np.int32)
    table = synth.normal_f16(16, 1, v, d, 0.02)
    proj = synth.normal_f16(16, 2, d, e, 1.0 / np.sqrt(d))
    got = orc.f16_to_f32(rt.embed_pooled(rt.to_device(tokens), rt.to_device(mask), rt.to_device(table),
                                         rt.to_device(proj)).download())
    _, want32 = orc.embed(tokens, mask, table, proj_f16=proj)
    assert np.all(got[0] == 0) and np.all(want32[0] == 0)
    assert _cos_rows(got[1:], want32[1:]).min() >= 0.9999


@pytest.mark.parametrize("b,t,d", [(3, 9, 64), (5, 200, 256), (16, 128, 384), (2, 300, 512), (9, 257, 192),
                                   (4, 70, 160), (3, 40, 96)])
def test_embed_one_round_shapes(rt, b, t, d):
    """The small-batch pooled embed (f16 projection, e = 384) at K its
    one-round kernel takes (64 to 512: one to eight 64-k blocks), K it
    leaves to the ring kernel (96, 160), sequences longer than
    one 128-row tile (published per-tile counts), ragged masks, and both
    workgroup orders (a tile count that is a multiple of 8 or not)."""
    e, v = 384, 700
    tokens = synth.uniform_i32(17, b, b * t, 0, v).reshape(b, t)
    lengths = synth.uniform_i32(17, 100 + b, b, 1, t + 1)
    lengths[0] = t
    mask = (np.arange(t)[None, :] < lengths[:, None]).astype(np.int32)
    table = synth.normal_f16(17, 1, v, d, 0.02)
    proj = synth.normal_f16(17, 2, d, e, 1.0 / np.sqrt(d))
    got = orc.f16_to_f32(rt.embed_pooled(rt.to_device(tokens), rt.to_device(mask), rt.to_device(table),
                                         rt.to_device(proj)).download())
    want16, want32 = orc.embed(tokens, mask, table, proj_f16=proj)
    assert _cos_rows(got, want32).min() >= 0.9999
    ulp = np.spacing(np.abs(orc.f16_to_f32(want16)).astype(np.float16)).astype(np.float32)
    assert np.all(np.abs(got - orc.f16_to_f32(want16)) <= 2 * ulp + 1e-7)
    # a second call on the same runtime (the tickets were reset) agrees bit for bit
    again = orc.f16_to_f32(rt.embed_pooled(rt.to_device(tokens), rt.to_device(mask), rt.to_device(table),
                                           rt.to_device(proj)).download())
    np.testing.assert_array_equal(again, got)


@pytest.mark.parametrize("d,e", [(64, 64), (384, 384)])
def test_embed_out_of_range_token(rt, d, e):
    tokens, mask, table, proj = synth.config1(b=4, t=32, vocab=100, d=d, e=e)
    tokens[2, 31] = 100
    mask[2, 31] = 0  # the reference gathers every position, masked or not
    rt.embed_pooled(rt.to_device(tokens), rt.to_device(mask), rt.to_device(table), rt.to_device(proj))
    with pytest.raises(MantaRocmError, match="gather index 100 out of range"):
        rt.synchronize()
    with pytest.raises(orc.OracleError, match="gather index 100 out of range"):
        orc.embed(tokens, mask, table, proj_f16=proj)


def test_step_by_step_pipeline_matches_fused(rt):
    """gather -> matmul -> mean_pool -> normalize as separate device steps
    (the reference's step list) agrees with the fused entry point."""
    tokens, mask, table, proj = synth.config1(b=8, t=128)
    b, t = tokens.shape
    g = rt.gather_rows_f16(rt.to_device(table), rt.to_device(tokens.reshape(-1)))
    y = rt.matmul_f16(g, rt.to_device(proj))
    y.shape = (b, t, proj.shape[1])
    pooled = rt.mean_pool_masked(y, rt.to_device(mask))
    rt.normalize_rows(pooled)
    steps = pooled.download()
    fused = orc.f16_to_f32(rt.embed_pooled(rt.to_device(tokens), rt.to_device(mask), rt.to_device(table),
                                           rt.to_device(proj)).download())
    _, want32 = orc.embed(tokens, mask, table, proj_f16=proj)
    assert _cos_rows(steps, want32).min() >= 0.9999
    assert _cos_rows(fused, steps).min() >= 0.9999


@pytest.mark.parametrize("nq,t,q8", [(512, 64, True), (256, 128, False), (128, 256, True)])
def test_embed_large_batch_whole_sequence_tiles(rt, nq, t, q8):
    """Batches large enough for 256-row workgroups of whole sequences
    (T = 64, 128, 256), ragged and empty sequences, q8 and f16 projections."""
    d = e = 384
    tokens = synth.uniform_i32(17, 0, nq * t, 0, 32000).reshape(nq, t)
    lengths = synth.uniform_i32(17, 1, nq, 0, t + 1)
    lengths[::37] = 0
    lengths[1::41] = t
    mask = (np.arange(t)[None, :] < lengths[:, None]).astype(np.int32)
    table = synth.normal_f16(17, 2, 32000, d, 0.02)
    if q8:
        pcodes = synth.uniform_i8(17, 3, d * e, -127, 127).reshape(d, e)
        cs = (np.arange(e, dtype=np.float32) + 1.0) / (127.0 * np.sqrt(d) * e)
        got = rt.embed_pooled(rt.to_device(tokens), rt.to_device(mask), rt.to_device(table),
                              rt.to_device(pcodes), rt.to_device(cs.astype(np.float32))).download()
        _, want32 = orc.embed(tokens, mask, table, proj_codes=pcodes, col_scale=cs.astype(np.float32))
    else:
        proj = synth.normal_f16(17, 3, d, e, 1.0 / np.sqrt(d))
        got = rt.embed_pooled(rt.to_device(tokens), rt.to_device(mask), rt.to_device(table),
                              rt.to_device(proj)).download()
        _, want32 = orc.embed(tokens, mask, table, proj_f16=proj)
    g = orc.f16_to_f32(got)
    empty = lengths == 0
    assert np.all(g[empty] == 0) and np.all(want32[empty] == 0)
    assert _cos_rows(g[~empty], want32[~empty]).min() >= 0.9999


# ---------------------------------------------------------------------------
# Projections prepared once (manta_rocm_prepare_projection): the same GEMMs
# read the prepared f16 [e, d] operand, so the outputs equal the per-call
# transpose path bit for bit.

@pytest.mark.parametrize("nq,t,q8", [(512, 64, True), (256, 128, False), (6, 100, True), (5, 70, False)])
def test_embed_prepared_projection_bit_identical(rt, nq, t, q8):
    """Whole-sequence tiles (the first two) and the partial-sum path (the
    last two, e = 256 so the single-pass f16 kernel does not apply)."""
    d, e = (384, 384) if nq >= 256 else (128, 256)
    tokens = synth.uniform_i32(19, 0, nq * t, 0, 32000).reshape(nq, t)
    lengths = synth.uniform_i32(19, 1, nq, 0, t + 1)
    mask = (np.arange(t)[None, :] < lengths[:, None]).astype(np.int32)
    table = rt.to_device(synth.normal_f16(19, 2, 32000, d, 0.02))
    td, md = rt.to_device(tokens), rt.to_device(mask)
    if q8:
        proj = rt.to_device(synth.uniform_i8(19, 3, d * e, -127, 127).reshape(d, e))
        cs = rt.to_device(((np.arange(e) + 1.0) / (127.0 * np.sqrt(d) * e)).astype(np.float32))
    else:
        proj = rt.to_device(synth.normal_f16(19, 3, d, e, 1.0 / np.sqrt(d)))
        cs = None
    pp = rt.prepare_projection(proj)
    assert pp.data.shape == (e, d)
    want = rt.embed_pooled(td, md, table, proj, cs).download()
    got = rt.embed_pooled(td, md, table, pp, cs).download()
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("q8", [False, True])
def test_matmul_prepared_projection(rt, q8):
    m, k, n = 300, 256, 256
    a = synth.normal_f16(21, 0, m, k, 0.02)
    ad = rt.to_device(a)
    if q8:
        codes = synth.uniform_i8(21, 1, k * n, -127, 127).reshape(k, n)
        csh = ((np.arange(n) + 1.0) / (127.0 * np.sqrt(k) * n)).astype(np.float32)
        rhs, cs = rt.to_device(codes), rt.to_device(csh)
        w = codes.astype(np.float32) * csh[None, :]
    else:
        wf = synth.normal_f16(21, 1, k, n, 1.0 / np.sqrt(k))
        rhs, cs = rt.to_device(wf), None
        w = orc.f16_to_f32(wf)
    want = rt.matmul_f16(ad, rhs, cs).download()
    got = rt.matmul_f16(ad, rt.prepare_projection(rhs), cs).download()
    np.testing.assert_array_equal(got, want)
    af = orc.f16_to_f32(a)
    assert np.all(np.abs(got - orc.matmul(af, w)) <= _matmul_bound(af, w))


def test_prepared_projection_errors(rt):
    """A prepared operand serves only the pipelined GEMM's shapes; a prepared
    kind cannot be prepared again."""
    a = rt.to_device(synth.normal_f16(23, 0, 10, 64, 0.02))
    proj = rt.to_device(synth.normal_f16(23, 1, 64, 96, 0.1))
    pp = rt.prepare_projection(proj)
    with pytest.raises(MantaRocmError, match="prepared projection needs k % 32 == 0 and n % 128 == 0"):
        rt.matmul_f16(a, pp)
    from manta_amd import _lib
    import ctypes as C
    k = C.c_int()
    with pytest.raises(MantaRocmError, match="is not a \\[d, e\\] projection"):
        _lib.call("manta_rocm_prepare_projection", rt.handle, pp.data.ptr, C.c_int(_lib.PROJ_F16_T), C.c_int64(64),
                  C.c_int64(96), pp.data.ptr, C.byref(k))
