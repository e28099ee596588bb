"""GPU parity of the encoder forward (manta_rocm_encoder_pooled) against the
CPU oracle's restatement of examples/encoder_trainable_q8.manta
(embed_pooled_batch).  Bar: per-row cosine >= 0.9999 with the oracle's f32
embedding and max abs error below 2e-3 (the device output is f16; the
device's reductions run in tree order)."""
import numpy as np
import pytest

from manta_amd._lib import MantaRocmError
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _pack_cols(w):
    """q8 with an f32 scale per column: code = round(w / s), s = maxabs / 127."""
    s = (np.abs(w).max(0) / 127.0).astype(np.float32)
    s[s == 0] = 1.0
    codes = np.clip(np.round(w / s), -127, 127).astype(np.int8)
    return codes, s


def _case(seed, b, t, vocab, d, h, empty_row=True):
    rng = np.random.default_rng(seed)
    tokens = rng.integers(0, vocab, size=(b, t), dtype=np.int32)
    lengths = rng.integers(1, t + 1, size=b)
    if empty_row:
        lengths[0] = 0  # a fully masked sequence pools to zeros
    mask = (np.arange(t)[None, :] < lengths[:, None]).astype(np.int32)
    table = (rng.standard_normal((vocab, d)) * 0.5).astype(np.float32)
    tcodes, tscales = orc.pack_q8_rows(table)
    ws = [(rng.standard_normal(s) / np.sqrt(s[0])).astype(np.float32)
          for s in [(d, d), (d, d), (d, d), (d, d), (d, h), (h, d)]]
    packed = [_pack_cols(w) for w in ws]
    return tokens, mask, tcodes, tscales, packed


def _run(rt, tokens, mask, tcodes, tscales, packed):
    dev = [(rt.to_device(c), rt.to_device(s)) for c, s in packed]
    out = rt.encoder_pooled(rt.to_device(tokens), rt.to_device(mask), rt.to_device(tcodes), rt.to_device(tscales),
                            dev)
    return out.download().view(np.float16).astype(np.float32)


def _want(tokens, mask, tcodes, tscales, packed):
    table = (tcodes.astype(np.float32) * tscales[:, None]).astype(np.float32)
    ws = [(c.astype(np.float32) * s[None, :]).astype(np.float32) for c, s in packed]
    return orc.encoder_pooled(tokens, mask, table, *ws)


@pytest.mark.parametrize("b,t,vocab,d,h", [(6, 16, 50, 64, 128), (5, 24, 70, 96, 160), (3, 1, 9, 32, 64),
                                           # d and h multiples of 128: the weight GEMMs on f16 MFMA (the
                                           # second with 120 rows, not a multiple of the 64-row tiles)
                                           (8, 64, 300, 384, 1536), (3, 40, 100, 128, 384),
                                           # d, h and t not multiples of 16: the scalar staging path of the
                                           # q8-weight and transposed-K GEMMs, with their bounds-checked K tails
                                           (4, 24, 40, 40, 72)])
def test_encoder_matches_oracle(rt, b, t, vocab, d, h):
    case = _case(b * 100 + t, b, t, vocab, d, h)
    got = _run(rt, *case)
    want = _want(*case)
    assert np.all(got[0] == 0.0) and np.all(want[0] == 0.0)  # the fully masked row
    live = np.linalg.norm(want, axis=1) > 0
    cos = (got[live] * want[live]).sum(1) / (np.linalg.norm(got[live], axis=1) * np.linalg.norm(want[live], axis=1))
    assert cos.min() >= 0.9999, cos.min()
    assert np.abs(got - want).max() < 2e-3


def test_encoder_token_out_of_range_is_reported(rt):
    tokens, mask, tcodes, tscales, packed = _case(7, 2, 8, 10, 32, 64, empty_row=False)
    tokens[1, 3] = 10
    dev = [(rt.to_device(c), rt.to_device(s)) for c, s in packed]
    rt.encoder_pooled(rt.to_device(tokens), rt.to_device(mask), rt.to_device(tcodes), rt.to_device(tscales), dev)
    with pytest.raises(MantaRocmError, match="gather index 10 out of range"):
        rt.synchronize()


def _run_layers(rt, layers, tokens, mask, tcodes, tscales, packed):
    dev = [(rt.to_device(c), rt.to_device(s)) for c, s in packed]
    out = rt.encoder_pooled(rt.to_device(tokens), rt.to_device(mask), rt.to_device(tcodes), rt.to_device(tscales),
                            dev, layers=layers)
    return out


def _want_layers(layers, tokens, mask, tcodes, tscales, packed):
    table = (tcodes.astype(np.float32) * tscales[:, None]).astype(np.float32)
    ws = [(c.astype(np.float32) * s[None, :]).astype(np.float32) for c, s in packed]
    return orc.encoder_pooled(tokens, mask, table, *ws, layers=layers)


@pytest.mark.parametrize("b,t,vocab,d,h", [(6, 16, 50, 64, 128), (8, 64, 300, 384, 1536), (4, 24, 40, 40, 72)])
def test_two_layer_encoder_matches_oracle(rt, b, t, vocab, d, h):
    """encoder_trainable_q8x2 (the block twice, shared weights) at the same
    bar as one layer."""
    case = _case(b * 77 + t, b, t, vocab, d, h)
    got = _run_layers(rt, 2, *case).download().view(np.float16).astype(np.float32)
    want = _want_layers(2, *case)
    assert np.all(got[0] == 0.0) and np.all(want[0] == 0.0)
    live = np.linalg.norm(want, axis=1) > 0
    cos = (got[live] * want[live]).sum(1) / (np.linalg.norm(got[live], axis=1) * np.linalg.norm(want[live], axis=1))
    assert cos.min() >= 0.9999, cos.min()
    assert np.abs(got - want).max() < 2e-3
    one = _run_layers(rt, 1, *case).download().view(np.float16).astype(np.float32)
    assert np.abs(one - got).max() > 1e-2  # the second block ran


def test_encoder_output_feeds_score_topk(rt):
    """The encoder's device output is the query matrix of the fused score +
    top-k with no host round trip; the result equals the reference scoring
    of those embeddings (cosineRows on the dequantized candidates)."""
    from manta_amd import synth
    b, t, vocab, d, h = 16, 32, 200, 128, 256
    case = _case(91, b, t, vocab, d, h, empty_row=False)
    emb = _run_layers(rt, 2, *case)  # f16 [b, d] on device
    codes, scales = synth.q8_rows(91, 5, 20000, d, normalize=True)
    cands = rt.bind_q8(codes, scales)
    ids, scores, _ = rt.score_topk(cands, "cosine", emb, 25)
    q = emb.download()
    ref = orc.cosine_rows(orc.f16_to_f32(q), orc.dequant_q8(codes, scales))
    want = orc.topk(ref, 25)
    np.testing.assert_array_equal(ids.download(), want)
    np.testing.assert_array_equal(scores.download(), np.take_along_axis(ref, want, 1))
