"""The codec front half's own kernels through the C ABI against the oracle: the RVQ lookup-sum
(bit-exact: the same f32 additions in codebook order, one rounding), the depthwise conv +
LayerNorm (one f16 ulp plus 1e-5 per element: the channel sums run in another order, which
moves outputs near zero by a few of their tiny ulps), and the conv epilogue's
GELU and per-channel scale at ConvNeXt's pointwise shapes (the conv bar: max-abs 2e-2 and one
ulp plus f32 summation-order error per element)."""
import numpy as np
import pytest
import torch

import oracle
from dtts import DttsError, nlc, ops, synth

from _util import to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,n_books,size,dim,first", [(48 * 75, 16, 2048, 256, 1), (7, 5, 33, 8, 2)])
def test_rvq_lookup_sum_bit_exact(dev, rows, n_books, size, dim, first):
    books = synth.normal(30, "books", (n_books, size, dim))
    codes = synth.randint(30, "codes", (rows, n_books), 0, size - 1).astype(np.int32)
    got = to_host(ops.rvq_lookup_sum(to_dev(codes, dev), to_dev(books, dev), first))
    assert np.array_equal(got, oracle.rvq_lookup_sum_f16(codes, books, first))


@pytest.mark.parametrize("lanes,length,c,k", [(2, 300, 1024, 7), (3, 41, 64, 7), (1, 17, 2048, 3), (2, 5, 8, 7)])
def test_depthwise_layernorm_matches_oracle(dev, lanes, length, c, k):
    x = synth.f16_bits(synth.normal(31, "x", (lanes, length, c)))
    taps = synth.normal(31, "taps", (c, k), 0, 0.3)
    bias = synth.normal(31, "bias", (c,), 0, 0.1)
    w = synth.uniform(31, "w", (c,), 0.5, 1.5)
    b = synth.normal(31, "b", (c,), 0, 0.1)
    got = to_host(ops.depthwise_layernorm(to_dev(x, dev), to_dev(taps, dev), to_dev(bias, dev), to_dev(w, dev),
                                          to_dev(b, dev), 1e-6))
    want = synth.from_f16_bits(oracle.depthwise_layernorm_f16(x, taps, bias, w, b, 1e-6)).astype(np.float64)
    g = synth.from_f16_bits(got).astype(np.float64)
    bad = np.abs(g - want) > np.abs(want) * 2.0 ** -10 + 1e-5
    assert not bad.any(), f"{int(bad.sum())} elements off, worst {np.max(np.abs(g - want)):.3e}"


def _close_elementwise(got, want):
    g = synth.from_f16_bits(got).astype(np.float64)
    w = synth.from_f16_bits(want).astype(np.float64)
    assert np.max(np.abs(g - w)) <= 2e-2
    bad = np.abs(g - w) > np.abs(w) * 2.0 ** -10 + 1e-4
    assert not bad.any(), f"{int(bad.sum())} elements off"


@pytest.mark.parametrize("lanes,length,cin,cout", [(2, 200, 1024, 4096), (1, 70, 256, 512)])
def test_pointwise_gelu(dev, lanes, length, cin, cout):
    x = synth.f16_bits(synth.normal(32, "x", (lanes, length, cin)))
    w = synth.f16_bits(synth.normal(32, "w", (cout, cin), 0, 1 / np.sqrt(cin)))
    b = synth.f16_bits(synth.normal(32, "b", (cout,), 0, 0.1))
    got = to_host(nlc.conv1d(to_dev(x, dev), to_dev(w, dev), to_dev(b, dev), k=1, act="gelu"))
    want = oracle.conv1d_nlc_f16(x, np.ascontiguousarray(w.T), b, 1, act="gelu")
    _close_elementwise(got, want)


@pytest.mark.parametrize("lanes,length,cin,cout", [(2, 200, 4096, 1024), (1, 33, 96, 64)])
def test_pointwise_scale_residual(dev, lanes, length, cin, cout):
    x = synth.f16_bits(synth.normal(33, "x", (lanes, length, cin)))
    w = synth.f16_bits(synth.normal(33, "w", (cout, cin), 0, 1 / np.sqrt(cin)))
    b = synth.f16_bits(synth.normal(33, "b", (cout,), 0, 0.1))
    r = synth.f16_bits(synth.normal(33, "r", (lanes, length, cout)))
    s = synth.uniform(33, "s", (cout,), 0.05, 0.15)
    got = to_host(nlc.conv1d(to_dev(x, dev), to_dev(w, dev), to_dev(b, dev), k=1, residual=to_dev(r, dev),
                             scale=to_dev(s, dev)))
    want = oracle.conv1d_nlc_f16(x, np.ascontiguousarray(w.T), b, 1, res_bits=r, scale=s)
    _close_elementwise(got, want)


def test_front_ops_reject_bad_arguments(dev):
    x = torch.zeros((1, 4, 12), dtype=torch.float16, device=dev)
    f = torch.zeros(12, dtype=torch.float32, device=dev)
    with pytest.raises(DttsError, match="multiple of 8"):
        ops.depthwise_layernorm(x, torch.zeros((12, 7), device=dev), f, f, f, 1e-6)
    codes = torch.zeros((3, 4), dtype=torch.int32, device=dev)
    with pytest.raises(DttsError, match="codes per row"):
        ops.rvq_lookup_sum(codes, torch.zeros((5, 8, 4), device=dev), 1)


def _rows_close(got, want, ulp_frac=2.0 ** -10, abs_tol=1e-4):
    g = synth.from_f16_bits(got).astype(np.float64)
    w = synth.from_f16_bits(want).astype(np.float64)
    bad = np.abs(g - w) > np.abs(w) * ulp_frac + abs_tol
    assert not bad.any(), f"{int(bad.sum())} elements off, worst {np.max(np.abs(g - w)):.3e}"


def test_rms_rows_and_swiglu_rows(dev):
    x = synth.f16_bits(synth.normal(34, "x", (97, 512)))
    g = synth.uniform(34, "g", (512,), 0.9, 1.1)
    got = to_host(ops_rms_rows(to_dev(x, dev), to_dev(g, dev), 1e-5))
    _rows_close(got, oracle.rms_norm_rows_f16(x, g, 1e-5), abs_tol=1e-5)
    gu = synth.f16_bits(synth.normal(34, "gu", (53, 2 * 1024)))
    y = torch.empty((53, 1024), dtype=torch.float16, device=dev)
    from dtts._lib import call, ptr, stream_handle
    gud = to_dev(gu, dev)  # held: a temporary's memory could be reused before the kernel runs
    call("dtts_swiglu_rows_f16", ptr(gud), ptr(y), 53, 1024, stream_handle())
    _rows_close(to_host(y), oracle.swiglu_rows_f16(gu), abs_tol=1e-6)


def ops_rms_rows(x, g, eps):
    from dtts._lib import call, ptr, stream_handle
    y = torch.empty_like(x)
    call("dtts_rms_norm_rows_f16", ptr(x), ptr(g), ptr(y), x.shape[0], x.shape[1], float(eps), stream_handle())
    return y


@pytest.mark.parametrize("lanes,length,heads,n_kv,window", [
    (2, 325, 16, 16, 72), (3, 70, 4, 2, 5), (1, 200, 8, 8, 192), (2, 1, 16, 16, 72), (1, 130, 4, 1, 1),
    (2, 150, 8, 4, 18), (1, 260, 4, 4, 100), (1, 300, 4, 2, 150), (1, 64, 2, 2, 17)])
def test_window_attention_matches_oracle(dev, lanes, length, heads, n_kv, window):
    """Every key-tile count (windows 1 to 192), lengths off the 64-query block, GQA 1/2/4. Bar: an
    f16 ulp (2^-10 of the value) plus 2e-4 per element -- the oracle keeps the kernel's f16 points
    (roped q and k, the unnormalised weights), so what differs is f32 summation order and exp's
    last bits, which can move a weight across an f16 rounding boundary."""
    from dtts._lib import call, ptr, stream_handle
    hd = 64
    qkv = synth.f16_bits(synth.normal(35, "qkv", (lanes, length, (heads + 2 * n_kv) * hd)))
    cos_t, sin_t = oracle.rope_table_f32(max(length, 8), hd, 1e4)
    scale = float(np.float32(1 / 8))
    out = torch.empty((lanes, length, heads * hd), dtype=torch.float16, device=dev)
    qd, cd, sd = to_dev(qkv, dev), to_dev(cos_t, dev), to_dev(sin_t, dev)  # held until the kernel has run
    call("dtts_window_attention_prefill_f16", ptr(qd), ptr(cd), ptr(sd), cos_t.shape[0], ptr(out), lanes, length,
         heads, n_kv, hd, window, scale, stream_handle())
    torch.cuda.synchronize()
    want = oracle.window_attention_prefill_f16(qkv, cos_t, sin_t, heads, n_kv, hd, window, scale)
    _rows_close(to_host(out), want, abs_tol=2e-4)


def test_front_decode_tiny_matches_oracle(dev):
    from dtts import codec_front
    from oracle import codec_front as ofront
    from _front_ref import TINY
    hw = codec_front.random_weights(TINY, 36)
    codes = synth.randint(36, "codes", (3, 17, TINY.n_books), 0, TINY.book_size - 1)
    front = codec_front.CodecFront(TINY, hw, dev)
    got = to_host(front.decode(codes))
    want = ofront.decode_f16(TINY, hw, codes)
    g, w = synth.from_f16_bits(got), synth.from_f16_bits(want)
    from _util import rel
    assert rel(g, w)[1] < 2e-3, rel(g, w)


def test_front_decode_codec_geometry(dev):
    """The Qwen3-TTS codec's own widths (16 books, latent 1024, 8 layers at 512, window 72, ratios
    2 and 2), 2 lanes x 90 frames (the window bites) against the oracle chain."""
    from dtts import codec_front
    from oracle import codec_front as ofront
    geo = codec_front.CODEC
    hw = codec_front.random_weights(geo, 37)
    codes = synth.randint(37, "codes", (2, 90, geo.n_books), 0, geo.book_size - 1)
    front = codec_front.CodecFront(geo, hw, dev)
    got = to_host(front.decode(codes))
    want = ofront.decode_f16(geo, hw, codes)
    from _util import rel
    assert got.shape == (2, 360, 1024)
    assert rel(synth.from_f16_bits(got), synth.from_f16_bits(want))[1] < 5e-3


def test_front_decode_rejects_bad_codes(dev):
    from dtts import codec_front
    from _front_ref import TINY
    front = codec_front.CodecFront(TINY, codec_front.random_weights(TINY, 38), dev)
    codes = np.zeros((1, 4, TINY.n_books), np.int32)
    codes[0, 2, 1] = TINY.book_size
    with pytest.raises(DttsError, match="outside"):
        front.decode(codes)


@pytest.mark.parametrize("n,chunk,context", [(14, 4, 2), (5, 4, 2), (3, 4, 2)])
def test_document_decode_matches_oracle(dev, n, chunk, context):
    """Codec::decode's chunked document (codec.rs:562-604) at a tiny front half and clamped waveform
    stack, against the oracle's window-by-window decode: all windows run as lanes of one length
    here, so for n < span the later windows are right-padded where the reference does not pad."""
    from dtts import codec, codec_front
    from oracle import codec as ocodec
    from oracle import codec_front as ofront
    from _doc_ref import TINY, TINY_WAVE, wave_weights
    from _util import rel
    hw, w = codec_front.random_weights(TINY, 62), wave_weights(62)
    codes = synth.randint(62, "codes", (n, TINY.n_books), 0, TINY.book_size - 1)
    front = codec_front.CodecFront(TINY, hw, dev)
    wave = codec.Codec(TINY_WAVE, w, dev)
    got = codec_front.decode_document(front, wave, codes, chunk, context).cpu().numpy()
    want = ofront.decode_document_f32(TINY, hw, TINY_WAVE, ocodec.prepare(TINY_WAVE, w), codes, chunk, context)
    assert got.shape == want.shape == (n * TINY.upsample * TINY_WAVE.hop,)
    assert np.max(np.abs(got - want)) <= 2e-2 and rel(got, want)[1] < 1e-2, (np.max(np.abs(got - want)),
                                                                            rel(got, want))


@pytest.mark.parametrize("n,chunk,context", [(14, 4, 2), (5, 4, 2)])
def test_document_decode_f32_wave_meets_the_reference_gate(dev, n, chunk, context):
    """The document decode with an f32 waveform stack (dtts_codec_create_f32, the reference's
    WAV_DTYPE) against the oracle's window-by-window decode through the f32 stack on the same f16
    front-half latent: within validate.rs's codec.wav gate, max|d| <= 5e-3
    (crates/qwen3tts/src/bin/validate.rs:315)."""
    from dtts import codec, codec_front
    from oracle import codec as ocodec
    from oracle import codec_front as ofront
    from _doc_ref import TINY, TINY_WAVE, wave_weights
    hw, w = codec_front.random_weights(TINY, 65), wave_weights(65)
    codes = synth.randint(65, "codes", (n, TINY.n_books), 0, TINY.book_size - 1)
    front = codec_front.CodecFront(TINY, hw, dev)
    wave = codec.Codec(TINY_WAVE, w, dev, dtype="f32")
    got = codec_front.decode_document(front, wave, codes, chunk, context).cpu().numpy()
    want = ofront.decode_document_f32(TINY, hw, TINY_WAVE, ocodec.prepare(TINY_WAVE, w), codes, chunk, context,
                                      wave="f32")
    assert got.shape == want.shape == (n * TINY.upsample * TINY_WAVE.hop,)
    assert np.max(np.abs(got - want)) <= 5e-3, np.max(np.abs(got - want))
    assert np.std(want) > 0.02


def test_document_decode_equals_its_windows(dev):
    """The batched document decode keeps, bit for bit, what each padded window decoded on its own
    (one lane through dtts_codec_front_decode and dtts_codec_decode) gives for its chunk."""
    from dtts import codec, codec_front
    from oracle import codec_front as ofront
    from _doc_ref import TINY, TINY_WAVE, wave_weights
    n, chunk, context = 23, 6, 3
    front = codec_front.CodecFront(TINY, codec_front.random_weights(TINY, 63), dev)
    wave = codec.Codec(TINY_WAVE, wave_weights(63), dev)
    codes = synth.randint(63, "codes", (n, TINY.n_books), 0, TINY.book_size - 1)
    got = codec_front.decode_document(front, wave, codes, chunk, context).cpu().numpy()
    spf = TINY.upsample * TINY_WAVE.hop
    for frm, to, length, drop, keep in ofront.document_windows(n, chunk, context):
        idx = np.minimum(np.arange(frm, frm + length), to - 1)
        lat = front.decode(codes[idx][None])
        wav = wave.decode(lat).float().cpu().numpy()[0]
        start = frm + drop
        assert np.array_equal(got[start * spf:(start + keep) * spf], wav[drop * spf:(drop + keep) * spf])


def test_document_decode_rejects_bad_arguments(dev):
    from dtts import DttsError, codec, codec_front
    from _doc_ref import TINY, TINY_WAVE, wave_weights
    front = codec_front.CodecFront(TINY, codec_front.random_weights(TINY, 64), dev)
    wave = codec.Codec(TINY_WAVE, wave_weights(64), dev)
    codes = np.zeros((9, TINY.n_books), np.int32)
    with pytest.raises(DttsError, match="bad sizes"):
        codec_front.decode_document(front, wave, codes, chunk=0, context=2)
    with pytest.raises(DttsError, match="max_frames"):
        codec_front.decode_document(front, wave, np.zeros((TINY.max_frames + 10, TINY.n_books), np.int32),
                                    chunk=TINY.max_frames, context=5)
    codes[7, 3] = -1
    with pytest.raises(DttsError, match="outside"):
        codec_front.decode_document(front, wave, codes, chunk=4, context=2)
