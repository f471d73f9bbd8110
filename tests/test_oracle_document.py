"""Pins the oracle's chunked document decode (oracle/codec_front.py: document_windows and
decode_document_f32, Codec::decode at crates/qwen3tts/src/codec.rs:562-604):

* the windows against the reference loop's own arithmetic at its constants (chunk 300, left
  context 25): starts every chunk, context dropped, padding to the span only when n >= span;
* a document no longer than one chunk is exactly one plain forward;
* the decoder is causal, so each window's kept audio equals the same frames' audio from an
  unpadded forward over frames[from:end] -- which fails if the padding went on the left, the
  drop were miscounted, or a window's codes were taken from the wrong place."""
import numpy as np
import pytest

from oracle import codec as ocodec
from oracle import codec_front as ofront
from dtts import codec_front, synth

from _doc_ref import TINY, TINY_WAVE, wave_weights


@pytest.mark.parametrize("n,want", [
    (700, [(0, 325, 325, 0, 300), (275, 600, 325, 25, 300), (575, 700, 325, 25, 100)]),
    (100, [(0, 100, 100, 0, 100)]),
    (325, [(0, 325, 325, 0, 300), (275, 325, 325, 25, 25)]),
    (300, [(0, 300, 300, 0, 300)]),
    (0, []),
])
def test_windows_at_reference_constants(n, want):
    got = ofront.document_windows(n, codec_front.CHUNK_FRAMES, codec_front.CHUNK_LEFT_CONTEXT)
    assert got == want
    kept = [(f + d, f + d + k) for f, _, _, d, k in got]
    assert sum(k for *_, k in got) == n
    assert all(a[1] == b[0] for a, b in zip(kept, kept[1:]))


def _setup(seed, n):
    hw = codec_front.random_weights(TINY, seed)
    w = wave_weights(seed)
    prep = ocodec.prepare(TINY_WAVE, w)
    codes = synth.randint(seed, "codes", (n, TINY.n_books), 0, TINY.book_size - 1)
    return hw, prep, codes


def _forward(hw, prep, codes):
    lat = ofront.decode_f16(TINY, hw, np.asarray(codes)[None])
    return ocodec.decode_f16(TINY_WAVE, prep, lat)[0].view(np.float16).astype(np.float32)


def test_one_chunk_document_is_one_forward():
    hw, prep, codes = _setup(60, 4)
    got = ofront.decode_document_f32(TINY, hw, TINY_WAVE, prep, codes, chunk=4, context=2)
    assert np.array_equal(got, _forward(hw, prep, codes))


@pytest.mark.parametrize("n,chunk,context", [(14, 4, 2), (5, 4, 2)])
def test_kept_audio_equals_unpadded_causal_forward(n, chunk, context):
    hw, prep, codes = _setup(61, n)
    spf = TINY.upsample * TINY_WAVE.hop
    got = ofront.decode_document_f32(TINY, hw, TINY_WAVE, prep, codes, chunk, context)
    assert got.shape == (n * spf,)
    wins = ofront.document_windows(n, chunk, context)
    # n >= span: the last window is padded by two repeats of frame 13; n < span: nothing is padded
    assert wins[-1] == ((10, 14, 6, 2, 2) if n == 14 else (2, 5, 3, 2, 1))
    for frm, _, _, drop, keep in wins:
        start = frm + drop
        plain = _forward(hw, prep, codes[frm:start + keep])
        assert np.array_equal(got[start * spf:(start + keep) * spf], plain[drop * spf:])
    assert 0.01 < np.std(got) < 0.99 and np.max(np.abs(got)) <= 1.0


def test_reference_fixture_shapes():
    """The reference's codec fixture manifest (fixtures/qwen3tts/oracle.json: codes [147, 16] ->
    quantized [1, 512, 147] -> pre_tf [1, 147, 1024] -> wav [1, 1, 282240]; the long case
    [400, 16] -> [1, 1, 768000], chunked and not) restated as this build's geometry: 16 books, the
    512-wide quantizer sum, the 1024-wide latent, 1920 samples per frame, and Codec::decode's
    windows covering both documents exactly once."""
    from dtts import codec

    g, w = codec_front.CODEC, codec.CONFIG5
    assert g.n_books == 16 and g.codebook_dim == 512 and g.latent_dim == 1024
    assert g.upsample * w.hop == 1920
    for n, samples in ((147, 282240), (400, 768000)):
        wins = ofront.document_windows(n, codec_front.CHUNK_FRAMES, codec_front.CHUNK_LEFT_CONTEXT)
        assert sum(k for *_, k in wins) * g.upsample * w.hop == samples
    assert ofront.document_windows(400, 300, 25) == [(0, 325, 325, 0, 300), (275, 400, 325, 25, 100)]
