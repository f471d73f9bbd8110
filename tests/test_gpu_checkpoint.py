"""Weight formats on the device (dtts_convert_*) and Codec::load from a checkpoint
(dtts_codec_model_load), through the C ABI.

Conversions are bit-exact against the host restatements: the element permutations of
dtts_tap_major_weight / dtts_transpose_tap_major_weight / dtts_transpose_bias (themselves pinned
against torch's conv1d and conv_transpose1d), numpy's round-to-nearest-even casts, numpy's f32
division for the codebook fold, the float64 exp rounded once for SnakeBeta's fold, and the host
Q8_0 quantiser byte for byte -- for f32, f16, bf16 and f64 sources. A whole codec loaded from a
checkpoint in the reference's naming decodes bit for bit like the same weights uploaded by the
Python host path, from f32 and from bf16 files."""
import ctypes

import numpy as np
import pytest
import torch

import _ckpt
import oracle
from dtts import checkpoint, codec, codec_front, nlc, synth
from dtts._lib import call, ptr

pytestmark = pytest.mark.gpu

DTYPES = ["F32", "F16", "BF16", "F64"]
CODE = {"F32": 0, "F16": 1, "BF16": 2, "F64": 3}


def _src(a, dtype, dev):
    """(device tensor in `dtype`, the f32 values it holds)."""
    t = torch.from_numpy(np.ascontiguousarray(a, np.float64))
    t = {"F32": t.float(), "F16": t.half(), "BF16": t.bfloat16(), "F64": t}[dtype]
    return t.to(dev), t.double().float().numpy()


def _f16(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("dtype", DTYPES)
def test_layout_conversions_bit_exact(dev, dtype):
    rng = np.random.default_rng(7)
    code = CODE[dtype]
    # tap-major conv weight
    w, w32 = _src(rng.standard_normal((48, 40, 7)), dtype, dev)
    out = torch.empty(48 * 7 * 40, dtype=torch.float16, device=dev)
    checkpoint.convert("tap_major_f16", ptr(w), code, ptr(out), 48, 40, 7)
    torch.cuda.synchronize()
    assert np.array_equal(_f16(out), synth.f16_bits(nlc.tap_major_weight(w32)).ravel())
    # polyphase transposed conv (kernel 2 * stride and kernel = stride)
    for cin, cout, kernel, stride in [(24, 16, 10, 5), (32, 32, 2, 2), (8, 6, 12, 3)]:
        w, w32 = _src(rng.standard_normal((cin, cout, kernel)), dtype, dev)
        out = torch.empty(cin * cout * kernel, dtype=torch.float16, device=dev)
        checkpoint.convert("transpose_tap_major_f16", ptr(w), code, ptr(out), cin, cout, kernel, stride)
        torch.cuda.synchronize()
        assert np.array_equal(_f16(out), synth.f16_bits(nlc.transpose_tap_major_weight(w32, stride)).ravel())
    # bias repeated per phase
    bsrc, b32 = _src(rng.standard_normal(37), dtype, dev)
    out = torch.empty(37 * 4, dtype=torch.float16, device=dev)
    checkpoint.convert("repeat_f16", ptr(bsrc), code, ptr(out), 37, 4)
    torch.cuda.synchronize()
    assert np.array_equal(_f16(out), synth.f16_bits(nlc.transpose_bias(b32, 4)).ravel())
    # [out, in] -> [in, out] (host_layout), off the 32-tile
    m, m32 = _src(rng.standard_normal((70, 45)), dtype, dev)
    out = torch.empty(45 * 70, dtype=torch.float16, device=dev)
    checkpoint.convert("transpose_f16", ptr(m), code, ptr(out), 70, 45)
    torch.cuda.synchronize()
    assert np.array_equal(_f16(out), synth.f16_bits(np.ascontiguousarray(m32.T)).ravel())
    # columns into a wider destination; plain casts
    out = torch.zeros(70 * 100, dtype=torch.float16, device=dev)
    checkpoint.convert("f16_cols", ptr(m), code, ptr(out), 70, 45, 100, 30)
    torch.cuda.synchronize()
    want = np.zeros((70, 100), np.float32)
    want[:, 30:75] = m32
    assert np.array_equal(_f16(out), synth.f16_bits(want).ravel())
    o32 = torch.empty(70 * 45, dtype=torch.float32, device=dev)
    checkpoint.convert("f32", ptr(m), code, ptr(o32), 70 * 45)
    torch.cuda.synchronize()
    assert np.array_equal(o32.cpu().numpy(), m32.ravel())


@pytest.mark.parametrize("dtype", DTYPES)
def test_folds_bit_exact(dev, dtype):
    rng = np.random.default_rng(8)
    code = CODE[dtype]
    a, a32 = _src(rng.uniform(np.log(0.03), np.log(3.0), 1000), dtype, dev)
    b, b32 = _src(rng.uniform(-3.0, 3.0, 1000), dtype, dev)
    alpha = torch.empty(1000, dtype=torch.float32, device=dev)
    brecip = torch.empty_like(alpha)
    checkpoint.convert("snake_fold", ptr(a), ptr(b), code, ptr(alpha), ptr(brecip), 1000)
    torch.cuda.synchronize()
    wa, wr = _ckpt._snake_fold(a32, b32)
    assert np.array_equal(alpha.cpu().numpy(), wa)
    assert np.array_equal(brecip.cpu().numpy(), wr)
    s, s32 = _src(rng.standard_normal((50, 24)), dtype, dev)
    u, u32 = _src(np.concatenate([rng.uniform(0.5, 2.0, 47), [0.0, 1e-7, 3e-6]]), dtype, dev)
    books = torch.empty(50 * 24, dtype=torch.float32, device=dev)
    checkpoint.convert("codebook_fold", ptr(s), ptr(u), code, ctypes.c_float(1e-5), ptr(books), 50, 24)
    torch.cuda.synchronize()
    assert np.array_equal(books.cpu().numpy(), codec_front.fold_codebook(s32, u32).ravel())


@pytest.mark.parametrize("dtype", DTYPES)
def test_q8_0_device_matches_host(dev, dtype):
    rng = np.random.default_rng(9)
    rows, k = 37, 256
    x = rng.standard_normal((rows, k)) * rng.uniform(0.01, 3.0, (rows, 1))
    x[3, 32:64] = 0.0            # an all-zero block
    x[5, 0:32] = 0.5             # ties at .5 after scaling (amax / 127 steps)
    x[6, 64] = -7.0              # amax at a block's first element
    w, w32 = _src(x, dtype, dev)
    blocks = torch.zeros(rows * k // 32 * 34, dtype=torch.uint8, device=dev)
    checkpoint.convert("q8_0", ptr(w), CODE[dtype], ptr(blocks), rows, k)
    torch.cuda.synchronize()
    host = np.zeros(rows * k // 32 * 34, np.uint8)
    src = np.ascontiguousarray(w32, np.float32)
    call("dtts_q8_0_quantize", src.ctypes.data_as(ctypes.c_void_p), host.ctypes.data_as(ctypes.c_void_p), rows, k)
    assert np.array_equal(blocks.cpu().numpy(), host)


def test_q8_0_device_ties_round_half_away(dev):
    """dtts_convert_q8_0 on exact ties (amax 127, so d = id = 1): away from zero, as the oracle's
    closed form and ggml's roundf / candle's f32::round give."""
    from test_oracle_gemm_q8 import TIE_CODES, tie_block_weights

    w32 = tie_block_weights()
    rows, k = w32.shape
    w = torch.from_numpy(w32).to(dev)
    blocks = torch.zeros(rows * k // 32 * 34, dtype=torch.uint8, device=dev)
    checkpoint.convert("q8_0", ptr(w), CODE["F32"], ptr(blocks), rows, k)
    torch.cuda.synchronize()
    got = blocks.cpu().numpy().reshape(rows, k // 32, 34)
    q = got[..., 2:].view(np.int8).astype(np.int32)
    assert np.array_equal(q[0, 0, :12], TIE_CODES)
    assert np.array_equal(q[1, 1, :12], TIE_CODES)
    assert np.array_equal(got, oracle.q8_0_quantize(w32))


def _python_models(fw, ww, dev):
    return (codec_front.CodecFront(_ckpt.TINY_CKPT_FRONT, fw, dev), codec.Codec(_ckpt.TINY_WAVE, ww, dev))


@pytest.mark.parametrize("dtype", ["F32", "BF16"])
def test_codec_model_load_decodes_like_host_upload(dev, tmp_path, dtype):
    T, fw, ww = _ckpt.build(_ckpt.TINY_CKPT_FRONT, _ckpt.TINY_WAVE, seed=3, dtype=dtype)
    path = tmp_path / "codec.safetensors"
    _ckpt.write(path, T, dtype)
    with checkpoint.Checkpoint(path) as ck:
        model = checkpoint.CodecModel(ck, _ckpt.TINY_CKPT_FRONT, _ckpt.TINY_WAVE, dev)
    front, wave = _python_models(fw, ww, dev)
    codes = synth.randint(3, "ck.codes", (2, 9, _ckpt.TINY.n_books), 0, _ckpt.TINY.book_size - 1)
    got = _f16(model.latent(codes))
    want = _f16(front.decode(codes))
    assert np.array_equal(got, want)
    doc = synth.randint(3, "ck.doc", (23, _ckpt.TINY.n_books), 0, _ckpt.TINY.book_size - 1)
    a = model.decode(doc, chunk=6, context=3).cpu().numpy()
    b = codec_front.decode_document(front, wave, doc, 6, 3).cpu().numpy()
    assert a.shape == (23 * _ckpt.TINY.upsample * _ckpt.TINY_WAVE.hop,)
    assert np.array_equal(a, b) and np.isfinite(a).all() and 0.01 < np.std(a) < 0.99
    assert model.nbytes > 0
    model.close()


def test_f64_source_rounds_through_f32(dev):
    """An f64 tensor cast to f16 is rounded to f32 first, as the reference's to_dtype(F32) then
    to_dtype(F16) is: 0.745849579666197 is 0.7458496 in f32, whose f16 is 0.746; one f64 -> f16
    rounding would give 0.7456."""
    x = torch.tensor([0.745849579666197, -0.745849579666197], dtype=torch.float64, device=dev)
    out = torch.empty(2, dtype=torch.float16, device=dev)
    checkpoint.convert("f16", ptr(x), CODE["F64"], ptr(out), 2)
    torch.cuda.synchronize()
    want = np.float32([0.745849579666197, -0.745849579666197]).astype(np.float16)
    assert np.array_equal(out.cpu().numpy(), want) and want[0] != np.float16(0.745849579666197)


@pytest.mark.parametrize("which,weight", [("SMALL", "f16"), ("WINDOWED", "f16"), ("SMALL", "f32"),
                                          ("WINDOWED", "f32"), ("SMALL", "q8_0"), ("SMALL", "q8_0_a32")])
def test_stack_model_load_decodes_like_host_upload(dev, tmp_path, which, weight):
    """Stack::load(.., how, ..) from a checkpoint (QK-norm with D = 128; LayerScale with a window
    at D = 64), for each weight kind: f16, f32, and Q8_0 quantized on the device (the device
    quantizer is the host's bit for bit), steps bit for bit like the same weights uploaded by the
    host path, over two steps."""
    import _stack_ref
    from dtts import stack

    geo = getattr(_stack_ref, which)
    layers, fn = stack.random_weights(geo, 12)
    prefix = "talker.model." if geo.qk_norm else "decoder.pre_transformer."
    path = tmp_path / "stack.safetensors"
    _ckpt.write(path, _ckpt.stack_tensors(geo, layers, fn, prefix))
    with checkpoint.Checkpoint(path) as ck:
        model = checkpoint.StackModel(ck, prefix, geo, dev, weight=weight)
    host = stack.Stack(geo, layers, fn, dev, weight=weight)
    lanes, cap = 3, geo.capacity
    sa, sb = model.stack.new_state(lanes, cap), host.new_state(lanes, cap)
    pos = np.array([0, 7, cap - 3], np.int32)
    for s in range(2):
        x = torch.from_numpy(synth.normal(12 + s, "ck.x", (lanes, geo.dim))).to(dev)
        a = model.stack.decode(x, sa, pos + s).cpu().numpy()
        b = host.decode(x, sb, pos + s).cpu().numpy()
        assert np.array_equal(a, b) and np.isfinite(a).all()
    assert model.nbytes > 0
    model.close()


def test_codec_model_load_full_geometry(dev, tmp_path):
    """The Qwen3-TTS codec's own geometry end to end: a 457 MB f32 checkpoint in the reference's
    naming (16 books of 2048 x 256, the 8-layer windowed transformer at 512, two ConvNeXt stages at
    1024, the 1536 -> 96 waveform stack, clamped output) loaded by dtts_codec_model_load, then a
    two-window document (40 frames, chunk 30, context 5) decoded bit for bit like the host-upload
    models."""
    import time
    from dataclasses import replace

    wave_geo = replace(codec.CONFIG5, out_clamp=True)
    T, fw, ww = _ckpt.build(codec_front.CODEC, wave_geo, seed=4)
    path = tmp_path / "full.safetensors"
    _ckpt.write(path, T)
    del T
    t0 = time.perf_counter()
    with checkpoint.Checkpoint(path) as ck:
        model = checkpoint.CodecModel(ck, codec_front.CODEC, wave_geo, dev)
    print(f"load: {time.perf_counter() - t0:.2f} s, arena {model.nbytes / 1e6:.1f} MB")
    doc = synth.randint(4, "ck.fulldoc", (40, codec_front.CODEC.n_books), 0, codec_front.CODEC.book_size - 1)
    a = model.decode(doc, chunk=30, context=5).cpu().numpy()
    front, wave = codec_front.CodecFront(codec_front.CODEC, fw, dev), codec.Codec(wave_geo, ww, dev)
    b = codec_front.decode_document(front, wave, doc, 30, 5).cpu().numpy()
    assert a.shape == (40 * 1920,) and np.array_equal(a, b)
    assert np.isfinite(a).all() and np.max(np.abs(a)) <= 1.0
    model.close()
