"""The codec waveform stack at the reference's own precision (dtts_codec_create_f32 /
dtts_codec_decode_f32): every activation, weight and sum f32, as the reference keeps its stack
(WAV_DTYPE = F32, crates/qwen3tts/src/codec.rs:33-43).

Bar: the reference's own gate for the decoded waveform, max|d| <= 5e-3 (`codec.wav`,
crates/qwen3tts/src/bin/validate.rs:315), against the oracle's f32 restatement of the reference
CPU route (oracle.codec.decode_f32_reference: pad + cat + GEMM per conv, polyphase transposed
convs) and against an independent float64 build from torch's conv1d / conv_transpose1d. Held at a
small geometry and at the full config-5 length on the first and last lanes of 48.
"""
import numpy as np
import pytest
import torch

from oracle import codec as ocodec
from dtts import DttsError, codec, synth

from _codec_ref import torch_decode
from _util import to_dev, to_host

pytestmark = pytest.mark.gpu

GATE = 5e-3  # validate.rs:315, codec.wav
SMALL = codec.Geometry(latent_dim=128, head_kernel=7, channels=(384, 192, 96), rates=(4, 3),
                       ru_kernel=7, ru_dilations=(1, 3, 9), out_kernel=7)


def _weights(geo, seed):
    w = codec.random_weights(geo, seed=seed)
    w.out_w = (w.out_w * 0.05).astype(np.float32)  # keep tanh off saturation so errors show
    return w


@pytest.mark.parametrize("geo,lanes,frames,check", [(SMALL, 3, 40, [0, 1, 2]), (codec.CONFIG5, 48, 250, [0, 47])],
                         ids=["small", "config5-full"])
def test_f32_codec_meets_the_reference_gate(dev, geo, lanes, frames, check):
    w = _weights(geo, 11)
    latent = synth.normal(11, "latent", (lanes, frames, geo.latent_dim))
    model = codec.Codec(geo, w, dev, dtype="f32")
    got = to_host(model.decode(to_dev(latent, dev)))
    assert got.shape == (lanes, frames * geo.hop) and np.isfinite(got).all()
    prep = ocodec.prepare(geo, w)
    for li in check:
        want = ocodec.decode_f32_reference(geo, prep, latent[li])
        exact = torch_decode(geo, w, latent[li])
        d_oracle = float(np.max(np.abs(got[li] - want)))
        d_exact = float(np.max(np.abs(got[li] - exact)))
        print(f"lane {li}: max|gpu - oracle f32| {d_oracle:.2e}, max|gpu - f64| {d_exact:.2e}, "
              f"max|oracle f32 - f64| {np.max(np.abs(want - exact)):.2e}")
        assert d_oracle <= GATE and d_exact <= GATE
        assert 0.02 < np.std(exact) < 0.95


def test_f32_and_f16_codecs_refuse_each_others_decode(dev):
    geo = SMALL
    w = _weights(geo, 12)
    m32 = codec.Codec(geo, w, dev, dtype="f32")
    m16 = codec.Codec(geo, w, dev)
    lat16 = torch.zeros((1, 4, geo.latent_dim), dtype=torch.float16, device=dev)
    with pytest.raises(DttsError, match="f32"):
        m32.decode(lat16)
    from dtts._lib import call
    import ctypes
    ws, need = m16.workspace(1, 4)
    out = torch.empty((1, 4 * geo.hop), dtype=torch.float32, device=dev)
    with pytest.raises(DttsError, match="dtts_codec_create \\(decode it with dtts_codec_decode\\)"):
        call("dtts_codec_decode_f32", m16.handle, ctypes.c_void_p(lat16.data_ptr()), ctypes.c_void_p(out.data_ptr()),
             1, 4, ctypes.c_void_p(ws.data_ptr()), ctypes.c_size_t(need), None)


def test_f32_codec_profile_names_the_split_kernels(dev):
    """The f32 codec runs its convs on the f16 matrix cores with split operands: a stage storing
    the latent split, every conv on conv_split_mfma, the output conv on the f32 window kernel
    reading split input; profiled launches give the decode's audio bit for bit."""
    geo = SMALL
    model = codec.Codec(geo, _weights(geo, 13), dev, dtype="f32")
    latent = to_dev(synth.normal(13, "latent", (2, 8, geo.latent_dim)), dev)
    ref = to_host(model.decode(latent))
    audio = torch.empty((2, 8 * geo.hop), dtype=torch.float32, device=dev)
    stages = model.profile(latent, out=audio)
    assert np.array_equal(to_host(audio), ref)
    assert len(stages) == 3 + sum(1 + 6 for _ in geo.channels[1:])  # every residual unit as two convs
    assert stages[0]["kernel"] == "split_act_kernel" and stages[-1]["kernel"] == "conv_nlc_f32_narrow<true>"
    assert all(s["kernel"].startswith("conv_split_mfma<") for s in stages[1:-1])
    assert sum(s["flops"] for s in stages) == pytest.approx(2 * 8 * geo.flops_per_frame(), rel=1e-9)


def test_split_and_f32_kernels_agree(dev, monkeypatch):
    """The split-operand codec against the plain-f32 one (DTTS_F32_CODEC_KERNEL=f32 at create: f32
    tensors, f32 matrix cores): both f32-accurate, so they differ by f32 summation order and the
    dropped lo.lo products (~2^-22 of each term), amplified by the SnakeBeta chain; bar 1e-4 of the
    audio's scale (the codec.wav gate is 5e-3)."""
    geo = SMALL
    w = _weights(geo, 14)
    latent = to_dev(synth.normal(14, "latent", (3, 24, geo.latent_dim)), dev)
    split = codec.Codec(geo, w, dev, dtype="f32")
    monkeypatch.setenv("DTTS_F32_CODEC_KERNEL", "f32")
    plain = codec.Codec(geo, w, dev, dtype="f32")
    a, b = to_host(split.decode(latent)), to_host(plain.decode(latent))
    assert "conv_split_mfma" in split.profile(latent)[1]["kernel"]
    assert "conv_nlc_f32_mfma" in plain.profile(latent)[1]["kernel"]
    d = float(np.max(np.abs(a - b)))
    print(f"max|split - f32| {d:.2e}, audio max {np.max(np.abs(b)):.3f}")
    assert d <= 1e-4 * max(1.0, float(np.max(np.abs(b))))
