"""Pins the oracle's codec chains against an independent float64 build of the same stack from
torch's CPU conv1d / conv_transpose1d (library routines) in torch's own NCL layout and
parameter layouts -- so weight layouts, the transposed conv's crop, padding, residual wiring and
the activation order are all checked, not just the arithmetic.
"""
import numpy as np
import oracle
from oracle import codec as ocodec
from dtts import codec, synth

from _codec_ref import torch_decode as _torch_decode

GEO = codec.Geometry(latent_dim=64, head_kernel=7, channels=(96, 64, 32), rates=(2, 3),
                     ru_kernel=7, ru_dilations=(1, 3, 9), out_kernel=7)


def test_geometry_flops_match_survey_config5():
    # 298.9 GFLOP per lane at 250 frames (head 5.5, convT 9.4/11.8/11.8/8.85, RU triples ...)
    f = codec.CONFIG5.flops_per_frame() * 250
    assert abs(f / 1e9 - 298.9) < 0.6
    assert codec.CONFIG5.hop == 480


def small_weights(seed):
    """Test weights: the output conv scaled down so tanh stays off saturation and shows errors."""
    w = codec.random_weights(GEO, seed=seed)
    w.out_w = (w.out_w * 0.05).astype(np.float32)
    return w


def test_oracle_codec_chains_match_torch_f64():
    w = small_weights(5)
    prep = ocodec.prepare(GEO, w)
    lanes, frames = 2, 12
    latent = synth.normal(5, "latent", (lanes, frames, GEO.latent_dim))
    want = np.stack([_torch_decode(GEO, w, latent[i]) for i in range(lanes)])
    got32 = np.stack([ocodec.decode_f32_reference(GEO, prep, latent[i]) for i in range(lanes)])
    assert np.max(np.abs(got32 - want)) < 1e-4
    assert 0.05 < np.std(want) < 0.9  # not saturated
    got16 = synth.from_f16_bits(ocodec.decode_f16(GEO, prep, synth.f16_bits(latent)))
    want16 = np.stack([_torch_decode(GEO, w, synth.from_f16_bits(synth.f16_bits(latent[i])))
                       for i in range(lanes)])
    # f16 storage points through 14 activations: a few f16 ulps of the unit-range waveform
    assert np.max(np.abs(got16 - want16)) < 2e-2
    assert got16.shape == (lanes, frames * GEO.hop)


def test_oracle_f32_chain_clamps_like_codec_forward():
    """out_clamp: Codec::forward's clamp to [-1, 1] (codec.rs:433-436) in place of tanh, against
    the float64 build; the output conv is scaled up so the clamp is reached."""
    from dataclasses import replace
    geo = replace(GEO, out_clamp=True)
    w = codec.random_weights(geo, seed=6)
    w.out_w = (w.out_w * 3.0).astype(np.float32)
    prep = ocodec.prepare(geo, w)
    latent = synth.normal(6, "latent", (10, geo.latent_dim))
    want = _torch_decode(geo, w, latent)
    got = ocodec.decode_f32_reference(geo, prep, latent)
    assert np.max(np.abs(got - want)) < 1e-4
    assert np.mean(np.abs(want) == 1.0) > 0.01  # the clamp is active
