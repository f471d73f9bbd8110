"""The codec decoder stack (dtts_codec_decode) against the oracle's f16-storage chain.

The GPU stack stores exactly the tensors the oracle's composed chain stores (all f16), so the
two differ only by f32 summation order inside each conv -- and SnakeBeta amplifies any input
difference through the stack (the reference's reason for keeping its codec f32,
crates/qwen3tts/src/codec.rs:33-43). Bar: the GPU no further from the oracle than f16 storage
itself puts the oracle from exact float64 arithmetic on the same inputs (torch's conv1d /
conv_transpose1d) -- in RMS, and at the worst sample within 2e-2 absolute (the f16 tolerance at
unit scale) or 1.5x the oracle's own worst-sample distance from float64, whichever is larger. Each conv is held exactly to its oracle stage in test_gpu_conv.py. The
geometries cover both SnakeBeta placements (stored snaked copy for stages wider than 96
channels, conv prologue at 96) and every kernel path.
"""
import numpy as np
import pytest
import torch

from oracle import codec as ocodec
from dtts import codec, synth

from _codec_ref import torch_decode
from _util import to_dev, to_host

pytestmark = pytest.mark.gpu

SMALL = codec.Geometry(latent_dim=128, head_kernel=7, channels=(384, 192, 96), rates=(4, 3),
                       ru_kernel=7, ru_dilations=(1, 3, 9), out_kernel=7)


def _weights(geo, seed):
    w = codec.random_weights(geo, seed=seed)
    w.out_w = (w.out_w * 0.05).astype(np.float32)  # keep tanh off saturation so errors show
    return w


@pytest.mark.parametrize("geo,lanes,frames", [(SMALL, 3, 40), (codec.CONFIG5, 2, 3)],
                         ids=["small", "config5-geometry"])
def test_codec_decode_matches_oracle(dev, geo, lanes, frames):
    w = _weights(geo, 7)
    latent = synth.f16_bits(synth.normal(7, "latent", (lanes, frames, geo.latent_dim)))
    model = codec.Codec(geo, w, dev)
    got = synth.from_f16_bits(to_host(model.decode(to_dev(latent, dev))))
    want = synth.from_f16_bits(ocodec.decode_f16(geo, ocodec.prepare(geo, w), latent))
    assert got.shape == (lanes, frames * geo.hop)
    assert np.isfinite(got).all()
    exact = np.stack([torch_decode(geo, w, synth.from_f16_bits(latent[i])) for i in range(lanes)])
    err = np.abs(got - want)
    rms_gpu = float(np.sqrt(np.mean((got - want) ** 2)))
    rms_f16 = float(np.sqrt(np.mean((want - exact) ** 2)))
    max_f16 = float(np.max(np.abs(want - exact)))
    msg = (f"max {np.max(err):.3e} (oracle-f64 {max_f16:.3e}) rms(gpu-oracle) {rms_gpu:.3e} "
           f"rms(oracle-f64) {rms_f16:.3e}")
    print(msg)
    assert np.max(err) <= max(2e-2, 1.5 * max_f16), msg
    assert rms_gpu <= 2.0 * rms_f16 + 1e-4, msg
    assert 0.02 < np.std(want) < 0.95


def test_codec_lanes_are_independent(dev):
    """A lane's audio does not depend on its batch neighbours (no cross-lane taps)."""
    geo = SMALL
    w = _weights(geo, 8)
    model = codec.Codec(geo, w, dev)
    latent = synth.f16_bits(synth.normal(8, "latent", (4, 16, geo.latent_dim)))
    full = to_host(model.decode(to_dev(latent, dev)))
    one = to_host(model.decode(to_dev(latent[2:3].copy(), dev)))
    assert np.array_equal(full[2:3], one)


def test_codec_profile_covers_every_launch(dev):
    geo = SMALL
    model = codec.Codec(geo, _weights(geo, 9), dev)
    latent = to_dev(synth.f16_bits(synth.normal(9, "latent", (2, 8, geo.latent_dim))), dev)
    ref = to_host(model.decode(latent))
    audio = torch.empty((2, 8 * geo.hop), dtype=torch.float16, device=dev)
    stages = model.profile(latent, out=audio)
    assert np.array_equal(to_host(audio), ref)
    fused = [c in (96, 192) for c in geo.channels[1:]]  # residual units run as one kernel there
    assert len(stages) == 2 + sum(1 + (3 if f else 6) for f in fused)
    assert all(s["ms"] > 0 for s in stages)
    assert stages[0]["name"] == "head" and stages[-1]["name"] == "out"
    assert sum(s["flops"] for s in stages) == pytest.approx(2 * 8 * geo.flops_per_frame(), rel=1e-9)


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_codec_empty_and_single_frame_decodes(dev, dtype):
    """No lanes or no frames: nothing is enqueued and nothing is written. One lane of one frame
    (every conv's grid a single, mostly padded tile) matches the oracle chain under the bar above
    (f16), or, f32, the oracle's f32 route and float64 within the reference's 5e-3 gate."""
    geo = SMALL
    w = _weights(geo, 10)
    model = codec.Codec(geo, w, dev, dtype=dtype)
    tdt = torch.float16 if dtype == "f16" else torch.float32
    for lanes, frames in ((0, 5), (2, 0)):
        lat = torch.zeros((lanes, frames, geo.latent_dim), dtype=tdt, device=dev)
        out = torch.full((lanes, frames * geo.hop), 7.0, dtype=tdt, device=dev)
        assert model.decode(lat, out=out).shape == (lanes, frames * geo.hop)
    canary = torch.full((3, geo.hop), 7.0, dtype=tdt, device=dev)
    model.decode(torch.zeros((1, 0, geo.latent_dim), dtype=tdt, device=dev), out=canary[:1, :0])
    torch.cuda.synchronize()
    assert bool((canary == 7.0).all())

    latent = synth.f16_bits(synth.normal(10, "latent", (1, 1, geo.latent_dim)))
    lat32 = synth.from_f16_bits(latent)
    exact = torch_decode(geo, w, lat32[0])[None]
    if dtype == "f16":
        got = synth.from_f16_bits(to_host(model.decode(to_dev(latent, dev))))
        want = synth.from_f16_bits(ocodec.decode_f16(geo, ocodec.prepare(geo, w), latent))
        max_f16 = float(np.max(np.abs(want - exact)))
        assert np.max(np.abs(got - want)) <= max(2e-2, 1.5 * max_f16)
    else:  # the reference's codec.wav gate (validate.rs:315), against its f32 route and float64
        got = to_host(model.decode(torch.from_numpy(lat32).to(dev)))
        want = ocodec.decode_f32_reference(geo, ocodec.prepare(geo, w), lat32[0])[None]
        assert np.max(np.abs(got - want)) <= 5e-3 and np.max(np.abs(got - exact)) <= 5e-3
    assert got.shape == (1, geo.hop) and np.isfinite(got).all()


def test_codec_decode_from_two_host_threads(dev):
    """Two host threads decode through one codec at once, each on its own stream with its own
    workspace: every decode equals the single-thread decode of the same latent bit for bit (the
    codec's lock keeps each call's fork and join events its own)."""
    import threading

    from dtts._lib import call, lib, ptr, stream_handle

    geo, lanes, frames, reps = SMALL, 4, 24, 12
    model = codec.Codec(geo, _weights(geo, 9), dev)
    lats = [to_dev(synth.f16_bits(synth.normal(9, f"latent{i}", (lanes, frames, geo.latent_dim))), dev)
            for i in range(2)]
    want = [to_host(model.decode(lat)) for lat in lats]
    need = int(lib().dtts_codec_workspace_bytes(model.handle, lanes, frames))
    torch.cuda.synchronize()
    got, errors = [None, None], []

    def worker(i):
        try:
            s = torch.cuda.Stream(device=dev)
            with torch.cuda.stream(s):
                ws = torch.empty(need, dtype=torch.uint8, device=dev)
                audio = torch.empty((lanes, frames * geo.hop), dtype=torch.float16, device=dev)
                outs = []
                for _ in range(reps):
                    call("dtts_codec_decode", model.handle, ptr(lats[i]), ptr(audio), lanes, frames, ptr(ws),
                         need, stream_handle())
                    outs.append(audio.clone())
            s.synchronize()
            got[i] = [to_host(o) for o in outs]
        except Exception as e:  # reported on the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i in range(2):
        assert len(got[i]) == reps
        for r, out in enumerate(got[i]):
            assert np.array_equal(out, want[i]), (i, r)
