"""Small geometries for Codec::decode's chunked path (crates/qwen3tts/src/codec.rs:562-604): the
tiny front half of _front_ref and a waveform stack over its latent width, clamped like
Codec::forward (codec.rs:433-436)."""
from dtts import codec

from _front_ref import TINY  # noqa: F401  (latent 64, upsample 6)

TINY_WAVE = codec.Geometry(latent_dim=64, head_kernel=7, channels=(96, 64, 32), rates=(3, 2), ru_kernel=7,
                           ru_dilations=(1, 3, 9), out_kernel=7, out_clamp=True)


def wave_weights(seed):
    import numpy as np

    w = codec.random_weights(TINY_WAVE, seed=seed)
    w.out_w = (w.out_w * 0.05).astype(np.float32)  # keep the clamp off its rails so errors show
    return w
