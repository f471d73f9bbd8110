"""An independent float64 codec stack built from torch's CPU conv1d / conv_transpose1d in
torch's NCL layout and checkpoint parameter layouts (test helper)."""
import numpy as np
import torch
import torch.nn.functional as F


def _snake(x, a, r):
    a = torch.from_numpy(np.asarray(a, np.float64))[None, :, None]
    r = torch.from_numpy(np.asarray(r, np.float64))[None, :, None]
    return x + r * torch.sin(a * x) ** 2


def _causal(x, w, b, dil=1):
    k = w.shape[2]
    return F.conv1d(F.pad(x, ((k - 1) * dil, 0)), torch.from_numpy(w).double(),
                    torch.from_numpy(b).double(), dilation=dil)


def torch_decode(geo, w, latent):
    """latent [frames, dim] -> [frames*hop], float64; tanh, or the clamp for geo.out_clamp."""
    x = torch.from_numpy(np.ascontiguousarray(latent.T)).double()[None]
    x = _causal(x, w.head_w, w.head_b)
    for i, blk in enumerate(w.blocks):
        r = geo.rates[i]
        s = _snake(x, *blk["act"])
        y = F.conv_transpose1d(s, torch.from_numpy(blk["up_w"]).double(),
                               torch.from_numpy(blk["up_b"]).double(), stride=r)
        u = y[:, :, : s.shape[2] * r]  # causal: drop the trailing k - stride
        for j, un in enumerate(blk["units"]):
            h = _causal(_snake(u, *un["act1"]), un["w1"], un["b1"], geo.ru_dilations[j])
            u = u + _causal(_snake(h, *un["act2"]), un["w2"], un["b2"])
        x = u
    y = _causal(_snake(x, *w.out_act), w.out_w, w.out_b)
    if getattr(geo, "out_clamp", False):
        return torch.clamp(y, -1.0, 1.0)[0, 0].numpy()
    return torch.tanh(y)[0, 0].numpy()
