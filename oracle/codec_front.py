"""CPU oracle of the codec's front half -- TEST INFRASTRUCTURE ONLY.

Restates Codec::forward up to the waveform stack (drmhse/dream-tts crates/qwen3tts/src/
codec.rs:401-424) op by op with the f16 storage points the GPU path keeps (every activation stored
in f16, every op computed in f32 and rounded once):

  q   = Rvq(semantic) + Rvq(acoustic)      lookups summed per stack (codec.rs:296-313), the two
                                           output projections over the stacks' joined width
  h   = pre_conv(q)                        causal, k = 3 (codec.rs:416)
  h   = input_proj(h)                      (codec.rs:418)
  h   = the windowed transformer           per layer (qwen3.rs:339-463): rms_norm, q|k|v, RoPE and
                                           windowed attention (prefill branch, qwen3.rs:420-443),
                                           o_proj * attn_scale + h, rms_norm, gate|up, SiLU*mul,
                                           down * mlp_scale + h; then the final rms_norm (qwen3.rs:466)
  h   = output_proj(h)                     (codec.rs:419)
  per upsampling ratio r (codec.rs:421-423):
      u = TransConv(h)                     kernel = stride = r, one tap over r phases (codec.rs:153-158)
      h = u + gamma * pw2(gelu(pw1(LN(depthwise(u)))))   ConvNext::forward (codec.rs:186-195)
"""
from __future__ import annotations

import numpy as np

from . import (conv1d_nlc_f16, depthwise_layernorm_f16, rms_norm_rows_f16, rope_table_f32,
               rvq_lookup_sum_f16, swiglu_rows_f16, tap_weight_f32, transpose_bias_f32,
               transpose_tap_weight_f32, window_attention_prefill_f16)


def _f16(a):
    return np.ascontiguousarray(np.asarray(a, np.float32).astype(np.float16).view(np.uint16))


def _lin(w_out_in):
    """A Linear's [out, in] weight as the conv oracle's tap layout [1, in, out], f16 bits."""
    return _f16(np.ascontiguousarray(np.asarray(w_out_in, np.float32).T)[None])


def decode_f16(geo, hw, codes):
    """codes [lanes, frames, n_books] int -> latent [lanes, frames * prod(up_ratios), latent] f16 bits."""
    codes = np.ascontiguousarray(codes, np.int32)
    lanes, frames, nb = codes.shape
    s = rvq_lookup_sum_f16(codes.reshape(lanes * frames, nb), hw.codebooks, geo.n_first)
    s = s.reshape(lanes, frames, 2 * geo.book_dim)
    w_out = np.concatenate([hw.out_proj_sem[:, :, 0], hw.out_proj_ac[:, :, 0]], axis=1)
    q = conv1d_nlc_f16(s, _lin(w_out), None, 1)
    h = conv1d_nlc_f16(q, _f16(tap_weight_f32(hw.pre_w)), _f16(hw.pre_b), 1)
    h = conv1d_nlc_f16(h, _lin(hw.in_w), _f16(hw.in_b), 1)
    cos_t, sin_t = rope_table_f32(max(frames, 1), geo.tf_head_dim, geo.tf_rope_base)
    scale = np.float32(1.0 / np.sqrt(np.float64(geo.tf_head_dim)))
    for L in hw.layers:
        a = rms_norm_rows_f16(h, L["attn_norm"], geo.tf_eps)
        qkv = conv1d_nlc_f16(a, _lin(np.concatenate([L["wq"], L["wk"], L["wv"]], 0)), None, 1)
        att = window_attention_prefill_f16(qkv, cos_t, sin_t, geo.tf_heads, geo.tf_n_kv, geo.tf_head_dim,
                                           geo.tf_window, float(scale))
        h = conv1d_nlc_f16(att, _lin(L["wo"]), None, 1, res_bits=h, scale=L["attn_scale"])
        a = rms_norm_rows_f16(h, L["ffn_norm"], geo.tf_eps)
        gu = conv1d_nlc_f16(a, _lin(np.concatenate([L["gate"], L["up"]], 0)), None, 1)
        t = swiglu_rows_f16(gu)
        h = conv1d_nlc_f16(t, _lin(L["down"]), None, 1, res_bits=h, scale=L["mlp_scale"])
    a = rms_norm_rows_f16(h, hw.tf_norm, geo.tf_eps)
    x = conv1d_nlc_f16(a, _lin(hw.out_w), _f16(hw.out_b), 1)
    for i, U in enumerate(hw.up):
        r = geo.up_ratios[i]
        u = conv1d_nlc_f16(x, _f16(transpose_tap_weight_f32(U["up_w"], r)), _f16(transpose_bias_f32(U["up_b"], r)), 1)
        lanes_, length, _ = u.shape
        u = u.reshape(lanes_, length * r, geo.latent_dim)
        dn = depthwise_layernorm_f16(u, U["dw_w"][:, 0, :], U["dw_b"], U["ln_w"], U["ln_b"], geo.ln_eps)
        p = conv1d_nlc_f16(dn, _lin(U["pw1_w"]), _f16(U["pw1_b"]), 1, act="gelu")
        x = conv1d_nlc_f16(p, _lin(U["pw2_w"]), _f16(U["pw2_b"]), 1, res_bits=u, scale=U["gamma"])
    return x


def document_windows(n, chunk, context):
    """Codec::decode's windows (codec.rs:582-603): (from, to, length, drop, keep) per window, in
    frames -- frames[from:to] right-padded with frame to-1 up to `length` (the full span when
    n >= span), of whose forward the audio of frames drop .. drop + keep is kept."""
    out, span, start = [], chunk + context, 0
    while start < n:
        end = min(start + chunk, n)
        frm = max(start - context, 0)
        to = min(frm + span, n)
        length = span if n >= span else to - frm
        out.append((frm, to, length, start - frm, end - start))
        start = end
    return out


def decode_document_f32(front_geo, front_hw, codec_geo, codec_prep, codes, chunk, context, wave="f16"):
    """codes [n, n_books] -> audio [n * samples_per_frame] f32: every window through this module's
    decode_f16 and the waveform oracle, one at a time, the kept audio concatenated. wave "f16":
    oracle.codec.decode_f16 (f16 storage); "f32": oracle.codec.decode_f32_reference on the latent
    widened from f16 (the reference's WAV_DTYPE = F32 stack)."""
    from .codec import decode_f16 as wave_f16
    from .codec import decode_f32_reference as wave_f32
    codes = np.ascontiguousarray(codes, np.int32)
    spf = front_geo.upsample * codec_geo.hop
    parts = []
    for frm, to, length, drop, keep in document_windows(codes.shape[0], chunk, context):
        idx = np.minimum(np.arange(frm, frm + length), to - 1)
        lat = decode_f16(front_geo, front_hw, codes[idx][None])
        if wave == "f32":
            wav = wave_f32(codec_geo, codec_prep, lat[0].view(np.float16).astype(np.float32))
            parts.append(np.asarray(wav[drop * spf:(drop + keep) * spf], np.float32))
            continue
        wav = wave_f16(codec_geo, codec_prep, lat)[0]
        parts.append(wav[drop * spf:(drop + keep) * spf].view(np.float16).astype(np.float32))
    return np.concatenate(parts) if parts else np.zeros(0, np.float32)
