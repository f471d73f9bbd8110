"""The safetensors reader (dtts_checkpoint_*, Weights at crates/tts-nn/src/lib.rs:143-360) against
the safetensors package's own writer, on the CPU: names, dtypes, shapes and bytes of every tensor,
metadata skipped, and the errors for damaged files (bad header length, bad JSON, offsets outside
the buffer, sizes that disagree with the shape, unknown dtypes, missing names). The codec model
loader's checks run before any device work, so its refusals of a checkpoint with a missing or
misshapen tensor are tested here too."""
import json
import struct

import numpy as np
import pytest

from dtts import DttsError, checkpoint


def _write_raw(path, header: dict, payload: bytes):
    h = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + payload)


def test_reader_matches_safetensors(tmp_path):
    import torch
    from safetensors.torch import save_file

    rng = np.random.default_rng(0)
    tensors = {
        "a.weight": torch.from_numpy(rng.standard_normal((3, 5, 7)).astype(np.float32)),
        "b.half": torch.from_numpy(rng.standard_normal((11,)).astype(np.float16)),
        "c.bf16": torch.from_numpy(rng.standard_normal((4, 6)).astype(np.float32)).to(torch.bfloat16),
        "d.i64": torch.arange(9, dtype=torch.int64).reshape(3, 3),
        "e.u8": torch.arange(5, dtype=torch.uint8),
        "f.scalar": torch.tensor(2.5, dtype=torch.float64),
        "g.empty": torch.zeros((0, 4), dtype=torch.float32),
        "name \"quoted\" é": torch.ones(2, dtype=torch.float32),
    }
    path = tmp_path / "t.safetensors"
    save_file(tensors, str(path), metadata={"format": "pt", "note": "x"})
    with checkpoint.Checkpoint(path) as ck:
        assert len(ck) == len(tensors)
        assert ck.names() == sorted(tensors)
        codes = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.float64: 3, torch.int64: 4,
                 torch.uint8: 8}
        for name, t in tensors.items():
            info = ck.info(name)
            assert info.name.decode() == name
            assert info.dtype == codes[t.dtype]
            assert info.dims == tuple(t.shape)
            assert info.bytes == t.numel() * t.element_size()
            got = ck.host(name)
            want = t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()
            assert got.shape == tuple(t.shape) and np.array_equal(got, want)
        with pytest.raises(DttsError, match="missing tensor nope"):
            ck.info("nope")
        with pytest.raises(DttsError, match="index 8 outside"):
            ck.info(8)


@pytest.mark.parametrize("case,match", [
    ("short", "not a safetensors file"),
    ("hlen", "exceeds the file"),
    ("json", "header"),
    ("offsets", "outside the 8-byte buffer"),
    ("size", "8 bytes for 4 elements"),
    ("wrap", "shape too large"),          # 2^61 + 1 doubles: numel * 8 wraps to 8 in 64 bits
    ("wrap2", "shape too large"),         # the same count over two dimensions
    ("dtype", "unknown dtype"),
    ("dup", "header"),
    ("missing", "mapping"),
])
def test_reader_refuses_damaged_files(tmp_path, case, match):
    path = tmp_path / "bad.safetensors"
    good = {"x": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}
    if case == "short":
        path.write_bytes(b"\x01\x00")
    elif case == "hlen":
        path.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    elif case == "json":
        h = b'{"x": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]'
        path.write_bytes(struct.pack("<Q", len(h)) + h + bytes(8))
    elif case == "offsets":
        _write_raw(path, {"x": {"dtype": "F32", "shape": [2], "data_offsets": [0, 16]}}, bytes(8))
    elif case == "size":
        _write_raw(path, {"x": {"dtype": "F32", "shape": [4], "data_offsets": [0, 8]}}, bytes(8))
    elif case == "wrap":
        _write_raw(path, {"x": {"dtype": "F64", "shape": [(1 << 61) + 1], "data_offsets": [0, 8]}}, bytes(8))
    elif case == "wrap2":
        _write_raw(path, {"x": {"dtype": "F64", "shape": [(1 << 31), (1 << 30) + 1], "data_offsets": [0, 8]}},
                   bytes(8))
    elif case == "dtype":
        _write_raw(path, {"x": {"dtype": "F33", "shape": [2], "data_offsets": [0, 8]}}, bytes(8))
    elif case == "dup":
        h = b'{"x": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}, "x": {"dtype": "F32", "shape": [2], ' \
            b'"data_offsets": [0, 8]}}'
        path.write_bytes(struct.pack("<Q", len(h)) + h + bytes(8))
        match = "listed twice"
    elif case == "missing":
        path = tmp_path / "absent.safetensors"
    else:
        _write_raw(path, good, bytes(8))
    with pytest.raises(DttsError, match=match):
        checkpoint.Checkpoint(path)


def test_reader_reads_metadata_free_and_empty_headers(tmp_path):
    p = tmp_path / "e.safetensors"
    _write_raw(p, {}, b"")
    with checkpoint.Checkpoint(p) as ck:
        assert len(ck) == 0
    _write_raw(p, {"__metadata__": {"k": "v", "n": "1"}, "y": {"dtype": "I32", "shape": [], "data_offsets": [0, 4]}},
               struct.pack("<i", -7))
    with checkpoint.Checkpoint(p) as ck:
        assert ck.names() == ["y"] and int(ck.host("y")) == -7


def test_model_loader_refuses_missing_and_misshapen_tensors(tmp_path):
    """The loader's checks run before anything touches the device: a checkpoint lacking a tensor,
    or holding one of the wrong shape, is refused with the tensor's name."""
    import _ckpt
    from dtts import codec, codec_front

    T, _, _ = _ckpt.build(_ckpt.TINY_CKPT_FRONT, _ckpt.TINY_WAVE, seed=1)
    name = "decoder.pre_transformer.layers.1.mlp.up_proj.weight"
    t2 = dict(T)
    del t2[name]
    p = tmp_path / "m.safetensors"
    _ckpt.write(p, t2)
    with checkpoint.Checkpoint(p) as ck:
        with pytest.raises(DttsError, match="missing tensor " + name.replace(".", r"\.")):
            checkpoint.CodecModel(ck, _ckpt.TINY_CKPT_FRONT, _ckpt.TINY_WAVE, None)
    t2 = dict(T)
    t2["decoder.decoder.2.block.3.conv1.conv.weight"] = np.zeros((32, 32, 5), np.float32)
    _ckpt.write(p, t2)
    with checkpoint.Checkpoint(p) as ck:
        with pytest.raises(DttsError, match=r"decoder\.decoder\.2\.block\.3\.conv1\.conv\.weight: shape \[32, 32, 5\], "
                                             r"expected \[32, 32, 7\]"):
            checkpoint.CodecModel(ck, _ckpt.TINY_CKPT_FRONT, _ckpt.TINY_WAVE, None)
    bad = codec.Geometry(**{**_ckpt.TINY_WAVE.__dict__, "latent_dim": 32})
    _ckpt.write(p, T)
    with checkpoint.Checkpoint(p) as ck:
        with pytest.raises(DttsError, match="latent"):
            checkpoint.CodecModel(ck, _ckpt.TINY_CKPT_FRONT, bad, None)
    assert isinstance(codec_front.CODEC, codec_front.Geometry)


def test_stack_loader_refuses_missing_qk_norm(tmp_path):
    import _ckpt
    from _stack_ref import SMALL
    from dtts import stack

    layers, fn = stack.random_weights(SMALL, 5)
    T = _ckpt.stack_tensors(SMALL, layers, fn, "talker.model.")
    del T["talker.model.layers.1.self_attn.k_norm.weight"]
    p = tmp_path / "s.safetensors"
    _ckpt.write(p, T)
    with checkpoint.Checkpoint(p) as ck:
        with pytest.raises(DttsError, match=r"missing tensor talker\.model\.layers\.1\.self_attn\.k_norm\.weight"):
            checkpoint.StackModel(ck, "talker.model.", SMALL, None)
        with pytest.raises(DttsError, match=r"missing tensor talker\.code_predictor\.model\.layers\.0"):
            checkpoint.StackModel(ck, "talker.code_predictor.model.", SMALL, None)
