"""Every public struct of include/dtts.h has the same layout in its two bindings.

A probe compiled with gcc against the header prints sizeof and offsetof of every member. The
ctypes mirrors in dream-tts_amd/dtts/ and the Rust #[repr(C)] mirrors in INTEGRATION.md (the
binding a tts-nn maintainer would paste) must name the same members in the same order at the
same offsets with the same total size. A mirror that drops a member (ConvDesc without out_scale,
say) hands the library a short struct whose tail it then reads as pointers.
"""
import ctypes
import os
import re
import subprocess

import pytest

from dtts import checkpoint, codec, codec_front, nlc, stack

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dtts.h")

CTYPES = {
    "dtts_conv_desc": nlc.ConvDesc, "dtts_ru_desc": nlc.RuDesc,
    "dtts_stack_geometry": stack._Geometry, "dtts_stack_layer": stack._Layer, "dtts_stack_cache": stack._Cache,
    "dtts_codec_front_geometry": codec_front._Geometry, "dtts_codec_front_layer": codec_front._Layer,
    "dtts_codec_front_up": codec_front._Up, "dtts_codec_front_weights": codec_front._Weights,
    "dtts_codec_geometry": codec._Geometry, "dtts_codec_unit": codec._Unit, "dtts_codec_block": codec._Block,
    "dtts_codec_weights": codec._Weights, "dtts_codec_stage": codec._Stage, "dtts_tensor_info": checkpoint.TensorInfo,
}
RUST = {
    "dtts_conv_desc": "ConvDesc", "dtts_ru_desc": "RuDesc",
    "dtts_stack_geometry": "StackGeometry", "dtts_stack_layer": "StackLayer", "dtts_stack_cache": "StackCache",
    "dtts_codec_front_geometry": "FrontGeometry", "dtts_codec_front_layer": "FrontLayer",
    "dtts_codec_front_up": "FrontUp", "dtts_codec_front_weights": "FrontWeights",
    "dtts_codec_geometry": "CodecGeometry", "dtts_codec_unit": "CodecUnit", "dtts_codec_block": "CodecBlock",
    "dtts_codec_weights": "CodecWeights", "dtts_codec_stage": "CodecStage", "dtts_tensor_info": "TensorInfo",
}


def _strip_c_comments(text):
    return re.sub(r"/\*.*?\*/", "", text, flags=re.S)


def header_structs():
    """{struct: [member, ...]} in declaration order, parsed from the header."""
    text = _strip_c_comments(open(HEADER).read())
    out = {}
    for name, body in re.findall(r"typedef struct (\w+)\s*\{(.*?)\}\s*\1\s*;", text, flags=re.S):
        members = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            for piece in decl.split(","):
                m = re.search(r"(\w+)\s*(\[[^\]]*\])?\s*$", piece.strip())
                assert m, f"{name}: cannot parse {piece!r}"
                members.append(m.group(1))
        out[name] = members
    return out


@pytest.fixture(scope="module")
def c_layout(tmp_path_factory):
    """{struct: (sizeof, [(member, offset, size), ...])} from a gcc-compiled probe."""
    structs = header_structs()
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "dtts.h"', "int main(void) {"]
    for s, members in structs.items():
        lines.append(f'  printf("S {s} %zu\\n", sizeof({s}));')
        for m in members:
            lines.append(f'  printf("M {s} {m} %zu %zu\\n", offsetof({s}, {m}), sizeof((({s} *)0)->{m}));')
    lines += ["  return 0;", "}"]
    d = tmp_path_factory.mktemp("abi")
    src, exe = d / "probe.c", d / "probe"
    src.write_text("\n".join(lines) + "\n")
    subprocess.run(["gcc", "-std=c11", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"),
                    "-I", "/opt/rocm/include", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    layout = {}
    for line in out.splitlines():
        f = line.split()
        if f[0] == "S":
            layout[f[1]] = (int(f[2]), [])
        else:
            layout[f[1]][1].append((f[2], int(f[3]), int(f[4])))
    return layout


def test_every_public_struct_has_both_mirrors():
    structs = set(header_structs())
    assert structs == set(CTYPES) == set(RUST), (structs ^ set(CTYPES), structs ^ set(RUST))


@pytest.mark.parametrize("name", sorted(CTYPES))
def test_ctypes_mirror_matches_header(c_layout, name):
    size, members = c_layout[name]
    cls = CTYPES[name]
    assert [f[0] for f in cls._fields_] == [m[0] for m in members], name
    for m, off, sz in members:
        assert (getattr(cls, m).offset, getattr(cls, m).size) == (off, sz), f"{name}.{m}"
    assert ctypes.sizeof(cls) == size, name


# ---------------------------------------------------------------- the Rust mirrors in INTEGRATION.md

_PRIM = {"i64": 8, "u64": 8, "usize": 8, "isize": 8, "f64": 8, "i32": 4, "u32": 4, "f32": 4,
         "c_int": 4, "i16": 2, "u16": 2, "i8": 1, "u8": 1, "c_char": 1}


def rust_structs():
    """{RustName: [(field, type), ...]} from every #[repr(C)] struct in INTEGRATION.md's rust blocks."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```rust\n(.*?)```", text, flags=re.S)
    out = {}
    for b in blocks:
        b = re.sub(r"//[^\n]*", "", b)
        for name, body in re.findall(r"#\[repr\(C\)\]\s*pub struct (\w+)\s*\{(.*?)\}", b, flags=re.S):
            fields, depth, cur = [], 0, ""
            for ch in body:
                if ch == "[":
                    depth += 1
                elif ch == "]":
                    depth -= 1
                if ch == "," and depth == 0:
                    fields.append(cur)
                    cur = ""
                else:
                    cur += ch
            fields.append(cur)
            parsed = []
            for f in fields:
                f = " ".join(f.split())
                if not f:
                    continue
                m = re.fullmatch(r"pub (\w+): (.+)", f)
                assert m, f"{name}: cannot parse field {f!r}"
                parsed.append((m.group(1), m.group(2)))
            assert name not in out, f"{name} defined twice"
            out[name] = parsed
    return out


def _rust_size_align(ty, structs, consts):
    ty = ty.strip()
    if ty.startswith("*const ") or ty.startswith("*mut "):
        return 8, 8
    if ty in _PRIM:
        return _PRIM[ty], _PRIM[ty]
    m = re.fullmatch(r"\[(.+);\s*([\w+ ]+)\]", ty)
    if m:
        n = eval(m.group(2), {}, dict(consts))
        s, a = _rust_size_align(m.group(1), structs, consts)
        return s * n, a
    assert ty in structs, f"unknown Rust type {ty!r}"
    return _rust_layout(ty, structs, consts)[0:2]


def _rust_layout(name, structs, consts):
    off, align, members = 0, 1, []
    for field, ty in structs[name]:
        s, a = _rust_size_align(ty, structs, consts)
        off = (off + a - 1) // a * a
        members.append((field, off, s))
        off += s
        align = max(align, a)
    size = (off + align - 1) // align * align
    return size, align, members


def _rust_consts():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    return dict((n, int(v)) for n, v in re.findall(r"pub const (\w+): usize = (\d+);", text))


@pytest.mark.parametrize("name", sorted(RUST))
def test_rust_mirror_in_integration_guide_matches_header(c_layout, name):
    structs = rust_structs()
    rname = RUST[name]
    assert rname in structs, f"INTEGRATION.md has no #[repr(C)] struct {rname}"
    size, _, members = _rust_layout(rname, structs, _rust_consts())
    want_size, want = c_layout[name]
    assert [m[0] for m in members] == [m[0] for m in want], rname
    assert members == want, rname
    assert size == want_size, rname
