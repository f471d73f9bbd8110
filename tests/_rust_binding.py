"""The Rust declaration a binding crate writes for each C prototype of include/dtts.h.

The type mapping is the one the binding guide uses: pointers stay raw pointers of the element
type (f16 as u16), the library's opaque handles are c_void, descriptor structs go by their
#[repr(C)] names, and `int` is c_int as a return value and i32 as a parameter.
"""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dtts.h")
GUIDE = os.path.join(ROOT, "INTEGRATION.md")

STRUCTS = {
    "dtts_conv_desc": "ConvDesc", "dtts_ru_desc": "RuDesc", "dtts_stack_geometry": "StackGeometry",
    "dtts_stack_layer": "StackLayer", "dtts_stack_cache": "StackCache",
    "dtts_codec_front_geometry": "FrontGeometry", "dtts_codec_front_weights": "FrontWeights",
    "dtts_codec_geometry": "CodecGeometry", "dtts_codec_weights": "CodecWeights",
    "dtts_codec_stage": "CodecStage", "dtts_tensor_info": "TensorInfo",
}
OPAQUE = {"dtts_stack", "dtts_codec_front", "dtts_codec", "dtts_checkpoint", "dtts_codec_model",
          "dtts_stack_model"}
SCALARS = {"int64_t": "i64", "int32_t": "i32", "int": "i32", "size_t": "usize", "float": "f32",
           "double": "f64", "hipStream_t": "HipStream", "dtts_f16": "u16", "char": "c_char",
           "void": "c_void", "uint8_t": "u8"}


def _rust_type(ctype, ret=False):
    t = " ".join(ctype.replace("*", " * ").split())
    stars = t.count("*")
    base = t.replace("*", "").strip()
    const = base.startswith("const ")
    base = base.replace("const ", "").strip()
    if stars == 0:
        if ret and base == "int":
            return "c_int"
        if ret and base == "void":
            return None
        return SCALARS[base]
    elem = "c_void" if base in OPAQUE else STRUCTS.get(base) or SCALARS[base]
    out = ("*const " if const else "*mut ") + elem
    for _ in range(stars - 1):
        out = "*mut " + out
    return out


def header_prototypes():
    """{name: (rust return type or None, [(param name, rust type)])} for every function."""
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
    src = re.sub(r"//[^\n]*", " ", src)
    src = "\n".join(l for l in src.splitlines() if not l.lstrip().startswith("#"))
    src = src.replace('extern "C" {', " ")
    protos = {}
    for ret, name, args in re.findall(r"([A-Za-z_][\w\s\*]*?)\b(dtts_[a-z0-9_]+)\s*\(([^;{()]*)\)\s*;", src):
        ret = " ".join(ret.split())
        ret = ret.split("}")[-1].strip() if "}" in ret else ret
        params = []
        for a in args.split(","):
            a = " ".join(a.split())
            if a in ("", "void"):
                continue
            m = re.match(r"(.*?)([A-Za-z_]\w*)$", a)
            params.append((m.group(2), _rust_type(m.group(1))))
        protos[name] = (_rust_type(ret, ret=True), params)
    return protos


def rust_decl(name, proto):
    ret, params = proto
    args = ", ".join(f"{n}: {t}" for n, t in params)
    return f"pub fn {name}({args})" + (f" -> {ret}" if ret else "") + ";"


def guide_declarations():
    """{name: [(return type or None, [param types])]} for every `pub fn dtts_*` in the guide."""
    text = open(GUIDE).read()
    out = {}
    for name, args, ret in re.findall(r"pub fn (dtts_[a-z0-9_]+)\s*\(([^)]*)\)\s*(?:->\s*([^;]+))?;", text, flags=re.S):
        types = []
        for a in args.split(","):
            a = " ".join(a.split())
            if a:
                types.append(a.split(":", 1)[1].strip())
        out.setdefault(name, []).append((" ".join(ret.split()) or None if ret else None, types))
    return out
