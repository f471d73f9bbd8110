"""The binding guide against the header: every C prototype of include/dtts.h has a Rust
declaration in INTEGRATION.md, and every declaration there has its prototype's parameter and
return types, in order (a binding with a missing or reordered argument passes the wrong values
through the C ABI without any error). CPU only."""
import _rust_binding as rb


def test_every_prototype_has_a_binding():
    protos = rb.header_prototypes()
    guide = rb.guide_declarations()
    assert len(protos) > 90
    missing = sorted(n for n in protos if n not in guide)
    assert not missing, f"no Rust declaration in INTEGRATION.md for {missing}"


def test_every_binding_matches_its_prototype():
    protos = rb.header_prototypes()
    for name, decls in rb.guide_declarations().items():
        assert name in protos, f"INTEGRATION.md declares {name}, which include/dtts.h does not"
        ret, params = protos[name]
        want = (ret, [t for _, t in params])
        for got in decls:
            assert got == want, f"{name}: INTEGRATION.md has {got}, the header gives {want}"


def test_mapping_reads_pointers_and_handles():
    """The mapping itself on prototypes of each kind: a handle out-parameter, a struct pointer,
    an f16 buffer, a size return and a void return."""
    protos = rb.header_prototypes()
    assert rb.rust_decl("dtts_codec_create", protos["dtts_codec_create"]) == (
        "pub fn dtts_codec_create(geo: *const CodecGeometry, weights: *const CodecWeights, "
        "out: *mut *mut c_void) -> c_int;")
    ret, params = protos["dtts_snake_nlc_f16"]
    assert ret == "c_int" and params[0][1] == "*const u16" and params[3][1] == "*mut u16"
    assert params[-1][1] == "HipStream"
    assert protos["dtts_codec_workspace_bytes"][0] == "usize"
    assert protos["dtts_codec_destroy"] == (None, [("codec", "*mut c_void")])
