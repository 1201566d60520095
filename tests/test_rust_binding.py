"""The Rust crate gemma4-rs_amd/llm-backend-hip against the C declarations it
binds, on the CPU (no Rust toolchain is needed; the checks read the sources):

- its `extern "C"` block declares every function of include/g4attn.h, and
  nothing else under the g4_ prefix, with each parameter's Rust type the one
  the C type maps to (pointer constness included) and the same return type;
- `G4Hparams` has the header struct's fields, in order, with mapped types,
  and the status constants the header enum's values;
- it declares nothing else: device memory comes from the library
  (g4_alloc, g4_copy_*, g4_free), and the build script links libg4attn alone;
- every `ffi::name(...)` call in the crate names a declared function and
  passes its declared number of arguments.
"""
import glob
import os
import re


from rust_binding import (RUST_KEYWORDS, c_to_rust, parse_header, parse_header_enum, parse_header_struct,
                          parse_rust_externs, rust_calls, strip_rust_comments)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "g4attn.h")
CRATE = os.path.join(ROOT, "gemma4-rs_amd", "llm-backend-hip")
FFI = os.path.join(CRATE, "src", "ffi.rs")


def test_mapping_of_c_types():
    assert c_to_rust("const float **") == "*mut *const f32"
    assert c_to_rust("g4_ctx **") == "*mut *mut G4Ctx"
    assert c_to_rust("const g4_kv_cache *") == "*const G4KvCache"
    assert c_to_rust("g4_stream") == "*mut c_void"
    assert c_to_rust("void") == "()"
    assert c_to_rust("const int8_t *") == "*const i8"
    assert c_to_rust("void **") == "*mut *mut c_void"
    assert c_to_rust("const void *") == "*const c_void"


def test_every_header_function_is_bound_with_its_types():
    header = parse_header(HEADER)
    rust = parse_rust_externs(FFI)
    assert len(header) >= 40
    names = [n for n, _, _ in header]
    assert len(set(names)) == len(names)
    for name, ret, params in header:
        assert name in rust, f"{name} is not declared in ffi.rs"
        rret, rparams = rust[name]
        assert rret == c_to_rust(ret), (name, rret, ret)
        assert len(rparams) == len(params), (name, len(rparams), len(params))
        for i, ((ctype, cname), (rname, rtype)) in enumerate(zip(params, rparams)):
            assert rtype == c_to_rust(ctype), (name, i, cname, ctype, rtype)
            assert rname == cname.lower() and rname not in RUST_KEYWORDS, (name, cname, rname)
    extra = sorted(n for n in rust if n.startswith("g4_") and n not in names)
    assert not extra, extra


def test_hparams_struct_and_status_codes():
    text = strip_rust_comments(open(FFI).read())
    body = re.search(r"pub struct G4Hparams \{(.*?)\}", text, flags=re.S).group(1)
    fields = re.findall(r"pub (\w+): ([^,]+),", body)
    header_fields = parse_header_struct(HEADER, "g4_hparams")
    assert [(n, t.strip()) for n, t in fields] == [(n, c_to_rust(t)) for t, n in header_fields]
    assert "#[repr(C)]\n#[derive(Clone, Copy, Debug, PartialEq)]\npub struct G4Hparams" in text
    consts = {k: int(v) for k, v in re.findall(r"pub const (G4_\w+): c_int = (\d+);", text)}
    assert consts == parse_header_enum(HEADER)


def test_the_crate_binds_the_library_alone():
    """No runtime below the C ABI: every extern function is a g4_ entry point
    of the header, and the build script links libg4attn only."""
    rust = parse_rust_externs(FFI)
    assert all(n.startswith("g4_") for n in rust), sorted(n for n in rust if not n.startswith("g4_"))
    build = open(os.path.join(CRATE, "build.rs")).read()
    assert re.findall(r"cargo:rustc-link-lib=dylib=(\w+)", build) == ["g4attn"]


def test_every_ffi_call_in_the_crate_passes_the_declared_arguments():
    rust = parse_rust_externs(FFI)
    calls = []
    for path in sorted(glob.glob(os.path.join(CRATE, "src", "*.rs"))):
        if path == FFI:
            continue
        calls += [(os.path.basename(path), n, k) for n, k in rust_calls(open(path).read())]
    assert len(calls) >= 40
    for path, name, count in calls:
        assert name in rust, (path, name)
        assert count == len(rust[name][1]), (path, name, count, len(rust[name][1]))
    # every entry point of the header has a safe wrapper except the raw
    # scheduling / preparation / two-step-quantized forms listed here
    called = {n for _, n, _ in calls}
    raw_only = {"g4_kv_append", "g4_prefill_schedule", "g4_rms_norm_rows", "g4_rope_neox_rows", "g4_prepare_qkv",
                "g4_decode_step_fused", "g4_last_error", "g4_last_error_fields"}
    missing = sorted(n for n, _, _ in parse_header(HEADER) if n not in called and n not in raw_only)
    assert not missing, missing


def test_crate_layout():
    cargo = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert re.search(r'^name = "llm-backend-hip"$', cargo, flags=re.M)
    assert re.search(r'^links = "g4attn"$', cargo, flags=re.M)
    assert "llm-eng.workspace = true" in cargo
    lib_rs = open(os.path.join(CRATE, "src", "lib.rs")).read()
    for module in ("attention", "device", "error", "ffi", "kv", "matvec", "port"):
        assert f"pub mod {module};" in lib_rs
        assert os.path.exists(os.path.join(CRATE, "src", module + ".rs"))
    port = open(os.path.join(CRATE, "src", "port.rs")).read()
    impl = re.search(r"impl ComputePort for HipPort \{(.*)\n\}", port, flags=re.S).group(1)
    assert re.findall(r"\n    fn (\w+)\(", impl) == ["matmul", "rms_norm", "softmax", "rope", "add"]
    assert "type Buffer = DevBuf;" in impl
