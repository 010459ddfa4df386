"""The Rust shim source (rust/src/hip/ffi.rs, mod.rs) against the C header.

No Rust toolchain exists here, so the shim is checked as text: ffi.rs
declares every function of include/rustllm_hip.h with the same argument
names, count and C-equivalent types, the status constants carry the header's
values, and the #[repr(C)] structs list the header's fields in order.
mod.rs maps every status code to its TinyError variant (src/error.rs:4-43),
rebuilding the three data-carrying variants from rl_last_error_payload.
"""

import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rustllm_hip.h")
FFI = os.path.join(ROOT, "rust", "src", "hip", "ffi.rs")
MOD = os.path.join(ROOT, "rust", "src", "hip", "mod.rs")

SCALARS = {"uint64_t": "u64", "uint32_t": "u32", "int32_t": "i32", "float": "f32",
           "rl_status": "rl_status", "char": "c_char", "void": "c_void"}


def c_to_rust(ctype: str) -> str:
    """The Rust spelling of a C parameter type (const T* -> *const T, T** -> *mut *mut T)."""
    t = " ".join(ctype.split())
    const = t.startswith("const ")
    if const:
        t = t[len("const "):]
    stars = t.count("*")
    base = SCALARS.get(t.replace("*", "").strip(), t.replace("*", "").strip())
    for i in range(stars):
        base = ("*const " if const and i == 0 else "*mut ") + base
    return base


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for ret, name, args in re.findall(
            r"^(rl_status|void|const char\*|int32_t|uint64_t|void\*)\s+(rl_[a-z0-9_]+)\s*\(([^;]*?)\);",
            text, flags=re.M | re.S):
        params = []
        args = " ".join(args.split())
        if args != "void":
            for a in args.split(","):
                m = re.match(r"(.*?)([A-Za-z_][A-Za-z0-9_]*)$", a.strip())
                params.append((m.group(2), c_to_rust(m.group(1))))
        out[name] = (params, None if ret == "void" else c_to_rust(ret))
    return out


def rust_functions():
    text = open(FFI).read()
    block = text.split('extern "C" {', 1)[1]
    out = {}
    for name, args, ret in re.findall(r"pub fn (rl_[a-z0-9_]+)\((.*?)\)\s*(?:->\s*([^;]+))?;",
                                      block, flags=re.S):
        params = []
        for a in " ".join(args.split()).split(","):
            a = a.strip()
            if a:
                n, t = a.split(":", 1)
                params.append((n.strip(), " ".join(t.split())))
        out[name] = (params, ret.strip() if ret else None)
    return out


def test_ffi_declares_every_header_function_with_its_signature():
    hdr, rs = header_functions(), rust_functions()
    assert len(hdr) >= 70
    assert set(rs) == set(hdr), (set(hdr) ^ set(rs))
    for name, (params, ret) in hdr.items():
        assert rs[name] == (params, ret), f"{name}: {rs[name]} vs {(params, ret)}"


def test_status_constants_match_the_header():
    hdr = dict(re.findall(r"#define (RL_(?:OK|ERR_[A-Z_]+)) (\d+)", open(HEADER).read()))
    rs = dict(re.findall(r"pub const (RL_(?:OK|ERR_[A-Z_]+)): rl_status = (\d+);",
                         open(FFI).read()))
    assert hdr == rs


def struct_fields(text, name, c_style):
    """[(field, Rust type)] of a struct, in order; C array fields T x[N]
    become [T'; N]."""
    if c_style:
        body = re.search(r"typedef struct %s \{(.*?)\}" % name, text, flags=re.S).group(1)
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        out = []
        for ctype, field, dim in re.findall(
                r"([A-Za-z_][A-Za-z0-9_ ]*?\**)\s*([A-Za-z_][A-Za-z0-9_]*)(?:\[([A-Z_0-9]+)\])?;",
                body):
            t = c_to_rust(ctype)
            out.append((field, f"[{t}; {dim}]" if dim else t))
        return out
    body = re.search(r"pub struct %s \{(.*?)\n\}" % name, text, flags=re.S).group(1)
    return [(f, " ".join(t.split())) for f, t in re.findall(r"pub ([a-z_]+): ([^,]+),", body)]


def test_repr_c_structs_follow_the_header_field_order_and_types():
    h, r = open(HEADER).read(), open(FFI).read()
    for name in ("rl_buffer", "rl_profile", "rl_error_payload"):
        assert struct_fields(h, name, True) == struct_fields(r, name, False), name
        assert f"#[repr(C)]\npub struct {name}" in r.replace("#[derive", "\n#[derive") or \
            re.search(r"#\[repr\(C\)\][^{]*pub struct %s \{" % name, r), name
    assert "#define RL_ERROR_MAX_RANK 16" in h and "RL_ERROR_MAX_RANK: usize = 16" in r


def test_check_maps_every_status_to_its_tinyerror_variant():
    text = open(MOD).read()
    body = text.split("pub(crate) fn check(", 1)[1].split("\n}\n", 1)[0]
    for code, variant in [("RL_ERR_INVALID_ARGUMENT", "InvalidArgument"),
                          ("RL_ERR_INVALID_SHAPE", "InvalidShape"),
                          ("RL_ERR_SHAPE_MISMATCH", "ShapeMismatch {"),
                          ("RL_ERR_INVALID_DIMENSION", "InvalidDimension"),
                          ("RL_ERR_UNSUPPORTED_DTYPE", "UnsupportedDType"),
                          ("RL_ERR_NON_CONTIGUOUS", "NonContiguousTensor"),
                          ("RL_ERR_POSITION_OUT_OF_RANGE", "PositionOutOfRange {"),
                          ("RL_ERR_MODEL_FORMAT", "ModelFormat"),
                          ("RL_ERR_INVALID_TOKEN_ID", "InvalidTokenId {")]:
        assert re.search(r"%s(?: if has_payload)? => TinyError::%s" % (code, re.escape(variant)),
                         body), code
    assert "rl_last_error_payload" in body
    # RL_ERR_DEVICE (and a data-carrying code without its payload) is the
    # reference's Metal variant: the device error
    assert re.search(r"_ => TinyError::Metal\(message\)", body)
    for field in ("left", "right", "start_pos", "seq_len", "max_seq_len", "token_id",
                  "vocab_size"):
        assert f"{field}:" in body, field


def test_shim_keeps_the_reference_type_names():
    text = open(MOD).read()
    for item in ("pub struct MetalContext", "pub struct MetalBuffer", "pub struct MetalExecution",
                 "pub fn begin_decode_submission_profile", "pub fn take_decode_submission_profile",
                 "pub fn from_slice", "pub fn from_f16_slice", "pub fn empty_with_element_size",
                 "pub fn as_slice", "pub fn as_f16_slice", "pub fn command_buffer",
                 "pub fn finish"):
        assert item in text, item
