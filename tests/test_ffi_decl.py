"""The three declarations of the C ABI agree: include/tl_hip.h, the Rust extern block a TL
maintainer adds (integration/tl_hip_ffi.rs) and the ctypes binding the tests use
(tl_amd/_lib.py) -- names, arity, and the C type of every parameter and result.  The
IDevice adapters (integration/device_impl.rs) call only declared functions, with the
declared arity.  The same kind of check as the reference's scripts/check_ffi_signatures.py,
which keeps TL's codegen declarations and its runtime's extern "C" functions in step.  CPU only."""
import ctypes as C
import os
import re

import pytest

from tl_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

_BASE = {"float": "f32", "double": "f64", "int": "i32", "int32_t": "i32", "int64_t": "i64", "uint32_t": "u32",
         "uint64_t": "u64", "size_t": "usize", "uint8_t": "u8", "uint16_t": "u16", "char": "c_char",
         "void": "c_void", "tl_hip_tensor": "tl_hip_tensor", "tl_hip_qtensor": "tl_hip_qtensor",
         "tl_hip_llama": "tl_hip_llama", "tl_hip_gguf": "tl_hip_gguf"}
_RUST_SCALARS = {"f32", "f64", "i32", "i64", "u32", "u64", "usize", "u8", "u16", "c_char", "c_void"} | \
    {"tl_hip_tensor", "tl_hip_qtensor", "tl_hip_llama", "tl_hip_gguf"}


def _c_type(t):
    """'const float*' -> ('*const', 'f32'); 'int64_t' -> ('', 'i64')."""
    t = " ".join(t.split())
    const = t.startswith("const ")
    if const:
        t = t[6:]
    stars = t.count("*")
    base = _BASE[t.replace("*", "").strip()]
    assert stars <= 1, t
    return ("*const" if const else "*mut") if stars else "", base


def header_decls():
    src = open(os.path.join(ROOT, "include", "tl_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    out = {}
    for ret, name, args in re.findall(r"([A-Za-z_][A-Za-z0-9_ \*]*?)\b(tl_hip_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", src):
        params = []
        args = " ".join(args.split())
        if args and args != "void":
            for a in args.split(","):
                m = re.match(r"(.*?)([A-Za-z_][A-Za-z0-9_]*)$", a.strip())
                params.append(_c_type(m.group(1)))
        out[name] = (_c_type(ret), params)
    return out


def _rust_type(t):
    t = " ".join(t.split())
    for q in ("*const", "*mut"):
        if t.startswith(q + " "):
            base = t[len(q) + 1:].replace("ffi::", "")
            assert base in _RUST_SCALARS, t
            return q, base
    assert t in _RUST_SCALARS, t
    return "", t


def rust_decls():
    src = open(os.path.join(ROOT, "integration", "tl_hip_ffi.rs")).read()
    block = src[src.index('extern "C" {'):]
    out = {}
    for name, params, ret in re.findall(r"pub fn (\w+)\((.*?)\)\s*(?:->\s*([^;]+?))?\s*;", block, flags=re.S):
        ps = [p.strip() for p in params.split(",") if p.strip()]
        out[name] = (_rust_type(ret) if ret else ("", "c_void"), [_rust_type(p.split(":", 1)[1]) for p in ps])
    return out


def test_rust_extern_block_matches_the_header():
    hd, rs = header_decls(), rust_decls()
    assert len(hd) > 90
    assert sorted(hd) == sorted(rs), f"only in header: {sorted(set(hd) - set(rs))}, only in Rust: {sorted(set(rs) - set(hd))}"
    for name in hd:
        (hret, hps), (rret, rps) = hd[name], rs[name]
        assert len(hps) == len(rps), f"{name}: arity {len(hps)} in the header, {len(rps)} in Rust"
        assert hret == rret, f"{name}: result {hret} vs {rret}"
        for i, (a, b) in enumerate(zip(hps, rps)):
            assert a == b, f"{name}: parameter {i} is {a} in the header, {b} in Rust"


def _balanced_args(src, start):
    depth, i, args, cur = 1, start, [], ""
    while depth:
        ch = src[i]
        if ch == "(":
            depth += 1
        elif ch == ")":
            depth -= 1
            if depth == 0:
                break
        if ch == "," and depth == 1:
            args.append(cur)
            cur = ""
        else:
            cur += ch
        i += 1
    if cur.strip():
        args.append(cur)
    return args


def test_device_adapters_call_declared_functions_with_their_arity():
    rs = rust_decls()
    src = open(os.path.join(ROOT, "integration", "device_impl.rs")).read()
    calls = [(m.group(1), m.end()) for m in re.finditer(r"ffi::(tl_hip_\w+)\(", src)]
    assert len(calls) > 30
    for name, pos in calls:
        assert name in rs, f"device_impl.rs calls undeclared {name}"
        assert len(_balanced_args(src, pos)) == len(rs[name][1]), f"{name}: wrong argument count"
    # the hot-path IDevice methods of the reference (device.rs) are all adapted
    for m in ["tensor_new", "tensor_zeros", "tensor_to_vec_f32", "tensor_release", "tensor_acquire", "tensor_matmul",
              "tensor_transpose_2d", "tensor_matmul_4d", "tensor_rms_norm", "tensor_rope_new_cos",
              "tensor_rope_new_sin", "tensor_apply_rope", "tensor_softmax", "tensor_silu", "tensor_mul",
              "tensor_scale", "tensor_repeat_interleave", "tensor_cat_4d", "tensor_narrow", "tensor_embedding",
              "tensor_scaled_dot_product_attention", "tensor_sample", "tensor_repetition_penalty"]:
        assert re.search(rf"pub fn {m}\(", src), f"IDevice::{m} has no adapter"


# (kind, bytes) of each scalar: ctypes aliases (c_size_t is c_ulong, c_int64 is c_long) are
# told apart only by size and signedness, which is what the ABI fixes
_KIND = {"f32": ("f", 4), "f64": ("f", 8), "i32": ("i", 4), "i64": ("i", 8), "u32": ("u", 4), "u64": ("u", 8),
         "usize": ("u", 8), "u8": ("u", 1), "u16": ("u", 2)}


def _kind(ct):
    if ct in (C.c_float, C.c_double):
        return "f", C.sizeof(ct)
    return ("i" if ct(-1).value < 0 else "u"), C.sizeof(ct)


def _ctypes_ok(ct, want):
    q, base = want
    if ct is None:
        return want == ("", "c_void")
    if ct is C.c_void_p:
        return q != ""
    if ct is C.c_char_p:
        return q != "" and base == "c_char"
    if isinstance(ct, type) and issubclass(ct, C._Pointer):
        return q != "" and base in _KIND and _kind(ct._type_) == _KIND[base]
    return q == "" and base in _KIND and _kind(ct) == _KIND[base]


@pytest.mark.parametrize("name", sorted(header_decls()))
def test_ctypes_prototypes_match_the_header(name):
    ret, params = header_decls()[name]
    res, args = _lib.PROTOS[name]
    assert len(args) == len(params), f"{name}: ctypes arity"
    assert _ctypes_ok(res, ret), f"{name}: ctypes result {res} vs {ret}"
    for i, (ct, want) in enumerate(zip(args, params)):
        assert _ctypes_ok(ct, want), f"{name}: ctypes parameter {i} {ct} vs {want}"
