"""The two bindings of the C ABI -- the Julia extension (onionop.jl_amd/julia/NNopAMDGPUExt.jl)
and the Python mirror's ctypes table -- against include/onionop.h, without Julia.

Every `ccall` in the extension is parsed and checked against include/onionop.h and the
built library: the symbol is declared and exported; the argument-type tuple has one entry
per C parameter, each of the same ABI class (pointer, int, int64_t, size_t, float); the
return type matches; and each call passes exactly as many arguments as it declares types.
This pins the drop-in binding's calling convention, which no Julia run checks here.
"""
import ctypes
import os
import re

from nnop import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "onionop.h")
JL = os.path.join(ROOT, "onionop.jl_amd", "julia", "NNopAMDGPUExt.jl")


def _c_class(decl):
    decl = decl.strip()
    if "*" in decl:
        return "ptr"
    base = re.sub(r"\b(const|unsigned)\b", "", decl).split()
    t = base[0] if base else ""
    return {"int": "int", "int64_t": "int64", "size_t": "size_t", "float": "float", "void": "void"}[t]


def header_decls():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    text = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("#"))  # preprocessor
    text = re.sub(r"extern\s+\"C\"\s*\{|\benum\b[^;]*;", ";", text)
    decls = {}
    for stmt in text.split(";"):
        m = re.match(r"\s*([\w\s\*]+?)\b(onionop_\w+)\s*\((.*)\)\s*$", stmt, flags=re.S)
        if not m:
            continue
        ret, name, params = m.groups()
        ps = [p for p in (x.strip() for x in params.split(",")) if p]
        if ps == ["void"]:
            ps = []
        # the parameter's type is the declaration without its name
        classes = [_c_class(re.sub(r"\b\w+\s*$", "", p) if not p.strip().endswith("*") else p) for p in ps]
        decls[name] = (_c_class(ret), classes)
    return decls


def _split_top(s):
    """Split s at commas outside (), {} and []."""
    out, depth, cur = [], 0, ""
    for ch in s:
        if ch in "({[":
            depth += 1
        elif ch in ")}]":
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur.strip())
    return out


def _balanced(text, start):
    """The text inside the parenthesis that opens at text[start]."""
    depth = 0
    for i in range(start, len(text)):
        if text[i] == "(":
            depth += 1
        elif text[i] == ")":
            depth -= 1
            if depth == 0:
                return text[start + 1:i]
    raise ValueError("unbalanced")


_JL_CLASS = {"Cint": "int", "Int64": "int64", "Csize_t": "size_t", "Cfloat": "float", "Cvoid": "void",
             "Cstring": "ptr"}


def _jl_class(t):
    t = t.strip()
    return "ptr" if t.startswith("Ptr{") else _JL_CLASS[t]


def julia_ccalls(text=None):
    text = open(JL).read() if text is None else text
    text = re.sub(r"#[^\n]*", "", text)  # comments
    calls = []
    for m in re.finditer(r"ccall\(", text):
        body = _balanced(text, m.end() - 1)
        parts = _split_top(body)
        sym = re.match(r"\(:(\w+),\s*libonionop\)", parts[0])
        assert sym, parts[0]
        types = parts[2].strip()
        assert types.startswith("(") and types.endswith(")"), types
        tlist = _split_top(types[1:-1])
        calls.append((sym.group(1), _jl_class(parts[1]), [_jl_class(t) for t in tlist], parts[3:]))
    return calls


def test_extension_ccalls_match_the_header():
    decls = header_decls()
    calls = julia_ccalls()
    assert len(calls) >= 20
    L = _lib.lib()
    for name, ret, types, args in calls:
        assert name in decls, f"{name}: not declared in include/onionop.h"
        assert hasattr(L, name), f"{name}: not exported by the library"
        cret, cparams = decls[name]
        assert ret == cret or (ret == "ptr" and cret == "ptr"), f"{name}: return {ret} vs {cret}"
        assert types == cparams, f"{name}: argument classes {types} vs header {cparams}"
        assert len(args) == len(types), f"{name}: {len(args)} arguments for {len(types)} types"


def test_extension_binds_every_launcher():
    """Each reference launcher the extension replaces, and the library's extras, are bound."""
    names = {c[0] for c in julia_ccalls()}
    for n in ("onionop_flash_attn_fwd", "onionop_flash_attn_bwd", "onionop_flash_attn_bwd_workspace",
              "onionop_softmax_fwd", "onionop_softmax_bwd", "onionop_softmax_bwd_bwd", "onionop_rms_norm_fwd",
              "onionop_rms_norm_bwd", "onionop_rms_norm_bwd_workspace", "onionop_layer_norm_fwd",
              "onionop_layer_norm_bwd", "onionop_layer_norm_bwd_workspace", "onionop_llama_rope",
              "onionop_device_lds_bytes", "onionop_last_error", "onionop_abi_version",
              "onionop_flash_attn_varlen_fwd", "onionop_flash_attn_varlen_bwd", "onionop_flash_attn_bwd_rope",
              "onionop_flash_attn_varlen_bwd_rope", "onionop_llama_rotary_embedding"):
        assert n in names, f"{n} is not bound by the Julia extension"


def _mismatches(text):
    decls = header_decls()
    return [name for name, ret, types, args in julia_ccalls(text)
            if types != decls[name][1] or len(args) != len(types)]


def test_parser_catches_a_wrong_binding():
    """The checks fail on the extension with an Int64 narrowed to Cint, or with a pointer
    argument dropped from a call and its type tuple."""
    src = open(JL).read()
    assert _mismatches(src) == []
    call = "(Ptr{Cvoid}, Cint, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid}), _stream(), _dt(T), N, M, x, y)"
    assert src.count(call) == 1
    narrowed = src.replace(call, call.replace("Cint, Int64, Int64", "Cint, Cint, Int64"))
    assert _mismatches(narrowed) == ["onionop_softmax_fwd"]
    dropped = src.replace(call, "(Ptr{Cvoid}, Cint, Int64, Int64, Ptr{Cvoid}), _stream(), _dt(T), N, M, x)")
    assert _mismatches(dropped) == ["onionop_softmax_fwd"]
    unbalanced = src.replace(call, "(Ptr{Cvoid}, Cint, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid}), _stream(), _dt(T), N, M, x)")
    assert _mismatches(unbalanced) == ["onionop_softmax_fwd"]


_CT_CLASS = {ctypes.c_void_p: "ptr", ctypes.c_char_p: "ptr", ctypes.c_int: "int", ctypes.c_int64: "int64",
             ctypes.c_size_t: "size_t", ctypes.c_float: "float"}


def _ct_class(t):
    return "ptr" if isinstance(t, type) and issubclass(t, ctypes._Pointer) else _CT_CLASS[t]


def test_python_signatures_match_the_header():
    """The Python mirror's ctypes table (nnop._lib.SIGNATURES) against the header, by the
    same ABI classes: every declared function is there, with its return and argument
    classes."""
    decls = header_decls()
    assert set(_lib.SIGNATURES) == set(decls)
    for name, (res, args) in _lib.SIGNATURES.items():
        cret, cparams = decls[name]
        assert _ct_class(res) == cret, f"{name}: return"
        assert [_ct_class(a) for a in args] == cparams, f"{name}: arguments"
