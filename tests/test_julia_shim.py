"""The Julia ``ccall`` binding (``qwendecisioncore.jl_amd/julia/amdgpu_hip.jl``)
against the C header it binds (``include/qdc_hip.h``), on the CPU.

Julia is not installed here, so the shim cannot run; what can be checked is the
part that breaks silently when the header changes: every ``ccall`` names a
declared entry point, with the header's return type and exactly its argument
C types in order, and every declared entry point except the benchmark's copy
has a binding.  A pointer must bind with its pointee type (``Ptr{Cvoid}`` for
``void *`` and ``hipStream_t``, ``Ptr{Float32}`` for ``float *`` ...).
"""
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "qdc_hip.h")
SHIM = os.path.join(ROOT, "qwendecisioncore.jl_amd", "julia", "amdgpu_hip.jl")
# the benchmark's ceilings and the row-scale self-checks: no reference counterpart
UNBOUND = {"qdc_copy", "qdc_copy_grid", "qdc_copy_pair", "qdc_copy_rows", "qdc_empty",
           "qdc_row_scale", "qdc_row_scale_check"}

_SCALARS = {"int32_t": "Int32", "int64_t": "Int64", "uint32_t": "UInt32", "float": "Float32",
            "hipStream_t": "Ptr{Cvoid}"}
_POINTEES = {"void": "Cvoid", "float": "Float32", "int32_t": "Int32", "int64_t": "Int64",
             "uint64_t": "UInt64"}


def _strip_comments(text):
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def _julia_type(c_decl: str, is_return: bool = False) -> str:
    """Julia ccall type of one C parameter (name included) or return type."""
    c = " ".join(c_decl.replace("*", " * ").split())
    words = [w for w in c.split() if w != "const"]
    if "*" in words:
        base = words[0]
        if base == "char":
            return "Cstring"
        return f"Ptr{{{_POINTEES[base]}}}"
    base = words[0]
    return _SCALARS[base]


def header_prototypes() -> dict:
    """name -> (return type, [argument types]) in Julia spelling."""
    text = _strip_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"((?:const\s+)?\w+\s*\*?)\s*(qdc_\w+)\s*\(([^)]*)\)\s*;", text, re.S):
        ret, name, params = m.group(1), m.group(2), m.group(3).strip()
        args = [] if params in ("", "void") else [_julia_type(p) for p in params.split(",")]
        out[name] = (_julia_type(ret, True), args)
    return out


def _balanced(text: str, start: int) -> int:
    """Index just past the parenthesis group opening at text[start]."""
    depth = 0
    for i in range(start, len(text)):
        if text[i] in "({":
            depth += 1
        elif text[i] in ")}":
            depth -= 1
            if depth == 0:
                return i + 1
    raise AssertionError("unbalanced parentheses in the shim")


def _split_top(inner: str) -> list:
    parts, depth, cur = [], 0, ""
    for ch in inner:
        if ch in "({":
            depth += 1
        elif ch in ")}":
            depth -= 1
        if ch == "," and depth == 0:
            parts.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        parts.append(cur.strip())
    return parts


def _julia_code(text: str) -> str:
    """The shim without comments and string literals."""
    text = re.sub(r'"(?:\\.|[^"\\])*"', '""', text)
    return re.sub(r"#[^\n]*", "", text)


def shim_ccalls() -> list:
    """(name, return type, [argument types], number of arguments passed)."""
    text = _julia_code(open(SHIM).read())
    calls = []
    for m in re.finditer(r"ccall\(\s*qdc_sym\(:(qdc_\w+)\)\s*,", text):
        close = _balanced(text, m.start() + len("ccall"))
        parts = _split_top(text[m.start() + len("ccall") + 1:close - 1])
        ret, types = parts[1], parts[2]
        assert types.startswith("(") and types.endswith(")"), (m.group(1), types)
        arg_types = _split_top(types[1:-1])
        calls.append((m.group(1), ret, arg_types, len(parts) - 3))
    return calls


def test_header_parses():
    protos = header_prototypes()
    assert len(protos) == 26, sorted(protos)
    assert protos["qdc_version"] == ("Cstring", [])
    assert protos["qdc_check_ids"] == ("Int32", ["Ptr{Int64}", "Int64", "Int64"])


def test_every_ccall_matches_the_header():
    protos = header_prototypes()
    calls = shim_ccalls()
    assert calls
    for name, ret, types, passed in calls:
        assert name in protos, f"{name} is not declared in include/qdc_hip.h"
        want_ret, want_args = protos[name]
        assert ret == want_ret, (name, ret, want_ret)
        assert types == want_args, (name, types, want_args)
        assert passed == len(want_args), (name, passed, len(want_args))


def test_every_entry_point_is_bound_once():
    names = [c[0] for c in shim_ccalls()]
    assert len(names) == len(set(names)), sorted(n for n in names if names.count(n) > 1)
    assert set(names) == set(header_prototypes()) - UNBOUND


def test_shim_brackets_balance():
    text = _julia_code(open(SHIM).read())
    for a, b in ("()", "[]", "{}"):
        assert text.count(a) == text.count(b), (a, b)


@pytest.mark.parametrize("mutation", ["drop", "swap"])
def test_checker_catches_a_changed_signature(mutation, monkeypatch):
    """The comparison fails when the header and a binding disagree."""
    protos = header_prototypes()
    name = "qdc_swiglu"
    ret, args = protos[name]
    # drop the last argument, or swap a pointer with an integer
    changed = args[:-1] if mutation == "drop" else [args[3]] + args[1:3] + [args[0]] + args[4:]
    monkeypatch.setitem(protos, name, (ret, changed))
    monkeypatch.setattr(__import__(__name__), "header_prototypes", lambda: protos)
    with pytest.raises(AssertionError):
        test_every_ccall_matches_the_header()


def _fallbacks(code: str) -> list:
    """Places where an overriding method hands its work to another method of the
    same function instead of the library: ``invoke(...)`` (the generic method)
    and a short-circuit ``|| return QwenDecisionCore.f(...)``."""
    pats = (r"\binvoke\s*\(", r"\|\|\s*return\s+(?:QwenDecisionCore\.)?\w+\s*\(")
    return [code[m.start():m.start() + 60] for p in pats for m in re.finditer(p, code)]


def test_shim_has_no_generic_fallback():
    """No in-scope operator of the shim falls back to a generic AMDGPU.jl method;
    unsupported shapes raise instead."""
    code = _julia_code(open(SHIM).read())
    assert _fallbacks(code) == []
    assert "throw(ArgumentError" in code


@pytest.mark.parametrize("planted", [
    "cfg.key_dim <= 256 || return invoke(QwenDecisionCore.delta_attention,\n"
    "    Tuple{Any,Any,Any,Any}, attention, x, mask, cfg)\n",
    "cfg.key_dim <= 256 || return QwenDecisionCore.delta_attention(attention, x, mask, cfg)\n",
])
def test_fallback_check_catches_a_planted_fallback(planted):
    code = _julia_code(open(SHIM).read() + planted)
    assert _fallbacks(code)


def test_shim_version_is_the_header_version():
    """The shim refuses a library built from another header: its constant must be
    the header's QDC_HIP_VERSION."""
    header = re.search(r'#define\s+QDC_HIP_VERSION\s+"([^"]+)"', open(HEADER).read()).group(1)
    shim = re.search(r'const QDC_HIP_VERSION = "([^"]+)"', open(SHIM).read()).group(1)
    assert shim == header
