"""The Rust FFI module INTEGRATION.md ships as text (no Rust toolchain exists
here) against include/qa.h, mechanically:
  * every `#[repr(C)] pub struct qa_*` block: field names in the C struct's
    order, and the offsets and size the Rust repr(C) rules give (computed
    from the field types) equal to offsetof / sizeof from a C program compiled
    from qa.h;
  * every `pub fn qa_*` in the `extern "C"` block: declared in qa.h with the
    same parameter and return types, and every qa.h function is bound;
  * the status-code constants equal qa.h's enum, and `open_towers` maps the
    crate's device policy (`gpu::Backend`, src/gpu.rs:121-153) as
    `load_backend_with_dtype` does (src/align_inference.rs:331-345): `Auto`
    falls back to the CPU towers on QA_EDEVICE / QA_EUNSUPPORTED only, `Gpu`
    returns every error, `Cpu` opens nothing, and every DeviceSelector
    variant (src/gpu.rs:30-51) is handled.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DOC = os.path.join(ROOT, "INTEGRATION.md")
HDR = os.path.join(ROOT, "include", "qa.h")

# Rust type -> (C spelling, size, alignment) on x86-64 / the LP64 ABI
RUST = {"u32": ("uint32_t", 4), "i32": ("int", 4), "c_int": ("int", 4), "f32": ("float", 4),
        "i64": ("int64_t", 8), "u64": ("uint64_t", 8), "usize": ("size_t", 8), "f64": ("double", 8)}


def _rust_c_type(t: str) -> str:
    t = " ".join(t.split())
    m = re.fullmatch(r"\*(const|mut)\s+(.+)", t)
    if m:
        inner = _rust_c_type(m.group(2))
        base = {"c_void": "void", "c_char": "char"}.get(m.group(2), inner)
        return ("const " if m.group(1) == "const" else "") + base + "*" if not inner.endswith("*") \
            else inner + "*"
    if t in RUST:
        return RUST[t][0]
    return t  # a struct name


def _c_norm(t: str) -> str:
    t = " ".join(t.replace("*", " * ").split())
    t = t.replace(" *", "*").replace("* ", "*")
    return {"int32_t": "int"}.get(t, t)


def _rust_structs():
    text = open(DOC).read()
    out = {}
    for m in re.finditer(r"#\[repr\(C\)\]\s*(?:#\[derive\([^)]*\)\]\s*)?pub struct (qa_\w+)\s*\{([^}]*)\}",
                         text):
        fields = re.findall(r"pub\s+(\w+)\s*:\s*([^,]+?)\s*(?:,|$)", m.group(2))
        out[m.group(1)] = [(n, " ".join(t.split())) for n, t in fields]
    return out


def _rust_layout(fields):
    off, offs, align = 0, [], 1
    for _, t in fields:
        size = 8 if t.startswith("*") else RUST[t][1]
        off = (off + size - 1) // size * size
        offs.append(off)
        off += size
        align = max(align, size)
    return offs, (off + align - 1) // align * align


def test_rust_structs_match_the_c_layout():
    if not shutil.which("gcc"):
        pytest.skip("gcc not available")
    structs = {k: v for k, v in _rust_structs().items() if v}  # qa_ctx is opaque
    assert len(structs) >= 12, sorted(structs)
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "qa.h"', "int main(void) {"]
    for cname, fields in structs.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for fname, _ in fields:
            lines.append(f'printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "l.c"), os.path.join(d, "l")
        open(src, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-std=c11", "-I", os.path.dirname(HDR), src, "-o", exe], check=True)
        got = dict(l.rsplit(" ", 1) for l in subprocess.run([exe], capture_output=True, text=True,
                                                            check=True).stdout.splitlines())
    hdr = open(HDR).read()
    for cname, fields in structs.items():
        offs, size = _rust_layout(fields)
        assert int(got[cname]) == size, (cname, size, got[cname])
        for (fname, _), off in zip(fields, offs):
            assert int(got[f"{cname}.{fname}"]) == off, (cname, fname, off)
        # same field order as the C struct
        body = re.search(r"typedef struct " + cname + r"\s*\{(.*?)\}\s*" + cname + ";", hdr, re.S)
        cfields = re.findall(r"(\w+)\s*(?:\[[^\]]*\])?\s*[,;]", re.sub(r"/\*.*?\*/", "", body.group(1),
                                                                      flags=re.S))
        assert cfields == [f for f, _ in fields], (cname, cfields)


def _c_prototypes():
    text = re.sub(r"/\*.*?\*/", "", open(HDR).read(), flags=re.S)
    text = " ".join(text.split())
    out = {}
    for m in re.finditer(r"([\w\s\*]+?)\b(qa_\w+)\s*\(([^()]*)\)\s*;", text):
        ret, name, args = m.group(1).strip(), m.group(2), m.group(3).strip()
        ret = ret.split("}")[-1].split(";")[-1].strip()
        params = [] if args in ("", "void") else [
            _c_norm(re.sub(r"\b\w+$", "", a.strip())) for a in args.split(",")]
        out[name] = (_c_norm(ret), params)
    return out


def _rust_fns():
    text = open(DOC).read()
    block = re.search(r'extern "C" \{(.*?)\n\}', text, re.S).group(1)
    out = {}
    for m in re.finditer(r"pub fn (qa_\w+)\s*\(([^)]*)\)\s*(?:->\s*([^;]+))?;", block):
        args = [a.split(":", 1)[1] for a in m.group(2).split(",") if a.strip()]
        ret = _rust_c_type(m.group(3).strip()) if m.group(3) else "void"
        out[m.group(1)] = (_c_norm(ret), [_c_norm(_rust_c_type(a.strip())) for a in args])
    return out


def test_rust_functions_match_the_c_prototypes():
    c, rust = _c_prototypes(), _rust_fns()
    assert set(rust) == set(c), (sorted(set(c) - set(rust)), sorted(set(rust) - set(c)))
    for name, sig in rust.items():
        assert sig == c[name], (name, sig, c[name])


def _rust_block(text, start):
    """The brace-balanced block that follows `start` in text."""
    i = text.index(start)
    j = text.index("{", i)
    depth = 0
    for k in range(j, len(text)):
        depth += {"{": 1, "}": -1}.get(text[k], 0)
        if depth == 0:
            return text[j + 1:k]
    raise AssertionError(f"unbalanced block after {start}")


def _arm(body, pattern):
    """Text of the match arm starting at `pattern`, up to the next top-level arm."""
    m = re.search(pattern, body)
    assert m, pattern
    rest = body[m.end():]
    nxt = re.search(r"\n        Backend::\w+", rest)
    return rest[:nxt.start()] if nxt else rest


def test_status_constants_match_the_header():
    doc = open(DOC).read()
    rust = {n: int(v) for n, v in re.findall(r"pub const (QA_E\w+|QA_OK): c_int = (-?\d+);", doc)}
    hdr = re.sub(r"/\*.*?\*/", "", open(HDR).read(), flags=re.S)
    c = {n: int(v) for n, v in re.findall(r"\b(QA_E[A-Z]+|QA_OK)\s*=\s*(-?\d+)\s*[,}]", hdr)}
    assert rust == c and len(c) == 5, (rust, c)


def test_backend_policy_binding():
    doc = open(DOC).read()
    body = _rust_block(doc, "pub fn open_towers(")
    cpu = _arm(body, r"Backend::Cpu\s*=>")
    assert "Towers::Cpu" in cpu and "QaGpu" not in cpu
    auto = _arm(body, r"Backend::Auto\s*=>")
    assert "QaGpu::open(" in auto
    fallback = re.search(r"Err\(e\) if (.*?)=>\s*\{(.*?)\n\s*\}", auto, re.S)
    assert fallback, auto
    assert set(re.findall(r"QA_E\w+", fallback.group(1))) == {"QA_EDEVICE", "QA_EUNSUPPORTED"}
    assert "Ok(Towers::Cpu)" in fallback.group(2)
    assert re.search(r"Err\(e\)\s*=>\s*Err\(", auto), "other errors must be returned"
    gpu = _arm(body, r"Backend::Gpu\(sel\)\s*=>")
    assert "Towers::Cpu" not in gpu, "Backend::Gpu never falls back"
    assert "?" in gpu and "QaGpu::open(" in gpu
    # every DeviceSelector variant of src/gpu.rs:30-51 is handled
    for variant in ("Auto", "Runtime", "Cpu", "Index", "Name"):
        assert re.search(r"DeviceSelector::" + variant + r"\b", gpu), variant
