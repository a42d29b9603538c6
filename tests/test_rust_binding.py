"""The Rust binding a Langtrain maintainer adds (integration/ltkv-sys) stays in
step with include/ltkv.h: its extern "C" block declares every entry point of
the header and nothing else, each with the header's argument and return types
mapped to Rust's C types, and its constants carry the header's values. (There
is no Rust toolchain here; this parse is the check the crate gets.)"""

from __future__ import annotations

import os
import re

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "ltkv.h")
CRATE = os.path.join(ROOT, "integration", "ltkv-sys")
LIB_RS = os.path.join(CRATE, "src", "lib.rs")

_BASE = {"size_t": "usize", "uint32_t": "u32", "int32_t": "i32", "uint64_t": "u64", "int64_t": "i64",
         "uint16_t": "u16", "int": "c_int", "unsigned": "c_uint", "float": "f32", "void": "c_void",
         "char": "c_char", "ltkv_cache": "ltkv_cache"}


def _c_type(decl: str, has_name: bool = True) -> str | None:
    """Rust spelling of a C parameter or return type ('const uint32_t *seqs'
    -> '*const u32'; arrays decay to pointers; 'void' return -> None)."""
    decl = " ".join(decl.split())
    arr = re.match(r"^(.*?)\s*\[\d*\]$", decl)
    stars = decl.count("*")
    if arr:
        decl, stars = arr.group(1), stars + 1
    words = decl.replace("*", " ").split()
    if has_name:
        words = words[:-1]
    const = words[0] == "const"
    base = _BASE[[w for w in words if w != "const"][0]]
    if stars == 0:
        return None if base == "c_void" else base
    inner = ("*const " if const else "*mut ") + base
    return "*mut " * (stars - 1) + inner


def _header():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"LTKV_API\s+([^;]*?)\b(ltkv_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.S):
        args = [a for a in (x.strip() for x in m.group(3).split(",")) if a and a != "void"]
        out[m.group(2)] = (_c_type(m.group(1), has_name=False), [_c_type(a) for a in args])
    return out, text


def _rust():
    text = open(LIB_RS).read()
    block = re.search(r'extern "C" \{(.*?)\n    \}', text, flags=re.S).group(1)
    block = re.sub(r"//[^\n]*", "", block)
    out = {}
    for m in re.finditer(r"pub fn (\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S):
        args = [" ".join(a.split(":", 1)[1].split()) for a in m.group(2).split(",") if a.strip()]
        ret = " ".join(m.group(3).split()) if m.group(3) else None
        out[m.group(1)] = (ret, args)
    return out, text


def test_crate_files_exist():
    for f in ("Cargo.toml", "build.rs", os.path.join("src", "lib.rs")):
        assert os.path.exists(os.path.join(CRATE, f)), f


def test_extern_block_declares_exactly_the_header():
    h, _ = _header()
    r, _ = _rust()
    assert len(h) >= 40
    assert set(r) == set(h), {"missing in lib.rs": sorted(set(h) - set(r)), "extra": sorted(set(r) - set(h))}


def test_argument_and_return_types_match():
    h, _ = _header()
    r, _ = _rust()
    for name, (ret, args) in h.items():
        rret, rargs = r[name]
        assert rret == ret, f"{name}: returns {rret}, header {ret}"
        assert len(rargs) == len(args), f"{name}: {len(rargs)} arguments, header {len(args)}"
        for i, (a, b) in enumerate(zip(rargs, args)):
            assert a == b, f"{name} argument {i}: {a}, header {b}"


def test_constants_match_the_header():
    _, htext = _header()
    _, rtext = _rust()
    hvals = {}
    for m in re.finditer(r"\b(LTKV_\w+)\s*=\s*(-?\d+)", htext):
        hvals[m.group(1)] = int(m.group(2))
    for m in re.finditer(r"#define\s+(LTKV_\w+)\s+\(?\s*(?:\(size_t\))?\s*\(?(-?\d+)\)?(?:\s*<<\s*(\d+))?", htext):
        hvals[m.group(1)] = int(m.group(2)) << int(m.group(3) or 0)
    for m in re.finditer(r"#define\s+(LTKV_\w+)\s+(\d+)u\b", htext):  # unsigned flags
        hvals[m.group(1)] = int(m.group(2))
    consts = dict((m.group(1), eval(m.group(2))) for m in
                  re.finditer(r"pub const (LTKV_\w+): \w+ = ([^;]+);", rtext))
    assert len(consts) >= 12
    for k, v in consts.items():
        assert k in hvals, k
        assert v == hvals[k], (k, v, hvals[k])


def test_fallible_wrappers_return_results():
    """The safe wrapper returns the library's status as a Result where the
    reference's kv.rs panics or errs: write (kv.rs:123-131), append, rows."""
    _, text = _rust()
    for sig in (r"pub fn write\(&mut self, layer: usize, block: usize, slot: usize, k: &\[f32\], v: &\[f32\]\)"
                r"\s*->\s*anyhow::Result<\(\)>",
                r"pub fn append\(&mut self, seq: u32, pos: usize\)\s*->\s*anyhow::Result<\(usize, usize\)>",
                r"pub fn rows\(&mut self, layer: usize, seq: u32, n: usize\)\s*->\s*anyhow::Result"):
        assert re.search(sig, text), sig
    assert text.count("check(") >= 30
