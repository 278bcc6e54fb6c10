"""The Rust feature crate (rust/whisper-tensor-hip) declares the C ABI of
include/wrs_attn.h exactly: the same functions with the same parameter count
and types, the same #[repr(C)] structs and the same status/dtype constants.
No Rust toolchain is needed: both files are parsed as text."""
from __future__ import annotations

import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "wrs_attn.h"
CRATE = ROOT / "rust" / "whisper-tensor-hip"
LIB_RS = CRATE / "src" / "lib.rs"

# C type (whitespace-normalized) -> the Rust type that binds it
C_TO_RUST = {
    "int": "c_int", "int *": "*mut c_int", "void": "()", "size_t": "usize", "int64_t": "i64",
    "float": "f32",
    "const float *": "*const f32", "float *": "*mut f32",
    "const void *": "*const c_void", "void *": "*mut c_void", "void **": "*mut *mut c_void",
    "const char *": "*const c_char",
    "wrs_attn_ctx *": "*mut WrsCtx", "wrs_attn_ctx **": "*mut *mut WrsCtx",
    "wrs_kv *": "*mut WrsKv", "wrs_kv **": "*mut *mut WrsKv",
    "const wrs_layout *": "*const WrsLayout", "const wrs_reserve *": "*const WrsReserve",
    "size_t *": "*mut usize", "const size_t *": "*const usize",
    "const void *const *": "*const *const c_void", "const float *const *": "*const *const f32",
    "void *const *": "*const *mut c_void",
}


def _norm_c(t: str) -> str:
    t = " ".join(t.replace("*", " * ").split())
    t = t.replace("* *", "**").replace("* const *", "*const *")
    return t.replace(" *", " *").strip()


def _c_type(param: str) -> str:
    param = " ".join(param.split())
    m = re.match(r"(.*?)([A-Za-z_][A-Za-z0-9_]*)$", param)
    t = m.group(1) if m else param
    t = t.replace("*", " * ")
    t = " ".join(t.split())
    t = re.sub(r"\* \*", "**", t)
    t = t.replace("* const *", "*const *")
    return t.strip()


def header_functions() -> dict[str, tuple[str, list[str]]]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for ret, name, args in re.findall(
            r"([A-Za-z_][A-Za-z0-9_ \*]*?)\b(wrs_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, re.S):
        params = [] if args.strip() in ("", "void") else [_c_type(p) for p in args.split(",")]
        out[name] = (_c_type(ret + " x"), params)
    return out


def rust_functions() -> dict[str, tuple[str, list[str]]]:
    text = LIB_RS.read_text()
    m = re.search(r'extern\s+"C"\s*\{(.*?)\n    \}', text, re.S)
    assert m, "no extern \"C\" block in the crate"
    block = re.sub(r"//[^\n]*", "", m.group(1))
    out = {}
    for name, args, ret in re.findall(
            r"pub fn (wrs_[a-z0-9_]+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", block, re.S):
        params = []
        for p in args.split(","):
            p = " ".join(p.split())
            if not p:
                continue
            params.append(p.split(":", 1)[1].strip())
        out[name] = ((ret or "()").strip(), params)
    return out


def test_crate_files_exist():
    for f in ("Cargo.toml", "build.rs", "src/lib.rs"):
        assert (CRATE / f).is_file(), f


def test_extern_block_matches_header():
    h, r = header_functions(), rust_functions()
    assert set(h) == set(r), (sorted(set(h) - set(r)), sorted(set(r) - set(h)))
    for name, (cret, cparams) in h.items():
        rret, rparams = r[name]
        assert len(cparams) == len(rparams), f"{name}: arity {len(cparams)} vs {len(rparams)}"
        assert C_TO_RUST[cret] == rret, f"{name}: return {cret!r} vs {rret!r}"
        for i, (ct, rt) in enumerate(zip(cparams, rparams)):
            assert ct in C_TO_RUST, f"{name} arg {i}: unmapped C type {ct!r}"
            assert C_TO_RUST[ct] == rt, f"{name} arg {i}: {ct!r} binds {C_TO_RUST[ct]!r}, not {rt!r}"


def _c_struct(name: str) -> list[tuple[str, str]]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    m = re.search(r"typedef struct " + name + r"\s*\{(.*?)\}\s*" + name + ";", text, re.S)
    assert m, name
    return [(f.split()[-1], " ".join(f.split()[:-1])) for f in
            (x.strip() for x in m.group(1).split(";")) if f]


def _rust_struct(name: str) -> list[tuple[str, str]]:
    m = re.search(r"pub struct " + name + r"\s*\{(.*?)\}", LIB_RS.read_text(), re.S)
    assert m, name
    return [tuple(x.strip() for x in f.replace("pub ", "").split(":")) for f in
            (y.strip() for y in m.group(1).split(",")) if f]


def test_repr_c_structs_match():
    for c_name, r_name in (("wrs_layout", "WrsLayout"), ("wrs_reserve", "WrsReserve")):
        cf, rf = _c_struct(c_name), _rust_struct(r_name)
        assert [n for n, _ in cf] == [n for n, _ in rf], c_name
        for (n, ct), (_, rt) in zip(cf, rf):
            assert C_TO_RUST[ct] == rt, f"{c_name}.{n}: {ct} vs {rt}"
    assert "#[repr(C)]" in LIB_RS.read_text()


def test_constants_match():
    hdr = dict(re.findall(r"#define (WRS_[A-Z0-9_]+) \(?(-?\d+)\)?", HEADER.read_text()))
    rs = dict(re.findall(r"pub const (WRS_[A-Z0-9_]+): c_int = (-?\d+);", LIB_RS.read_text()))
    assert hdr and hdr == rs


def test_crate_passes_the_reference_architecture_gate_by_construction():
    # scripts/check_pure_rust.sh check 3 rejects *-sys and C-builder crates in
    # `cargo tree`; check 4 rejects extern "C" blocks under crates/ src/ tests/
    # examples/ bindings/. The crate has no dependencies, is not a -sys crate,
    # and sits outside those directories.
    cargo = (CRATE / "Cargo.toml").read_text()
    assert re.search(r'^name = "whisper-tensor-hip"$', cargo, re.M)
    deps = cargo.split("[dependencies]", 1)[1].split("[", 1)[0]
    assert not [l for l in deps.splitlines() if l.strip() and not l.strip().startswith("#")]
    assert CRATE.relative_to(ROOT).parts[0] not in ("crates", "src", "tests", "examples",
                                                    "bindings")
