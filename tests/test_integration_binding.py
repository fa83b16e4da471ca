"""The Rust FFI crate a maintainer would add to flour (`rust/flour-hip-sys`: Cargo.toml, build.rs,
src/lib.rs) declares every function exactly as include/flour_hip.h and include/flour_cache.h
do: same names, same number of parameters, same kind of each parameter (pointer, 32-bit int,
64-bit int, size, float) and the same return kind. No Rust toolchain exists here, so this is
what pins the binding to the ABI the library exports.
"""
from __future__ import annotations

import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def _c_decls() -> dict[str, tuple[str, list[str]]]:
    text = ""
    for h in ("flour_hip.h", "flour_cache.h"):
        src = (ROOT / "include" / h).read_text()
        src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
        src = re.sub(r"//[^\n]*", " ", src)
        text += src + "\n"
    out = {}
    pat = re.compile(r"([A-Za-z_][\w\s\*]*?)\b(flour_\w+)\s*\(([^;{]*?)\)\s*;", re.S)
    for ret, name, params in pat.findall(text):
        ps = [p.strip() for p in params.split(",") if p.strip() and p.strip() != "void"]
        out[name] = (_c_kind(ret.strip() + " _"), [_c_kind(p) for p in ps])
    return out


def _c_kind(decl: str) -> str:
    t = " ".join(decl.split())
    if "*" in t:
        return "ptr"
    t = t.rsplit(" ", 1)[0]  # drop the parameter name
    t = t.replace("const ", "")
    return {"int": "i32", "int32_t": "i32", "uint32_t": "i32", "int64_t": "i64",
            "size_t": "usize", "float": "f32", "void": "void"}[t]


def _rust_kind(ty: str) -> str:
    t = ty.strip()
    if t.startswith("*"):
        return "ptr"
    return {"c_int": "i32", "i32": "i32", "u32": "i32", "i64": "i64", "usize": "usize",
            "f32": "f32", "": "void"}[t]


CRATE = ROOT / "rust" / "flour-hip-sys"


def _rust_decls() -> dict[str, tuple[str, list[str]]]:
    src = (CRATE / "src" / "lib.rs").read_text()
    out = {}
    for ext in re.findall(r'extern "C" \{(.*?)\n\}', src, flags=re.S):
        for name, params, ret in re.findall(
                r"fn\s+(flour_\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", ext, flags=re.S):
            ps = [p.split(":", 1)[1] for p in params.split(",") if ":" in p]
            out[name] = (_rust_kind(ret or ""), [_rust_kind(p) for p in ps])
    return out


def test_rust_binding_matches_the_headers():
    c, rust = _c_decls(), _rust_decls()
    assert len(rust) >= 15, sorted(rust)
    for name, (ret, params) in rust.items():
        assert name in c, f"{name}: bound in INTEGRATION.md, not declared in include/"
        c_ret, c_params = c[name]
        assert len(params) == len(c_params), f"{name}: {len(params)} vs {len(c_params)} params"
        assert params == c_params, f"{name}: parameter kinds {params} vs {c_params}"
        assert ret == c_ret, f"{name}: returns {ret} vs {c_ret}"


def test_rust_binding_covers_every_declared_function():
    c, rust = _c_decls(), _rust_decls()
    missing = sorted(n for n in c if n not in rust)
    assert not missing, f"header functions without a Rust declaration: {missing}"


def test_crate_builds_the_library_from_this_repository():
    cargo = (CRATE / "Cargo.toml").read_text()
    assert 'name = "flour-hip-sys"' in cargo and 'links = "flour_hip"' in cargo
    build = (CRATE / "build.rs").read_text()
    assert '"flour_amd.build"' in build and "rustc-link-lib=dylib=flour_hip" in build
    # the package path build.rs resolves by default is this repository's root
    assert (CRATE / "../.." / "flour_amd" / "build.py").resolve().is_file()
