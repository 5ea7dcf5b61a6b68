"""INTEGRATION.md's Rust `-sys` block declares every function and constant of
include/midman_hip.h with the same arguments (count, order and C type mapped
to the Rust FFI type), so the binding a maintainer copies is complete."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

C_TO_RUST = {"mmh_handle": "mmh_handle", "int32_t": "i32", "uint32_t": "u32",
             "int64_t": "i64", "uint64_t": "u64", "float": "f32", "double": "f64",
             "void": "c_void", "char": "c_char", "uint8_t": "u8"}


def c_type_to_rust(t):
    t = " ".join(t.split())
    if t == "const char *const *":
        return "*const *const c_char"
    const = t.startswith("const ")
    if const:
        t = t[len("const "):]
    stars = t.count("*")
    base = C_TO_RUST[t.replace("*", "").strip()]
    if stars == 0:
        return base
    if stars == 1:
        return ("*const " if const else "*mut ") + base
    assert stars == 2 and not const, t
    return "*mut *mut " + base


def header_functions():
    src = open(os.path.join(ROOT, "include", "midman_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    out = {}
    for ret, name, args in re.findall(
            r"\b(int32_t|uint32_t|const char \*)\s*(mmh_[a-z0-9_]+)\s*\(([^)]*)\);", src):
        types = []
        if args.strip() != "void":
            for a in args.split(","):
                m = re.match(r"(.*?)([A-Za-z_][A-Za-z0-9_]*)(\[\d+\])?$", " ".join(a.split()))
                ty = m.group(1).strip() + (" *" if m.group(3) else "")
                types.append(c_type_to_rust(ty))
        out[name] = types
    return out, dict(re.findall(r"#define (MMH_[A-Z0-9_]+) \(?(-?\d+)u?\)?", src))


def rust_block():
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    m = re.search(r"```rust\n//! Raw bindings.*?```", doc, flags=re.S)
    assert m, "the -sys block is missing"
    block = m.group(0)
    assert "..." not in block, "the block elides declarations"
    fns = {}
    for name, args in re.findall(r"pub fn (mmh_[a-z0-9_]+)\(([^)]*)\)", block, flags=re.S):
        types = [a.split(":", 1)[1].strip() for a in args.split(",") if a.strip()]
        assert name not in fns, f"{name} declared twice"
        fns[name] = types
    consts = dict(re.findall(r"pub const (MMH_[A-Z0-9_]+): [iu]32 = (-?\d+);", block))
    return fns, consts


def test_rust_sys_block_declares_the_whole_header():
    want_fns, want_consts = header_functions()
    got_fns, got_consts = rust_block()
    assert len(want_fns) >= 90
    assert set(got_fns) == set(want_fns), set(got_fns) ^ set(want_fns)
    for name, types in want_fns.items():
        assert got_fns[name] == types, (name, got_fns[name], types)
    assert got_consts == want_consts, set(got_consts.items()) ^ set(want_consts.items())
