"""The Rust crate's raw binding (rust/mrml-hip/src/ffi.rs) against the C ABI
(include/mrml_hip.h): every declared function is bound, under its symbol, with
the header's parameter and return types mapped one to one.  CPU only (the
image has no Rust toolchain, so this is the crate's build-independent check).
"""

from __future__ import annotations

import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]

# C parameter types (whitespace-normalised, const kept) -> the Rust spelling
_SCALARS = {"int32_t": "i32", "int64_t": "i64", "uint32_t": "u32", "uint64_t": "u64", "uint16_t": "u16",
            "uint8_t": "u8", "size_t": "usize", "float": "f32", "int": "c_int", "char": "c_char", "void": "c_void"}
_HANDLES = {"mrml_hip_ctx": "Ctx", "mrml_hip_gemma2": "Model", "mrml_gguf": "Gguf"}
_STRUCTS = {"mrml_hip_device_info": "MrmlHipDeviceInfo", "mrml_hip_gemma2_config": "MrmlHipGemma2Config",
            "mrml_hip_gemma2_layer": "MrmlHipGemma2Layer", "mrml_hip_sampler": "MrmlHipSampler",
            "mrml_gguf_tensor_info": "MrmlGgufTensorInfo"}


def rust_type(c: str) -> str:
    c = " ".join(c.replace("*", " * ").split())
    stars = c.count("*")
    const = c.startswith("const ")
    base = c.replace("const ", "").replace("*", "").split()[0]
    if base in _HANDLES:  # opaque handles travel as *mut c_void aliases, const or not
        t = _HANDLES[base]
        stars -= 1
    else:
        t = _SCALARS.get(base) or _STRUCTS[base]
        if stars:
            t = ("*const " if const else "*mut ") + t
            stars -= 1
    for _ in range(stars):
        t = "*mut " + t
    return t


def header_prototypes() -> dict:
    s = (ROOT / "include" / "mrml_hip.h").read_text()
    s = re.sub(r"/\*.*?\*/", "", s, flags=re.S)
    out = {}
    for ret, name, args in re.findall(r"\n\s*((?:const\s+)?[a-z_0-9]+\s*\*?\s*)(mrml_(?:hip|gguf)_[a-z0-9_]+)\s*\(([^;]*?)\);",
                                      s, flags=re.S):
        params = []
        a = " ".join(args.split())
        if a not in ("", "void"):
            for p in a.split(","):
                p = p.strip()
                m = re.match(r"(.*?)([A-Za-z_][A-Za-z_0-9]*)$", p)
                params.append(rust_type(m.group(1).strip()))
        out[name] = (params, rust_type(ret.strip()))
    return out


def rust_table() -> dict:
    s = (ROOT / "rust" / "mrml-hip" / "src" / "ffi.rs").read_text()
    body = s[s.index("api! {"):]
    out = {}
    for args, ret, sym in re.findall(r"\w+: fn\((.*?)\) -> (.*?) = \"(mrml_[a-z0-9_]+)\";", body):
        params = [" ".join(a.split()) for a in args.split(",") if a.strip()]
        out[sym] = (params, " ".join(ret.split()))
    return out


def test_every_header_function_is_bound():
    h, r = header_prototypes(), rust_table()
    assert len(h) >= 79
    assert sorted(h) == sorted(r), (sorted(set(h) - set(r)), sorted(set(r) - set(h)))


def test_parameter_and_return_types_match():
    h, r = header_prototypes(), rust_table()
    bad = {n: (h[n], r[n]) for n in h if h[n] != r[n]}
    assert not bad, bad


def test_struct_fields_match_header_order():
    s = (ROOT / "include" / "mrml_hip.h").read_text()
    rs = (ROOT / "rust" / "mrml-hip" / "src" / "ffi.rs").read_text()

    def c_fields(struct: str) -> list[str]:
        body = re.search(r"typedef struct (?:%s )?\{(.*?)\}\s*%s;" % (struct, struct), s, flags=re.S).group(1)
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        names = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            decl = re.sub(r"\[\d+\]", "", decl)
            parts = decl.replace("*", " ").split()
            rest = " ".join(parts[1:]) if parts[0] != "const" else " ".join(parts[2:])
            names += [n.strip() for n in rest.split(",")]
        return names

    def rust_fields(struct: str) -> list[str]:
        body = re.search(r"pub struct %s \{(.*?)\}" % struct, rs, flags=re.S).group(1)
        return re.findall(r"pub (\w+):", body)

    rename = {"type": "type_id"}
    for c, r in _STRUCTS.items():
        assert [rename.get(f, f) for f in c_fields(c)] == rust_fields(r), c


def _call_args(src: str, start: int) -> list[str]:
    """Top-level comma-separated arguments of the call whose '(' is at start."""
    depth, args, cur = 0, [], []
    for ch in src[start:]:
        if ch in "([{":
            depth += 1
            if depth == 1:
                continue
        elif ch in ")]}":
            depth -= 1
            if depth == 0:
                args.append("".join(cur).strip())
                return [a for a in args if a]
        elif ch == "," and depth == 1:
            args.append("".join(cur).strip())
            cur = []
            continue
        cur.append(ch)
    raise AssertionError("unbalanced call")


def test_crate_calls_match_the_table():
    """Every `api.<name>` the crate calls is a field of its api! table, called
    with as many arguments as that entry point takes (the crate is not
    compiled here, so this is its argument-count check)."""
    s = (ROOT / "rust/mrml-hip/src/ffi.rs").read_text()
    body = s[s.index("api! {"):]
    arity = {name: len([a for a in args.split(",") if a.strip()])
             for name, args in re.findall(r"(\w+): fn\((.*?)\) -> .*? = \"mrml_[a-z0-9_]+\";", body)}
    calls = 0
    for path in sorted((ROOT / "rust/mrml-hip/src").glob("*.rs")):
        src = path.read_text()
        for m in re.finditer(r"\bapi\.(\w+)\)\s*\(", src):
            name = m.group(1)
            assert name in arity, f"{path.name}: api.{name} is not in the api! table"
            args = _call_args(src, m.end() - 1)
            assert len(args) == arity[name], f"{path.name}: api.{name} called with {len(args)} arguments, takes {arity[name]}"
            calls += 1
    assert calls > 50
