"""The Rust binding (crates/headshot-hip) against include/headshot_hip.h, on
the CPU without a Rust toolchain: the `extern "C"` block that links
headshot_hip declares exactly the header's functions with the same
argument count, argument types (C types mapped to their Rust FFI
equivalents) and return types, and every `ffi::hs_*` call in the safe layer
passes as many arguments as the function takes."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "headshot_hip.h")
CRATE = os.path.join(ROOT, "crates", "headshot-hip")
FFI_RS = os.path.join(CRATE, "src", "ffi.rs")
LIB_RS = os.path.join(CRATE, "src", "lib.rs")

# C type (whitespace-normalised) -> Rust FFI type, as ffi.rs documents it
C_TO_RUST = {
    "hs_stream_t": "HsStream",
    "hs_dtype": "HsDtype",
    "hs_status": "HsStatus",
    "int32_t": "i32",
    "int64_t": "i64",
    "float": "f32",
    "const void*": "*const c_void",
    "void*": "*mut c_void",
    "const float*": "*const f32",
    "float*": "*mut f32",
    "const char*": "*const c_char",
    "void": None,  # no return value
}


def _norm_c(t: str) -> str:
    t = re.sub(r"\s+", " ", t.strip())
    return re.sub(r"\s*\*", "*", t)


def header_decls(path=HEADER) -> dict:
    """name -> (return C type, [(arg name, arg C type)])."""
    text = re.sub(r"/\*.*?\*/", "", open(path).read(), flags=re.S)
    text = re.sub(r"#.*", "", text)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(hs_\w+)\s*\(([^)]*)\)\s*;", text):
        ret, name, args = _norm_c(m.group(1)), m.group(2), m.group(3).strip()
        params = []
        if args and args != "void":
            for a in args.split(","):
                a = a.strip()
                pm = re.match(r"(.*?)([A-Za-z_]\w*)$", a)
                params.append((pm.group(2), _norm_c(pm.group(1))))
        out[name] = (ret, params)
    return out


def _extern_block(text: str, link: str) -> str:
    m = re.search(r'#\[link\(name\s*=\s*"%s"\)\]\s*extern\s+"C"\s*\{' % re.escape(link), text)
    assert m, f"no extern block linking {link}"
    depth, i = 1, m.end()
    while depth:
        depth += {"{": 1, "}": -1}.get(text[i], 0)
        i += 1
    return text[m.end():i - 1]


def rust_decls(path=FFI_RS) -> dict:
    """name -> (return Rust type or None, [(arg name, arg Rust type)]) of the
    extern block that links headshot_hip."""
    block = re.sub(r"//[^\n]*", "", _extern_block(open(path).read(), "headshot_hip"))
    out = {}
    for m in re.finditer(r"pub\s+fn\s+(\w+)\s*\(([^)]*)\)\s*(->\s*([^;]+))?;", block):
        name, args, ret = m.group(1), m.group(2).strip(), m.group(4)
        params = []
        for a in filter(None, (x.strip() for x in args.split(","))):
            an, at = a.split(":", 1)
            params.append((an.strip(), re.sub(r"\s+", " ", at.strip())))
        out[name] = (None if ret is None else ret.strip(), params)
    return out


def _call_args(text: str, start: int) -> list:
    """Top-level comma-separated arguments of the call whose '(' is at start."""
    depth, i, args, cur = 0, start, [], ""
    while True:
        c = text[i]
        if c in "([{":
            depth += 1
            if depth > 1:
                cur += c
        elif c in ")]}":
            depth -= 1
            if depth == 0:
                break
            cur += c
        elif c == "," and depth == 1:
            args.append(cur.strip())
            cur = ""
        else:
            cur += c
        i += 1
    if cur.strip():
        args.append(cur.strip())
    return args


@pytest.fixture(scope="module")
def decls():
    return header_decls(), rust_decls()


def test_crate_files_exist():
    for f in ("Cargo.toml", "build.rs", "src/ffi.rs", "src/lib.rs"):
        assert os.path.exists(os.path.join(CRATE, f)), f


def test_same_functions(decls):
    h, r = decls
    assert len(h) >= 29
    assert sorted(r) == sorted(h), (f"only in header: {sorted(set(h) - set(r))}; "
                                    f"only in ffi.rs: {sorted(set(r) - set(h))}")


def test_same_signatures(decls):
    h, r = decls
    for name, (cret, cparams) in h.items():
        rret, rparams = r[name]
        assert C_TO_RUST[cret] == rret, f"{name} returns {cret} in C, {rret} in Rust"
        assert len(cparams) == len(rparams), f"{name}: {len(cparams)} args in C, {len(rparams)}"
        for i, ((cn, ct), (rn, rt)) in enumerate(zip(cparams, rparams)):
            assert C_TO_RUST[ct] == rt, f"{name} arg {i} ({cn}): C {ct} -> {C_TO_RUST[ct]}, Rust {rt}"
            assert cn == rn, f"{name} arg {i}: named {cn} in C, {rn} in Rust"


def test_constants_match_header():
    hdr = open(HEADER).read()
    rs = open(FFI_RS).read()
    consts = dict(re.findall(r"#define (HS_\w+) \(?(-?\d+)\)?", hdr))
    consts.update({m[0]: m[1] for m in re.findall(r"\b(HS_F32|HS_F16) = (\d+)", hdr)})
    for k, v in consts.items():
        m = re.search(r"pub const %s: \w+ = (-?\d+);" % k, rs)
        assert m, f"{k} missing from ffi.rs"
        assert m.group(1) == v, f"{k}: header {v}, Rust {m.group(1)}"


def test_safe_layer_calls_match_arity(decls):
    h, _ = decls
    text = re.sub(r"//[^\n]*", "", open(LIB_RS).read())
    called = set()
    for m in re.finditer(r"ffi::(hs_\w+)\s*\(", text):
        name = m.group(1)
        assert name in h, f"lib.rs calls undeclared {name}"
        args = _call_args(text, m.end() - 1)
        assert len(args) == len(h[name][1]), f"lib.rs: {name} called with {len(args)} args, takes {len(h[name][1])}"
        called.add(name)
    missing = sorted(set(h) - called)
    assert not missing, f"exports with no safe-layer method: {missing}"


def test_parser_catches_a_changed_declaration(tmp_path, decls):
    """The comparison is not vacuous: a dropped argument and a changed type
    in a copy of ffi.rs are both reported."""
    h, _ = decls
    src = open(FFI_RS).read()
    bad = src.replace("rows: i64, dim: i32, eps: f32)", "rows: i64, dim: i32)", 1)
    assert bad != src
    p = tmp_path / "ffi.rs"
    p.write_text(bad)
    r = rust_decls(str(p))
    assert len(r["hs_layernorm"][1]) == len(h["hs_layernorm"][1]) - 1
    bad2 = src.replace("total: i64) -> HsStatus;", "total: i32) -> HsStatus;", 1)
    p.write_text(bad2)
    r2 = rust_decls(str(p))
    diffs = [n for n in h if [C_TO_RUST[t] for _, t in h[n][1]] != [t for _, t in r2[n][1]]]
    assert diffs, "a changed argument type must show"
