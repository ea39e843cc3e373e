"""The Rust backend files (longctx100m_amd/rust/) against the C ABI they bind.

cargo and rustc are not in this image, so the files are not compiled here.
What can be checked without them is checked: every `extern "C"` function
amd_attn.rs declares exists in include/longctx100m_attn.h with the same
parameter list (count, order, pointer depth and constness, element types),
the `#[repr(C)]` ring descriptor has the header struct's fields in order with
the same widths, and build.rs compiles with the flags of longctx100m_amd/build.py.
Their exact call sequence runs from C in tests/c/abi_ring.c (mode customop3).
"""

import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
RS = (ROOT / "longctx100m_amd" / "rust" / "amd_attn.rs").read_text()
BUILD_RS = (ROOT / "longctx100m_amd" / "rust" / "build.rs").read_text()
HEADER = (ROOT / "include" / "longctx100m_attn.h").read_text()

# element types: Rust name -> C name
ELEM = {"c_void": "void", "f32": "float", "i32": "int32_t", "u32": "uint32_t",
        "i64": "int64_t", "c_char": "char", "LcRingDesc": "lc_ring_desc_t",
        "usize": "size_t"}
C_SYNONYM = {"int": "int32_t"}


def _strip_c_comments(text):
    return re.sub(r"/\*.*?\*/", " ", text, flags=re.S)


def _c_param(p):
    """'const void* const* qs' -> ('void', ('const', 'const')) : element type and,
    per pointer level from the outermost, whether the pointee is const."""
    p = re.sub(r"\b\w+$", "", p.strip()).strip() if re.search(r"[\w\]]\s*$", p) and \
        len(p.replace("*", " ").split()) > 1 else p.strip()
    toks = p.replace("*", " * ").split()
    # C reads right to left: "const void * const *" = pointer to const pointer to const void
    levels = []
    base_const = False
    elem = None
    i = 0
    while i < len(toks):
        t = toks[i]
        if t == "const":
            if elem is None:
                base_const = True
            else:
                levels[-1] = (levels[-1][0], True) if levels else None
        elif t == "*":
            levels.append(("*", False))
        else:
            elem = C_SYNONYM.get(t, t)
        i += 1
    # pointee constness per level: level 0 (innermost pointer) points at elem (base_const),
    # level k points at the pointer of level k-1 (whose const flag says so)
    consts = []
    for k in range(len(levels)):
        consts.append(base_const if k == 0 else levels[k - 1][1])
    return elem, tuple(reversed(consts))


def _rs_param(p):
    """'qs: *const *const c_void' -> ('void', (True, True))."""
    ty = p.split(":", 1)[1].strip()
    consts = []
    while ty.startswith("*"):
        m = re.match(r"\*(const|mut)\s+", ty)
        consts.append(m.group(1) == "const")
        ty = ty[m.end():]
    return ELEM.get(ty.strip(), ty.strip()), tuple(consts)


def _c_decls():
    out = {}
    text = _strip_c_comments(HEADER)
    for m in re.finditer(r"([\w\s\*]+?)\b(lc_\w+)\s*\(([^;{]*?)\)\s*;", text):
        params = [p for p in m.group(3).replace("\n", " ").split(",") if p.strip()]
        if params == ["void"] or [p.strip() for p in params] == ["void"]:
            params = []
        out[m.group(2)] = [_c_param(p) for p in params]
    return out


def _rs_decls():
    block = re.search(r'extern "C" \{(.*?)\n\}', RS, re.S).group(1)
    out = {}
    for m in re.finditer(r"fn (lc_\w+)\((.*?)\)", block, re.S):
        params = [p for p in m.group(2).replace("\n", " ").split(",") if p.strip()]
        out[m.group(1)] = [_rs_param(p) for p in params]
    return out


def test_extern_declarations_match_the_header():
    c, rs = _c_decls(), _rs_decls()
    assert {"lc_ring_fwd_with_stats_host", "lc_ring_bwd_host", "lc_last_error"} <= set(rs)
    for name, params in rs.items():
        assert name in c, f"{name} is not declared in include/longctx100m_attn.h"
        assert params == c[name], (name, params, c[name])


def test_ring_descriptor_layout_matches_the_header():
    rs_body = re.search(r"#\[repr\(C\)\]\s*struct LcRingDesc \{(.*?)\}", RS, re.S).group(1)
    rs_fields = [(n, ELEM[t]) for n, t in re.findall(r"(\w+):\s*(\w+)", rs_body)]
    c_body = re.search(r"typedef struct lc_ring_desc \{(.*?)\} lc_ring_desc_t;",
                       _strip_c_comments(HEADER), re.S).group(1)
    c_fields = [(n, t) for t, n in re.findall(r"(\w+)\s+(\w+);", c_body)]
    assert rs_fields == c_fields


def test_dtype_codes_match_the_header():
    for name in ("LC_DTYPE_F32", "LC_DTYPE_BF16"):
        rs = re.search(rf"const {name}: i32 = (\d+);", RS).group(1)
        c = re.search(rf"{name}\s*=\s*(\d+)", HEADER).group(1)
        assert rs == c


def test_build_rs_uses_the_library_build_flags():
    from longctx100m_amd import build

    flags = re.search(r"cmd\.args\(\[(.*?)\]\)", BUILD_RS, re.S).group(1)
    rs_flags = re.findall(r'"([^"]+)"', flags)
    want = [f for f in build.COMMON_FLAGS if not f.startswith(("-W", "-I"))]
    assert rs_flags == want
    contract_off = set(re.findall(r'name == "([\w.]+)"', BUILD_RS))
    assert contract_off == {k for k, v in build.EXTRA_FLAGS.items() if "-ffp-contract=off" in v}
