"""The C ABI as C, and its two bindings against it, on the CPU (no device).

* Every header of include/ compiles alone and together as strict C99
  (gcc -std=c99 -pedantic -Werror -Wall -Wextra), as a C caller such as the
  Rust -sys crate's build or a cgo/N-API binding would compile it.
* A generated C program prints sizeof, alignof and the offsetof of every
  field of every public struct; the Rust crate's #[repr(C)] structs
  (ark_amd/host/ark-opt-sys/src/lib.rs) and the Python ctypes structs
  (ark_amd/_abi.py) must reproduce those layouts field for field (the Rust
  layout is computed by repr(C)'s rules, since no Rust toolchain is here).
* The crate declares exactly the functions of the headers, with the same
  parameter and return types, and the same values for the constants.
"""
import ctypes as C
import os
import re
import subprocess

import pytest

from ark_amd import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")
CRATE = os.path.join(ROOT, "ark_amd", "host", "ark-opt-sys", "src", "lib.rs")
HEADERS = sorted(h for h in os.listdir(INCLUDE) if h.endswith(".h"))
CFLAGS = ["-std=c99", "-pedantic", "-Werror", "-Wall", "-Wextra"]


def _c_text(h):
    t = open(os.path.join(INCLUDE, h)).read()
    return re.sub(r"/\*.*?\*/", " ", t, flags=re.S)


def _c_decl(decl):
    """'const uint16_t *src' -> ('const uint16_t *', 'src')."""
    decl = " ".join(decl.replace("*", " * ").split())
    m = re.match(r"^(.*?)\s*(\w+)$", decl)
    return m.group(1).replace(" *", "*").replace("* ", "*"), m.group(2)


def c_structs():
    """{name: [(ctype, field), ...]} of every typedef struct with a body."""
    out = {}
    for h in HEADERS:
        for m in re.finditer(r"typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*(\w+)\s*;", _c_text(h),
                             flags=re.S):
            assert m.group(1) == m.group(3), m.group(0)
            out[m.group(1)] = [_c_decl(f) for f in m.group(2).split(";") if f.strip()]
    return out


def c_functions():
    """{name: (return ctype, [param ctypes])} of every ark_* prototype."""
    out = {}
    for h in HEADERS:
        for m in re.finditer(r"^\s*((?:const\s+)?\w+\s*\**)\s*(ark_\w+)\s*\(([^)]*)\)\s*;",
                             _c_text(h), flags=re.M | re.S):
            params = " ".join(m.group(3).split())
            types = [] if params == "void" else [_c_decl(p)[0] for p in params.split(",")]
            out[m.group(2)] = (" ".join(m.group(1).split()).replace(" *", "*"), types)
    return out


def c_defines():
    """{name: int value} of every numeric ARK_* macro."""
    out = {}
    for h in HEADERS:
        for m in re.finditer(r"^#define\s+(ARK_\w+)\s+(.+)$", _c_text(h), flags=re.M):
            expr = re.sub(r"(0x[0-9A-Fa-f]+|\d+)(?:ull|ul|u|ll)\b", r"\1", m.group(2)).strip()
            if re.fullmatch(r"[()0-9xA-Fa-f\s<\-]+", expr):
                out[m.group(1)] = int(eval(expr))
    return out


# C scalar types -> the Rust types the crate must use for them
C_TO_RUST = {"uint16_t": "u16", "uint32_t": "u32", "uint64_t": "u64", "int32_t": "i32",
             "int": "c_int", "float": "f32", "double": "f64", "size_t": "usize",
             "char": "c_char", "void": "c_void"}


def rust_type_of_c(ct):
    """'const uint16_t*' -> '*const u16'; 'ark_opt_handle**' -> '*mut *mut ark_opt_handle'."""
    stars = ct.count("*")
    base = ct.replace("*", "").strip()
    const = base.startswith("const ")
    base = base[6:] if const else base
    rt = C_TO_RUST.get(base, base)
    for k in range(stars):
        rt = ("*const " if (const and k == 0) else "*mut ") + rt
    return rt


def _rust_text():
    t = open(CRATE).read()
    return re.sub(r"//[^\n]*", "", t)


def rust_structs():
    out = {}
    for m in re.finditer(r"pub struct (\w+)\s*\{(.*?)\}", _rust_text(), flags=re.S):
        fields = re.findall(r"pub (\w+):\s*([^,]+),", m.group(2))
        if fields:
            out[m.group(1)] = [(" ".join(t.split()), n) for n, t in fields]
    return out


def rust_functions():
    out = {}
    for m in re.finditer(r"pub fn (\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", _rust_text(),
                         flags=re.S):
        args = [a.strip() for a in m.group(2).split(",") if a.strip()]
        types = [" ".join(a.split(":", 1)[1].split()) for a in args]
        out[m.group(1)] = (" ".join((m.group(3) or "()").split()), types)
    return out


def rust_consts():
    out = {}
    for m in re.finditer(r"pub const (ARK_\w+):\s*\w+\s*=\s*([^;]+);", _rust_text()):
        out[m.group(1)] = int(eval(m.group(2).replace("_", "")))
    return out


def _gcc(args, cwd):
    r = subprocess.run(["gcc"] + args, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True)
    assert r.returncode == 0, r.stdout
    return r


@pytest.mark.parametrize("header", HEADERS + ["all"])
def test_headers_compile_as_strict_c99(header, tmp_path):
    incs = HEADERS if header == "all" else [header]
    src = tmp_path / "use.c"
    src.write_text("".join(f'#include "{h}"\n' for h in incs) +
                   "int ark_c_abi_probe(void);\nint ark_c_abi_probe(void) { return 0; }\n")
    _gcc(CFLAGS + ["-I", INCLUDE, "-c", str(src), "-o", str(tmp_path / "use.o")], tmp_path)


@pytest.fixture(scope="module")
def c_layout(tmp_path_factory):
    """{struct: (size, align, [(field, offset, size), ...])} from the C compiler."""
    d = tmp_path_factory.mktemp("layout")
    structs = c_structs()
    lines = ["#include <stdio.h>", "#include <stddef.h>", "#include <stdalign.h>"]
    lines += [f'#include "{h}"' for h in HEADERS]
    lines.append("int main(void) {")
    for s, fields in structs.items():
        lines.append(f'  printf("S {s} %zu %zu\\n", sizeof({s}), alignof({s}));')
        for _, f in fields:
            lines.append(f'  printf("F {s} {f} %zu %zu\\n", offsetof({s}, {f}), '
                         f"sizeof((({s} *)0)->{f}));")
    lines.append("  return 0;\n}")
    (d / "layout.c").write_text("\n".join(lines) + "\n")
    _gcc(["-std=c11", "-Wall", "-Werror", "-I", INCLUDE, "layout.c", "-o", "layout"], d)
    out = {}
    for ln in subprocess.run([str(d / "layout")], stdout=subprocess.PIPE, text=True,
                             check=True).stdout.splitlines():
        k = ln.split()
        if k[0] == "S":
            out[k[1]] = (int(k[2]), int(k[3]), [])
        else:
            out[k[1]][2].append((k[2], int(k[3]), int(k[4])))
    assert set(out) == set(structs) and len(out) >= 9
    return out


RUST_SCALARS = {"u16": 2, "i16": 2, "u32": 4, "i32": 4, "f32": 4, "c_int": 4, "u64": 8,
                "i64": 8, "f64": 8, "usize": 8}


def _rust_layout(name, structs, memo):
    """(size, align, [(field, offset, size)]) by repr(C): fields in order, each
    at the next multiple of its alignment, the size rounded to the largest."""
    if name in memo:
        return memo[name]
    off, align, fields = 0, 1, []
    for t, f in structs[name]:
        if t.startswith("*"):
            sz = al = 8
        elif t in RUST_SCALARS:
            sz = al = RUST_SCALARS[t]
        else:
            sz, al, _ = _rust_layout(t, structs, memo)
        off = (off + al - 1) // al * al
        fields.append((f, off, sz))
        off += sz
        align = max(align, al)
    memo[name] = ((off + align - 1) // align * align, align, fields)
    return memo[name]


def test_rust_struct_layouts_match_c(c_layout):
    public = rust_structs()
    assert set(public) == set(c_layout), (set(public) ^ set(c_layout))
    memo = {}
    cs = c_structs()
    for name, (size, align, fields) in c_layout.items():
        assert _rust_layout(name, public, memo) == (size, align, fields), name
        # and the field types correspond
        for (ct, f), (rt, rf) in zip(cs[name], public[name]):
            assert f == rf and rust_type_of_c(ct) == rt, (name, f, ct, rt)
    opaque = set(re.findall(r"pub struct (\w+)\s*\{\s*_private:", _rust_text()))
    text = "".join(_c_text(h) for h in HEADERS)
    assert opaque == set(re.findall(r"typedef\s+struct\s+(\w+)\s+\1\s*;", text))


def test_ctypes_struct_layouts_match_c(c_layout):
    # ark_opt_struct_sizes order: the first five from ark_opt.h, then the others
    names = ["ark_opt_tensor", "ark_opt_hparams", "ark_opt_state", "ark_opt_step_info",
             "ark_opt_timing", "ark_codec_span", "ark_ckpt_record", "ark_ckpt_info",
             "ark_grad_span"]
    assert set(names) == set(c_layout)
    for cls, name in zip(_abi.ALL_STRUCTS, names):
        size, align, fields = c_layout[name]
        assert C.sizeof(cls) == size and C.alignment(cls) == align, name
        got = [(f, getattr(cls, f).offset, getattr(cls, f).size) for f, _ in cls._fields_]
        assert [(o, s) for _, o, s in got] == [(o, s) for _, o, s in fields], name
        assert [f for f, _, _ in got] == [f for f, _, _ in fields], name


def test_rust_declares_every_function_with_the_c_types():
    cf, rf = c_functions(), rust_functions()
    assert set(cf) == set(rf), (set(cf) - set(rf), set(rf) - set(cf))
    for name, (ret, params) in cf.items():
        rret, rparams = rf[name]
        assert rust_type_of_c(ret) == rret, (name, ret, rret)
        assert [rust_type_of_c(p) for p in params] == rparams, (name, params, rparams)
    # the library exports exactly these (tests/test_abi.py checks the .so side)
    assert len(cf) >= 37


def test_rust_constants_match_c():
    cd, rc = c_defines(), rust_consts()
    # every numeric constant of the headers except the include guards
    want = {k: v for k, v in cd.items() if not k.endswith("_H")}
    assert set(rc) == set(want), (set(rc) ^ set(want))
    for k, v in want.items():
        assert rc[k] == v, (k, rc[k], v)
