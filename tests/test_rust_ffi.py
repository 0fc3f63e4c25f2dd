"""The Rust FFI crate (rust/burn_dragon_hip) cannot be compiled here (no Rust
toolchain), so its raw bindings are checked against include/bdh_hip.h as
text: every C function has an extern "C" declaration with the same
parameter names, count and types (int64_t -> i64, int32_t -> i32, float ->
f32, double -> f64, T* -> *mut T, const T* -> *const T, void* -> *mut
c_void), the same return type, and every C struct has a #[repr(C)] Rust
struct with the same fields in the same order and types."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "bdh_hip.h")
FFI = os.path.join(ROOT, "rust", "burn_dragon_hip", "src", "ffi.rs")

SCALARS = {"int64_t": "i64", "int32_t": "i32", "uint64_t": "u64", "uint32_t": "u32",
           "float": "f32", "double": "f64", "char": "c_char", "void": "c_void"}


def c_to_rust(ctype: str) -> str:
    t = " ".join(ctype.replace("*", " * ").split())
    # pointer levels, innermost first: "const float * const *" -> *const *const f32
    parts = t.split("*")
    base = parts[0].split()
    const_base = "const" in base
    name = [w for w in base if w != "const"][0]
    rust = SCALARS.get(name, name)
    if len(parts) == 1:
        return rust
    out = ("*const " if const_base else "*mut ") + rust
    for quals in parts[1:-1]:
        out = ("*const " if "const" in quals.split() else "*mut ") + out
    return out


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    funcs = {}
    for m in re.finditer(r"([\w\s\*]+?)\b(bdh_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        ret = m.group(1).strip().split("\n")[-1].strip()
        params = [] if m.group(3).strip() in ("", "void") else \
            [" ".join(p.split()) for p in m.group(3).split(",")]
        parsed = []
        for p in params:
            mm = re.match(r"(.*?)(\w+)$", p)
            parsed.append((mm.group(2), c_to_rust(mm.group(1))))
        funcs[m.group(2)] = (c_to_rust(ret), parsed)
    return funcs


def header_structs():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"typedef struct\s*\{([^}]*)\}\s*(\w+)\s*;", text):
        fields = []
        for decl in m.group(1).split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            if "*" in decl or decl.startswith("const "):
                mm = re.match(r"(.*?)(\w+)$", decl)  # one pointer field: "const float* name"
                fields.append((mm.group(2), c_to_rust(mm.group(1))))
                continue
            typ, names = decl.split(" ", 1)
            for n in names.split(","):
                fields.append((n.strip(), SCALARS.get(typ, typ)))
        out[m.group(2)] = fields
    return out


def rust_functions():
    text = re.sub(r"//.*", "", open(FFI).read())
    block = text[text.index('extern "C"'):]
    funcs = {}
    for m in re.finditer(r"pub fn (bdh_\w+)\s*\(([^)]*)\)\s*(->\s*([^;]+))?;", block, flags=re.S):
        params = []
        for p in [x for x in m.group(2).split(",") if x.strip()]:
            name, typ = p.split(":", 1)
            params.append((name.strip(), " ".join(typ.split())))
        ret = " ".join(m.group(4).split()) if m.group(4) else "c_void"
        funcs[m.group(1)] = (ret, params)
    return funcs


def rust_structs():
    text = re.sub(r"//.*", "", open(FFI).read())
    out = {}
    for m in re.finditer(r"pub struct (\w+)\s*\{([^}]*)\}", text):
        fields = []
        for f in m.group(2).split(","):
            f = f.strip()
            if not f:
                continue
            name, typ = f.replace("pub ", "").split(":")
            fields.append((name.strip(), typ.strip()))
        out[m.group(1)] = fields
    return out


def test_c_to_rust_type_mapping():
    assert c_to_rust("const float*") == "*const f32"
    assert c_to_rust("float* const*") == "*const *mut f32"
    assert c_to_rust("const float* const*") == "*const *const f32"
    assert c_to_rust("void*") == "*mut c_void"
    assert c_to_rust("int64_t") == "i64"


def test_every_c_function_has_a_matching_rust_declaration():
    c, r = header_functions(), rust_functions()
    assert set(c) == set(r), (set(c) ^ set(r))
    for name, (ret, params) in c.items():
        rret, rparams = r[name]
        assert rret == ret.replace("bdh_status", "i32"), (name, rret, ret)
        assert len(rparams) == len(params), name
        for (cn, ct), (rn, rt) in zip(params, rparams):
            assert cn == rn, (name, cn, rn)
            assert rt == ct, (name, cn, ct, rt)


def test_every_c_struct_has_a_matching_repr_c_struct():
    c, r = header_structs(), rust_structs()
    for name, fields in c.items():
        assert name in r, name
        assert r[name] == fields, (name, r[name], fields)
