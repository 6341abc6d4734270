"""The Rust crate's extern block (lightx2v-rs_amd/crates/lightx2v-hip/src/
ffi.rs) against the C header (include/lightx2v_hip.h): the same entry
points, each with the same arity, argument kinds (integer width, float,
pointer constness and pointee) and return type; the same enum values and
#[repr(C)] struct fields.  No Rust toolchain is in this image, so this
check is what keeps the binding in step with the ABI; the trait impl
(src/lib.rs) is checked for every required Backend method by name.
"""

import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lightx2v_hip.h")
CRATE = os.path.join(ROOT, "lightx2v-rs_amd", "crates", "lightx2v-hip")

OPAQUE = {"lx2v_hip_ctx": "Ctx", "lx2v_hip_buf": "RawBuf", "lx2v_hip_weight": "RawWeight",
          "lx2v_hip_mask": "RawMask", "lx2v_hip_kv": "RawKv", "lx2v_hip_graph": "RawGraph"}
SCALAR_C = {"int": "int", "size_t": "usize", "float": "f32", "double": "f64", "uint64_t": "u64",
            "uint8_t": "u8", "int8_t": "i8", "char": "char", "void": "void"}
SCALAR_R = {"c_int": "int", "usize": "usize", "c_float": "f32", "f32": "f32", "c_double": "f64", "u64": "u64",
            "u8": "u8", "i8": "i8", "c_char": "char", "c_void": "void"}


def _strip_c_comments(s):
    s = re.sub(r"/\*.*?\*/", " ", s, flags=re.S)
    return re.sub(r"//[^\n]*", " ", s)


def _c_type(t):
    """A C parameter / return type (name removed) as (base, [const flags per pointer level])."""
    t = t.strip()
    stars = t.count("*")
    # constness of the outermost pointee: `const T *` or `T const *`
    const = bool(re.match(r"^const\b", t))
    base = re.sub(r"\bconst\b|\*|\bstruct\b", " ", t).split()
    base = base[0]
    base = OPAQUE.get(base, SCALAR_C.get(base, base))
    # levels: the innermost pointer's constness is `const`; outer levels are mutable
    return base, ["const" if (const and i == stars - 1) else "mut" for i in range(stars)]


def _c_decls():
    text = _strip_c_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"([\w\s\*]+?)\b(lx2v_hip_\w+)\s*\(([^;{]*?)\)\s*;", text, re.S):
        ret, name, args = m.group(1), m.group(2), m.group(3).strip()
        params = []
        if args and args != "void":
            for a in args.split(","):
                a = a.strip()
                # drop the parameter name (the last identifier)
                a = re.sub(r"\b\w+\s*$", "", a) if not a.endswith("*") else a
                params.append(_c_type(a))
        out[name] = (_c_type(ret), params)
    return out


def _r_type(t):
    t = t.strip()
    levels = []
    while t.startswith("*"):
        m = re.match(r"\*(const|mut)\s+(.*)$", t)
        levels.append(m.group(1))
        t = m.group(2).strip()
    base = t.split("::")[-1]
    base = SCALAR_R.get(base, base)
    # Rust lists pointer levels outermost first; the C parse innermost last
    return base, levels


def _r_decls():
    text = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    block = text[text.index('extern "C" {'):]
    out = {}
    for m in re.finditer(r"pub fn (lx2v_hip_\w+)\s*\((.*?)\)\s*->\s*([^;]+);", block, re.S):
        name, args, ret = m.group(1), m.group(2), m.group(3)
        params = [_r_type(a.split(":", 1)[1]) for a in args.split(",") if a.strip()]
        out[name] = (_r_type(ret), params)
    return out


def test_same_entry_points():
    c, r = _c_decls(), _r_decls()
    assert len(c) >= 70
    assert set(c) == set(r), (sorted(set(c) - set(r)), sorted(set(r) - set(c)))


@pytest.mark.parametrize("name", sorted(_c_decls()))
def test_signature(name):
    (cret, cargs), (rret, rargs) = _c_decls()[name], _r_decls()[name]
    assert cret == rret, f"{name}: return {cret} vs {rret}"
    assert len(cargs) == len(rargs), f"{name}: {len(cargs)} C arguments, {len(rargs)} Rust"
    for i, (ca, ra) in enumerate(zip(cargs, rargs)):
        assert ca == ra, f"{name} argument {i}: C {ca} vs Rust {ra}"


def test_enum_values():
    text = _strip_c_comments(open(HEADER).read())
    rs = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    consts = dict((m.group(1), int(m.group(2))) for m in re.finditer(r"pub const (\w+): \w+ = (\d+);", rs))
    seen = 0
    for m in re.finditer(r"\b(LX2V_(\w+))\s*=\s*(\d+)", text):
        name = m.group(2)
        assert consts.get(name) == int(m.group(3)), f"LX2V_{name}"
        seen += 1
    assert seen >= 27
    ver = int(re.search(r"#define LX2V_HIP_ABI_VERSION (\d+)", text).group(1))
    assert consts["ABI_VERSION"] == ver


@pytest.mark.parametrize("cname,rname", [("lx2v_hip_weight_info_t", "lx2v_hip_weight_info_t"),
                                         ("lx2v_hip_norm_t", "lx2v_hip_norm_t"),
                                         ("lx2v_hip_memrope_t", "lx2v_hip_memrope_t")])
def test_struct_fields(cname, rname):
    text = _strip_c_comments(open(HEADER).read())
    body = re.search(r"typedef struct\s*\{([^{}]*)\}\s*" + cname + r"\s*;", text, re.S).group(1)
    cfields = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        m = re.match(r"((?:const\s+)?[\w]+)\s*(.*)$", decl)
        base = m.group(1)
        for v in m.group(2).split(","):
            v = v.strip()
            cfields.append((v.strip("* "), _c_type(base + " " + "*" * v.count("*"))))
    rs = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    rbody = re.search(r"pub struct " + rname + r"\s*\{(.*?)\}", rs, re.S).group(1)
    rfields = [(f.split(":")[0].replace("pub", "").strip(), _r_type(f.split(":", 1)[1]))
               for f in rbody.split(",") if f.strip()]
    assert cfields == rfields


def test_trait_methods_present():
    """Every method of lightx2v_core::backend::Backend without a default
    (crates/lightx2v-core/src/backend.rs:145-307) has an impl, and the
    associated types are set."""
    rs = open(os.path.join(CRATE, "src", "lib.rs")).read()
    impl = rs[rs.index("impl Backend for HipBackend"):]
    required = ["name", "alloc", "upload", "write", "download", "buf_len", "copy", "weight", "weight_q8",
                "weight_q4", "weight_fp8", "sync", "linear", "layer_norm", "residual_norm", "gate_residual",
                "head_split", "attention", "causal_attention", "sparse_prepare", "sparse_attention",
                "kv_cache_new", "kv_cache_append", "kv_cache_put", "kv_cache_len", "kv_cache_temporal",
                "kv_cache_kv", "kv_cache_memrope_update", "patchify", "unpatchify", "dmd_step", "conv2d",
                "tanh_clamp"]
    for m in required:
        assert re.search(r"\bfn " + m + r"\s*\(", impl), m
    for t in ("Buf = HipBuf", "Weight = HipWeight", "KvCache = HipKv", "Sparse = SparseSpec"):
        assert "type " + t in impl, t


def test_every_extern_is_declared_in_the_header_once():
    rs = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    names = re.findall(r"pub fn (lx2v_hip_\w+)", rs)
    assert len(names) == len(set(names))
