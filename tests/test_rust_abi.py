"""The Rust declarations of crates/kapel-hip (src/abi.rs) against the C
header include/kapel_hip.h: the same functions with the same argument and
return types in the same order, the same constants and the same layout of
kh_weight; the device patch applies to the Kapel sources it is written for
only where those sources exist (not on the GPU box).  No Rust toolchain is
needed: both files are parsed as text."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kapel_hip.h")
ABI = os.path.join(ROOT, "crates", "kapel-hip", "src", "abi.rs")

# C type -> Rust type of the FFI.
C_TO_RUST = {
    "uint32_t": "u32", "uint64_t": "u64", "int64_t": "i64", "int": "c_int",
    "const kh_weight *": "*const KhWeight", "const void *": "*const c_void", "void *": "*mut c_void",
    "const char *": "*const c_char", "int8_t *": "*mut i8", "const int8_t *": "*const i8",
    "float *": "*mut f32", "const float *": "*const f32", "int32_t *": "*mut i32",
    "const uint32_t *": "*const u32", "uint8_t *": "*mut u8",
}


def c_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    out = {}
    for m in re.finditer(r"^([a-z_0-9 ]+?\*?)\s*\b(kh_[a-z_0-9]+)\(([^)]*)\);", text, re.M | re.S):
        ret, name, args = m.group(1).strip(), m.group(2), m.group(3)
        params = []
        if args.strip() != "void":
            for a in args.split(","):
                a = " ".join(a.split())
                ty = re.sub(r"\b[a-z_0-9]+$", "", a).strip()
                ty = ty.replace(" *", " *").replace("*", " *").replace("  ", " ").strip()
                ty = re.sub(r"\s+\*", " *", ty)
                params.append(ty)
        out[name] = (re.sub(r"\s+\*", " *", ret.replace("*", " *")).strip(), params)
    return out


def rust_functions():
    text = open(ABI).read()
    body = text[text.index("unsafe extern \"C\" {"):]
    out = {}
    for m in re.finditer(r"pub fn (kh_[a-z_0-9]+)\(([^)]*)\)\s*(?:->\s*([^;]+))?;", body, re.S):
        name, args, ret = m.group(1), m.group(2), (m.group(3) or "()").strip()
        params = []
        for a in args.split(","):
            a = " ".join(a.split())
            if not a:
                continue
            params.append(a.split(":", 1)[1].strip())
        out[name] = (ret, params)
    return out


def test_the_same_functions_with_the_same_types():
    c, r = c_functions(), rust_functions()
    assert len(c) >= 14
    assert sorted(c) == sorted(r)
    for name, (ret, params) in c.items():
        rret, rparams = r[name]
        assert C_TO_RUST[ret] == rret, (name, ret, rret)
        assert [C_TO_RUST[p] for p in params] == rparams, (name, params, rparams)


def test_the_same_constants():
    header = re.sub(r"/\*.*?\*/", " ", open(HEADER).read(), flags=re.S)
    c = {m.group(1): int(m.group(2)) for m in re.finditer(r"#define (KH_[A-Z0-9_]+) \(?(\d+)u?", header)}
    c["KH_STATIC_SCRATCH_BYTES"] = 32 << 20
    rust = open(ABI).read()
    r = {}
    for m in re.finditer(r"pub const (KH_[A-Z0-9_]+): [a-z_0-9]+ = ([0-9 <]+);", rust):
        r[m.group(1)] = eval(m.group(2))  # literals and a shift only
    assert sorted(c) == sorted(r)
    for name, value in c.items():
        assert r[name] == value, name


def test_the_weight_struct_has_the_same_layout():
    header = open(HEADER).read()
    c_fields = re.search(r"typedef struct kh_weight \{(.*?)\} kh_weight;", header, re.S).group(1)
    c_fields = [(m.group(2), m.group(1)) for m in re.finditer(r"^\s*([a-z_0-9 ]+?\*?)\s*\b([a-z]+);", c_fields, re.M)]
    rust = open(ABI).read()
    r_block = re.search(r"#\[repr\(C\)\][^{]*pub struct KhWeight \{(.*?)\}", rust, re.S).group(1)
    r_fields = re.findall(r"pub ([a-z]+): ([^,]+),", r_block)
    assert [f for f, _ in c_fields] == [f for f, _ in r_fields]
    types = {"uint32_t": "u32", "uint64_t": "u64", "const void *": "*const c_void"}
    for (cf, ct), (rf, rt) in zip(c_fields, r_fields):
        ct = re.sub(r"\s*\*", " *", ct).strip()
        assert types[ct] == rt.strip(), cf


def test_the_crate_declares_the_backend_of_the_catalogue():
    lib = open(os.path.join(ROOT, "crates", "kapel-hip", "src", "backend.rs")).read()
    for trait in ("Run<QuantizedMatmul> for Hip", "Run<ExpertMatmul> for Hip", "Transfer for Hip",
                  "Write for Hip", "Record for Hip", "Recurrent for Hip", "Update for Hip",
                  "impl Storage for HipStorage"):
        assert trait in lib, trait
    # Every operation of kapel_ops::Backend (crates/kapel-ops/src/lib.rs:165-197)
    # other than the two products runs on the host.
    ops = ["Unary", "Glu", "Binary", "Affine", "Cast", "Contiguous", "Concat", "Matmul", "Sum",
           "Mean", "Max", "ArgMax", "Softmax", "LogSoftmax", "CrossEntropy", "LayerNorm",
           "RmsNorm", "Attention", "PagedAttention", "Rope", "GatherRows", "ScatterAddRows",
           "TopK", "GatherColumns"]
    hosted = re.search(r"on_the_host!\((.*?)\);", lib, re.S).group(1)
    assert [o.strip() for o in hosted.split(",") if o.strip()] == ops


@pytest.mark.skipif(not os.path.isdir("/root/reference/crates"), reason="the Kapel sources are not here")
def test_the_device_patch_applies_to_kapel():
    import subprocess
    patch = os.path.join(ROOT, "crates", "kapel-hip", "patches", "device-hip.patch")
    r = subprocess.run(["git", "apply", "--check", "-p1", patch], cwd="/root/reference",
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout
