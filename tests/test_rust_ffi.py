"""CPU: the Rust FFI crate (volta-hip-sys/src/lib.rs) declares exactly the C ABI
of include/volta_hip.h -- same functions in the same order, same parameter
counts and types, same constants.  (cargo is not in this image, so the crate
is checked as source.)"""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "volta_hip.h")
RUST = os.path.join(ROOT, "volta-hip-sys", "src", "lib.rs")

# C parameter type -> Rust FFI type
TYPES = {"int": "c_int", "const void*": "*const c_void", "void*": "*mut c_void", "int64_t": "i64",
         "size_t": "usize", "float": "f32", "const float*": "*const f32", "float*": "*mut f32",
         "void**": "*mut *mut c_void", "int*": "*mut c_int", "const char*": "*const c_char"}


def header_decls():
    body = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = []
    for ret, name, args in re.findall(r"^\s*(int|const char\*)\s+(vh_\w+)\s*\(([^)]*)\)\s*;", body, re.M):
        types = []
        for a in (x.strip() for x in args.split(",")):
            if not a or a == "void":
                continue
            ty = re.match(r"(.*?)\w+$", " ".join(a.split())).group(1).replace(" *", "*").strip()
            types.append(TYPES[ty])
        out.append((name, "c_int" if ret == "int" else "*const c_char", types))
    return out


def rust_decls():
    src = open(RUST).read()
    block = re.search(r'extern "C" \{(.*?)\n\}', src, re.S).group(1)
    out = []
    for name, args, ret in re.findall(r"pub fn (vh_\w+)\(([^)]*)\)\s*->\s*([^;]+);", block, re.S):
        types = [a.split(":", 1)[1].strip() for a in args.split(",") if a.strip()]
        out.append((name, ret.strip(), types))
    return out


def test_extern_block_matches_header():
    h, r = header_decls(), rust_decls()
    assert [d[0] for d in r] == [d[0] for d in h], "function names / order differ from the header"
    for hd, rd in zip(h, r):
        assert rd == hd, f"{hd[0]}: header {hd[1:]} vs Rust {rd[1:]}"
    assert len(h) >= 50


def test_constants_match_header():
    hdr = open(HEADER).read()
    src = open(RUST).read()
    enum = dict((k, int(v)) for k, v in re.findall(r"(VH_\w+)\s*=\s*(\d+)", hdr))
    enum.update((k, int(v)) for k, v in re.findall(r"#define\s+(VH_(?:UNARY|OPT)_\w+)\s+(\d+)", hdr))
    rust = dict((k, int(v)) for k, v in re.findall(r"pub const (VH_\w+): c_int = (\d+);", src))
    for k, v in rust.items():
        assert enum.get(k) == v, f"{k}: Rust {v}, header {enum.get(k)}"
    for k in ("VH_OK", "VH_ERR_CAPTURE", "VH_ALGO_AUTO", "VH_BF16", "VH_OPT_ADAM"):
        assert k in rust, k
    scratch = re.search(r"#define VH_NOALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << (\d+)\)", hdr)
    rs = re.search(r"VH_NOALLOC_SCRATCH_BYTES: usize = (\d+) << (\d+);", src)
    assert scratch and rs and scratch.groups() == rs.groups()


def test_build_script_uses_the_library_makefile():
    build = open(os.path.join(ROOT, "volta-hip-sys", "build.rs")).read()
    assert '"make"' in build and "csrc" in build and "rustc-link-lib=dylib=volta_hip" in build
    mk = open(os.path.join(ROOT, "volta_amd", "csrc", "Makefile")).read()
    assert "--offload-arch=$(ARCH)" in mk and "ARCH ?= gfx950" in mk
