"""CPU: the Rust FFI crate (volta-hip-sys/src/lib.rs) declares exactly the C ABI
of include/volta_hip.h -- same functions in the same order, same parameter
counts and types, same constants.  (cargo is not in this image, so the crate
is checked as source.)"""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "volta_hip.h")
RUST = os.path.join(ROOT, "volta-hip-sys", "src", "lib.rs")

# C parameter type -> Rust FFI type
TYPES = {"int": "c_int", "const void*": "*const c_void", "void*": "*mut c_void", "int64_t": "i64",
         "size_t": "usize", "float": "f32", "const float*": "*const f32", "float*": "*mut f32",
         "void**": "*mut *mut c_void", "int*": "*mut c_int", "const char*": "*const c_char",
         "size_t*": "*mut usize"}


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


# ------------------------------------------------------------------ the safe gpu_* layer
SAFE = os.path.join(ROOT, "volta-hip-sys", "src", "gpu_ops.rs")
REF_GPU_OPS = "/root/reference/src/ops/gpu_ops.rs"

_CONV = ["batch_size", "in_channels", "out_channels", "height", "width", "kernel_h", "kernel_w", "stride_h",
         "stride_w", "pad_h", "pad_w", "h_out", "w_out"]
_COL = ["batch_size", "channels", "height", "width", "kernel_h", "kernel_w", "stride_h", "stride_w", "h_out",
        "w_out"]
# The reference's RawTensor::gpu_* functions on the path (src/ops/gpu_ops.rs, the
# line of each signature), their tensor and dimension parameters in order, and the
# one extern "C" entry each safe body calls.
EXPECTED = {
    "gpu_matmul": (151, ["a", "b"], ["m", "k", "n"], "vh_matmul_alloc"),
    "gpu_matmul_backward_a": (408, ["grad", "b"], ["m", "k", "n"], "vh_matmul_backward_a_alloc"),
    "gpu_matmul_backward_b": (430, ["a", "grad"], ["m", "k", "n"], "vh_matmul_backward_b_alloc"),
    "gpu_im2col": (515, ["input"], _COL, "vh_im2col_alloc"),
    "gpu_col2im": (546, ["col"], _COL, "vh_col2im_alloc"),
    "gpu_direct_conv": (574, ["input", "weight"], _CONV, "vh_direct_conv_alloc"),
    "gpu_igemm": (622, ["input", "weight"], _CONV, "vh_igemm_alloc"),
    "gpu_conv_backward_input": (670, ["out_grad", "weight"], _CONV, "vh_conv_backward_input_alloc"),
    "gpu_conv_backward_weight": (718, ["out_grad", "input"], _CONV, "vh_conv_backward_weight_alloc"),
    "gpu_igemm_backward_input": (766, ["out_grad", "weight"], _CONV, "vh_igemm_backward_input_alloc"),
    "gpu_igemm_backward_weight": (814, ["out_grad", "input"], _CONV, "vh_igemm_backward_weight_alloc"),
}


def _rust_fns(src, prefix):
    """name -> ([(param, type)], return type, body) of every `pub fn` / `pub(crate) fn` named prefix*."""
    out = {}
    for m in re.finditer(r"pub(?:\(crate\))? fn (" + prefix + r"\w*)\s*\((.*?)\)\s*->\s*([^{]+?)\s*\{", src, re.S):
        params, depth, cur = [], 0, ""
        for ch in m.group(2) + ",":  # split at top-level commas (types such as &[(usize, usize)])
            depth += {"(": 1, "[": 1, "<": 1, ")": -1, "]": -1, ">": -1}.get(ch, 0)
            if ch == "," and depth == 0:
                a = " ".join(cur.split())
                if a:
                    name, ty = a.split(":", 1)
                    params.append((name.strip(), ty.strip()))
                cur = ""
            else:
                cur += ch
        # the body: up to the brace that closes the function
        depth, i = 1, m.end()
        while depth:
            depth += {"{": 1, "}": -1}.get(src[i], 0)
            i += 1
        out[m.group(1)] = (params, m.group(3).strip(), src[m.end():i - 1])
    return out


def test_safe_layer_mirrors_reference_signatures():
    src = open(SAFE).read()
    fns = _rust_fns(src, "gpu_")
    for name, (_, tensors, dims, _) in EXPECTED.items():
        assert name in fns, f"{name} has no body in the crate"
        params, ret, _ = fns[name]
        want = [(t, "&DeviceBuffer") for t in tensors] + [(d, "usize") for d in dims]
        assert params == want, f"{name}: {params} vs {want}"
        assert ret == "Option<DeviceBuffer>", f"{name} returns {ret}"
    # the glue entries keep the reference's parameters too
    assert fns["gpu_unary"][0] == [("input", "&DeviceBuffer"), ("op", "&str")]
    assert fns["gpu_unary_backward"][0] == [("out_grad", "&DeviceBuffer"), ("x", "&DeviceBuffer"), ("op", "&str")]
    assert fns["gpu_sum_reduce"][0] == [("data", "&DeviceBuffer")] and fns["gpu_sum_reduce"][1] == "Option<f32>"
    assert fns["gpu_sum_backward"][0] == [("grad", "f32"), ("input_size", "usize")]


def test_safe_bodies_call_one_entry_point_and_map_status_to_none():
    src = open(SAFE).read()
    fns = _rust_fns(src, "gpu_")
    externs = {d[0] for d in rust_decls()}
    for name, (_, _, _, entry) in EXPECTED.items():
        body = fns[name][2]
        called = [c for c in re.findall(r"\b(vh_\w+)\b", body) if c in externs]
        assert called == [entry], f"{name} calls {called}, expected [{entry}]"
        assert "alloc_out(" in body or "conv_call(" in body, name
    # a non-zero status or a null output is None; the buffer frees itself
    alloc_out = re.search(r"fn alloc_out<F>.*?\n\}", src, re.S).group(0)
    assert "status != VH_OK || out.is_null()" in alloc_out and "return None" in alloc_out
    drop = re.search(r"impl Drop for DeviceBuffer \{.*?\n\}", src, re.S).group(0)
    assert "vh_free(self.ptr)" in drop
    assert "pub mod gpu_ops;" in open(RUST).read()


@pytest.mark.skipif(not os.path.exists(REF_GPU_OPS), reason="reference tree not present")
def test_expected_table_matches_reference_source():
    """The embedded table above against the reference's own gpu_ops.rs, when it is present."""
    src = open(REF_GPU_OPS).read()
    fns = _rust_fns(src, "gpu_")
    lines = src.splitlines()
    for name, (line, tensors, dims, _) in EXPECTED.items():
        params, ret, _ = fns[name]
        assert params == [(t, "&Storage") for t in tensors] + [(d, "usize") for d in dims], name
        assert ret == "Option<Storage>", name
        assert f"fn {name}(" in lines[line - 1], f"{name} not at gpu_ops.rs:{line}"
