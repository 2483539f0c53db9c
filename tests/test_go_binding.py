"""The Go side of the drop-in (ingot_amd/go: the cgo package kernels/rocm and the rocm GPUSession in graph/)
checked against include/ingot_rocm.h on the CPU.

No Go toolchain exists in this image, so the Go sources cannot be compiled here. These checks pin what a
compile against the header would: every C.ingot_rocm_* function they call is declared, with the same number of
arguments; every field of C.ingot_rocm_gemm_args they set exists; the constants they mirror (status codes,
dtypes, activations, C broadcast modes, math types) equal the header's #defines; build tags and the GPUSession
surface of graph/gpu_other.go:13-37 (the stub the rocm files replace) are present.
"""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ingot_rocm.h")
GO = os.path.join(ROOT, "ingot_amd", "go")
BINDING = os.path.join(GO, "kernels", "rocm", "rocm.go")
GRAPH = [os.path.join(GO, "graph", f) for f in ("gpu_rocm.go", "gpuops_rocm.go", "gpuhalf_rocm.go")]


def header_text():
    return re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)


def split_top(s):
    """Splits an argument list at top-level commas."""
    out, depth, cur = [], 0, ""
    for ch in s:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur)
    return [a.strip() for a in out]


def balanced(text, start):
    """The text inside the parentheses opening at text[start]."""
    depth = 0
    for i in range(start, len(text)):
        if text[i] == "(":
            depth += 1
        elif text[i] == ")":
            depth -= 1
            if depth == 0:
                return text[start + 1:i]
    raise ValueError("unbalanced")


def header_functions():
    text = header_text()
    fns = {}
    for m in re.finditer(r"\b(ingot_rocm_[a-z0-9_]+)\s*\(", text):
        params = balanced(text, m.end() - 1)
        args = split_top(params)
        fns[m.group(1)] = 0 if args == ["void"] else len(args)
    return fns


def header_defines():
    return {m.group(1): m.group(2) for m in re.finditer(r"#define\s+(INGOT_[A-Z0-9_]+)\s+(\S+)", header_text())}


def go_calls(path):
    text = open(path).read()
    calls = []
    for m in re.finditer(r"\bC\.(ingot_rocm_[a-z0-9_]+)\s*\(", text):
        calls.append((m.group(1), split_top(balanced(text, m.end() - 1))))
    return calls


def test_go_sources_exist_with_build_tags():
    for p in [BINDING] + GRAPH:
        first = open(p).readline().strip()
        assert first == "//go:build linux && amd64 && rocm && cgo", f"{p}: build tag {first!r}"
    assert "package rocm" in open(BINDING).read()
    for p in GRAPH:
        assert re.search(r"^package graph$", open(p).read(), re.M)


def test_every_c_call_is_declared_with_matching_arity():
    fns = header_functions()
    calls = go_calls(BINDING)
    assert len(calls) >= 25
    for name, args in calls:
        assert name in fns, f"C.{name} is not declared in include/ingot_rocm.h"
        assert len(args) == fns[name], f"C.{name}: {len(args)} arguments, the header declares {fns[name]}"
    # the kernel-layer entry points a GPU session needs are all bound
    bound = {n for n, _ in calls}
    for required in ["ingot_rocm_open", "ingot_rocm_close", "ingot_rocm_sync", "ingot_rocm_last_error",
                     "ingot_rocm_device_alloc", "ingot_rocm_device_free", "ingot_rocm_memcpy_h2d",
                     "ingot_rocm_memcpy_d2h", "ingot_rocm_weight_upload", "ingot_rocm_weight_free",
                     "ingot_rocm_gemm", "ingot_rocm_gemm_dynamic_b", "ingot_rocm_gemv_bf16",
                     "ingot_rocm_matmul_integer", "ingot_rocm_qlinear_matmul", "ingot_rocm_dequantize_linear",
                     "ingot_rocm_activation", "ingot_rocm_timer_start", "ingot_rocm_timer_stop"]:
        assert required in bound, f"{required} is not bound"
    # the graph package reaches the library only through kernels/rocm
    for p in GRAPH:
        assert "C.ingot_rocm" not in open(p).read()


def test_gemm_args_fields_exist():
    text = header_text()
    body = re.search(r"typedef struct ingot_rocm_gemm_args\s*\{(.*?)\}\s*ingot_rocm_gemm_args;", text, re.S).group(1)
    fields = set()
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        # "int64_t M, N, K" / "const void* d_a": the last identifier of each declarator
        for part in decl.split(","):
            fields.add(re.findall(r"[A-Za-z_][A-Za-z0-9_]*", part)[-1])
    go = open(BINDING).read()
    fn = go[go.index("func (g *Gemm) args() C.ingot_rocm_gemm_args {"):]
    fn = fn[:fn.index("\n}\n")]
    used = set(re.findall(r"\ba\.([A-Za-z_][A-Za-z0-9_]*)", fn))
    assert used, "no field of the argument block is set"
    missing = used - fields
    assert not missing, f"fields not in ingot_rocm_gemm_args: {sorted(missing)}"
    # every field the header declares is filled (a zero left in one would be a silent default)
    assert fields - used <= set(), f"fields never set: {sorted(fields - used)}"


@pytest.mark.parametrize("go_name,c_name", [
    ("statusOK", "INGOT_OK"), ("statusInval", "INGOT_EINVAL"), ("statusDeclined", "INGOT_EDECLINED"),
    ("statusDevice", "INGOT_EDEVICE"), ("statusNoMem", "INGOT_ENOMEM"),
    ("F32", "INGOT_DT_F32"), ("F16", "INGOT_DT_F16"), ("BF16", "INGOT_DT_BF16"), ("I8", "INGOT_DT_I8"),
    ("U8", "INGOT_DT_U8"), ("I16", "INGOT_DT_I16"), ("I32", "INGOT_DT_I32"), ("I64", "INGOT_DT_I64"),
    ("Bool", "INGOT_DT_BOOL"), ("PackI8G", "INGOT_PACK_I8G"),
    ("ActNone", "INGOT_ACT_NONE"), ("ActRelu", "INGOT_ACT_RELU"), ("ActGeluErf", "INGOT_ACT_GELU_ERF"),
    ("ActGeluTanh", "INGOT_ACT_GELU_TANH"), ("ActSigmoid", "INGOT_ACT_SIGMOID"), ("ActSiLU", "INGOT_ACT_SILU"),
    ("ActHardSwish", "INGOT_ACT_HARDSWISH"), ("ActHardSigmoid", "INGOT_ACT_HARDSIGMOID"),
    ("ActClip", "INGOT_ACT_CLIP"), ("ActLeakyRelu", "INGOT_ACT_LEAKYRELU"),
    ("CNone", "INGOT_C_NONE"), ("CFull", "INGOT_C_FULL"), ("CRow", "INGOT_C_ROW"), ("CCol", "INGOT_C_COL"),
    ("CScalar", "INGOT_C_SCALAR"), ("MathAuto", "INGOT_MATH_AUTO"), ("MathF32", "INGOT_MATH_F32"),
    ("MathBF16", "INGOT_MATH_BF16"),
])
def test_go_constants_match_header(go_name, c_name):
    go = open(BINDING).read()
    m = re.search(r"^\s*%s\s*=\s*(\d+)" % re.escape(go_name), go, re.M)
    assert m, f"{go_name} not defined in kernels/rocm"
    assert m.group(1) == header_defines()[c_name], f"{go_name} = {m.group(1)}, {c_name} = {header_defines()[c_name]}"


def test_gpusession_surface():
    """graph/gpu_other.go:13-37's GPUSession surface (CompileGPU, Run, Close, Stage, Release via the embedded
    Session, the GPUSteps/CPUSteps/Flushes/GPUTime/FlushedBy/Profile/OpTime/NodeTime counters) plus Check mode
    and Mismatches (graph/gpu_darwin_arm64.go:61-83)."""
    src = open(GRAPH[0]).read()
    for sig in [r"func CompileGPU\(g \*Graph, opts \.\.\.GPUOption\) \(\*GPUSession, error\)",
                r"func \(s \*GPUSession\) Run\(feeds map\[string\]\*tensor\.Tensor\) \(res map\[string\]\*tensor\.Tensor, err error\)",
                r"func \(s \*GPUSession\) Close\(\)", r"func \(s \*GPUSession\) Stage\(t \*tensor\.Tensor\) \*tensor\.Tensor"]:
        assert re.search(sig, src), sig
    struct = src[src.index("type GPUSession struct {"):]
    struct = struct[:struct.index("\n}\n")]
    assert "\t*Session\n" in struct
    # field declarations, whatever gofmt's column alignment
    decls = {re.sub(r"\s+", " ", ln.split("//")[0]).strip() for ln in struct.splitlines()}
    for field in ["GPUTime time.Duration", "GPUSteps, CPUSteps, Flushes int", "FlushedBy []string", "Profile bool",
                  "OpTime map[string]time.Duration", "NodeTime map[*Node]time.Duration", "Check bool",
                  "Mismatches []Mismatch", "bf16 bool"]:
        assert field in decls, field
    # the bisecting switches of graph/gpu_darwin_arm64.go:133-146
    assert 'os.Getenv("INGOT_GPU_SKIP")' in src and 'os.Getenv("INGOT_GPU_NOHALF")' in src


def test_go_sources_are_balanced():
    """A cheap syntax guard without a Go compiler: braces, brackets and parentheses balance in every file,
    outside strings, runes and comments."""
    for p in [BINDING] + GRAPH:
        text = open(p).read()
        text = re.sub(r"//[^\n]*", "", text)
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r'"(\\.|[^"\\])*"', '""', text)
        text = re.sub(r"'(\\.|[^'\\])*'", "''", text)
        text = re.sub(r"`[^`]*`", "``", text)
        stack = []
        pairs = {")": "(", "]": "[", "}": "{"}
        for i, ch in enumerate(text):
            if ch in "([{":
                stack.append(ch)
            elif ch in ")]}":
                assert stack and stack[-1] == pairs[ch], f"{p}: unbalanced {ch!r} at offset {i}"
                stack.pop()
        assert not stack, f"{p}: unclosed {stack[-1]!r}"
