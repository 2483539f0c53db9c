"""The C-ABI library loads and exports every symbol include/ingot_rocm.h declares.

CPU-only: no compute call is made. The product must not fall back to any CPU
path, so the Python binding refuses to run without the built library.
"""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ingot_rocm.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ingot_rocm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ["ingot_rocm_open", "ingot_rocm_close", "ingot_rocm_last_error", "ingot_rocm_weight_upload",
                     "ingot_rocm_gemm", "ingot_rocm_gemv_bf16", "ingot_rocm_matmul_integer",
                     "ingot_rocm_dequantize_linear", "ingot_rocm_op_create", "ingot_rocm_op_run"]:
        assert required in names


def test_library_exports_every_declared_symbol():
    from ingot_amd import _lib

    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_bindings_cover_the_header():
    from ingot_amd import _lib

    assert sorted(_lib.SIGNATURES) == declared_functions()
    _lib.load()  # every signature binds


def test_struct_layout_matches_header(tmp_path):
    """ctypes mirrors of the C structs have the sizes and offsets gcc gives them."""
    import subprocess

    from ingot_amd import _lib

    fields = [f for f, _ in _lib.GemmArgs._fields_]
    qfields = [f for f, _ in _lib.QconvArgs._fields_]
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "%s"\nint main(void){\n' % HEADER
        + 'printf("%zu %zu %zu\\n", sizeof(ingot_rocm_gemm_args), sizeof(ingot_rocm_tensor), '
          'sizeof(ingot_rocm_qconv_args));\n'
        + "".join('printf("%%zu\\n", offsetof(ingot_rocm_gemm_args, %s));\n' % f for f in fields)
        + "".join('printf("%%zu\\n", offsetof(ingot_rocm_qconv_args, %s));\n' % f for f in qfields)
        + "return 0;}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    assert int(out[0]) == ctypes.sizeof(_lib.GemmArgs)
    assert int(out[1]) == ctypes.sizeof(_lib.Tensor)
    assert int(out[2]) == ctypes.sizeof(_lib.QconvArgs)
    offs = out[3:]
    for f, off in zip(fields, offs[:len(fields)]):
        assert getattr(_lib.GemmArgs, f).offset == int(off), f
    for f, off in zip(qfields, offs[len(fields):]):
        assert getattr(_lib.QconvArgs, f).offset == int(off), f


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from ingot_amd import _lib

    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(RuntimeError, match="missing"):
        _lib.load()


def test_version_and_error_without_compute():
    from ingot_amd import _lib

    lib = _lib.load()
    assert b"gfx950" in lib.ingot_rocm_version()
    # invalid arguments are reported, not crashed on
    assert lib.ingot_rocm_close(None) == 0
    rc = lib.ingot_rocm_sync(None)
    assert rc == _lib.EINVAL and b"nil session" in lib.ingot_rocm_last_error()


def test_header_is_strict_c99(tmp_path):
    """include/ingot_rocm.h compiles as strict C99 (what cgo and other FFIs include)."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if not gcc:
        pytest.skip("gcc not available")
    src = tmp_path / "only_header.c"
    src.write_text('#include "%s"\nint main(void) { return INGOT_OK; }\n' % HEADER)
    r = subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic", "-fsyntax-only", str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
