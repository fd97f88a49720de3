"""The C-ABI library loads without a GPU and exports every symbol the
headers declare (no compute calls here)."""

import ctypes
import os
import re
import subprocess

import pytest

import feattn

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(fe_\w+)\s*\(", text, flags=re.M)))


HEADERS = {"fe_attn.h": feattn.C_SYMBOLS, "fe_driver.h": feattn.DRIVER_SYMBOLS, "fe_ops.h": feattn.OPS_SYMBOLS}


def test_header_matches_binding_list():
    assert sorted(os.listdir(os.path.join(ROOT, "include"))) == sorted(
        list(HEADERS) + ["fe_native_hip.hpp"])
    for header, symbols in HEADERS.items():
        names = header_functions(os.path.join(ROOT, "include", header))
        assert names == sorted(symbols), header


def test_library_exports_every_c_symbol():
    lib = feattn.lib()
    for header in HEADERS:
        for name in header_functions(os.path.join(ROOT, "include", header)):
            assert hasattr(lib, name), name
    assert feattn.version().startswith("feattn-hip-gfx950")


def test_library_exports_reference_namespace():
    """fe::cuda:: symbols with the reference's exact parameter lists -- every
    function of include/fe/native_cuda.hpp:7-15 -- so cuda_model.cpp can link
    unchanged."""
    out = subprocess.run(["nm", "-DC", feattn.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    want = [
        "fe::cuda::create_plan(int, int, int, int, int, int, bool, int)",
        "fe::cuda::destroy_plan(fe::cuda::AttentionPlan*)",
        "fe::cuda::prepare_plan(fe::cuda::AttentionPlan*, int const*, int const*, int const*, "
        "int const*, int, int, bool, void*)",
        "fe::cuda::attention(fe::cuda::AttentionPlan*, void*, void*, void*, void*, bool, void*)",
        "fe::cuda::rope(void*, void*, long const*, float const*, int, int, int, int, bool, void*, int)",
        "fe::cuda::store(void const*, void const*, void*, void*, long const*, int, int, bool, void*, int)",
        "fe::cuda::norm(void const*, void const*, void const*, void*, void*, int, int, float, bool, void*)",
        "fe::cuda::silu_mul(void const*, void*, int, int, bool, void*)",
        "fe::cuda::accept(long const*, long const*, long*, int, int, void*)",
    ]
    for w in want:
        assert w in out, w


def test_library_links_only_the_hip_runtime():
    """No torch or CUDA in the product library's dependencies."""
    out = subprocess.run(["readelf", "-d", feattn.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    needed = re.findall(r"Shared library: \[(.+?)\]", out)
    assert any(n.startswith("libamdhip64") for n in needed)
    assert not any("torch" in n or "cuda" in n or "c10" in n for n in needed), needed


def test_error_reporting_without_device():
    """create rejects a bad head size before touching the device."""
    lib = feattn.lib()
    h = ctypes.c_void_p()
    rc = lib.fe_attn_plan_create(32, 8, 64, 16, 4, 4, 1, 16, ctypes.byref(h))
    assert rc == feattn.FE_EINVAL
    assert b"128" in lib.fe_attn_last_error()
    rc = lib.fe_attn_plan_create(32, 8, 128, 24, 4, 4, 1, 16, ctypes.byref(h))
    assert rc == feattn.FE_EINVAL and b"page" in lib.fe_attn_last_error()
    rc = lib.fe_attn_plan_create(30, 8, 128, 16, 4, 4, 1, 16, ctypes.byref(h))
    assert rc == feattn.FE_EINVAL



def test_headers_are_c99_and_resolve(tmp_path):
    """The C headers compile as strict C99, and every function they declare
    resolves against libfeattn.so from a C program (C linkage, exact names)."""
    import shutil

    if shutil.which("gcc") is None:
        pytest.skip("no C compiler")
    names = sorted({n for h in HEADERS for n in header_functions(os.path.join(ROOT, "include", h))})
    src = "".join(f'#include "{h}"\n' for h in HEADERS)
    src += "typedef void (*fn)(void);\nstatic const fn table[] = {\n"
    src += ",\n".join(f"  (fn)&{n}" for n in names)
    src += "\n};\nint main(void) { return table[0] == 0; }\n"
    c = tmp_path / "abi.c"
    c.write_text(src)
    lib_dir = os.path.dirname(feattn.LIB_PATH)
    r = subprocess.run(["gcc", "-std=c99", "-pedantic", "-Wall", "-Wextra", "-Werror",
                        "-I" + os.path.join(ROOT, "include"), str(c), "-o", str(tmp_path / "abi"),
                        "-L" + lib_dir, "-lfeattn", "-Wl,-rpath-link,/opt/rocm/lib"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
