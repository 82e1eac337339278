"""CPU-side checks of the drop-in boundary: the built library loads, exports
every entry point include/pfhip.h declares, and the product package never
reaches into the test oracle. No GPU calls."""
import ctypes as C
import os
import re

import pytest

from textsift_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    src = open(os.path.join(ROOT, "include", "pfhip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(pfhip_[a-z_0-9]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the ctypes table covers the same set
    assert sorted(n for n, _, _ in _native.EXPORTS) == names


def test_version_and_kernel_table_need_no_gpu():
    lib = _native.lib()
    assert b"gfx950" in lib.pfhip_version()
    table = lib.pfhip_kernel_names().decode().split("\n")
    names = {l.split()[0] for l in table if l}
    reference_kernels = {"rms_norm", "zero_f32", "cast_fp16_to_f32", "cast_f32_to_fp16_scaled", "add_fp16",
                         "add_rmsnorm_fp16_to_f32", "embed_lookup_int4", "matmul_int4_fp16_f16",
                         "matmul_int4_f32_f32", "rope_apply", "banded_attention", "router_topk", "qmoe_gate_up",
                         "swiglu_clamp", "qmoe_down_scatter"}
    assert reference_kernels <= names


def test_create_backend_fails_cleanly_without_a_gpu():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU device node is present")
    err = C.create_string_buffer(1024)
    h = _native.lib().pfhip_create_backend(0, err, 1024)
    assert not h and err.value  # error text, no abort


def test_product_package_does_not_use_the_oracle():
    pkg = os.path.join(ROOT, "textsift_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h", ".cuh", ".js", ".cc")):
                text = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"\boracle\b|liboracle|pf_oracle", text), os.path.join(dirpath, f)
