"""Checks on the gfx950 machine code this repository builds (CPU only).

The objects under textsift_amd/_build/ are disassembled (llvm-objdump from the
ROCm toolchain) and scanned for instruction forms the kernels must not use:
  * packed FP32 arithmetic (v_pk_fma_f32, v_pk_mul_f32, v_pk_add_f32): the
    build disables the feature;
  * scalar memory writes (s_store*, s_buffer_store*, s_atomic*,
    s_dcache_wb*): every store is a vector store;
  * fused mixed-precision conversions to fp16 (v_fma_mixlo_f16,
    v_fma_mixhi_f16): they round a product once to fp16 where the reference
    rounds to f32 first. They are allowed only in the RoPE epilogue
    instances, whose products (fp16 x fp16) are exact in f32. v_fma_mix_f32
    (an f32 result) widens its fp16 operands exactly and rounds once to f32:
    it is the f32 fma of the widened values and is allowed anywhere.
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "textsift_amd", "_build")
LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


def _objects():
    """Objects of the .hip sources (the .cpp ones carry no device code)."""
    from textsift_amd import build
    names = [os.path.splitext(s)[0] + ".o" for s in build.SOURCES if s.endswith(".hip")]
    objs = [os.path.join(BUILD, n) for n in names]
    if not all(os.path.exists(o) for o in objs):
        build.build()
    return objs


def _disassemble(obj, tmp_path):
    fatbin = tmp_path / (os.path.basename(obj) + ".fatbin")
    scratch = tmp_path / (os.path.basename(obj) + ".host.o")
    subprocess.run([f"{LLVM}/llvm-objcopy", f"--dump-section=.hip_fatbin={fatbin}", obj, str(scratch)], check=True)
    code = tmp_path / (os.path.basename(obj) + ".co")
    subprocess.run([f"{LLVM}/clang-offload-bundler", "--unbundle", "--type=o", f"--input={fatbin}",
                    f"--targets={TARGET}", f"--output={code}"], check=True)
    out = subprocess.run([f"{LLVM}/llvm-objdump", "-d", "--mcpu=gfx950", str(code)], check=True,
                         capture_output=True, text=True).stdout
    return out


def _by_function(asm):
    """{function symbol: [instruction mnemonics]}"""
    funcs, cur = {}, None
    for line in asm.splitlines():
        m = re.match(r"^[0-9a-f]+ <(.+)>:$", line)
        if m:
            cur = m.group(1)
            funcs[cur] = []
            continue
        if cur is None:
            continue
        parts = line.strip().split()
        if parts and re.match(r"^[vs]_[a-z0-9_]+$", parts[0]):
            funcs[cur].append(parts[0])
    return funcs


@pytest.fixture(scope="module")
def device_code(tmp_path_factory):
    if not os.path.exists(f"{LLVM}/llvm-objdump"):
        pytest.skip("ROCm llvm tools not installed")
    tmp = tmp_path_factory.mktemp("co")
    code = {}
    for obj in _objects():
        code.update(_by_function(_disassemble(obj, tmp)))
    return code


def test_objects_have_device_code(device_code):
    names = " ".join(device_code)
    for kernel in ("k_gemm_w4", "k_gemm_int4", "k_banded_attention", "k_moe_combine", "k_embed"):
        assert kernel in names


def test_no_packed_fp32(device_code):
    bad = {f: [i for i in ins if i in ("v_pk_fma_f32", "v_pk_mul_f32", "v_pk_add_f32")]
           for f, ins in device_code.items()}
    assert not {f: b for f, b in bad.items() if b}


def test_no_scalar_memory_writes(device_code):
    pat = re.compile(r"^s_(store|buffer_store|scratch_store|atomic|buffer_atomic|dcache_wb)")
    bad = {f: [i for i in ins if pat.match(i)] for f, ins in device_code.items()}
    assert not {f: b for f, b in bad.items() if b}


def test_fused_mixed_conversions_only_in_rope(device_code):
    bad = {f for f, ins in device_code.items() if any(i.startswith(("v_fma_mixlo", "v_fma_mixhi")) for i in ins)
           and "Epi)2" not in f and "EpiE2" not in f}
    assert not bad, sorted(bad)
