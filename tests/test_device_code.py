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
    it is the f32 fma of the widened values and is allowed anywhere;
  * an LDS DMA (global_load_lds) in the cycle after the write of M0 that
    holds its LDS address: it needs one wait state in between (the
    compiler's own sequences always have one);
  * reads of an MFMA result too soon after the MFMA: the matrix cores write
    the result several cycles after the instruction issues and the hardware
    does not stall a dependent read, so it needs wait states (8 for the
    gfx950 MFMAs used here: the fewest the compiler itself leaves before one
    of its own reads). The compiler counts them only for instructions it
    sees; inline assembly reading accumulators does not get them.
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


def _by_function(asm, operands=False):
    """{function symbol: [instruction mnemonics]} (with operands=True, whole
    instructions: mnemonic and operand text)"""
    funcs, cur = {}, None
    for line in asm.splitlines():
        m = re.match(r"^[0-9a-f]+ <(.+)>:$", line)
        if m:
            cur = m.group(1)
            funcs[cur] = []
            continue
        if cur is None:
            continue
        text = line.split("//")[0].strip()
        parts = text.split()
        if not parts:
            continue
        if operands:
            if re.match(r"^(v|s|global|buffer|ds|flat|scratch)_[a-z0-9_]+$", parts[0]):
                funcs[cur].append(text)
        elif re.match(r"^[vs]_[a-z0-9_]+$", parts[0]):
            funcs[cur].append(parts[0])
    return funcs


@pytest.fixture(scope="module")
def disassembly(tmp_path_factory):
    if not os.path.exists(f"{LLVM}/llvm-objdump"):
        pytest.skip("ROCm llvm tools not installed")
    tmp = tmp_path_factory.mktemp("co")
    return [_disassemble(obj, tmp) for obj in _objects()]


@pytest.fixture(scope="module")
def device_code(disassembly):
    code = {}
    for asm in disassembly:
        code.update(_by_function(asm))
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


def _vgprs(tok):
    m = re.match(r"^v\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"^v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _instructions(asm):
    """{function: [(address, instruction text)]} from llvm-objdump output."""
    funcs, cur = {}, None
    for line in asm.splitlines():
        m = re.match(r"^[0-9a-f]+ <(.+)>:$", line)
        if m:
            cur = m.group(1)
            funcs[cur] = []
            continue
        if cur is None or "//" not in line:
            continue
        text, comment = line.split("//", 1)
        am = re.match(r"\s*([0-9A-Fa-f]+):", comment)
        if text.strip() and am:
            funcs[cur].append((int(am.group(1), 16), text.strip()))
    return funcs


MFMA_READ_WAIT_STATES = 8


def _early_mfma_reads(ins):
    """(mfma, reader, wait states) for every path from an MFMA, through
    branches, to the first non-MFMA instruction reading its destination
    with fewer than MFMA_READ_WAIT_STATES wait states in between."""
    at = {a: i for i, (a, _) in enumerate(ins)}
    found = []
    for i, (_, text) in enumerate(ins):
        if not text.startswith("v_mfma"):
            continue
        dst = _vgprs(text.split(None, 1)[1].split(",")[0].strip())
        stack, seen = [(i + 1, 0)], set()
        while stack:
            j, waits = stack.pop()
            if j >= len(ins) or waits >= MFMA_READ_WAIT_STATES or (j, waits) in seen:
                continue
            seen.add((j, waits))
            addr, nxt = ins[j]
            parts = nxt.split(None, 1)
            op = parts[0]
            if op == "s_nop":
                stack.append((j + 1, waits + int(parts[1], 0) + 1))
                continue
            if op.startswith(("s_cbranch", "s_branch")):
                tgt = at.get(addr + 4 + 4 * int(parts[1].split()[0], 0))
                if tgt is not None:
                    stack.append((tgt, waits + 1))
                if op.startswith("s_cbranch"):
                    stack.append((j + 1, waits + 1))
                continue
            if op.startswith(("s_setpc", "s_endpgm")):
                continue
            if not op.startswith("v_mfma"):  # MFMA operands forward (the compiler orders these)
                args = [a.strip().split()[0] for a in parts[1].split(",") if a.strip()] if len(parts) > 1 else []
                reads = args[1:] if op.startswith("v_") else args  # a vector op's first operand is written
                if any(_vgprs(a) & dst for a in reads):
                    found.append((text, nxt, waits))
                    continue
            stack.append((j + 1, waits + 1))
    return found


def test_mfma_results_read_after_wait_states(disassembly):
    """On every path from an MFMA, the first instruction other than an MFMA
    that reads its destination registers comes at least 8 wait states after
    it (an instruction counts 1, s_nop N counts N + 1)."""
    bad = []
    for asm in disassembly:
        for f, ins in _instructions(asm).items():
            bad += [(f[:80],) + b for b in _early_mfma_reads(ins)]
    assert not bad, bad[:10]


def test_lds_dma_after_m0_write(disassembly):
    """No LDS DMA directly after an instruction that writes M0."""
    bad = []
    for asm in disassembly:
        for f, ins in _instructions(asm).items():
            for (_, a), (_, b) in zip(ins, ins[1:]):
                if re.match(r"^s_\w+ m0,", a) and b.startswith("global_load_lds"):
                    bad.append((f[:80], a, b))
    assert not bad, bad[:10]
