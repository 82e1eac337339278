"""CPU checks of bench.py's report helpers: the kernel-symbol labels the
profile summaries are grouped by, the algorithmic FLOPs behind the roofline
line, and the committed HBM-traffic figure the bench line quotes."""
import importlib.util
import os

import pytest

from textsift_amd.config import PF_CONFIG

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


# kernel symbols as rocprofv3 prints them (the forward's launches at 16 x 2048)
SYMBOLS = {
    "void pf::(anonymous namespace)::k_gemm_w4<4, 128, 1, (pf::Epi)4, true, 4, 0, false, false, false>(pf::GemmArgs)":
        "gemm_moe_gate_up",
    "void pf::(anonymous namespace)::k_gemm_w4<4, 128, 1, (pf::Epi)0, true, 4, 0, false, false, false>(pf::GemmArgs)":
        "gemm_moe_down",
    "void pf::(anonymous namespace)::k_gemm_w4<4, 128, 1, (pf::Epi)2, false, 4, 0, false, false, false>(pf::GemmArgs)":
        "gemm_qkv_rope",
    "void pf::(anonymous namespace)::k_gemm_w4_rownorm<7>(pf::GemmArgs, unsigned short const*)": "gemm_o_add_rmsnorm",
    "void pf::(anonymous namespace)::k_gemm_w4<2, 64, 1, (pf::Epi)5, false, 4, 0, false, false, false>(pf::GemmArgs)":
        "gemm_router",
    "void pf::(anonymous namespace)::k_gemm_w4<1, 64, 1, (pf::Epi)0, false, 4, 0, false, false, false>(pf::GemmArgs)":
        "gemm_classifier",
    "void pf::(anonymous namespace)::k_banded_attention_hw<64, 9, 8, false>(pf::AttnArgs)": "banded_attention",
    "void pf::(anonymous namespace)::k_moe_combine<0, 4, 3, true, true>(int const*, float const*)": "moe_combine_norm",
    "pf::(anonymous namespace)::k_moe_route_counts(int const*, int const*, int)": "moe_route",
    "void pf::(anonymous namespace)::k_embed_rms_norm4<5>(unsigned char const*, unsigned short const*)":
        "embed_rms_norm",
    "void pf::(anonymous namespace)::k_embed<true>(unsigned char const*, unsigned short const*)": "embed_lookup_int4",
    "void pf::(anonymous namespace)::k_rms_norm4<5>(unsigned short const*, unsigned short const*)": "rms_norm",
}


def test_kernel_labels(bench):
    for sym, label in SYMBOLS.items():
        assert bench.label_of(sym) == label, sym


def test_gate_up_flops(bench):
    M = 16 * 2048
    f = bench.gemm_flops(PF_CONFIG, M)
    # 4 routed rows per token, N = 2 x 640 (gate, up), K = 640
    assert f["gemm_moe_gate_up"] == 2.0 * 4 * M * 1280 * 640 == 214748364800.0
    assert f["gemm_moe_down"] == f["gemm_moe_gate_up"] / 2


def test_committed_traffic_is_read(bench):
    t = bench.read_traffic("gemm_moe_gate_up", 16, 2048)
    assert t is not None and 2.0e8 < t < 1.0e9
    assert bench.read_traffic("gemm_moe_gate_up", 1, 64) is None
    assert bench.read_traffic("no_such_kernel", 16, 2048) is None
