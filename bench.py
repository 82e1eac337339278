"""Benchmark: the privacy-filter encoder forward at 16 x 2048 tokens on one MI355X.

A step is one full forward (embed -> 8 MoE transformer blocks -> classifier)
over 16 sequences of 2048 tokens, with token ids
already resident in HBM and logits left in HBM. Weights are random-init in the
MatMulNBits / GatherBlockQuantized byte layouts (textsift_amd.synth); token
ids are uniform over the 200064-row vocabulary.

Prints one JSON line with the throughput, the roofline of the dominant kernel
(its algorithmic FLOPs per launch over its average launch time, measured with
HIP events on the backend's stream during the timed steps; the events bracket
that kernel only, so the timed region carries no per-launch instrumentation
of the others) and the CPU baseline (the oracle's C restatement of the WASM
path, multi-threaded with the reference's worker partitioning, on a bounded
sample). The per-kernel table comes from a separate profiled pass after the
warmup. roofline.traffic (HBM bytes per launch) is read from the committed
profiles/<kernel>_traffic.md, produced by the two rocprofv3 --pmc passes that
--traffic-report turns into that summary.

Modes beside the default:
  --copy-calibration-mb N   also run one plain device copy of N MiB (for the
                            PMC passes: the counters' bytes-per-byte factor)
  --traffic-report FETCH_CSV WRITE_CSV --copy-mb N
                            turn two rocprofv3 --pmc counter_collection.csv
                            files into the traffic summary (markdown)
"""
import argparse
import subprocess
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

MFMA_FP16_PEAK_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA
HBM_PEAK_GBS = 8000.0

# rocprofv3 kernel symbols -> the launch names the backend profiles under
KERNEL_LABELS = [
    ("gemm_moe_gate_up", ("k_gemm_w4<", "(pf::Epi)4, true")),
    ("gemm_moe_down", ("k_gemm_w4<", "(pf::Epi)0, true")),   # fp16 numerics: fp16 expert outputs
    ("gemm_moe_down", ("k_gemm_w4<", "(pf::Epi)1, true")),
    ("gemm_qkv_rope", ("k_gemm_w4<", "(pf::Epi)2, false")),
    ("gemm_o_add_rmsnorm", ("k_gemm_w4_rownorm",)),
    ("gemm_o", ("k_gemm_w4<4, 128", "(pf::Epi)0, false")),
    ("gemm_o", ("k_gemm_w4<1, 16", "(pf::Epi)0, false, 4, 7,")),      # all-K small tile, K = 896
    ("gemm_router", ("k_gemm_w4<2, ", "(pf::Epi)5, false")),
    ("gemm_router", ("k_gemm_w4<2, ", "(pf::Epi)1, false")),
    ("gemm_classifier", ("k_gemm_w4<1, 64", "(pf::Epi)0, false")),
    ("gemm_classifier", ("k_gemm_w4<1, 16", "(pf::Epi)0, false, 4, 5,")),  # all-K small tile, K = 640
    ("banded_attention", ("k_banded_attention",)),
    ("moe_combine_norm", ("k_moe_combine",)),
    ("add_rmsnorm_f16", ("k_add_rms_norm",)),
    ("router_topk", ("k_router_topk",)),
    ("moe_route", ("k_moe_route_small",)),
    ("moe_route", ("k_moe_route_counts",)),
    ("moe_count", ("k_moe_count",)),
    ("moe_scan", ("k_moe_scan",)),
    ("moe_scatter", ("k_moe_scatter",)),
    ("embed_rms_norm", ("k_embed_rms_norm",)),
    ("embed_lookup_int4", ("k_embed",)),
    ("rms_norm", ("k_rms_norm",)),
    ("copy_lds", ("k_copy16_lds",)),
    ("gather16", ("k_gather16",)),
    ("copy", ("k_copy16",)),
]
CALIBRATION = ("copy", "copy_lds", "gather16")


def short_symbol(sym):
    """A kernel symbol without namespace qualifiers and parameter list."""
    s = sym.replace("void ", "").replace("pf::(anonymous namespace)::", "").replace("pf::", "")
    depth = 0
    for i, ch in enumerate(s):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return s[:i]
    return s


LABELS = list(dict.fromkeys(lab for lab, _ in KERNEL_LABELS))  # unique, in order


def label_of(symbol):
    for label, parts in KERNEL_LABELS:
        if all(p in symbol for p in parts):
            return label
    return None


def read_counters(path, counter):
    """{dispatch id: (kernel symbol, value)} from a rocprofv3 counter_collection.csv."""
    import csv
    out = {}
    with open(path, newline="") as f:
        rows = csv.reader(f)
        header = next(rows)
        ci, vi = header.index("Counter_Name"), header.index("Counter_Value")
        ki, di = header.index("Kernel_Name"), header.index("Dispatch_Id")
        for r in rows:
            # kernel symbols may contain commas: fields after Kernel_Name are counted from the end
            name = ",".join(r[ki:len(r) - (len(header) - ki - 1)])
            tail = r[len(r) - (len(header) - ki - 1):]
            cn, cv = tail[ci - ki - 1], float(tail[vi - ki - 1])
            if cn != counter:
                continue
            d = int(r[di])
            prev = out.get(d, (name, 0.0))
            out[d] = (name, prev[1] + cv)
    return out


def traffic_report(fetch_csv, write_csv, copy_mb, raw=False):
    """Markdown summary: per kernel, FETCH_SIZE and WRITE_SIZE (KiB per
    dispatch) scaled by what the counters read for calibration workloads of
    known size run in the same process (--copy-calibration-mb): a plain copy
    of copy_mb MiB (the factor applied), the same copy with HBM -> LDS loads,
    and a gather of copy_mb MiB in scattered 16-byte units (reported, so a
    reader sees whether the factor depends on the load form).
    raw: kernels by their symbols instead of the forward's launch names."""
    fetch = read_counters(fetch_csv, "FETCH_SIZE")
    write = read_counters(write_csv, "WRITE_SIZE")
    expect_kib = copy_mb * 1024.0
    def key(name):
        lab = label_of(name)
        if lab in CALIBRATION or not raw:
            return lab
        return short_symbol(name)
    def per_label(d):
        acc = {}
        for name, v in d.values():
            lab = key(name)
            if lab:
                acc.setdefault(lab, []).append(v)
        return acc
    fl, wl = per_label(fetch), per_label(write)
    # calibration: bytes each workload moves (read, write) in KiB
    known = {"copy": (expect_kib, expect_kib), "copy_lds": (expect_kib, expect_kib),
             "gather16": (expect_kib * 1.25, expect_kib)}  # gather reads a 4-byte index per 16-byte unit
    factors = {}
    for c in CALIBRATION:
        if c in fl and c in wl:
            factors[c] = (max(fl[c]) / known[c][0], max(wl[c]) / known[c][1])
    kf, kw = factors.get("copy", (None, None))
    lines = ["| kernel | dispatches | FETCH_SIZE KiB/dispatch | WRITE_SIZE KiB/dispatch | HBM bytes/launch |",
             "|---|---|---|---|---|"]
    summary = {}
    for lab in sorted(set(fl) & set(wl), key=lambda x: (LABELS.index(x) if x in LABELS else len(LABELS), x)):
        if lab in CALIBRATION:
            continue
        f = sum(fl[lab]) / len(fl[lab])
        w = sum(wl[lab]) / len(wl[lab])
        hbm = (f / kf + w / kw) * 1024.0 if kf and kw else None
        summary[lab] = hbm
        lines.append(f"| {lab} | {len(fl[lab])} | {f:.1f} | {w:.1f} | {hbm:.4g} |" if hbm else
                     f"| {lab} | {len(fl[lab])} | {f:.1f} | {w:.1f} | - |")
    head = []
    for c, (a, b) in factors.items():
        head.append(f"calibration {c} of {copy_mb} MiB: FETCH_SIZE factor {a:.4f}, WRITE_SIZE factor {b:.4f}")
    head += ["HBM bytes/launch = (FETCH / copy FETCH factor + WRITE / copy WRITE factor) * 1024", ""] if kf and kw \
        else ["no calibration copy found", ""]
    tail = [""] + [f"hbm_bytes_per_launch {lab}: {int(v)}" for lab, v in summary.items() if v]
    return "\n".join(head + lines + tail)


def run_calibration(be, mib):
    """The counters' calibration workloads, copy_mb MiB each (see traffic_report)."""
    n = mib << 20
    src, dst = be.buffer(nbytes=n), be.buffer(nbytes=n)
    be.dispatch("copy16", [src, dst], np.array([n], np.uint32))
    be.dispatch("copy16_lds", [src, dst], np.array([n], np.uint32))
    units = n // 16
    idx = be.buffer(np.random.default_rng(0).integers(0, units, units).astype(np.int32))
    be.dispatch("gather16", [src, idx, dst], np.array([units, units], np.uint32))
    for b in (src, dst, idx):
        b.release()


SQ_PASS1 = "SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_VALU_MFMA_BUSY_CYCLES SQ_ACTIVE_INST_VALU SQ_WAIT_INST_ANY SQ_WAIT_ANY " \
           "SQ_ACTIVE_INST_LDS SQ_VALU_MFMA_COEXEC_CYCLES"
SQ_PASS2 = "SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS SQ_WAIT_INST_LDS SQ_LDS_BANK_CONFLICT SQ_ACTIVE_INST_ANY " \
           "SQ_INSTS_SALU SQ_WAVES"


def sq_report(p1_csv, p2_csv, cus=256, ses=32):
    """Markdown summary of the SQ counter passes, per kernel and dispatch:
    instructions per wave and MFMA pipe utilisation. SQ_BUSY_CYCLES sums
    the shader engines (ses of them), SQ_VALU_MFMA_BUSY_CYCLES all SIMDs
    (4 per CU), so MFMA busy = (MFMA_BUSY / (4 cus)) / (BUSY / ses)."""
    names = SQ_PASS1.split() + SQ_PASS2.split()
    per = {}
    for path, cnts in ((p1_csv, SQ_PASS1.split()), (p2_csv, SQ_PASS2.split())):
        for cn in cnts:
            for d, (sym, v) in read_counters(path, cn).items():
                lab = label_of(sym)
                if lab:
                    per.setdefault(lab, {}).setdefault(cn, {})[(path, d)] = v
    lines = ["| kernel | waves | VALU / wave | MFMA / wave | SALU / wave | LDS / wave | LDS conflict cycles / LDS instr | "
             "MFMA busy | wave time waiting on dependencies |", "|---|---|---|---|---|---|---|---|---|"]
    for lab in LABELS:
        if lab not in per or any(n not in per[lab] for n in names):
            continue
        a = {n: sum(per[lab][n].values()) / len(per[lab][n]) for n in names}
        w = a["SQ_WAVES"] or 1.0
        mfma_busy = (a["SQ_VALU_MFMA_BUSY_CYCLES"] / (4 * cus)) / (a["SQ_BUSY_CYCLES"] / ses)
        lines.append(f"| {lab} | {w:.0f} | {a['SQ_INSTS_VALU'] / w:.0f} | {a['SQ_INSTS_MFMA'] / w:.0f} | "
                     f"{a['SQ_INSTS_SALU'] / w:.0f} | {a['SQ_INSTS_LDS'] / w:.0f} | "
                     f"{a['SQ_LDS_BANK_CONFLICT'] / max(a['SQ_INSTS_LDS'], 1.0):.1f} | {100 * mfma_busy:.0f} % | "
                     f"{100 * a['SQ_WAIT_INST_ANY'] / a['SQ_WAVE_CYCLES']:.0f} % |")
    return "\n".join(lines)


def stats_report(stats_csv, top=20):
    """Markdown table of a rocprofv3 --stats kernel_stats.csv: per kernel
    symbol, calls and average/min/max duration, by total time."""
    import csv
    with open(stats_csv, newline="") as f:
        rows = list(csv.DictReader(f))
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    lines = ["| kernel | calls | avg us | min us | max us | % of GPU time |", "|---|---|---|---|---|---|"]
    for r in rows[:top]:
        name = r["Name"] if len(r["Name"]) <= 100 else r["Name"][:97] + "..."
        lines.append(f"| `{name}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                     f"{float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.2f} |")
    return "\n".join(lines)


def read_traffic(kernel, B, T):
    """HBM bytes per launch of `kernel` from the committed traffic summary, or
    None. The summary is of the 16 x 2048 headline forward, so other shapes get
    None."""
    if (B, T) != (16, 2048):
        return None
    path = os.path.join(ROOT, "profiles", "forward_16x2048_hbm_traffic.md")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith(f"hbm_bytes_per_launch {kernel}:"):
                return int(line.split(":")[1])
    return None


def gemm_flops(cfg, M):
    """Algorithmic FLOPs per launch of each GEMM kernel of the forward
    (2*M*N*K; the MoE GEMMs run on the M*topk routed rows)."""
    D, F, E, K = cfg.hidden_size, cfg.intermediate_size, cfg.num_experts, cfg.num_experts_per_tok
    hq, hk, hd = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
    S = M * K
    return {
        "gemm_qkv_rope": 2.0 * M * (hq + 2 * hk) * hd * D,
        "gemm_o": 2.0 * M * D * hq * hd,
        "gemm_o_add_rmsnorm": 2.0 * M * D * hq * hd,  # the O GEMM with the residual add + norm fused
        "gemm_router": 2.0 * M * E * D,
        "gemm_moe_gate_up": 2.0 * S * 2 * F * D,
        "gemm_moe_down": 2.0 * S * D * F,
        "gemm_classifier": 2.0 * M * cfg.num_classes * D,
    }


def attention_flops(cfg, B, T):
    """QK^T + PV over the band: 4 * head_dim FLOPs per (query, key) pair."""
    W = cfg.sliding_window
    t = np.arange(T)
    keys = np.minimum(T, t + W + 1) - np.maximum(0, t - W)
    return 4.0 * cfg.head_dim * cfg.num_heads * B * float(keys.sum())


BLAS_SHAPES = [  # (kernel of this build, what its launch also does)
    ("gemm_qkv_rope", "int4 W, bias, RoPE"),
    ("gemm_o_add_rmsnorm", "int4 W, bias, residual add, RMSNorm"),
    ("gemm_router", "int4 W, bias, f32 out, top-4 + softmax"),
    ("gemm_moe_gate_up", "int4 W, 128 experts grouped, bias, SwiGLU"),
    ("gemm_moe_down", "int4 W, 128 experts grouped, bias, fp16 out"),
]


def blas_shapes(cfg, M):
    D, F, E, K = cfg.hidden_size, cfg.intermediate_size, cfg.num_experts, cfg.num_experts_per_tok
    hq, hk, hd = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
    S = M * K
    return {"gemm_qkv_rope": (M, (hq + 2 * hk) * hd, D), "gemm_o_add_rmsnorm": (M, D, hq * hd),
            "gemm_router": (M, E, D), "gemm_moe_gate_up": (S, 2 * F, D), "gemm_moe_down": (S, D, F)}


def blas_torch_times(cfg, M, reps=20):
    """torch.matmul of a dense fp16 [M, K] x [K, N] product (hipBLASLt on
    ROCm; fp16 weights, no dequantisation, no expert grouping, fp16 output)
    for each forward GEMM shape: {kernel: average us}. Runs in its own
    process (torch's HIP runtime and the library's are separate)."""
    import torch
    dev = torch.device("cuda")
    out = {}
    for name, (m, n, k) in blas_shapes(cfg, M).items():
        a = torch.randn(m, k, device=dev, dtype=torch.float16)
        w = torch.randn(n, k, device=dev, dtype=torch.float16)
        for _ in range(3):
            torch.matmul(a, w.t())
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            torch.matmul(a, w.t())
        e1.record()
        torch.cuda.synchronize()
        out[name] = e0.elapsed_time(e1) * 1000.0 / reps
        del a, w
    return out


def blas_reference_table(cfg, M, prof, ref):
    """Each GEMM of the forward (its profiled average launch time, epilogue
    included) next to the dense fp16 torch.matmul of the same M x N x K."""
    rows = ["| kernel (this build) | its launch also does | M x N x K | this build us | TFLOP/s | "
            "torch.matmul fp16 us | TFLOP/s | torch / this |", "|---|---|---|---|---|---|---|---|"]
    shapes = blas_shapes(cfg, M)
    for name, what in BLAS_SHAPES:
        m, n, k = shapes[name]
        fl = 2.0 * m * n * k
        ours = prof.get(name)
        us = ours[1] * 1000.0 / ours[0] if ours else float("nan")
        us_ref = ref[name]
        rows.append(f"| `{name}` | {what} | {m} x {n} x {k} | {us:.1f} | {fl / us / 1e6:.0f} | {us_ref:.1f} | "
                    f"{fl / us_ref / 1e6:.0f} | {us_ref / us:.2f} |")
    return "\n".join(rows)


# The reference's published single-sequence forward latencies (ms) at small T
# (its README.md:172-184 and docs-site/src/content/docs/benchmarks.mdx:14-39):
# WebGPU on an Apple M3 Pro, Metal-direct on an Apple M2 Pro, synthetic weights.
REF_LATENCY_MS = {7: {"WebGPU M3 Pro": 8.9, "Metal M2 Pro": 5.2}, 25: {"WebGPU M3 Pro": 11.8, "Metal M2 Pro": 10.0},
                  32: {"Metal M2 Pro": 10.8}, 80: {"WebGPU M3 Pro": 22.0, "Metal M2 Pro": 23.8}}


def latency_measure(model, cfg, Ts=(7, 25, 32, 80), reps=50, weights=None, cpu_threads_n=0):
    """Median latency (ms) of one B=1 forward at each T: device-resident
    (token ids and logits in HBM) and host in/out (copies included), after 5
    warmups; with `weights`, also the oracle forward on the host (median of 3
    after one warmup, cpu_threads_n threads). {T: {"dev", "host"[, "cpu"]}}"""
    from textsift_amd import synth
    out = {}
    for T in Ts:
        ids = synth.tagged_token_ids(7 + T, T, cfg.vocab_size)
        mask = np.ones(T, np.uint8)
        for _ in range(5):
            model.forward(ids, mask, 1, T)
        host = []
        for _ in range(reps):
            t0 = time.perf_counter()
            model.forward(ids, mask, 1, T)
            host.append((time.perf_counter() - t0) * 1000.0)
        be = model.backend
        ib, lb = be.buffer(ids), be.buffer(nbytes=T * cfg.num_classes * 4)
        for _ in range(3):
            model.forward_device(ib, None, 1, T, lb)
        dev = []
        for _ in range(reps):
            t0 = time.perf_counter()
            model.forward_device(ib, None, 1, T, lb)
            dev.append((time.perf_counter() - t0) * 1000.0)
        ib.release()
        lb.release()
        out[T] = {"dev": round(float(np.median(dev)), 4), "host": round(float(np.median(host)), 4)}
        if weights is not None:
            import oracle
            nt = cpu_threads_n or 1
            oracle.model_forward(cfg, weights, ids, n_threads=nt)
            ts = []
            for _ in range(3):
                t0 = time.perf_counter()
                oracle.model_forward(cfg, weights, ids, n_threads=nt)
                ts.append((time.perf_counter() - t0) * 1000.0)
            out[T]["cpu"] = round(float(np.median(ts)), 2)
    return out


def latency_table(model, cfg, reps=50):
    """Markdown table of latency_measure at the token counts the reference
    publishes, next to its published numbers (other hardware)."""
    rows = ["| T | host in/out ms (median) | device-resident ms (median) | reference (other hardware) |",
            "|---|---|---|---|"]
    lat = latency_measure(model, cfg, tuple(sorted(REF_LATENCY_MS)), reps)
    for T in sorted(REF_LATENCY_MS):
        ref = ", ".join(f"{k} {v} ms" for k, v in REF_LATENCY_MS[T].items())
        rows.append(f"| {T} | {lat[T]['host']:.3f} | {lat[T]['dev']:.3f} | {ref} |")
    return "\n".join(rows)


def cpu_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


# ---------------------------------------------------------------- per-config measurement

CACHE_COLD_BYTES = 512 << 20   # rotate inputs over at least this much memory: 2x the 256 MB MALL


def host_cpu():
    """(threads this process may use, CPU model name) of the host."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return n, model


def ref_default_threads(n):
    """The reference's WASM worker count for a host of n cores,
    max(2, min(6, cores - 1)) (browser/backends/wasm.ts:659-661)."""
    return max(2, min(6, n - 1))


def timed_threads(fn, n_threads, reps=3):
    """Median wall time of fn(n_threads) over reps runs (after one warmup)."""
    fn(n_threads)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn(n_threads)
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def sliced(fn, total, n_threads):
    """Runs fn(lo, hi) over n_threads contiguous slices of range(total) on host
    threads (the oracle's C code releases the GIL), as the reference's MtPool
    partitions its work (T-slices for GEMMs, H_q-slices for attention)."""
    from concurrent.futures import ThreadPoolExecutor
    n = max(1, min(n_threads, total))
    bounds = [(total * i // n, total * (i + 1) // n) for i in range(n)]
    with ThreadPoolExecutor(max_workers=n) as ex:
        list(ex.map(lambda b: fn(*b), bounds))


def cpu_baseline_both(work_fn, units, unit, sample):
    """The oracle timed at the reference's default thread count and at all host
    cores (capped at 16, the box's CPU share): {value, unit, cores, ...}."""
    n, model = host_cpu()
    allc = max(1, min(n, 16))
    refc = ref_default_threads(n)
    t_all = timed_threads(work_fn, allc)
    t_ref = t_all if refc == allc else timed_threads(work_fn, refc)
    return {"value": round(units / t_all, 3), "unit": unit, "cores": allc, "kind": "port",
            "sample": sample, "host_nproc": n, "cpu_model": model,
            "reference_default_threads": {"cores": refc, "value": round(units / t_ref, 3)}}


def time_dispatch(be, name, make_bindings, push, copies, reps):
    """Median device time (HIP events around the whole named dispatch, on the
    backend's stream) of `reps` one-shot dispatches, rotating over `copies`
    binding sets; the first 3 dispatches are warmups (the reference's method,
    tests/native/forward-vulkan.js:518-559: median of >= 10 after 3 warmups)."""
    be.profile(True)
    be.profile_select("dispatch:" + name)
    ts = []
    for i in range(reps + 3):
        be.profile_reset()
        be.dispatch(name, make_bindings(i % copies), push)
        n, ms = be.profile_report()["dispatch:" + name]
        if i >= 3:
            ts.append(ms * 1000.0)
    be.profile(False)
    be.profile_select(None)
    return float(np.median(ts)), float(np.min(ts))


def kernel_times(be, name, make_bindings, push, copies, reps):
    """Per-kernel median device times (us) of one named dispatch's launches."""
    be.profile(True)
    be.profile_select(None)
    per = {}
    for i in range(reps + 3):
        be.profile_reset()
        be.dispatch(name, make_bindings(i % copies), push)
        if i >= 3:
            for k, (n, ms) in be.profile_report().items():
                if not k.startswith("dispatch:"):
                    per.setdefault(k, []).append(ms * 1000.0)
    be.profile(False)
    return {k: round(float(np.median(v)), 3) for k, v in per.items()}


def roof(achieved, peak, unit, traffic=None):
    return {"bound": "hbm" if unit == "GB/s" else "mfma", "achieved": round(achieved, 2), "peak": peak,
            "unit": unit, "frac": round(achieved / peak, 4), "traffic": traffic}


def bench_config(cfg_id, reps, variant="both", no_cpu=False, calib_mb=0):
    """BASELINE config 1-4 (each kernel on its own, cache-warm and cache-cold),
    with the roofline against MI355X peaks and the oracle CPU baseline at both
    thread settings: the dict of one JSON line."""
    import oracle
    from textsift_amd import _native, synth
    from textsift_amd.config import PF_CONFIG as cfg
    be = _native.Backend(0)
    if calib_mb:
        run_calibration(be, calib_mb)
    u32 = lambda *v: np.array(v, np.uint32).tobytes()
    keep = []
    nan2 = (float("nan"), float("nan"))
    do_warm, do_cold = variant in ("both", "warm"), variant in ("both", "cold")

    def buf(a=None, nbytes=None):
        b = be.buffer(a) if a is not None else be.buffer(nbytes=nbytes)
        keep.append(b)
        return b

    out = {"n_gpus": 1, "higher_is_better": False, "data": "synthetic (seeded)", "dtype": None}
    if cfg_id == 1:
        T, N, K = 512, 640, 640
        x = synth.to_fp16_bits(synth.normal(1, T * K)).reshape(T, K)
        w = synth.qweight(2, N, K, zp=8, bias_sigma=None)
        alg_bytes = T * K * 2 + N * K // 2 + N * (K // 32) * 2 + T * N * 2
        flops = 2.0 * T * N * K
        ws = alg_bytes + N * (K // 32) * 4
        copies = max(1, CACHE_COLD_BYTES // ws) if do_cold else 1
        sets = []
        for c in range(copies):
            wq, ws_, wz = buf(w["int4"]), buf(w["scales"]), buf(w["zp"])
            w4, sz = buf(nbytes=N * K // 2), buf(nbytes=N * (K // 32) * 4)
            be.dispatch("w4_prepare", [wq, ws_, wz, w4, sz], u32(N, K, 1, 0))
            for b_ in (wq, ws_, wz):
                b_.release()
            sets.append([buf(x), w4, sz, buf(w["bias"]), buf(nbytes=T * N * 2)])
        push = u32(T, N, K, 0, 0, 0)
        name = "matmul_w4"
        warm = time_dispatch(be, name, lambda i: sets[0], push, 1, reps) if do_warm else nan2
        cold = time_dispatch(be, name, lambda i: sets[i], push, copies, reps) if do_cold else nan2
        got = sets[0][4].read(np.uint16).reshape(T, N)
        ref = oracle.matmul(x, w["int4"], w["scales"], w["zp"], w["bias"], N, K, x_f32=False, out_f32=False)
        err = float(np.linalg.norm(got.view(np.float16).astype(np.float64) - ref.view(np.float16))
                    / np.linalg.norm(ref.view(np.float16).astype(np.float64)))

        def cpu(nt):
            sliced(lambda lo, hi: oracle.matmul(x[lo:hi], w["int4"], w["scales"], w["zp"], w["bias"], N, K, False,
                                                False), T, nt)
        reps_cpu = 20
        cpu_b = None if no_cpu else cpu_baseline_both(lambda nt: [cpu(nt) for _ in range(reps_cpu)], reps_cpu * flops / 1e9, "GFLOP/s",
                                  f"{reps_cpu} x the config's GEMM (oracle MatMulNBits, T-slices)")
        out.update({"metric": "int4 GEMM 512x640x640 (fp16 in/out, blk32, zp 8) us/launch", "dtype": "int4w/fp16/f32-acc",
                    "config": {"workload": "BASELINE config 1: MatMulNBits int4 GEMM T=512 N=640 K=640",
                               "kernel": "k_gemm_w4 all-K 16-token tile (the forward's choice at 512 rows)"},
                    "algorithmic": {"bytes": alg_bytes, "flops": flops},
                    "value": round(warm[0] if do_warm else cold[0], 3), "unit": "us", "rel_err_vs_oracle": err})
        for tag, (med, mn) in (("warm", warm), ("cold", cold)):
            out[tag] = {"median_us": round(med, 3), "min_us": round(mn, 3),
                        "hbm": roof(alg_bytes / (med * 1e-6) / 1e9, HBM_PEAK_GBS, "GB/s"),
                        "mfma": roof(flops / (med * 1e-6) / 1e12, MFMA_FP16_PEAK_TFLOPS, "TFLOP/s")}
        out["cold"]["rotating_copies"] = copies
        out["roofline"] = out["cold"]["hbm"]
        out["roofline_time_us"] = round(max(alg_bytes / (HBM_PEAK_GBS * 1e3), flops / (MFMA_FP16_PEAK_TFLOPS * 1e6)), 3)
        out["cpu_baseline"] = cpu_b
        out["gpu_cpu_ratio"] = round(flops / (warm[0] * 1e-6) / 1e9 / cpu_b["value"], 1) if cpu_b else None
    elif cfg_id == 2:
        V, D, T = cfg.vocab_size, cfg.hidden_size, 32768
        tab = synth.qweight(3, V, D, zp=8, bias_sigma=None)
        ids = synth.token_ids(4, T, V)
        rows = len(np.unique(ids))
        alg_bytes = T * 4 + rows * (D // 2 + (D // 32) * 2 + (D // 64)) + T * D * 2
        tab_bytes = tab["int4"].nbytes + tab["scales"].nbytes + tab["zp"].nbytes
        copies = max(1, -(-CACHE_COLD_BYTES // (tab_bytes + T * D * 2))) if do_cold else 1
        sets = [[buf(tab["int4"]), buf(tab["scales"]), buf(tab["zp"]), buf(ids), buf(nbytes=T * D * 2)]
                for _ in range(copies)]
        push = u32(T, V, D, 0)
        name = "embed_lookup_int4"
        warm = time_dispatch(be, name, lambda i: sets[0], push, 1, reps) if do_warm else nan2
        cold = time_dispatch(be, name, lambda i: sets[i], push, copies, reps) if do_cold else nan2
        got = sets[0][4].read(np.uint16).reshape(T, D)
        ref = oracle.embed_lookup(tab["int4"], tab["scales"], tab["zp"], ids, V, D)
        exact = bool(np.array_equal(got, ref))

        def cpu(nt):
            sliced(lambda lo, hi: oracle.embed_lookup(tab["int4"], tab["scales"], tab["zp"], ids[lo:hi], V, D), T, nt)
        reps_cpu = 10
        cpu_b = None if no_cpu else cpu_baseline_both(lambda nt: [cpu(nt) for _ in range(reps_cpu)], reps_cpu * alg_bytes / 1e9, "GB/s",
                                  f"{reps_cpu} x the config's gather (oracle embed_lookup_int4, T-slices)")
        out.update({"metric": "GatherBlockQuantized 32768 ids x 640 (int4 table 200064 rows) us/launch",
                    "dtype": "u4->fp16", "config": {"workload": "BASELINE config 2: GatherBlockQuantized embedding",
                                                    "kernel": "k_embed", "distinct_rows": rows},
                    "algorithmic": {"bytes": alg_bytes}, "value": round(warm[0] if do_warm else cold[0], 3), "unit": "us",
                    "bit_exact_vs_oracle": exact})
        for tag, (med, mn) in (("warm", warm), ("cold", cold)):
            out[tag] = {"median_us": round(med, 3), "min_us": round(mn, 3),
                        "hbm": roof(alg_bytes / (med * 1e-6) / 1e9, HBM_PEAK_GBS, "GB/s")}
        out["cold"]["rotating_copies"] = copies
        out["roofline"] = out["cold"]["hbm"]
        out["roofline_time_us"] = round(alg_bytes / (HBM_PEAK_GBS * 1e3), 3)
        out["cpu_baseline"] = cpu_b
        out["gpu_cpu_ratio"] = round(alg_bytes / (warm[0] * 1e-6) / 1e9 / cpu_b["value"], 1) if cpu_b else None
    elif cfg_id == 3:
        T, D, E, K, F = 2048, cfg.hidden_size, cfg.num_experts, cfg.num_experts_per_tok, cfg.intermediate_size
        x = synth.to_fp16_bits(synth.normal(5, T * D)).reshape(T, D)
        rw_, rb = synth.zipf_router(6, D, E)
        gu = synth.qweight(7, 2 * F, D, lead=(E,))
        dn = synth.qweight(8, D, F, lead=(E,))
        exp_bytes = sum(gu[k].nbytes for k in ("int4", "scales", "zp", "bias")) + \
            sum(dn[k].nbytes for k in ("int4", "scales", "zp", "bias"))
        prep_bytes = E * 2 * F * (D // 2 + (D // 32) * 4 + 2) + E * D * (F // 2 + (F // 32) * 4 + 2)
        copies = max(1, -(-CACHE_COLD_BYTES // prep_bytes)) if do_cold else 1
        wsets = []
        for c in range(copies):
            pw = []
            for qw, rows, kk in ((gu, 2 * F, D), (dn, D, F)):
                wq, ws_, wz = buf(qw["int4"]), buf(qw["scales"]), buf(qw["zp"])
                w4, sz = buf(nbytes=E * rows * kk // 2), buf(nbytes=E * rows * (kk // 32) * 4)
                be.dispatch("w4_prepare", [wq, ws_, wz, w4, sz], u32(E * rows, kk, 1, 0))
                for b_ in (wq, ws_, wz):
                    b_.release()
                pw += [w4, sz, buf(qw["bias"])]
            wsets.append(pw)
        # the router weight is transposed to [E][D] once (as a weight upload would); the layer then
        # runs the forward's fused router chain: 5 launches
        xb, rws, rbb = buf(x), buf(rw_), buf(rb)
        rwb = buf(nbytes=D * E * 2)
        be.dispatch("transpose_f16", [rws, rwb], u32(D, E))
        ob, ib, wb = buf(nbytes=T * D * 2), buf(nbytes=T * K * 4), buf(nbytes=T * K * 4)
        push = u32(T, D, E, K, F, 0, 0, 1)
        name = "moe_ffn_w4"
        mk = lambda i: [xb, rwb, rbb] + wsets[i] + [ob, ib, wb]
        warm = time_dispatch(be, name, lambda i: mk(0), push, 1, reps) if do_warm else nan2
        cold = time_dispatch(be, name, mk, push, copies, reps) if do_cold else nan2
        per_kernel = kernel_times(be, name, lambda i: mk(0), push, 1, max(5, reps // 2))
        ridx = ib.read(np.int32).reshape(T, K)
        rwt = wb.read(np.float32).reshape(T, K)
        y = ob.read(np.uint16).reshape(T, D)
        counts = np.bincount(ridx.ravel(), minlength=E)
        srt = np.sort(counts)[::-1]
        nz = srt[srt > 0][:32]  # the head: the tail's few-token counts are noise
        rank = np.arange(1, nz.size + 1)
        zipf_s = float(-np.polyfit(np.log(rank), np.log(nz), 1)[0])
        zref = np.arange(1, E + 1, dtype=np.float64) ** -1.1
        touched = int((counts > 0).sum())
        alg_flops = 2.0 * T * D * E + 2.0 * T * K * (2 * F * D + D * F)
        alg_bytes = int(touched / E * exp_bytes) + D * E * 2 + E * 2 + T * D * 2 * 2 + T * K * 8
        w = {}
        for kk, vv in gu.items():
            w[f"layers.0.experts.gate_up.{kk}"] = vv
        for kk, vv in dn.items():
            w[f"layers.0.experts.down.{kk}"] = vv
        for nm in ("attn.q_proj", "attn.k_proj", "attn.v_proj", "attn.o_proj", "router"):
            for kk, vv in synth.qweight(9, 64, 64).items():
                w[f"layers.0.{nm}.{kk}"] = vv
        w["layers.0.input_layernorm"] = w["layers.0.post_attention_layernorm"] = np.zeros(D, np.uint16)
        w["layers.0.attn.sinks"] = np.zeros(cfg.num_heads, np.float32)
        xf = oracle.fp16_to_f32(x)
        ref = oracle.expert_dispatch(cfg, w, 0, xf, ridx, rwt * np.float32(0.25), n_slices=8)
        err = float(np.linalg.norm(y.view(np.float16).astype(np.float64) - ref.view(np.float16))
                    / np.linalg.norm(ref.view(np.float16).astype(np.float64)))
        wr = oracle.fp16_to_f32(rw_).reshape(D, E)
        br = oracle.fp16_to_f32(rb)

        def cpu(nt):
            lg = np.empty((T, E), np.float32)
            sliced(lambda lo, hi: np.matmul(xf[lo:hi], wr, out=lg[lo:hi]), T, nt)
            lg += br
            ix, vals = oracle.topk(lg, T, E, K)
            sm = oracle.softmax(vals, T, K)
            oracle.expert_dispatch(cfg, w, 0, xf, ix, sm * np.float32(0.25), n_slices=nt)
        cpu_b = None if no_cpu else cpu_baseline_both(cpu, alg_flops / 1e9, "GFLOP/s",
                                  "the config's MoE layer: router (numpy f32), oracle top-k/softmax and expert-major "
                                  "dispatch (token slices)")
        out.update({"metric": "MoE FFN layer T=2048, 128 experts top-4, Zipf(1.1) router us/layer",
                    "dtype": "int4w/fp16-mfma/f32-acc",
                    "config": {"workload": "BASELINE config 3: one MoE FFN layer", "kernels": per_kernel,
                               "expert_tile": 64},
                    "algorithmic": {"flops": alg_flops, "bytes": alg_bytes, "experts_touched": touched},
                    "zipf": {"fitted_s_top32": round(zipf_s, 3), "max_load": int(srt[0]), "min_load": int(srt[-1]),
                             "top8_share": round(float(srt[:8].sum() / srt.sum()), 4),
                             "zipf_1.1_top8_share": round(float(zref[:8].sum() / zref.sum()), 4),
                             "loads_sorted": [int(v) for v in srt]},
                    "value": round(warm[0] if do_warm else cold[0], 3), "unit": "us", "rel_err_vs_oracle": err})
        for tag, (med, mn) in (("warm", warm), ("cold", cold)):
            out[tag] = {"median_us": round(med, 3), "min_us": round(mn, 3),
                        "hbm": roof(alg_bytes / (med * 1e-6) / 1e9, HBM_PEAK_GBS, "GB/s"),
                        "mfma": roof(alg_flops / (med * 1e-6) / 1e12, MFMA_FP16_PEAK_TFLOPS, "TFLOP/s")}
        out["cold"]["rotating_copies"] = copies
        out["roofline"] = out["cold"]["hbm"]
        out["roofline_time_us"] = round(max(alg_bytes / (HBM_PEAK_GBS * 1e3),
                                            alg_flops / (MFMA_FP16_PEAK_TFLOPS * 1e6)), 3)
        out["cpu_baseline"] = cpu_b
        out["gpu_cpu_ratio"] = round(alg_flops / (warm[0] * 1e-6) / 1e9 / cpu_b["value"], 1) if cpu_b else None
    elif cfg_id == 4:
        T, Hq, Hkv, hd, W = 8192, 14, 2, 64, 128
        q = synth.to_fp16_bits(synth.normal(10, T * Hq * hd)).reshape(T, Hq * hd)
        k = synth.to_fp16_bits(synth.normal(11, T * Hkv * hd)).reshape(T, Hkv * hd)
        v = synth.to_fp16_bits(synth.normal(12, T * Hkv * hd)).reshape(T, Hkv * hd)
        sinks = np.full(Hq, -np.inf, np.float32)
        alg_bytes = 2 * q.nbytes + k.nbytes + v.nbytes
        t = np.arange(T)
        keys = float((np.minimum(T, t + W + 1) - np.maximum(0, t - W)).sum())
        flops = 4.0 * hd * Hq * keys
        copies = max(1, -(-CACHE_COLD_BYTES // alg_bytes)) if do_cold else 1
        sets = [[buf(q), buf(k), buf(v), buf(sinks), buf(np.ones(T, np.uint8)), buf(nbytes=q.nbytes)]
                for _ in range(copies)]
        push = u32(T, Hq, Hkv, hd, W, 0) + np.array([0.125], np.float32).tobytes() + u32(1)
        name = "banded_attention"
        warm = time_dispatch(be, name, lambda i: sets[0], push, 1, reps) if do_warm else nan2
        cold = time_dispatch(be, name, lambda i: sets[i], push, copies, reps) if do_cold else nan2
        got = sets[0][5].read(np.uint16).reshape(T, Hq * hd)
        # scale 1/8 applied to Q in fp16 is exact (a power of two, no subnormal results for N(0,1) inputs)
        qs = synth.to_fp16_bits(oracle.fp16_to_f32(q) * np.float32(0.125)).reshape(T, Hq * hd)
        ref = oracle.banded_attention_wgsl(qs, k, v, sinks, None, T, Hq, Hkv, hd, W)
        err = float(np.linalg.norm(got.view(np.float16).astype(np.float64) - ref.view(np.float16))
                    / np.linalg.norm(ref.view(np.float16).astype(np.float64)))

        def cpu(nt):
            sliced(lambda h0, h1: oracle.banded_attention(qs, k, v, sinks, None, T, Hq, Hkv, hd, W, h0, h1), Hq, nt)
        cpu_b = None if no_cpu else cpu_baseline_both(cpu, flops / 1e9, "GFLOP/s",
                                  "the config's attention (oracle banded_attention, H_q slices, attention.ts:156-182)")
        out.update({"metric": "banded GQA attention T=8192 14/2 heads d=64 +-128 us/launch", "dtype": "fp16/f32-acc",
                    "config": {"workload": "BASELINE config 4: banded bidirectional GQA attention, scale 1/8, no sinks",
                               "kernel": "k_banded_attention_hw"},
                    "algorithmic": {"bytes": alg_bytes, "flops": flops}, "value": round(warm[0] if do_warm else cold[0], 3), "unit": "us",
                    "rel_err_vs_oracle": err})
        for tag, (med, mn) in (("warm", warm), ("cold", cold)):
            out[tag] = {"median_us": round(med, 3), "min_us": round(mn, 3),
                        "hbm": roof(alg_bytes / (med * 1e-6) / 1e9, HBM_PEAK_GBS, "GB/s"),
                        "mfma": roof(flops / (med * 1e-6) / 1e12, MFMA_FP16_PEAK_TFLOPS, "TFLOP/s")}
        out["cold"]["rotating_copies"] = copies
        out["roofline"] = out["cold"]["hbm"]
        out["roofline_time_us"] = round(max(alg_bytes / (HBM_PEAK_GBS * 1e3), flops / (MFMA_FP16_PEAK_TFLOPS * 1e6)), 3)
        out["cpu_baseline"] = cpu_b
        out["gpu_cpu_ratio"] = round(flops / (warm[0] * 1e-6) / 1e9 / cpu_b["value"], 1) if cpu_b else None
    else:
        raise SystemExit(f"unknown config {cfg_id}")
    for b_ in keep:
        b_.release()
    be.close()
    return out


def config_summary(out):
    """The compact per-config record the headline line carries: kernel time
    (median of the reference's method, us) warm and HBM-cold, the cold roofline
    fraction and its bound, the CPU baseline at all cores and at the
    reference's default thread count, and the parity check's result."""
    cpu = out.get("cpu_baseline")
    parity = ("bit-exact" if out.get("bit_exact_vs_oracle") else "NOT bit-exact") \
        if "bit_exact_vs_oracle" in out else f"rel-err {out.get('rel_err_vs_oracle', float('nan')):.2e}"
    rec = {"us": [out["warm"]["median_us"], out["cold"]["median_us"]],
           "frac": out["roofline"]["frac"], "bound": out["roofline"]["bound"],
           "roofline_us": out["roofline_time_us"], "parity": parity}
    if "mfma" in out["cold"]:
        rec["mfma_frac"] = out["cold"]["mfma"]["frac"]
    if cpu:
        rec["cpu"] = [cpu["value"], cpu["reference_default_threads"]["value"], cpu["unit"]]
    if "zipf" in out:
        rec["launches"] = len(out["config"]["kernels"])
    return rec


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--config", type=int, default=5, choices=[1, 2, 3, 4, 5],
                    help="BASELINE config: 5 = the full forward (default); 1-4 = one kernel on its own")
    ap.add_argument("--reps", type=int, default=20, help="timed dispatches per variant for --config 1-4")
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--seq", type=int, default=2048)
    ap.add_argument("--seed", type=int, default=20260101)
    ap.add_argument("--cpu-seqs", type=int, default=2,
                    help="CPU baseline sample: this many of the batch's sequences (full length) through the oracle")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-profile", action="store_true")
    ap.add_argument("--precision", choices=["fp16", "split"], default="fp16",
                    help="numerics of the forward: fp16 (the reference's GPU paths, the default) or split (its WASM path)")
    ap.add_argument("--profile-steps", type=int, default=2, help="steps of the all-kernel profiled pass")
    ap.add_argument("--copy-calibration-mb", type=int, default=0)
    ap.add_argument("--traffic-report", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"))
    ap.add_argument("--copy-mb", type=int, default=1024)
    ap.add_argument("--raw-symbols", action="store_true", help="--traffic-report: group by kernel symbol")
    ap.add_argument("--stats-report", metavar="KERNEL_STATS_CSV", help="markdown table of a rocprofv3 --stats csv")
    ap.add_argument("--variant", choices=["both", "warm", "cold"], default="both",
                    help="--config 1-4: which cache variants to time (one alone for rocprofv3 runs)")
    ap.add_argument("--sq-report", nargs=2, metavar=("PASS1_CSV", "PASS2_CSV"),
                    help="summarise two rocprofv3 --pmc passes of the counters in SQ_PASS1 / SQ_PASS2")
    ap.add_argument("--blas-reference", action="store_true",
                    help="print a table of each forward GEMM next to a dense fp16 torch.matmul (hipBLASLt) of "
                         "the same M x N x K, then exit")
    ap.add_argument("--blas-torch", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--recipe", choices=["spread", "uniform"], default="spread",
                    help="synthetic weights (textsift_amd.synth.make_model_weights): spread (the default) or the "
                         "earlier uniform recipe, whose routing collapses")
    ap.add_argument("--headline-only", action="store_true",
                    help="config 5 only: skip the small-T latencies, the collapsed-model comparison and configs 1-4")
    ap.add_argument("--latency", action="store_true",
                    help="single-sequence forward latency at the token counts the reference publishes, then exit")
    args = ap.parse_args()
    if args.copy_calibration_mb:
        # the counter calibration's copy and gather kernels are measurement tooling of the library
        os.environ["PFHIP_TOOLING"] = "1"

    if args.blas_torch:  # the torch half of --blas-reference, in a process of its own
        from textsift_amd.config import PF_CONFIG
        print(json.dumps(blas_torch_times(PF_CONFIG, args.batch * args.seq)))
        return
    blas_ref = None
    if args.blas_reference:
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--blas-torch", "--batch", str(args.batch),
                            "--seq", str(args.seq)], capture_output=True, text=True)
        if r.returncode != 0:
            print(r.stderr, file=sys.stderr)
            sys.exit(r.returncode)
        blas_ref = json.loads(r.stdout.strip().splitlines()[-1])

    if args.traffic_report:
        print(traffic_report(args.traffic_report[0], args.traffic_report[1], args.copy_mb, raw=args.raw_symbols))
        return
    if args.stats_report:
        print(stats_report(args.stats_report))
        return
    if args.sq_report:
        print(sq_report(args.sq_report[0], args.sq_report[1]))
        return

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(across GPUs the forward shards as independent sequences, one process per GPU)", file=sys.stderr)
        sys.exit(2)

    if args.config != 5:
        print(json.dumps(bench_config(args.config, args.reps, args.variant, args.no_cpu, args.copy_calibration_mb)))
        return

    from textsift_amd import _native, synth
    from textsift_amd.config import PF_CONFIG

    cfg = PF_CONFIG
    B, T = args.batch, args.seq
    M = B * T
    t_gen = time.time()
    weights = synth.make_model_weights(cfg, seed=args.seed, recipe=args.recipe)
    ids = (synth.tagged_token_ids(args.seed + 1, M) if args.recipe == "spread" else synth.token_ids(args.seed + 1, M))
    gen_s = time.time() - t_gen

    be = _native.Backend(0)
    prec = _native.PRECISION_FP16 if args.precision == "fp16" else _native.PRECISION_SPLIT
    model = load_model(be, cfg, weights, prec)
    ids_buf = be.buffer(ids)
    logits_buf = be.buffer(nbytes=M * cfg.num_classes * 4)

    if args.latency:
        print(latency_table(model, cfg))
        return

    for _ in range(args.warmup):
        model.forward_device(ids_buf, None, B, T, logits_buf)

    if args.copy_calibration_mb:
        run_calibration(be, args.copy_calibration_mb)

    # per-kernel table: a separate profiled pass with every launch bracketed
    prof, dom = {}, None
    if not args.no_profile and args.profile_steps > 0:
        be.profile(True)
        be.profile_select(None)
        be.profile_reset()
        for _ in range(args.profile_steps):
            model.forward_device(ids_buf, None, B, T, logits_buf)
        prof = be.profile_report()
        dom = max(prof.items(), key=lambda kv: kv[1][1])[0]
        # the timed region brackets the dominant kernel only
        be.profile_reset()
        be.profile_select(dom)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        model.forward_device(ids_buf, None, B, T, logits_buf)
    t1 = time.perf_counter()
    dom_prof = be.profile_report().get(dom) if dom else None
    be.profile(False)
    be.profile_select(None)
    ms_per_step = (t1 - t0) * 1000.0 / args.steps
    tok_s = M / (ms_per_step / 1000.0)

    if args.blas_reference:
        print(blas_reference_table(cfg, M, prof, blas_ref))
        return

    logits = logits_buf.read(np.float32).reshape(M, cfg.num_classes)
    finite = bool(np.isfinite(logits).all())
    am = np.argmax(logits, 1)
    argmax = {"classes": int(np.unique(am).size), "max_share": round(float(np.bincount(am).max() / M), 4)}
    if args.recipe == "spread":
        argmax["planted_tag_agreement"] = round(float(np.mean(am == ids % cfg.num_classes)), 5)

    # the realised expert load per layer (one forward with the routing taps on)
    model.enable_taps(True)
    model.forward_device(ids_buf, None, B, T, logits_buf)
    K, E = cfg.num_experts_per_tok, cfg.num_experts
    loads = [synth.routing_load(model.tap(f"ridx.{l}", np.int32, M * K), E) for l in range(cfg.num_layers)]
    model.enable_taps(False)
    routing = {"experts_touched": [r["touched"] for r in loads],
               "max_share": [round(r["max_share"], 4) for r in loads],
               "top20_share": [round(r["top20_share"], 3) for r in loads],
               "under_0p1pct": [r["under_0p1pct"] for r in loads]}

    # roofline of the dominant kernel
    flops = gemm_flops(cfg, M)
    flops["banded_attention"] = attention_flops(cfg, B, T) / 1.0  # per launch (one per layer)
    roof = None
    kernels = {}
    if prof:
        for name, (n, ms) in prof.items():
            kernels[name] = round(1000.0 * ms / n, 2)
    if dom_prof and dom in flops:
        n, ms = dom_prof
        avg_s = ms / n / 1000.0
        achieved = flops[dom] / avg_s / 1e12
        roof = {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_FP16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / MFMA_FP16_PEAK_TFLOPS, 4), "traffic": read_traffic(dom, B, T),
                "flops_per_launch": flops[dom], "avg_launch_us": round(avg_s * 1e6, 2),
                "launches_timed": n}
    total_flops = sum(flops[k] * cfg.num_layers for k in
                      ("gemm_qkv_rope", "gemm_o", "gemm_router", "gemm_moe_gate_up", "gemm_moe_down",
                       "banded_attention")) + flops["gemm_classifier"]

    n_host, cpu_model = host_cpu()
    thr = args.cpu_threads or cpu_threads()
    refc = ref_default_threads(n_host)
    extra = {}
    if not args.headline_only:
        # small T: the reference's published forward sizes, one sequence each
        extra["latency_ms"] = {str(t): v for t, v in latency_measure(
            model, cfg, (7, 25, 80), reps=30, weights=None if args.no_cpu else weights, cpu_threads_n=refc).items()}
    model.close()
    ids_buf.release()
    logits_buf.release()

    if not args.headline_only:
        # the collapsed model of the "uniform" recipe, same batch: labelled comparison value
        wu = synth.make_model_weights(cfg, seed=args.seed, recipe="uniform")
        mu = load_model(be, cfg, wu, prec)
        idu = synth.token_ids(args.seed + 1, M)
        ib, lb = be.buffer(idu), be.buffer(nbytes=M * cfg.num_classes * 4)
        for _ in range(args.warmup):
            mu.forward_device(ib, None, B, T, lb)
        steps_u = max(5, args.steps // 2)
        t2 = time.perf_counter()
        for _ in range(steps_u):
            mu.forward_device(ib, None, B, T, lb)
        ms_u = (time.perf_counter() - t2) * 1000.0 / steps_u
        mu.enable_taps(True)
        mu.forward_device(ib, None, B, T, lb)
        touched_u = [synth.routing_load(mu.tap(f"ridx.{l}", np.int32, M * K), E)["touched"]
                     for l in range(cfg.num_layers)]
        mu.close()
        ib.release()
        lb.release()
        del wu
        extra["collapsed_model"] = {
            "ms_per_step": round(ms_u, 3), "tokens_per_s": round(M / (ms_u / 1000.0), 1),
            "experts_touched": touched_u,
            "note": "earlier synthetic recipe (uniform nibbles 0-15, zp 8): routing collapses onto a few experts, "
                    "one class for every token; not the headline"}
    be.close()

    if not args.headline_only:
        # BASELINE configs 1-4, each kernel on its own (warm and HBM-cold), with their CPU baselines
        extra["configs"] = {}
        for c in (1, 2, 3, 4):
            extra["configs"][str(c)] = config_summary(bench_config(c, args.reps, "both", args.no_cpu))

    cpu = None
    if not args.no_cpu:
        # the oracle (C restatement of the WASM path, the reference's MtPool
        # partitioning) on whole sequences of the batch: all host cores (<= 16,
        # the box's CPU share) and the reference's default worker count; the
        # sequences run one after another as the reference runs its chunks, so
        # tokens/s of the sample is that of the whole 16-sequence batch
        import oracle

        def cpu_rate(nthr, nseq):
            t2 = time.perf_counter()
            for b in range(nseq):
                oracle.model_forward(cfg, weights, ids[b * T:(b + 1) * T], n_threads=nthr)
            return nseq * T / (time.perf_counter() - t2), time.perf_counter() - t2

        nseq = max(1, min(args.cpu_seqs, B))
        v_all, s_all = cpu_rate(thr, nseq)
        v_ref, s_ref = cpu_rate(refc, 1) if refc != thr else (v_all, 0.0)
        cpu = {"value": round(v_all, 2), "unit": "tokens/s", "cores": thr, "kind": "port",
               "sample": f"{nseq} of the batch's {B} sequences ({nseq}x{T} tokens, {s_all:.1f} s) through the oracle "
                         f"(C restatement of the WASM path, MtPool partitioning, {thr} threads); sequences run "
                         f"serially, so the rate extrapolates to all {B}",
               "host_nproc": n_host, "cpu_model": cpu_model,
               "reference_default_threads": {"cores": refc, "value": round(v_ref, 2),
                                             "sample": f"1 sequence ({T} tokens, {s_ref:.1f} s)"}}

    out = {
        "metric": "tokens/sec full encoder fwd @16x2048; int4 GEMM % HBM/MFMA roofline",
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4w/fp16-mfma/f32-acc" if args.precision == "fp16" else "int4w/f32-as-fp16x2-mfma/f32-acc",
        "precision": args.precision,
        "data": (f"synthetic: seeded random-init int4 weights ({args.recipe} recipe), token ids "
                 + ("uniform over the vocabulary, drawn as legal BIOES runs of the ids' planted classes"
                    if args.recipe == "spread" else "uniform")),
        "config": {"workload": "full synthetic 8-layer int4 MoE encoder forward (BASELINE config 5)",
                   "batch": B, "seq_len": T, "layers": cfg.num_layers, "experts": cfg.num_experts,
                   "topk": cfg.num_experts_per_tok, "vocab": cfg.vocab_size, "window": cfg.sliding_window},
        "roofline": roof,
        "cpu_baseline": cpu,
        "model_tflops_per_s": round(total_flops / (ms_per_step / 1000.0) / 1e12, 2),
        "routing": routing,
        "argmax": argmax,
        "kernels_us": kernels,
        "logits_finite": finite,
    }
    out.update(extra)
    print(json.dumps(out))


def load_model(be, cfg, weights, prec):
    from textsift_amd import _native
    model = _native.Model(be, cfg, precision=prec)
    for name, arr in weights.items():
        model.set_weight(name, arr)
    model.finalize()
    return model


if __name__ == "__main__":
    main()
