"""Benchmark of the NSA selection path on one MI355X.

A step is one pass of the hot path over one layer of BASELINE config 3 (Wan2.1-1.3B shape: one
81-frame clip = 32760 tokens, 12 heads x 128, bf16, 64-token blocks, groups of 64 queries,
top-16, causal by 4680-token chunks), inputs resident in HBM:

    k_cmp = block_pool(k, 64)                       # block compression
    ids   = parallel_nsa_topk(q, k_cmp, 16, ...)    # query pooling + scoring + top-k
    out   = sel_fwd(q, k, v, ids, ...)              # selection attention forward

All 30 layers of a forward have this shape, so a forward is 30 steps.  ``value`` is the useful
selection-attention TFLOP/s of the whole step (4 * D * visible selected tokens per query, summed,
divided by the step time); ``roofline`` is the selection-attention kernel alone, timed with HIP
events on the stream it runs on.  Config 2 (top-k alone) is timed beside it and reported as
``topk`` (GB/s of algorithmic bytes), and the selection backward of the same layer as ``sel_bwd``
(useful work 2.5x the forward's).  ``ms_per_ar_chunk`` runs the AR driver (configs 4 and 5).
``cpu_baseline`` times the reference's PyTorch CPU formulation (oracle/cpu_baseline.py) on a
bounded sample of the same workload.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from typing import Optional

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "sel-attn TFLOP/s + %MFMA peak; top-k GB/s; ms per AR chunk at 60s cache"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
PEAK_FP8_TFLOPS = 5000.0    # MI355X dense fp8 MFMA
PEAK_FP32_TFLOPS = 157.3    # MI355X dense fp32 MFMA

# config 3, one layer
M = N = 32760
H, D, BS, G, TOPK, CHUNK = 12, 128, 64, 64, 16, 4680
# config 2: 512 query blocks of 64 (32760 tokens + 8 pad), 512 compressed key blocks
C2_T, C2_NC = 32768, 512
C2_BYTES = C2_T * H * D * 2 + C2_NC * H * D * 2 + (C2_T // 64) * H * TOPK * 4


# Algorithmic work per dispatch of the kernels the rocprof summaries price (bytes for HBM-bound
# kernels, FLOPs for MFMA-bound ones), keyed by rocprofv3 kernel-name prefix, per workload.
# AR shapes: one 4680-token chunk, 12 heads x 128, 64-token pages (74 per chunk), 80 cached
# chunks (5920 pooled blocks), top-16, a window of 3 chunks.
_AR_C, _AR_PPC, _AR_HIST, _AR_WIN = CHUNK, -(-CHUNK // BS), 80, 3
ALGO = {
    "c3": {
        # config 2 and the config-3 layer's top-k (32768 / 32760 tokens: the same to 0.03 %)
        "topk_mfma_kernel<bf16_t, 128, true>": ("bytes", C2_BYTES),
        # K compression of the config-3 layer: read k, write k_cmp
        "pool_rows_kernel<bf16_t>": ("bytes", M * H * D * 2 + (M // BS + 1) * H * D * 2),
    },
    "ar": {
        # append of one layer-forward: read the chunk's K and V, write their pages (74 x 64
        # slots each) and pooled rows; fp8 writes 1-byte codes and a scale per (page, head)
        "paged_append_wg_kernel<false>": ("bytes", 2 * _AR_C * H * D * 2
                                          + 2 * _AR_PPC * BS * H * D * 2
                                          + 2 * _AR_PPC * H * D * 2),
        "paged_append_wg_kernel<true>": ("bytes", 2 * _AR_C * H * D * 2
                                         + 2 * _AR_PPC * BS * H * D + 2 * _AR_PPC * H * 4
                                         + 2 * _AR_PPC * H * D * 2),
        # the per-(page, head, K or V) append kernel that serves head dims 64 / 128: the same
        # bytes per dispatch; the fp8 caches also write the chunk's bf16 K / V into the window
        # ring from the kernel's registers
        "paged_append_kv_kernel<false>": ("bytes", 2 * _AR_C * H * D * 2
                                          + 2 * _AR_PPC * BS * H * D * 2
                                          + 2 * _AR_PPC * H * D * 2),
        "paged_append_kv_kernel<true>": ("bytes", 2 * _AR_C * H * D * 2
                                         + 2 * _AR_PPC * BS * H * D + 2 * _AR_PPC * H * 4
                                         + 2 * _AR_PPC * H * D * 2 + 2 * _AR_C * H * D * 2),
        # selection over the history (cache.select): 4680 queries x 12 heads x 16 pages x 64
        # tokens, 4 D FLOPs each (bf16 pages, some host-resident; fp8 pages)
        "sel_fwd_dma_kernel<bf16_t, PagedAcc<bf16_t>, 128, 2>": (
            "flops", 4 * D * _AR_C * H * TOPK * BS),
        "sel_fwd_mfma_kernel<bf16_t, PagedAcc<unsigned char>, 128, false>": (
            "flops", 4 * D * _AR_C * H * TOPK * BS),
        # the fp8 Q K^T variant: half the FLOPs (Q K^T) on fp8 MFMA, half (P V) on bf16
        "sel_fwd_mfma_kernel<bf16_t, PagedAcc<unsigned char>, 128, true>": (
            "flops_qk8", 4 * D * _AR_C * H * TOPK * BS),
        # bf16 window attention over the window's pages: 4680 queries x 3 chunks of keys
        "sel_fwd_dma_kernel<bf16_t, PagedAcc<bf16_t>, 128, 4>": (
            "flops", 4 * D * _AR_C * H * _AR_WIN * _AR_C),
        # gated mix after an fp8 selection: read the compressed, selected and window outputs
        # and the three gates, write the mixed output (in place over the selected one)
        "branch_mix_kernel": ("bytes", 4 * _AR_C * H * D * 2 + _AR_C * H * 3 * 2),
    },
}
# config 1 (bench.py --c1-only): useful FLOPs of the seeded fp32 call, counted from its ids by
# useful_flops (the queries as the last frame: every selected block visible)
ALGO["c1"] = {"sel_fwd_f32mfma_kernel<DenseAcc<float>, 128>": ("flops_fp32", 9602498560),
             "sel_fwd_f32split_kernel<DenseAcc<float>, 128>": ("flops_fp32", 9602498560)}
# kernels one call launches together, priced as a whole: the AR top-k (query pooling into the
# workspace, split scoring + selection, merge) reads the chunk's q and the pooled history
ALGO_GROUPS = {
    "ar": {
        "AR top-k call (pool_rows_wg + topk_mfma + merge)": (
            ["pool_rows_wg_kernel<bf16_t>", "topk_mfma_kernel<bf16_t, 128, false>",
             "topk_merge_kernel"],
            "bytes", _AR_C * H * D * 2 + _AR_HIST * _AR_PPC * H * D * 2
            + _AR_PPC * H * TOPK * 4),
    },
    # the split fp32 call: equal runs of selected blocks per workgroup, then the merge of the
    # split items' records
    "c1": {
        "config-1 call (f32split + f32merge)": (
            ["sel_fwd_f32split_kernel<DenseAcc<float>, 128>", "sel_fwd_f32merge_kernel<128>"],
            "flops_fp32", 9602498560),
    },
}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-seconds", type=float, default=15.0,
                   help="target duration of the CPU baseline sample")
    p.add_argument("--ar-history", type=int, default=80,
                   help="cached chunks before the timed AR steps (80 chunks = 240 latent frames)")
    p.add_argument("--ar-steps", type=int, default=3, help="timed AR chunks per cache dtype")
    p.add_argument("--no-ar", action="store_true", help="skip the AR (configs 4 and 5) leg")
    p.add_argument("--no-full", action="store_true",
                   help="skip the config-3 30-layer forward and the config-1 call")
    p.add_argument("--full-only", action="store_true",
                   help="only the config-3 30-layer forward and the config-1 call")
    p.add_argument("--c1-only", action="store_true",
                   help="only the config-1 fp32 selection call (its rocprof profile)")
    p.add_argument("--ar-only", action="store_true",
                   help="run only the AR leg (configs 4 and 5) and print its results (profiling "
                        "runs of the cache kernels)")
    p.add_argument("--rocprof-summary", nargs=2, metavar=("OUT", "DIR"),
                   help="summarise the rocprofv3 runs under DIR (stats/, fetch/, write/, "
                        "copy_fetch/, copy_write/) into OUT.json and OUT.md, then exit")
    p.add_argument("--rocprof-md", metavar="JSON",
                   help="rewrite the text form (.md) of a committed rocprof summary and exit")
    p.add_argument("--summary-command", default="",
                   help="the command lines that produced the runs, recorded in the summary")
    p.add_argument("--summary-workload", default="c3", choices=sorted(ALGO),
                   help="which algorithmic-work table prices the summary's kernels")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run 5 device copies of 256 MiB (the reference kernel for scaling "
                        "rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes) and exit")
    return p.parse_args()


def copy_calibration():
    """5 copies of a 256 MiB device buffer: a kernel of known traffic (256 MiB read + 256 MiB
    written per dispatch) for calibrating the HBM byte counters."""
    import torch
    n = 256 * 1024 * 1024
    a = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "copies": 5}))


def _short_kernel_name(n: str) -> str:
    n = n.replace("omm::(anonymous namespace)::", "").replace("omm::", "").replace("void ", "")
    depth = 0
    for i, ch in enumerate(n):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return n[:i]
    return n


def _csv_rows(d: str, suffix: str):
    import csv
    import glob
    for path in glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True):
        with open(path) as f:
            yield from csv.DictReader(f)


def rocprof_summary(out: str, d: str, command: str, workload: str = "c3"):
    """Kernel durations (``--kernel-trace --stats``) and HBM bytes per dispatch (``--pmc
    FETCH_SIZE`` / ``WRITE_SIZE``, medians in KiB, scaled by the same counters' reading of a
    256 MiB device copy) of every kernel of one workload, with the ALGO figures priced against
    the MI355X peaks."""
    import statistics
    stats = {}
    for r in _csv_rows(os.path.join(d, "stats"), "kernel_stats.csv"):
        stats[_short_kernel_name(r["Name"])] = (int(r["Calls"]), float(r["AverageNs"]))
    med = {}
    for c, sub in (("FETCH_SIZE", "fetch"), ("WRITE_SIZE", "write"),
                   ("COPY_FETCH", "copy_fetch"), ("COPY_WRITE", "copy_write")):
        vals = {}
        for r in _csv_rows(os.path.join(d, sub), "counter_collection.csv"):
            vals.setdefault(_short_kernel_name(r["Kernel_Name"]), []).append(
                float(r["Counter_Value"]))
        med[c] = {k: statistics.median(v) for k, v in vals.items()}
    scale = {}
    for c, cc in (("FETCH_SIZE", "COPY_FETCH"), ("WRITE_SIZE", "COPY_WRITE")):
        cp = [v for k, v in med[cc].items() if "copyBuffer" in k]
        scale[c] = (256 * 1024) / cp[0] if cp else None
    kernels = {}
    for name, (calls, avg_ns) in sorted(stats.items(), key=lambda kv: -kv[1][0] * kv[1][1]):
        if "at::native" in name or "copyBuffer" in name:
            continue
        k = {"calls": calls, "avg_us": round(avg_ns / 1e3, 2)}
        f, w = med["FETCH_SIZE"].get(name), med["WRITE_SIZE"].get(name)
        if f is not None and w is not None and scale["FETCH_SIZE"] and scale["WRITE_SIZE"]:
            k["FETCH_SIZE"], k["WRITE_SIZE"] = f, w
            k["hbm_bytes_scaled"] = round(1024 * (f * scale["FETCH_SIZE"] + w * scale["WRITE_SIZE"]))
            k["hbm_GBps"] = round(k["hbm_bytes_scaled"] / avg_ns, 1)
        algo = next((v for p_, v in ALGO[workload].items() if name.startswith(p_)), None)
        if algo is not None:
            unit, amount = algo
            if unit == "bytes":
                k["algorithmic_bytes"] = amount
                k["algorithmic_GBps"] = round(amount / avg_ns, 1)
                k["frac_hbm_8TBps"] = round(amount / avg_ns / PEAK_HBM_GBS, 4)
            elif unit == "flops_fp32":
                k["useful_flops"] = amount
                k["useful_TFLOPs"] = round(amount / avg_ns / 1e3, 1)
                k["frac_fp32_peak"] = round(amount / avg_ns / 1e3 / PEAK_FP32_TFLOPS, 4)
            else:
                k["useful_flops"] = amount
                k["useful_TFLOPs"] = round(amount / avg_ns / 1e3, 1)
                k["frac_bf16_peak"] = round(amount / avg_ns / 1e3 / PEAK_BF16_TFLOPS, 4)
                if unit == "flops_qk8":
                    # time at peak: the Q K^T half at the fp8 rate, the P V half at bf16's
                    ideal_ns = (amount / 2) / (PEAK_FP8_TFLOPS * 1e3) + \
                               (amount / 2) / (PEAK_BF16_TFLOPS * 1e3)
                    k["frac_mixed_fp8_bf16_peak"] = round(ideal_ns / avg_ns, 4)
        kernels[name] = k
    # further counter passes (directories pmc_*): medians per dispatch, and for MFMA kernels the
    # executed bf16 MFMA rate (SQ_INSTS_VALU_MFMA_MOPS_BF16 counts units of 512 FLOPs), the MFMA
    # busy share of the busy CU-SIMD cycles and VALU instructions per MFMA instruction
    import glob as _glob
    for sub in sorted(_glob.glob(os.path.join(d, "pmc_*"))):
        vals = {}
        for r in _csv_rows(sub, "counter_collection.csv"):
            vals.setdefault((_short_kernel_name(r["Kernel_Name"]), r["Counter_Name"]), []).append(
                float(r["Counter_Value"]))
        for (name, cname), v in vals.items():
            if name in kernels:
                kernels[name].setdefault("counters", {})[cname] = statistics.median(v)
    for name, k in kernels.items():
        c = k.get("counters", {})
        if "SQ_INSTS_VALU_MFMA_MOPS_BF16" in c:
            fl = 512.0 * c["SQ_INSTS_VALU_MFMA_MOPS_BF16"]
            k["mfma_bf16_executed_TFLOPs"] = round(fl / (k["avg_us"] * 1e6), 1)
            k["mfma_bf16_executed_frac_peak"] = round(fl / (k["avg_us"] * 1e6) / PEAK_BF16_TFLOPS, 4)
        if c.get("SQ_BUSY_CU_CYCLES") and "SQ_VALU_MFMA_BUSY_CYCLES" in c:
            k["mfma_busy_share"] = round(c["SQ_VALU_MFMA_BUSY_CYCLES"] /
                                         (4.0 * c["SQ_BUSY_CU_CYCLES"]), 4)
        if c.get("SQ_INSTS_MFMA") and "SQ_INSTS_VALU" in c:
            k["valu_insts_per_mfma"] = round(c["SQ_INSTS_VALU"] / c["SQ_INSTS_MFMA"], 2)
        if c.get("TCC_HIT_sum") is not None and c.get("TCC_MISS_sum") is not None:
            tot = c["TCC_HIT_sum"] + c["TCC_MISS_sum"]
            k["l2_hit_rate"] = round(c["TCC_HIT_sum"] / tot, 4) if tot else None
    groups = {}
    for gname, (members, unit, amount) in ALGO_GROUPS.get(workload, {}).items():
        if all(m in kernels for m in members):
            us = sum(kernels[m]["avg_us"] for m in members)
            if unit == "flops_fp32":
                groups[gname] = {"avg_us_sum": round(us, 2), "useful_flops": amount,
                                 "useful_TFLOPs": round(amount / (us * 1e6), 1),
                                 "frac_fp32_peak": round(amount / (us * 1e6) / PEAK_FP32_TFLOPS,
                                                         4)}
                continue
            groups[gname] = {"avg_us_sum": round(us, 2), "algorithmic_bytes": amount,
                             "algorithmic_GBps": round(amount / (us * 1e3), 1),
                             "frac_hbm_8TBps": round(amount / (us * 1e3) / PEAK_HBM_GBS, 4)}
    res = {"command": command, "counters": "FETCH_SIZE / WRITE_SIZE median KiB per dispatch",
           "calibration": {"copy_bytes": 256 * 1024 * 1024,
                           **{f"{c}_scale": round(v, 4) for c, v in scale.items() if v},
                           "note": "scale = true bytes of a 256 MiB device copy / counter "
                                   "reading of that copy"},
           "kernels": kernels, "groups": groups}
    with open(out + ".json", "w") as f:
        json.dump(res, f, indent=1)
    summary_md(res, out + ".md")


def summary_md(res: dict, path: str):
    """The short text form of a rocprof summary (kernel table, groups, counter passes)."""
    kernels, groups = res["kernels"], res.get("groups", {})
    title = os.path.splitext(os.path.basename(path))[0]
    lines = [f"# {title}", "", "Command:", "", "    " + res["command"], "",
             "| kernel | calls | avg µs | HBM bytes (scaled) | GB/s | algorithmic | achieved | frac |",
             "|---|---|---|---|---|---|---|---|"]
    for name, k in kernels.items():
        if k["calls"] * k["avg_us"] < 1.0 and "algorithmic_bytes" not in k and "useful_flops" not in k:
            continue
        alg = (f"{k['algorithmic_bytes']:,} B" if "algorithmic_bytes" in k else
               f"{k['useful_flops']:,} FLOP" if "useful_flops" in k else "")
        ach = (f"{k['algorithmic_GBps']} GB/s" if "algorithmic_bytes" in k else
               f"{k['useful_TFLOPs']} TFLOP/s" if "useful_flops" in k else "")
        frac = k.get("frac_hbm_8TBps", k.get("frac_mixed_fp8_bf16_peak",
                                              k.get("frac_bf16_peak", k.get("frac_fp32_peak", ""))))
        shown = name if len(name) <= 72 else name[:69] + "..."
        lines.append(f"| `{shown}` | {k['calls']} | {k['avg_us']} | "
                     f"{k.get('hbm_bytes_scaled', ''):,} | {k.get('hbm_GBps', '')} | {alg} | "
                     f"{ach} | {frac} |" if "hbm_bytes_scaled" in k else
                     f"| `{shown}` | {k['calls']} | {k['avg_us']} |  |  | {alg} | {ach} | {frac} |")
    for gname, g in groups.items():
        if "useful_flops" in g:
            lines.append(f"| {gname} | | {g['avg_us_sum']} | | | {g['useful_flops']:,} FLOP | "
                         f"{g['useful_TFLOPs']} TFLOP/s | {g['frac_fp32_peak']} |")
            continue
        lines.append(f"| {gname} | | {g['avg_us_sum']} | | | {g['algorithmic_bytes']:,} B | "
                     f"{g['algorithmic_GBps']} GB/s | {g['frac_hbm_8TBps']} |")
    derived = ("mfma_bf16_executed_TFLOPs", "mfma_bf16_executed_frac_peak", "mfma_busy_share",
               "valu_insts_per_mfma", "l2_hit_rate")
    rows = [(n, k) for n, k in kernels.items() if any(x in k for x in derived)]
    if rows:
        lines += ["", "Counter passes (medians per dispatch; MFMA FLOPs = 512 x "
                  "SQ_INSTS_VALU_MFMA_MOPS_BF16; busy share = SQ_VALU_MFMA_BUSY_CYCLES / "
                  "(4 x SQ_BUSY_CU_CYCLES); L2 hit = TCC_HIT_sum / (TCC_HIT_sum + TCC_MISS_sum)):", "",
                  "| kernel | " + " | ".join(derived) + " |", "|---|" + "---|" * len(derived)]
        for n, k in rows:
            lines.append(f"| `{n}` | " + " | ".join(str(k.get(x, "")) for x in derived) + " |")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")




def topk_prepooled(q2, k2, want, steps):
    """Config 2's kernel-only variant: the scoring and selection on already pooled queries
    (omm_topk on q_pool [1,512,12,128]; the mask keeps 4680-token chunks over 64-token groups),
    graph-replayed like the fused call.  Its 3.54 MB make it launch-bound.  The ids must equal
    the fused call's.  Returns a function that times one replay of the captured calls."""
    import torch
    from omnimem_amd import _lib
    from omnimem_amd.index_topk import _mask, block_pool
    qp = block_pool(q2, G)
    B, MG, Hh, _ = qp.shape
    NC = k2.shape[1]
    m = _mask(BS, G, CHUNK, CHUNK, True, 0, 0, False, False, 0, 0, 0, 0)
    out = torch.empty((B, MG, Hh, TOPK), dtype=torch.int32, device=qp.device)
    ws_n = _lib.lib().omm_topk_workspace_bytes(B, MG, Hh, NC, TOPK)
    ws = _lib.workspace(ws_n, qp.device)

    def call():
        _lib.call("omm_topk", _lib.view4(qp), _lib.view4(k2), _lib.dtype_code(qp), TOPK,
                  D ** -0.5, m, out.data_ptr(), ws.data_ptr(), ws_n, _lib.stream_of(qp))

    call()
    torch.cuda.synchronize()
    torch.testing.assert_close(out, want, rtol=0, atol=0)
    g = torch.cuda.CUDAGraph()
    s_cap = torch.cuda.Stream()
    s_cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s_cap):
        call()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s_cap):
            for _ in range(steps):
                call()
    torch.cuda.current_stream().wait_stream(s_cap)
    g.replay()
    torch.cuda.synchronize()
    torch.testing.assert_close(out, want, rtol=0, atol=0)
    nbytes = qp.numel() * 2 + k2.numel() * 2 + out.numel() * 4

    keep = (qp, k2, ws, out)  # the captured calls' buffers live as long as the graph is used

    def timed():
        assert all(t is not None for t in keep)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        torch.testing.assert_close(out, want, rtol=0, atol=0)
        return {"workload": "config 2 kernel only: q_pool [1,512,12,128] bf16 (pooled "
                            "beforehand), k_cmp [1,512,12,128], top-16, causal chunk 4680",
                "ms": round(ms, 4), "algorithmic_bytes": int(nbytes),
                "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                "timing": "HIP-graph replay, like the fused call; ids equal the fused call's"}
    return timed


def useful_flops(ids, M, N, G, BS, chunk, D, g0=0, causal=True):
    """4 * D * sum over queries and heads of the visible tokens of their selected blocks.

    ids holds query groups g0, g0+1, ... of a [B, ceil(M/G), H, T] index tensor."""
    import torch
    ids = ids.long()
    B, MG, Hh, T = ids.shape
    g = torch.arange(g0, g0 + MG, device=ids.device).view(1, MG, 1, 1)
    t0 = ids * BS
    n = torch.clamp(N - t0, max=BS)
    if causal:
        qc = (g * G) // chunk
        n = torch.minimum(n, (qc + 1) * chunk - t0)
        ok = (ids >= 0) & (t0 < N) & ((t0 // chunk) <= qc) & (n > 0)
    else:
        ok = (ids >= 0) & (t0 < N) & (n > 0)
    n = torch.where(ok, n, torch.zeros_like(n))
    nq = torch.clamp(M - g * G, max=G)
    return int((n.sum(-1, keepdim=True) * nq).sum().item()) * 4 * D


PMC_FILE = os.path.join(ROOT, "profiles", "config3_layer_kernels.json")


# rocprofv3 names of the kernels whose traffic the line reports (config 3 forward, config 2 top-k)
ROOFLINE_KERNEL = "sel_fwd_dma_kernel<bf16_t, DenseAcc<bf16_t>, 128, 2>"
TOPK_KERNEL = "topk_mfma_kernel<bf16_t, 128, true>"


def measured_traffic(kernel_prefix: str):
    """HBM bytes per launch of a kernel from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary of this benchmark (calibrated against a plain copy), or None."""
    try:
        with open(PMC_FILE) as f:
            kernels = json.load(f)["kernels"]
    except (OSError, ValueError, KeyError):
        return None
    for name, v in kernels.items():
        if name.startswith(kernel_prefix):
            return v.get("hbm_bytes_scaled")
    return None


def cpu_model() -> str:
    """The host CPU's model name from /proc/cpuinfo (platform's string if unreadable)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_threads():
    """(threads, note): every CPU this process may run on, bounded by OMP_NUM_THREADS when the
    host sets it (the GPU box gives each GPU a 16-thread CPU share and sets it so)."""
    nproc = os.cpu_count() or 1
    try:
        allowed = len(os.sched_getaffinity(0))
    except AttributeError:
        allowed = nproc
    omp = os.environ.get("OMP_NUM_THREADS")
    threads = allowed
    if omp and omp.isdigit() and int(omp) > 0:
        threads = min(threads, int(omp))
    note = (f"cpu={cpu_model()}, nproc={nproc}, affinity={allowed}, "
            f"OMP_NUM_THREADS={omp or 'unset'}, torch threads={threads}")
    return threads, note


def cpu_baseline(q, k, v, ids, seconds: float):
    """Time the reference's CPU formulation on random (query group, head) pairs until ~seconds."""
    import torch
    from oracle import cpu_baseline as CB
    threads, note = cpu_threads()
    torch.set_num_threads(threads)
    qc, kc, vc = (x.float().cpu() for x in (q, k, v))
    idc = ids.cpu().long()
    MG, Hh = idc.shape[1], idc.shape[2]
    pairs = torch.randperm(MG * Hh, generator=torch.Generator().manual_seed(0)).tolist()
    done, flops, t_total = 0, 0, 0.0
    for p in pairs:
        g, h = divmod(p, Hh)
        m0, m1 = g * G, min(M, g * G + G)
        qh = qc[:, m0:m1, h:h + 1]
        kh, vh = kc[:, :, h:h + 1], vc[:, :, h:h + 1]
        tok = CB.inflate_indices(idc[:, g:g + 1, h:h + 1], BS).expand(-1, m1 - m0, -1, -1)
        t = time.perf_counter()
        CB.select_attention_chunked(qh, kh, vh, tok, scale=D ** -0.5, causal=True,
                                    chunk_size=CHUNK)
        t_total += time.perf_counter() - t
        flops += useful_flops(idc[:, g:g + 1, h:h + 1], M, N, G, BS, CHUNK, D, g0=g)
        done += 1
        if t_total >= seconds:
            break
    return {
        "value": round(flops / t_total / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"reference select_attention_torch_chunk formulation (fp32, 32-query chunks) on "
                  f"{done} random (64-query group, head) pairs of the config-3 layer "
                  f"({100.0 * done / (MG * Hh):.1f}% of the step), {t_total:.1f} s of CPU time; "
                  + note,
    }


def cpu_baseline_ar(history: int = 80, q_small: int = 64, q_large: int = 256):
    """Config 4 on the CPU: one AR layer-forward of the selection path at ``history`` cached
    chunks (60 s of video at 80), the reference's CPU formulation: query pooling, block scoring
    + top-16 over the pooled history (window of 3 chunks excluded), then selection attention of
    the chunk's 4680 queries over their 16 blocks of the 374,400-token bf16 K/V (2.3 GB in RAM).

    The selection call costs a fixed part (the permute of the whole K/V, select_attention.py:85)
    plus one part per 32-query chunk (:88), so it is timed on ``q_small`` and ``q_large``
    queries and the line through the two points is evaluated at 4680 queries; the per-layer
    time is then x150 (5 forwards x 30 layers) for one AR chunk.  Both steps are extrapolations
    and are labelled so."""
    import torch
    from oracle import cpu_baseline as CB
    threads, note = cpu_threads()
    torch.set_num_threads(threads)
    C, P, Gq, W = CHUNK, BS, G, 3
    Ntok = history * C
    gdev = "cuda" if torch.cuda.is_available() else "cpu"
    g = torch.Generator(device=gdev).manual_seed(11)
    # the cache and the chunk come from the GPU's generator (faster than the CPU's), then live
    # in host memory
    k = torch.randn((1, Ntok, H, D), generator=g, device=gdev).to(torch.bfloat16).cpu()
    v = torch.randn((1, Ntok, H, D), generator=g, device=gdev).to(torch.bfloat16).cpu()
    q = torch.randn((1, C, H, D), generator=g, device=gdev).to(torch.bfloat16).cpu()
    nb = Ntok // P
    kc = k[:, :nb * P].reshape(1, nb, P, H, D).float().mean(2).to(torch.bfloat16)  # pooled history
    t = time.perf_counter()
    ng = -(-C // Gq)
    qp = torch.nn.functional.pad(q.float(), (0, 0, 0, 0, 0, ng * Gq - C)).view(
        1, ng, Gq, H, D).mean(2)
    # scores over the history with the progressive window of 3 chunks excluded (the query
    # chunk is the newest), then top-16 with the (score desc, id asc) rule
    sc = torch.einsum("bghd,bnhd->bghn", qp, kc.float()) * D ** -0.5
    sc[..., ((history - W + 1) * C) // P:] = float("-inf")
    val, idx = torch.topk(sc, TOPK, dim=-1)
    idx, order = torch.sort(idx, dim=-1)
    val = torch.gather(val, -1, order)
    val, order = torch.sort(val, dim=-1, descending=True, stable=True)
    ids = torch.gather(idx, -1, order)
    t_topk = time.perf_counter() - t
    tok = CB.inflate_indices(ids.repeat_interleave(Gq, dim=1)[:, :C], P)
    pts = []
    for m in (q_small, q_large):
        t = time.perf_counter()
        CB.select_attention_chunked(q[:, :m], k, v, tok[:, :m], scale=D ** -0.5, causal=False)
        pts.append(time.perf_counter() - t)
    qch = 32  # the formulation's query chunk
    per_qchunk = (pts[1] - pts[0]) / ((q_large - q_small) / qch)
    fixed = max(0.0, pts[0] - per_qchunk * q_small / qch)
    t_sel = fixed + per_qchunk * (-(-C // qch))
    layer = t_topk + t_sel
    del k, v, q, kc, sc, tok
    return {
        "ms_per_layer_forward": round(1e3 * layer, 1),
        "ms_per_ar_chunk_extrapolated": round(1e3 * layer * 150, 1),
        "unit": "ms",
        "cores": threads,
        "kind": "port",
        "sample": f"one AR layer-forward of the selection path at {history} cached chunks: query "
                  f"pooling + scores + top-16 over {nb} pooled blocks ({1e3 * t_topk:.0f} ms), "
                  f"and selection attention of {C} queries x {H} heads over {TOPK} x {P}-token "
                  f"blocks of a {Ntok}-token bf16 K/V cache in RAM, timed on {q_small} and "
                  f"{q_large} queries ({1e3 * pts[0]:.0f} / {1e3 * pts[1]:.0f} ms) and "
                  f"extrapolated linearly to {C} (fixed {1e3 * fixed:.0f} ms + "
                  f"{1e3 * per_qchunk:.0f} ms per 32-query chunk); x150 (5 forwards x 30 layers) "
                  f"= extrapolated ms per AR chunk; " + note,
    }


def run_config1(steps: int):
    """Config 1: one fp32 selection call, q [1,1560,12,128], k / v [1,4680,12,128] ~ N(0,1)/sqrt(128),
    64-token blocks, groups of 64, top-16 over 1560-token frame chunks, the queries read as the
    last frame (all three frames are candidates).  The attention call alone (its split and
    merge kernels), timed with events over back-to-back calls; useful FLOPs counted from the ids
    as for config 3."""
    import torch
    from omnimem_amd.index_topk import block_pool, parallel_nsa_topk
    from omnimem_amd.selection import sel_fwd
    gen = torch.Generator().manual_seed(1)
    Mq, Nk, Cf = 1560, 4680, 1560
    q, k, v = (torch.randn((1, L, H, D), generator=gen).div_(D ** 0.5).cuda() for L in (Mq, Nk, Nk))
    ids = parallel_nsa_topk(q, block_pool(k, BS), TOPK, block_size=BS, chunk_size=Cf,
                            causal=False, group_size=G)
    out = torch.empty_like(q)
    lse = torch.empty((1, H, Mq), dtype=torch.float32, device="cuda")
    for _ in range(3):
        sel_fwd(q, k, v, ids, BS, Cf, D ** -0.5, False, G, out=out, lse=lse)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        sel_fwd(q, k, v, ids, BS, Cf, D ** -0.5, False, G, out=out, lse=lse)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flops = useful_flops(ids, Mq, Nk, G, BS, Cf, D, causal=False)
    tf = flops / (ms * 1e-3) / 1e12
    return {"workload": "config 1: fp32 q [1,1560,12,128], k/v [1,4680,12,128], top-16 of "
                        "64-token blocks, groups of 64, queries as the last 1560-token frame",
            "kernel": "sel_fwd_f32split_kernel + sel_fwd_f32merge_kernel (fp32 MFMA, "
                      "v_mfma_f32_16x16x4_f32; the 300 (group, head) items' selected blocks cut "
                      "into 2 equal runs per CU, split items merged in a second pass)",
            "ms": round(ms, 4),
            "useful_flops": int(flops), "useful_gflop": round(flops / 1e9, 3), "useful_tflops": round(tf, 3),
            "peak_fp32_tflops": PEAK_FP32_TFLOPS, "frac_fp32_peak": round(tf / PEAK_FP32_TFLOPS, 4),
            "timing": "--steps back-to-back launches, HIP events"}


def run_config3_forward(frames: int = 21):
    """Config 3: the 30-layer full-sequence Wan2.1-1.3B NSA forward (omnimem_amd/wan_full.py) on
    seeded latents of one 81-frame 480x832 clip (32760 tokens), random-init weights.  One warm-up
    forward, then one timed forward with per-category event timers and an event pair around each
    layer's selection call (with the branch mix in its epilogue); selection TFLOP/s = useful
    selection FLOPs of the 30 calls / their summed time."""
    import torch
    from omnimem_amd.wan_ar import WanARConfig
    from omnimem_amd.wan_full import WanNSAFull
    cfg = WanARConfig()
    t0 = time.perf_counter()
    model = WanNSAFull(cfg, frames=frames, seed=7)
    t_init = time.perf_counter() - t0
    gen = torch.Generator(device="cuda").manual_seed(8)
    x = torch.randn((1, model.tokens, cfg.in_dim * cfg.patch), generator=gen,
                    device="cuda").to(torch.bfloat16)
    model.forward(x, 500.0)
    torch.cuda.synchronize()
    model.timers, model.sel_events = {}, []
    t0 = time.perf_counter()
    model.forward(x, 500.0)
    torch.cuda.synchronize()
    fwd_ms = 1e3 * (time.perf_counter() - t0)
    cats = {k: round(sum(a.elapsed_time(b) for a, b in v), 3) for k, v in sorted(model.timers.items())}
    sel_ms = sum(a.elapsed_time(b) for a, b in model.sel_events)
    flops = sum(useful_flops(ids, model.tokens, model.tokens, cfg.group_size, cfg.page_tokens,
                             cfg.chunk_tokens, cfg.head_dim) for ids in model.sel_ids)
    tf = flops / (sel_ms * 1e-3) / 1e12
    res = {"workload": f"config 3: {cfg.layers}-layer full-sequence forward, {model.tokens} "
                       f"tokens ({frames} latent frames), dim {cfg.dim}, {cfg.heads}x"
                       f"{cfg.head_dim} heads, RMSNorm q/k, top-{cfg.topk} of {cfg.page_tokens}-"
                       f"token blocks, groups of {cfg.group_size}, causal by {cfg.chunk_tokens}, "
                       f"window {cfg.window_chunks} chunks",
           "ms_per_forward": round(fwd_ms, 2),
           "selection_ms_per_forward": round(sel_ms, 3),
           "selection_useful_tflop_per_forward": round(flops / 1e12, 3),
           "selection_useful_tflops": round(tf, 3),
           "selection_frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4),
           "breakdown_ms_per_forward": cats,
           "setup_s": round(t_init, 1),
           "timing": "one forward after one warm-up; selection events around each layer's "
                     "sel_fwd_gated call, whose epilogue also mixes the three branches (the "
                     "mix's reads of o_cmp, o_swa and the gates are inside the selection time; "
                     "the selection alone is the top-level roofline)"}
    del model
    torch.cuda.empty_cache()
    return res


def run_ar(dtype, history: int, steps: int, budget_bytes: float = 48e9,
           keep_window_kv: Optional[bool] = None, qk_fp8: bool = False):
    """Configs 4 / 5: ms per AR chunk with ``history`` chunks cached, 48 GB HBM budget.  The
    sliding window of a bf16 cache is read from the cache's pages; an fp8 cache keeps a dense
    bf16 ring of the window (``keep_window_kv`` overrides either choice)."""
    import torch
    from omnimem_amd.block_cache import PagedKVCache
    from omnimem_amd.wan_ar import WanARConfig, WanNSAAR
    cfg = WanARConfig()
    warm = 1
    max_chunks = history + warm + steps + 2
    t0 = time.perf_counter()
    cache = PagedKVCache(cfg.layers, cfg.heads, cfg.head_dim, max_chunks=max_chunks,
                         chunk_len=cfg.chunk_tokens, page_tokens=cfg.page_tokens, dtype=dtype,
                         hbm_budget_bytes=int(budget_bytes), window_chunks=cfg.window_chunks,
                         keep_window_kv=(dtype == "fp8") if keep_window_kv is None
                         else keep_window_kv, qk_fp8=qk_fp8)
    model = WanNSAAR(cfg, cache, seed=4)
    t_alloc = time.perf_counter() - t0
    t0 = time.perf_counter()
    model.prefill(history, seed=5, student_t=(dtype == "fp8"))
    torch.cuda.synchronize()
    t_prefill = time.perf_counter() - t0
    gen = torch.Generator(device="cuda").manual_seed(6)
    noise = lambda: torch.randn((1, cfg.chunk_tokens, cfg.in_dim * cfg.patch), generator=gen,
                                device="cuda").to(torch.bfloat16)
    cid = history
    for _ in range(warm):
        model.step(cid, noise())
        cid += 1
    torch.cuda.synchronize()
    s0 = dict(cache.stats)
    times = []
    cats = {}
    # the timed chunks run back to back, as in an AR loop (a flush's copies on the move stream
    # overlap the next chunk), between two synchronisations of every stream, so the mean
    # includes the last flush's copies too; the chunks carry the per-category event timers
    # themselves, so the breakdown and the mean describe the same chunks
    xs = [noise() for _ in range(steps)]
    model.timers = {}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for x in xs:
        model.step(cid, x)
        cid += 1
    torch.cuda.synchronize()
    times.append(time.perf_counter() - t0)
    for name, pairs in model.timers.items():
        cats[name] = cats.get(name, 0.0) + sum(a.elapsed_time(b) for a, b in pairs)
    model.timers = None
    s1 = dict(cache.stats)
    breakdown = {k: round(v / steps, 3) for k, v in sorted(cats.items())}
    ms_chunk = 1e3 * sum(times) / steps
    moved = (s1["evicted_bytes"] - s0["evicted_bytes"]) + (s1["promoted_bytes"] - s0["promoted_bytes"])
    page_bytes = 2 * cfg.page_tokens * cfg.head_dim * cache.elem  # one K page + one V page
    d = lambda key: (s1[key] - s0[key]) // steps
    res = {
        "dtype": "fp8e4m3" if dtype == "fp8" else "bf16",
        "qk": "fp8 MFMA (queries quantised per row)" if qk_fp8 else "bf16 MFMA",
        "ms_per_ar_chunk": round(ms_chunk, 2),
        "steps": steps,
        "cached_chunks_at_start": history,
        "cached_tokens_per_layer": history * cfg.chunk_tokens,
        "cache_bytes_total": history * cfg.layers * cfg.heads * 2 * cache.unit_bytes,
        "hbm_budget_bytes": cache.hbm_budget_bytes,
        "hbm_unit_slots": cache.n_slots,
        "host_unit_slots": cache.n_host,
        # async: a flush's copies run on the cache's move stream, committed by the next flush
        "flush_copies": "async" if cache._async_ok() else "on the compute stream",
        "per_chunk": {
            "evicted_bytes": d("evicted_bytes"),
            "promoted_bytes": d("promoted_bytes"),
            "host_units_touched": d("host_units_touched"),
            "hbm_units_touched": d("hbm_units_touched"),
            # per-call unit accesses (the reference's LRU accesses) served by each pool
            "host_unit_accesses": d("misses"),
            "hbm_unit_accesses": d("hits"),
            # (layer, head, page) triples read from each pool, each counted once per chunk
            "host_pages_unique": d("host_pages_unique"),
            "hbm_pages_unique": d("hbm_pages_unique"),
            # page listings: a page selected by k (query group, forward) pairs counts k times
            "host_page_listings": d("host_page_reads"),
            "hbm_page_listings": d("hbm_page_reads"),
        },
        # host-link bytes per chunk: the evict / promote copies, plus the zero-copy reads of
        # host-resident pages between two bounds (each page once / each listing once)
        "host_link_bytes_per_chunk": {
            "moved": moved // steps,
            "zero_copy_unique_pages": page_bytes * d("host_pages_unique"),
            "zero_copy_listings_upper_bound": page_bytes * d("host_page_reads"),
        },
        "lru_hit_rate": round((s1["hits"] - s0["hits"]) /
                              max(1, (s1["hits"] - s0["hits"]) + (s1["misses"] - s0["misses"])), 4),
        "breakdown_ms_per_chunk": breakdown,
        "breakdown_sum_ms": round(sum(breakdown.values()), 2),
        "unattributed_ms": round(ms_chunk - sum(breakdown.values()), 2),
        "setup_s": {"alloc": round(t_alloc, 1), "prefill": round(t_prefill, 1)},
        "selection_useful_tflop_per_chunk": round(
            (cfg.denoise_steps + 1) * cfg.layers * 4 * cfg.chunk_tokens * cfg.heads * cfg.head_dim *
            cfg.topk * cfg.page_tokens / 1e12, 3),
    }
    del model
    cache.close()
    del cache
    torch.cuda.empty_cache()
    return res


def main():
    args = parse()
    if args.rocprof_md:
        with open(args.rocprof_md) as f:
            summary_md(json.load(f), os.path.splitext(args.rocprof_md)[0] + ".md")
        return
    if args.rocprof_summary:
        rocprof_summary(args.rocprof_summary[0], args.rocprof_summary[1], args.summary_command,
                        args.summary_workload)
        return
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); the selection path has no "
              "multi-GPU mode in this build", file=sys.stderr)
        sys.exit(2)
    import torch
    from omnimem_amd.index_topk import block_pool, parallel_nsa_topk
    from omnimem_amd.selection import sel_fwd

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.c1_only:
        print(json.dumps({"config1": run_config1(args.steps)}), flush=True)
        return
    if args.full_only:
        print(json.dumps({"config1": run_config1(args.steps),
                          "config3_forward": run_config3_forward()}), flush=True)
        return
    if args.ar_only:
        print(json.dumps({"ms_per_ar_chunk": {
            "bf16": run_ar(torch.bfloat16, args.ar_history, args.ar_steps),
            "fp8": run_ar("fp8", args.ar_history, args.ar_steps),
            "fp8_qk8": run_ar("fp8", args.ar_history, args.ar_steps, qk_fp8=True)}}), flush=True)
        return
    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn((1, L, H, D), generator=gen).to(torch.bfloat16).to(dev)
               for L in (M, N, N))
    q2 = torch.randn((1, C2_T, H, D), generator=gen).to(torch.bfloat16).to(dev)
    k2 = torch.randn((1, C2_NC, H, D), generator=gen).to(torch.bfloat16).to(dev)
    scale = D ** -0.5
    out = torch.empty_like(q)
    lse = torch.empty((1, H, M), dtype=torch.float32, device=dev)

    def step():
        kc = block_pool(k, BS)
        ids = parallel_nsa_topk(q, kc, TOPK, block_size=BS, chunk_size=CHUNK, causal=True,
                                group_size=G)
        sel_fwd(q, k, v, ids, BS, CHUNK, scale, True, G, out=out, lse=lse)
        return ids

    def topk_step():
        return parallel_nsa_topk(q2, k2, TOPK, block_size=BS, chunk_size=CHUNK, causal=True,
                                 group_size=G)

    ids = step()
    torch.cuda.synchronize()
    flops = useful_flops(ids, M, N, G, BS, CHUNK, D)

    # Measurement order.  The GPU's clock drops within milliseconds of idling (host work such as
    # the graph capture below) and takes about 20 ms of load to recover: the first ~20 steps after
    # an idle period run about 20% slower than the sustained rate.  So the host-side work comes
    # first, then the backward (about 30 ms of untimed calls, then the timed ones), the top-k
    # timings, and right after them the step's warm-up and timed steps, with no idle period in
    # between.
    #
    # config 2: top-k alone (pool + score + select).  One call is shorter than its host-side
    # enqueue, so back-to-back calls would time the host: the calls are captured once in a HIP
    # graph and the replays timed; the eager per-call time is reported beside it
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    g_topk = torch.cuda.CUDAGraph()
    s_cap = torch.cuda.Stream()
    s_cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s_cap):
        topk_step()  # allocations of the captured calls come from the graph's pool
        torch.cuda.synchronize()
        with torch.cuda.graph(g_topk, stream=s_cap):
            for _ in range(args.steps):
                topk_ids = topk_step()
    torch.cuda.current_stream().wait_stream(s_cap)
    torch.cuda.synchronize()
    g_topk.replay()
    torch.cuda.synchronize()
    torch.testing.assert_close(topk_ids, topk_step(), rtol=0, atol=0)  # replays are exact

    # selection backward on the same layer (dq, dk, dv from the step's out / lse): useful work is
    # 2.5x the forward's (S recomputed, dP, dQ, dK, dV: 5 products of the forward's 2)
    from omnimem_amd.selection import sel_bwd
    d_out = torch.randn(q.shape, generator=gen).to(torch.bfloat16).to(dev)
    # about 30 ms of untimed backward calls: the clock recovers from the graph capture's idle
    # period before the timed calls start
    for _ in range(30):
        sel_bwd(q, k, v, ids, out, lse, d_out, BS, CHUNK, scale, True, G)
    b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    b0.record()
    for _ in range(args.steps):
        sel_bwd(q, k, v, ids, out, lse, d_out, BS, CHUNK, scale, True, G)
    b1.record()
    e0.record()
    g_topk.replay()
    e1.record()
    torch.cuda.synchronize()
    bwd_ms = b0.elapsed_time(b1) / args.steps
    bwd_tflops = 2.5 * flops / (bwd_ms * 1e-3) / 1e12
    topk_ms = e0.elapsed_time(e1) / args.steps
    e0.record()
    for _ in range(args.steps):
        topk_step()
    e1.record()
    torch.cuda.synchronize()
    topk_eager_ms = e0.elapsed_time(e1) / args.steps
    del g_topk, d_out

    for _ in range(args.warmup):
        step()
        topk_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps

    # the selection kernel alone: the step's sel_fwd launched back to back, HIP events on its
    # stream around the batch, so the mean is the kernel's launch duration (the host enqueues
    # faster than a launch runs: no idle gaps between launches)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        sel_fwd(q, k, v, ids, BS, CHUNK, scale, True, G, out=out, lse=lse)
    e1.record()
    torch.cuda.synchronize()
    sel_ms = e0.elapsed_time(e1) / args.steps

    sel_tflops = flops / (sel_ms * 1e-3) / 1e12
    # the kernel-only top-k last: its graph capture idles the GPU (see above)
    prepooled = topk_prepooled(q2, k2, topk_ids, args.steps)()

    traffic = measured_traffic(ROOFLINE_KERNEL)
    res = {
        "metric": METRIC,
        "value": round(flops / dt / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) q/k/v resident in HBM",
        "config": {"workload": "config 3, one layer: pool + top-k + selection attention",
                   "tokens": M, "heads": H, "head_dim": D, "block_size": BS, "group_size": G,
                   "topk": TOPK, "chunk": CHUNK, "causal": True, "layers_per_forward": 30},
        "useful_gflop_per_step": round(flops / 1e9, 3),
        "roofline": {
            "kernel": "sel_fwd_dma_kernel",
            "bound": "mfma",
            "achieved": round(sel_tflops, 3),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(sel_tflops / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic,
            "kernel_ms": round(sel_ms, 4),
            "timing": "--steps back-to-back sel_fwd launches, HIP events on its stream",
            # the same launch seen from HBM: measured traffic over its time, against 8 TB/s
            "traffic_frac_hbm": (round(traffic / (sel_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)
                                 if traffic else None),
        },
        "topk": {
            "workload": "config 2: q [1,32768,12,128] bf16 pooled by 64, k_cmp [1,512,12,128], "
                        "top-16, causal chunk 4680",
            "ms": round(topk_ms, 4),
            "timing": "HIP-graph replay of --steps captured calls, events around the replay",
            "ms_eager_per_call": round(topk_eager_ms, 4),
            "algorithmic_bytes": C2_BYTES,
            "GB/s": round(C2_BYTES / (topk_ms * 1e-3) / 1e9, 1),
            "frac_hbm": round(C2_BYTES / (topk_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "traffic": measured_traffic(TOPK_KERNEL),
            "prepooled": prepooled,
        },
        "sel_bwd": {
            "workload": "config 3 layer backward (dq, dk, dv; dQ, block index and dK/dV kernels)",
            "ms": round(bwd_ms, 4),
            "useful_tflops": round(bwd_tflops, 3),
            "frac_bf16_peak": round(bwd_tflops / PEAK_BF16_TFLOPS, 4),
        },
        "config1": None,
        "config3_forward": None,
        "ms_per_ar_chunk": None,
        "cpu_baseline": None,
    }
    if not args.no_full:
        res["config1"] = run_config1(args.steps)
        res["config3_forward"] = run_config3_forward()
    if not args.no_ar:
        del q2, k2
        torch.cuda.empty_cache()
        res["ms_per_ar_chunk"] = {
            "bf16": run_ar(torch.bfloat16, args.ar_history, args.ar_steps),
            "fp8": run_ar("fp8", args.ar_history, args.ar_steps),
            "fp8_qk8": run_ar("fp8", args.ar_history, args.ar_steps, qk_fp8=True),
        }
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(q, k, v, ids, args.cpu_seconds)
        if not args.no_ar:
            del q, k, v, out, lse
            torch.cuda.empty_cache()
            res["cpu_baseline"]["config4_ar"] = cpu_baseline_ar(args.ar_history)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
