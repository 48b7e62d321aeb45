"""Benchmark of the MoE expert-FFN decode path on one MI355X.

    python bench.py [--config 1] [--steps K] [--warmup W] [--gpus 1]

A step is one decode token through the workload's MoE layers with all
inputs resident in HBM.  Workloads (synthetic data):
  0  gpt-oss-20b single MoE layer (rotating 8 distinct layer copies so the
     256 MB Infinity Cache cannot hold the active experts)
  1  gpt-oss-20b 24-layer MoE stack, Zipf(1.1) router bias   (default)
  2  gpt-oss-120b 36-layer stack, 128 experts, Zipf(1.1)
  3  Qwen3-30B-A3B 48-layer MoE stack: Q4_K gate/up, Q6_K down, top-8 of 128
  4  gpt-oss-20b layer, 512-token prefill: tokens grouped by expert, expert
     GEMMs on the matrix cores (8 rotating layer copies)
  5  Qwen3-30B-A3B layer, 512-token prefill on the int8 matrix cores (the
     batched k-quant path beside config 4)
  6  gpt-oss two-stage LM head, 201088 x 2880: Q4
     screen of every row, exact Q8 refine of 96 candidates, greedy
  7  gpt-oss-20b attention, 24 layers, one token at position 1024
  8  gpt-oss-20b whole decode step: 24 x (attention + MoE) + head, one graph
Prints one JSON line: value = expert-weight GB/s (algorithmic bytes of the
active experts + biases + router per token / time), plus tok/s, the roofline
of the dominant kernel (gate/up) and the CPU baseline (the oracle on the
host's cores over a bounded sample of the same workload).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

# HBM bytes per dispatch of the roofline kernel, from rocprofv3 FETCH_SIZE /
# WRITE_SIZE runs scaled by a 1 GiB copy; None where not yet measured.  The
# bench cannot read hardware counters itself (they need a profiler run of
# their own), so each line names the profile its figure comes from.
MEASURED_TRAFFIC = {"k_gateup_mx": 35_815_144, "k_gateup_kq": 14_418_124,
                    "k_gateup_grouped": 532_770_153, "k_gateup_kq_grouped": 282_353_586,
                    "head": 327_526_064}
TRAFFIC_SOURCE = {"k_gateup_mx": "profiles/hbm_traffic_config1_phased.md",
                  "k_gateup_kq": "profiles/hbm_traffic_config3_qwen.md",
                  "k_gateup_grouped": "profiles/mfma_hbm_config4_grouped.md",
                  "k_gateup_kq_grouped": "profiles/mfma_hbm_config4_grouped.md",
                  "head": "profiles/hbm_traffic_config6_head.md"}

METRIC = "expert-weight GB/s (% HBM peak) + MoE-layer tok/s, gpt-oss-20b shape, 1 GPU"
HBM_PEAK_GBS = 8000.0

CONFIGS = {
    0: dict(name="config0: gpt-oss-20b single MoE layer, decode batch 1 (8 rotating layer copies)",
            d=2880, dff=2880, ne=32, k=4, layers=8, per_step=1, zipf=None, norm=False),
    1: dict(name="config1: gpt-oss-20b 24-layer MoE stack (attention omitted), decode batch 1, Zipf(1.1) router bias",
            d=2880, dff=2880, ne=32, k=4, layers=24, per_step=24, zipf=1.1, norm=True),
    2: dict(name="config2: gpt-oss-120b 36-layer MoE stack, 128 experts, decode batch 1, Zipf(1.1) router bias",
            d=2880, dff=2880, ne=128, k=4, layers=36, per_step=36, zipf=1.1, norm=True),
    3: dict(name="config3: Qwen3-30B-A3B 48-layer MoE stack (attention omitted), decode batch 1, Q4_K gate/up, "
                 "Q6_K down, softmax then top-8 of 128",
            d=2048, dff=768, ne=128, k=8, layers=48, per_step=48, zipf=None, norm=True, family="qwen"),
    4: dict(name="config4: gpt-oss-20b MoE layer, 512-token prefill (batched), Zipf(1.1) router bias, tokens grouped "
                 "by expert, fp8 x fp4 scaled-MFMA expert GEMMs",
            d=2880, dff=2880, ne=32, k=4, layers=8, per_step=1, zipf=1.1, norm=True, n_tok=512),
    5: dict(name="config5: Qwen3-30B-A3B MoE layer, 512-token prefill (batched), Q4_K gate/up + Q6_K down, tokens "
                 "grouped by expert, int8 MFMA expert GEMMs",
            d=2048, dff=768, ne=128, k=8, layers=8, per_step=1, zipf=None, norm=True, n_tok=512, family="qwen"),
    6: dict(name="config6: gpt-oss two-stage LM head (output.weight 201088 x 2880 bf16 -> Q4 screen + Q8 refine of "
                 "12 x 8 candidates + greedy), one token",
            d=2880, dff=0, ne=0, k=0, layers=1, per_step=1, zipf=None, norm=True, family="head", vocab=201088),
    7: dict(name="config7: gpt-oss-20b attention, 24 layers (even: window 128, odd: full causal), decode one token "
                 "at position 1024 with the KV cache filled, Q8 projections",
            d=2880, dff=0, ne=0, k=0, layers=24, per_step=24, zipf=None, norm=True, family="attn", n_head=64,
            n_head_kv=8, swa=128, pos=1024),
    8: dict(name="config8: gpt-oss-20b whole decode step on the GPU: 24 x (attention at position 1024 + MoE, Zipf(1.1) "
                 "router bias) + two-stage LM head, one captured graph per token",
            d=2880, dff=2880, ne=32, k=4, layers=24, per_step=24, zipf=1.1, norm=True, family="step", n_head=64,
            n_head_kv=8, swa=128, pos=1024, vocab=201088),
}
for _c in CONFIGS.values():
    _c.setdefault("family", "gptoss")
    _c.setdefault("n_tok", 1)
MFMA_FP8_PEAK_TOPS = 5000.0   # MI355X dense fp8 / int8 (the f8f6f4 instructions run fp8 x fp4 at this rate)


def layer_bytes(c) -> dict:
    """Algorithmic bytes one token reads per layer (active experts only)."""
    d, dff, ne, k = c["d"], c["dff"], c["ne"], c["k"]
    if c["family"] == "qwen":
        gu = k * 2 * dff * (d // 256 * 144)                      # Q4_K gate + up rows
        dn = k * d * (dff // 256 * 210)                          # Q6_K down rows
        router = ne * d * 4 + (d * 4 if c["norm"] else 0)
    else:
        gu = k * 2 * dff * (d // 32 * 17) + k * 2 * dff * 4      # MXFP4 rows + fp32 biases
        dn = k * d * (dff // 32 * 17) + k * d * 4
        router = ne * d * 4 + ne * 4 + (d * 4 if c["norm"] else 0)
    return {"gate_up": gu, "down": dn, "router": router, "total": gu + dn + router}


def batched_result(c, args, ms, n_tok, kt) -> dict:
    """Bench line of a batched (prefill) step: one layer over n_tok tokens.
    The roofline is the gate/up GEMM's (the dominant kernel): every expert's
    gate/up weights are read (all experts hold pairs at this batch size)."""
    d, dff, ne, k = c["d"], c["dff"], c["ne"], c["k"]
    qwen = c["family"] == "qwen"
    if qwen:
        gu_w = ne * 2 * dff * (d // 256 * 144)
        dn_w = ne * d * (dff // 256 * 210)
        wbytes = gu_w + dn_w + ne * d * 4
    else:
        gu_w = ne * 2 * dff * (d // 32 * 17) + ne * 2 * dff * 4          # MXFP4 rows + biases
        dn_w = ne * d * (dff // 32 * 17) + ne * d * 4
        wbytes = gu_w + dn_w + ne * d * 4 + ne * 4
    macs = n_tok * k * (2 * dff * d + d * dff)                          # useful int8 multiply-adds
    sec = ms * 1e-3
    gbs = wbytes / sec / 1e9
    tops = 2 * macs / sec / 1e12
    gu_ms, gu_n = kt["gate_up"]
    dn_ms, dn_n = kt["down"]
    gu_us = gu_ms / max(gu_n, 1) * 1e3
    dn_us = dn_ms / max(dn_n, 1) * 1e3
    gu_gbs = gu_w / (gu_us * 1e-6) / 1e9
    gu_tops = 2 * n_tok * k * 2 * dff * d / (gu_us * 1e-6) / 1e12
    kern = "k_gateup_kq_grouped" if qwen else "k_gateup_grouped"
    return {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8" if qwen else "fp8 x fp4 (exact int8 x E2M1)", "data": "synthetic",
        "config": {"workload": c["name"], "tokens_per_step": n_tok, "d": d, "d_ff": dff, "n_expert": ne,
                   "top_k": k,
                   "weights": "Q4_K gate/up + Q6_K down (GGUF types 12/14)" if qwen else "MXFP4 (GGUF type 39)"},
        "tok_per_s": round(n_tok / sec, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "kernels_us": {"gate_up_gemm": round(gu_us, 2), "down_gemm": round(dn_us, 2)},
        "roofline": {"bound": "hbm", "kernel": kern, "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                     "traffic": MEASURED_TRAFFIC.get(kern), "traffic_source": TRAFFIC_SOURCE.get(kern),
                     "bytes_per_launch": gu_w,
                     "mfma_int8_equiv": {"achieved": round(gu_tops, 2), "peak": MFMA_FP8_PEAK_TOPS,
                                         "unit": "TOP/s", "frac": round(gu_tops / MFMA_FP8_PEAK_TOPS, 5)}},
        "mfma": {"achieved": round(tops, 2), "peak": MFMA_FP8_PEAK_TOPS, "unit": "TOP/s (useful int8-equivalent, whole layer)",
                 "frac": round(tops / MFMA_FP8_PEAK_TOPS, 5), "ops_per_step": 2 * macs},
    }


def grouping_padding(blk, c, tokens) -> dict:
    """Tile slots the grouped GEMMs compute for a batch (pairs grouped by
    expert, 32-token tiles, the last tile of each expert padded) against the
    (token, slot) pairs themselves.  The ids come from the per-token decode
    path, which the grouped path matches bit for bit."""
    import numpy as np
    counts = np.zeros(c["ne"], np.int64)
    for t in tokens:
        _, tr = blk.forward(0, t, c["norm"], trace=True)
        np.add.at(counts, tr["ids"], 1)
    pairs = int(counts.sum())
    tiles = int(np.ceil(counts / 32).sum())
    return {"pairs": pairs, "experts_used": int((counts > 0).sum()), "tiles": tiles, "tile_slots": 32 * tiles,
            "overhead": round(32 * tiles / pairs - 1, 4), "max_pairs_per_expert": int(counts.max())}


def calib_copy(args) -> None:
    """A copy kernel of known size: its FETCH_SIZE / WRITE_SIZE give the
    counter-to-bytes factor for the kernels of the same run."""
    if not args.calib_copy_mib:
        return
    import torch
    n = args.calib_copy_mib * (1 << 20) // 4
    src = torch.empty(n, dtype=torch.float32, device="cuda:0").uniform_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def _host_info() -> dict:
    """nproc, the cores this process may run on, and the CPU model: the
    model name as the host reports it (a virtual machine may shorten it),
    with the vendor, family / model / stepping numbers and lscpu's name."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k = k.strip()
            if k in ("model name", "vendor_id", "cpu family", "model", "stepping") and k not in info:
                info[k] = v.strip()
            if line.strip() == "" and info:
                break
    except OSError:
        pass
    model = info.get("model name", "")
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                ln = line.split(":", 1)[1].strip()
                if ln and ln != model:
                    model = f"{model} (lscpu: {ln})" if model else ln
    except Exception:
        pass
    ids = ", ".join(f"{k} {info[k]}" for k in ("vendor_id", "cpu family", "model", "stepping") if k in info)
    if ids:
        model = f"{model} [{ids}]"
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"nproc": os.cpu_count() or 1, "usable": usable, "model": model}


def cpu_baseline(host_layers, c, budget_s: float) -> dict:
    """Oracle (C restatement of the reference path, OpenMP over rows) on the
    host's cores, over the first layers of the same workload: threaded over
    every core this process may use (capped by OMP_NUM_THREADS, the host's
    per-GPU CPU share on the GPU boxes), and single-threaded."""
    import numpy as np
    from oracle import oracle as O
    from cpubrrr_amd import synth

    info = _host_info()
    threads = info["usable"]
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    fwd = O.qwen_moe if c["family"] == "qwen" else O.gptoss_moe
    lb = layer_bytes(c)["total"]

    def run(nth, budget):
        O.set_threads(nth)
        x = synth.token(c["d"], 0, 12345)
        n = 0
        t0 = time.perf_counter()
        # a batch of tokens is n_tok independent decodes for the reference path
        while time.perf_counter() - t0 < budget or n == 0:
            L = host_layers[n % len(host_layers)]
            x, _ = fwd(L, x, c["norm"])
            n += 1
        return n, time.perf_counter() - t0

    n, dt = run(threads, budget_s)
    n1, dt1 = run(1, budget_s / 2)
    per_layer, per_layer1 = dt / n, dt1 / n1
    tok_s = 1.0 / (per_layer * c["per_step"])
    f64 = None
    if c["family"] != "qwen":
        # the second mode: scripts/ffn_reference.py's float64 dequant algorithm
        # (scale 2^(e-128)) on the same layers and threads
        O.set_threads(threads)
        x = synth.token(c["d"], 0, 12345)
        nf, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget_s / 2 or nf == 0:
            x = O.gptoss_moe_f64(host_layers[nf % len(host_layers)], x, c["norm"])
            nf += 1
        pf = (time.perf_counter() - t0) / nf
        f64 = {"value": round(1.0 / (pf * c["per_step"]), 3), "unit": "tok/s", "cores": threads,
               "ms_per_layer": round(pf * 1e3, 3), "layers": nf,
               "algorithm": "scripts/ffn_reference.py float64 dequant (2^(e-128)), weights decoded per row"}
    return {"value": round(tok_s, 3), "unit": "tok/s", "cores": threads,
            "f64_dequant": f64,
            "kind": "port", "sample": f"{n} MoE layers ({len(host_layers)} distinct) of the same workload in "
                                       f"{dt:.1f} s on {threads} threads; {per_layer * 1e3:.2f} ms/layer, "
                                       f"{lb / per_layer / 1e9:.2f} GB/s algorithmic",
            "ms_per_layer": round(per_layer * 1e3, 3),
            "single_thread": {"value": round(1.0 / (per_layer1 * c["per_step"]), 3), "unit": "tok/s",
                              "ms_per_layer": round(per_layer1 * 1e3, 3), "layers": n1},
            "host": {"nproc": info["nproc"], "usable_cores": info["usable"], "cpu_model": info["model"],
                     "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}}


def bench_head(args, c) -> int:
    """config 6: the LM head on one token; value = screen bytes (Q4, or Q2
    with --head-screen 2: the reference's CPBRR_HEAD2 option) / time."""
    import numpy as np
    import torch

    from cpubrrr_amd import LmHead

    d, V = c["d"], c["vocab"]
    r = np.random.default_rng(0)
    w32 = (r.standard_normal((V, d)) * 0.02).astype(np.float32)
    w = ((w32.view(np.uint32).astype(np.uint64) + 0x7FFF + ((w32.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16)
    del w32
    nw = np.ones(d, np.float32)
    torch.cuda.set_device(0)
    hd = LmHead(d, V)
    t0 = time.perf_counter()
    hd.load(w, nw)
    log(f"head quantised in {time.perf_counter() - t0:.1f} s")
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    hd.set_stream(stream.cuda_stream)
    hd.set_screen(args.head_screen)
    calib_copy(args)
    x = torch.from_numpy((r.standard_normal(d) * 3).astype(np.float32)).to("cuda:0")
    ch = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    for _ in range(args.warmup):
        hd.forward_device(x.data_ptr(), ch.data_ptr())
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        hd.forward_device(x.data_ptr(), ch.data_ptr())
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    nb = d // 32
    q2 = args.head_screen == 2
    screen_bytes = V * nb * ((8 if q2 else 16) + 2)    # codes + bf16 scales of every row
    refine_bytes = 96 * (d + nb * 4)
    gbs = (screen_bytes + refine_bytes) / (ms * 1e-3) / 1e9
    out = {"metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "int8 x Q2 / Q8" if q2 else "int8 x Q4 / Q8", "data": "synthetic",
           "config": {"workload": c["name"] + (" [Q2 screen]" if q2 else ""), "d": d, "n_vocab": V, "n_slices": 12,
                      "n_cand": 8, "screen_bits": args.head_screen},
           "tok_per_s": round(1e3 / ms, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
           "roofline": {"bound": "hbm", "kernel": "whole head (norm, screen, top-k, refine)", "achieved": round(gbs, 1),
                        "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                        "traffic": MEASURED_TRAFFIC["head"] if (d, V) == (2880, 201088) and not q2 else None,
                        "traffic_source": TRAFFIC_SOURCE["head"] if not q2 else None,
                        "bytes_per_launch": screen_bytes + refine_bytes}}
    hd.close()
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline_head(w, nw, x.cpu().numpy(), args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


def attn_bytes(c) -> dict:
    """Algorithmic bytes of one token through one attention layer: the Q8
    weights of q / k / v / o (codes + fp32 scale per 32) and the cache rows
    the layer reads (window on even layers, every position on odd ones)."""
    d, nq, nkv = c["d"], c["n_head"] * 64, c["n_head_kv"] * 64
    w = ((nq + 2 * nkv) * d + d * nq) * (1 + 4 / 32)
    vec = 4 * (d + nq + 2 * nkv + d + c["n_head"])
    pos = c["pos"]
    kv_even = 2 * min(c["swa"], pos + 1) * nkv * 4
    kv_odd = 2 * (pos + 1) * nkv * 4
    return {"weights": int(w + vec), "kv_even": kv_even, "kv_odd": kv_odd,
            "per_token": int(c["layers"] * (w + vec) + c["layers"] // 2 * (kv_even + kv_odd))}


def bench_attn(args, c) -> int:
    """config 7: one token through the 24 attention layers; value = bytes / time."""
    import numpy as np
    import torch

    from cpubrrr_amd import Attention, synth

    d, nh, nkv, nl, pos = c["d"], c["n_head"], c["n_head_kv"], c["layers"], c["pos"]
    torch.cuda.set_device(0)
    at = Attention(d, nh, nkv, nl, max_seq=pos + 1, sliding_window=c["swa"], rope_base=150000.0, rms_eps=1e-5)
    t0 = time.perf_counter()
    host0 = None
    for il in range(nl):
        L = synth.attn_layer(d, nh, nkv, 64, seed=0, layer=il, swa=c["swa"])
        at.load_layer(il, L)
        if il == 0:
            host0 = L
    log(f"attention weights quantised in {time.perf_counter() - t0:.1f} s")
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    at.set_stream(stream.cuda_stream)
    calib_copy(args)
    x = torch.from_numpy(synth.token(d, 0, 7)).to("cuda:0")
    # fill the cache: positions 0 .. pos-1 through every layer
    for p in range(pos):
        for il in range(nl):
            at.forward_device(il, p, x.data_ptr())
        x.mul_(0.5)      # keep the residual bounded while the cache fills
    torch.cuda.synchronize()
    x0 = x.clone()

    def step():
        x.copy_(x0)
        for il in range(nl):
            at.forward_device(il, pos, x.data_ptr())
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    ab = attn_bytes(c)
    gbs = ab["per_token"] / (ms * 1e-3) / 1e9
    out = {"metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "int8 x Q8 (fp32 softmax)", "data": "synthetic",
           "config": {"workload": c["name"], "d": d, "n_head": nh, "n_head_kv": nkv, "layers": nl, "pos": pos,
                      "sliding_window": c["swa"]},
           "tok_per_s": round(1e3 / ms, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
           "roofline": {"bound": "hbm", "kernel": "whole block (norm, qkv, core, o-proj) x 24 layers",
                        "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "bytes_per_launch": ab["per_token"]}}
    at.close()
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline_attn(host0, c, args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


def bench_step(args, c) -> int:
    """config 8: one token through 24 x (attention + MoE) and the head, the
    whole step captured as one graph (the library's launches land in the
    caller's graph); value = bytes the step reads / time."""
    import numpy as np
    import torch

    from cpubrrr_amd import Attention, LmHead, MoeBlock, MoeConfig, synth

    d, nl, pos, V = c["d"], c["layers"], c["pos"], c["vocab"]
    torch.cuda.set_device(0)
    t0 = time.perf_counter()
    at = Attention(d, c["n_head"], c["n_head_kv"], nl, max_seq=pos + 1, sliding_window=c["swa"], rope_base=150000.0,
                   rms_eps=1e-5)
    cfg = MoeConfig.gptoss(d=d, n_expert=c["ne"], top_k=c["k"], d_ff=c["dff"], n_layer=nl)
    moe = MoeBlock(cfg)
    host_attn0 = host_moe0 = None
    for l in range(nl):
        A = synth.attn_layer(d, c["n_head"], c["n_head_kv"], 64, seed=0, layer=l, swa=c["swa"])
        at.load_layer(l, A)
        M = synth.gptoss_layer(d, c["dff"], c["ne"], c["k"], seed=0, layer=l, zipf=c["zipf"])
        moe.load_layer(l, M)
        if l == 0:
            host_attn0, host_moe0 = A, M
        del A, M
    r = np.random.default_rng(0)
    w32 = (r.standard_normal((V, d)) * 0.02).astype(np.float32)
    w_out = ((w32.view(np.uint32).astype(np.uint64) + 0x7FFF + ((w32.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16)
    del w32
    n_out = np.ones(d, np.float32)
    hd = LmHead(d, V)
    hd.load(w_out, n_out)
    log(f"loaded {nl} attention + MoE layers and the head in {time.perf_counter() - t0:.1f} s")
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    for h in (at, moe, hd):
        h.set_stream(stream.cuda_stream)
    x = torch.from_numpy(synth.token(d, 0, 7)).to("cuda:0")
    ch = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    # the cache: positions 0 .. pos-1 through the attention layers
    for p in range(pos):
        for l in range(nl):
            at.forward_device(l, p, x.data_ptr())
        x.mul_(0.5)
    torch.cuda.synchronize()
    x0 = torch.from_numpy(synth.token(d, 0, 8)).to("cuda:0")
    xs = x0.clone()
    torch.cuda.synchronize()

    def token_step():
        for l in range(nl):
            at.forward_device(l, pos, xs.data_ptr())
            moe.forward_device(l, 1, xs.data_ptr(), 1, True)
        hd.forward_device(xs.data_ptr(), ch.data_ptr())

    token_step()                           # eager once (the MoE layers' buffers exist before capture)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        token_step()
    for _ in range(args.warmup):
        xs.copy_(x0)
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        xs.copy_(x0)
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    assert torch.isfinite(xs).all().item()
    moe_b = layer_bytes(dict(c, family="gptoss"))["total"] * nl
    ab = attn_bytes(c)["per_token"]
    nb = d // 32
    head_b = V * nb * 18 + 96 * (d + nb * 4)
    total = moe_b + ab + head_b
    gbs = total / (ms * 1e-3) / 1e9
    out = {"metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "int8 x MXFP4 / Q8 / Q4 (fp32 softmax, routing)", "data": "synthetic",
           "config": {"workload": c["name"], "d": d, "layers": nl, "pos": pos, "n_expert": c["ne"], "top_k": c["k"],
                      "n_vocab": V},
           "tok_per_s": round(1e3 / ms, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
           "bytes_per_token": {"moe": moe_b, "attention": ab, "head": head_b},
           # the reference's own end-to-end decode figure, on its hardware (context, not the same metric)
           "reference_published": {"value": 90.1, "unit": "tok/s", "hardware": "Apple M4 Max CPU",
                                   "source": "the reference's README.md:19"},
           "roofline": {"bound": "hbm", "kernel": "whole decode step (24 x 6 kernels + 3)", "achieved": round(gbs, 1),
                        "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                        "bytes_per_launch": total}}
    for h in (hd, moe, at):
        h.close()
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline_step(host_attn0, host_moe0, w_out, n_out, c, args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


def cpu_baseline_step(A, M, w_out, n_out, c, budget_s: float) -> dict:
    """The oracle's decode step at the same shapes: attention (single-threaded
    C) and MoE (C, OpenMP) of one layer per step of the sample, scaled to the
    24 layers, plus the head on pre-quantised rows."""
    import numpy as np
    from oracle import oracle as O

    info = _host_info()
    threads = info["usable"]
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    O.set_threads(threads)
    pos, nkv = c["pos"], c["n_head_kv"]
    Lq = dict(A)
    for n in ("q", "k", "v", "o"):
        Lq["w" + n], Lq["s" + n] = O.q8_rows(A["w" + n])
    tab = O.rope_table(64, pos + 1, 150000.0)
    r = np.random.default_rng(1)
    kc = r.standard_normal((pos + 1, nkv, 64)).astype(np.float32)
    vc = r.standard_normal((pos + 1, nkv, 64)).astype(np.float32)
    x = r.standard_normal(c["d"]).astype(np.float32)
    pre = O.q4_quant_rows(w_out)
    n, t_layers, t_head = 0, 0.0, 0.0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s or n < 2:
        t1 = time.perf_counter()
        xa, _ = O.attn_layer(Lq, n % 2, pos, x, kc, vc, tab)
        xm, _ = O.gptoss_moe(M, xa, True)
        t2 = time.perf_counter()
        O.head(w_out, xm, n_out, 1e-5, pre=pre)
        t3 = time.perf_counter()
        t_layers += t2 - t1
        t_head += t3 - t2
        n += 1
    per_tok = t_layers / n * c["layers"] + t_head / n
    return {"value": round(1.0 / per_tok, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} (attention + MoE layer + head) evaluations in {t_layers + t_head:.1f} s on {threads} threads "
                      f"(attention single-threaded); {t_layers / n * 1e3:.1f} ms per layer, {t_head / n * 1e3:.1f} ms "
                      f"head, scaled to {c['layers']} layers + head",
            "ms_per_token": round(per_tok * 1e3, 2)}


def cpu_baseline_attn(L, c, budget_s: float) -> dict:
    """The oracle's attention step (single-threaded C, the reference's fp32
    order) at the same shape and position, on random cache contents."""
    import numpy as np
    from oracle import oracle as O

    pos, nkv = c["pos"], c["n_head_kv"]
    Lq = dict(L)
    for n in ("q", "k", "v", "o"):
        Lq["w" + n], Lq["s" + n] = O.q8_rows(L["w" + n])
    tab = O.rope_table(64, pos + 1, 150000.0)
    r = np.random.default_rng(1)
    kc = r.standard_normal((pos + 1, nkv, 64)).astype(np.float32)
    vc = r.standard_normal((pos + 1, nkv, 64)).astype(np.float32)
    x = r.standard_normal(c["d"]).astype(np.float32)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s or n < 2:
        O.attn_layer(Lq, n % 2, pos, x, kc, vc, tab)       # alternate window / full layers
        n += 1
    per_layer = (time.perf_counter() - t0) / n
    return {"value": round(1.0 / (per_layer * c["per_step"]), 3), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"{n} attention layer steps (alternating window / full) at pos {pos} in "
                      f"{per_layer * n:.1f} s on 1 thread; {per_layer * 1e3:.2f} ms/layer",
            "ms_per_layer": round(per_layer * 1e3, 3)}


def cpu_baseline_head(w, nw, x, budget_s: float) -> dict:
    """The oracle's head (C, OpenMP over the Q4 screen rows) on the same
    weights and hidden state."""
    from oracle import oracle as O

    info = _host_info()
    threads = info["usable"]
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    O.set_threads(threads)
    pre = O.q4_quant_rows(w)                  # load time, outside the sample
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s or n == 0:
        O.head(w, x, nw, 1e-5, pre=pre)
        n += 1
    per = (time.perf_counter() - t0) / n
    return {"value": round(1.0 / per, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} head evaluations with the Q4 screen (rows quantised beforehand, as at the reference's load) in "
                      f"{per * n:.1f} s on {threads} threads; {per * 1e3:.1f} ms each",
            "ms_per_token": round(per * 1e3, 2)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=1, choices=sorted(CONFIGS))
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--head-screen", type=int, default=4, choices=[4, 2],
                    help="config 6: the head's screen rows, Q4 (default) or Q2 (the reference's CPBRR_HEAD2)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="also run one plain device copy of this many MiB (HBM-traffic counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from cpubrrr_amd import MoeBlock, MoeConfig, synth

    c = CONFIGS[args.config]
    if c["family"] == "head":
        return bench_head(args, c)
    if c["family"] == "attn":
        return bench_attn(args, c)
    if c["family"] == "step":
        return bench_step(args, c)
    d, dff, ne, k, nl = c["d"], c["dff"], c["ne"], c["k"], c["layers"]
    qwen = c["family"] == "qwen"
    if qwen:
        cfg = MoeConfig.qwen3(d=d, n_expert=ne, top_k=k, d_ff=dff, n_layer=nl, max_tokens=c["n_tok"])
    else:
        cfg = MoeConfig.gptoss(d=d, n_expert=ne, top_k=k, d_ff=dff, n_layer=nl, max_tokens=c["n_tok"])
    dev = torch.device("cuda:0")
    torch.cuda.set_device(0)
    blk = MoeBlock(cfg, device=0)
    host_keep = []
    t0 = time.perf_counter()
    for l in range(nl):
        if qwen:
            L = synth.qwen_layer(d, dff, ne, k, seed=0, layer=l)
        else:
            L = synth.gptoss_layer(d, dff, ne, k, seed=0, layer=l, zipf=c["zipf"])
        blk.load_layer(l, L)
        if l < 8:
            host_keep.append(L)
        del L
    log(f"loaded {nl} layers in {time.perf_counter() - t0:.1f} s "
        f"({MoeBlock.layer_bytes(cfg) * nl / 1e9:.2f} GB of expert weights in HBM)")

    # a dedicated (non-default) stream: the library launches on it and the
    # timing events below are recorded on it
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    blk.set_stream(stream.cuda_stream)
    n_tok = c["n_tok"]
    if n_tok > 1:
        x = torch.from_numpy(np.stack([synth.token(d, 0, i) for i in range(n_tok)])).to(dev)
    else:
        x = torch.from_numpy(synth.token(d, 0, 0)).to(dev)
    calib_copy(args)

    def step(i):
        if c["per_step"] == nl:
            blk.forward_device(0, nl, x.data_ptr(), n_tok, c["norm"])
        else:
            blk.forward_device(i % nl, 1, x.data_ptr(), n_tok, c["norm"])

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(args.steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    assert torch.isfinite(x).all().item()

    # per-kernel durations over the same steps (HIP events on the launch stream)
    blk.timing(True)
    for i in range(args.steps):
        step(i)
    kt = blk.kernel_times()
    blk.timing(False)

    if n_tok > 1:
        out = batched_result(c, args, ms, n_tok, kt)
        # padding of the token tiles, on the step's initial batch
        out["padding"] = grouping_padding(blk, c, [synth.token(d, 0, i) for i in range(n_tok)])
        if not args.no_cpu:
            log("timing the CPU baseline ...")
            out["cpu_baseline"] = cpu_baseline(host_keep, c, args.cpu_seconds)
        blk.close()
        print(json.dumps(out), flush=True)
        return 0

    lb = layer_bytes(c)
    bytes_tok = lb["total"] * c["per_step"]
    gbs = bytes_tok / (ms * 1e-3) / 1e9
    tok_s = 1e3 / ms
    gu_ms, gu_n = kt["gate_up"]
    gu_avg_us = gu_ms / max(gu_n, 1) * 1e3
    dn_ms, dn_n = kt["down"]
    rt_ms, rt_n = kt["route"]
    gu_ach = lb["gate_up"] / (gu_avg_us * 1e-6) / 1e9
    out = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8" if qwen else "fp8 x fp4 (exact int8 x E2M1)", "data": "synthetic",
        "config": {"workload": c["name"], "layers_per_step": c["per_step"], "d": d, "d_ff": dff,
                   "n_expert": ne, "top_k": k, "batch": 1,
                   "weights": "Q4_K gate/up + Q6_K down (GGUF types 12/14)" if qwen else "MXFP4 (GGUF type 39)"},
        "tok_per_s": round(tok_s, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "bytes_per_token": bytes_tok,
        "kernels_us": {"route": round(rt_ms / max(rt_n, 1) * 1e3, 2), "gate_up": round(gu_avg_us, 2),
                       "down": round(dn_ms / max(dn_n, 1) * 1e3, 2)},
        "roofline": {"bound": "hbm", "kernel": "k_gateup_kq" if qwen else "k_gateup_mx", "achieved": round(gu_ach, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gu_ach / HBM_PEAK_GBS, 4),
                     "traffic": MEASURED_TRAFFIC["k_gateup_kq" if qwen else "k_gateup_mx"],
                     "traffic_source": TRAFFIC_SOURCE["k_gateup_kq" if qwen else "k_gateup_mx"],
                     "bytes_per_launch": lb["gate_up"]},
    }
    if not args.no_cpu:
        log("timing the CPU baseline ...")
        out["cpu_baseline"] = cpu_baseline(host_keep, c, args.cpu_seconds)
    blk.close()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
