#!/usr/bin/env python3
"""Benchmark of the MI355X Q4_K GEMV path (BASELINE.json metric).

Default workload: one synthetic 7B-class decode step at
batch 1 -- 28 layers x {q|k|v fused 4608x3584, o 3584x3584, gate|up fused
37888x3584, down 3584x18944} + lm_head 152064x3584 = 113 GEMV launches over
3.98 GB of resident Q4_K weights, replayed as one HIP graph per step. A "step"
is one token's matvec chain.

Prints ONE JSON line: value = whole-step algorithmic GB/s (weights + x + y
bytes / step time), plus tokens/s, a roofline object for the GEMV kernel
(HIP events around the graph replays) and a CPU baseline (the oracle's restatement of
the reference CPU GEMV, llm.rs:468-806, on a bounded sample). Progress goes to
stderr.

  python bench.py [--steps K] [--warmup W] [--workload decode7b|layer|gateup]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
METRIC = "Q4_K GEMV achieved HBM GB/s (% of peak); 7B-class decode tokens/sec"
BLOCK_BYTES, BLOCK_ELEMS = 144, 256

HIDDEN, INTER, NQ, NKV, HEAD, LAYERS, VOCAB = 3584, 18944, 28, 4, 128, 28, 152064


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gemv_bytes(n: int, k: int) -> int:
    return n * (k // BLOCK_ELEMS) * BLOCK_BYTES + 4 * k + 4 * n


def decode_step_shapes():
    """(name, out_dim, in_dim) of the 113 launches of one decode step."""
    qkv = NQ * HEAD + 2 * NKV * HEAD  # 3584 + 1024
    shapes = []
    for l in range(LAYERS):
        shapes += [(f"L{l}.qkv", qkv, HIDDEN), (f"L{l}.o", HIDDEN, NQ * HEAD),
                   (f"L{l}.gate_up", 2 * INTER, HIDDEN), (f"L{l}.down", HIDDEN, INTER)]
    shapes.append(("lm_head", VOCAB, HIDDEN))
    return shapes


def layer_shapes():
    """the 7 per-layer matvecs, unfused."""
    return [("q", HIDDEN, HIDDEN), ("k", NKV * HEAD, HIDDEN), ("v", NKV * HEAD, HIDDEN),
            ("o", HIDDEN, HIDDEN), ("gate", INTER, HIDDEN), ("up", INTER, HIDDEN),
            ("down", HIDDEN, INTER)]


def make_q4k(torch, n: int, k: int, gen) -> "torch.Tensor":
    """Seeded random Q4_K bytes on the GPU with finite, model-like d/dmin."""
    nblk = n * (k // BLOCK_ELEMS)
    w = torch.randint(0, 256, (nblk, BLOCK_BYTES), dtype=torch.uint8, device="cuda", generator=gen)
    dd = (torch.rand((nblk, 2), device="cuda", generator=gen) * 2e-3 + 1e-4).to(torch.float16)
    w[:, 0:4] = dd.view(torch.uint8).view(nblk, 4)
    return w.view(-1)


class Workload:
    def __init__(self, torch, shapes, copies: int = 1, seed: int = 0x514B00):
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed)
        self.launches = []  # (name, w, x, y, n, k)
        self.keep = []
        for c in range(copies):
            for name, n, k in shapes:
                w = make_q4k(torch, n, k, gen)
                x = torch.randn(k, device="cuda", generator=gen, dtype=torch.float32)
                y = torch.empty(n, device="cuda", dtype=torch.float32)
                self.keep += [w, x, y]
                self.launches.append((f"{name}#{c}" if copies > 1 else name, w, x, y, n, k))
        self.bytes_per_pass = sum(gemv_bytes(n, k) for _, _, _, _, n, k in self.launches)
        self.weight_bytes = sum(w.numel() for _, w, _, _, _, _ in self.launches)


def time_graph(torch, q4k, wl: Workload, steps: int, warmup: int):
    chain = q4k.Chain([(w.data_ptr(), x.data_ptr(), y.data_ptr(), n, k // BLOCK_ELEMS)
                       for _, w, x, y, n, k in wl.launches])
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        chain.launch(stream)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(steps):
        chain.launch(stream)
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    chain.close()
    return ms


def check_parity(torch, wl: Workload, rows: int = 256) -> str:
    """Recompute sampled rows of a few launches with the CPU oracle."""
    from oracle import oracle as orc
    worst = 0.0
    picks = [wl.launches[0], wl.launches[2], wl.launches[3], wl.launches[-1]]
    for name, w, x, y, n, k in picks:
        bpr = k // BLOCK_ELEMS
        rng = np.random.default_rng(n + k)
        idx = np.sort(rng.choice(n, size=min(rows, n), replace=False))
        wr = w.view(n, bpr * BLOCK_BYTES)[torch.from_numpy(idx).cuda()].cpu().numpy().ravel()
        y_ref, a = orc.gemv(wr, x.cpu().numpy(), idx.size, bpr)
        yg = y.cpu().numpy()[idx]
        r = np.abs(yg.astype(np.float64) - y_ref) / np.maximum(a, 1e-300)
        worst = max(worst, float(r.max()))
        if not np.all(r <= 1e-4):
            return f"FAIL {name}: max err/absdot {r.max():.3e}"
    return f"ok (max err/absdot {worst:.2e} <= 1e-4)"


def cpu_baseline(torch, wl: Workload, target_s: float, threads: int, launches: int = 32):
    """The reference CPU GEMV restated (oracle), on the first `launches`
    launches of the workload (8 decode layers = 1.05 GB, above any host
    cache, so the CPU streams from DRAM like the GPU streams from HBM)."""
    from oracle import oracle as orc
    sample = [(name, w.cpu().numpy(), x.cpu().numpy(), n, k)
              for name, w, x, _, n, k in wl.launches[:launches]]
    nbytes = sum(gemv_bytes(n, k) for _, _, _, n, k in sample)
    ys = [np.empty(n, np.float32) for _, _, _, n, _ in sample]
    for (name, w, x, n, k), y in zip(sample, ys):  # warm-up
        orc.cpu_matvec(w, x, y, n, k // BLOCK_ELEMS, threads)
    reps, t_total = 0, 0.0
    while t_total < target_s:
        t = time.perf_counter()
        for (name, w, x, n, k), y in zip(sample, ys):
            orc.cpu_matvec(w, x, y, n, k // BLOCK_ELEMS, threads)
        t_total += time.perf_counter() - t
        reps += 1
    gbs = nbytes * reps / t_total / 1e9
    names = f"{sample[0][0]}..{sample[-1][0]} ({len(sample)} launches)"
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{names}, {nbytes / 1e6:.1f} MB of Q4_K + activations, x {reps} passes, "
                      f"{t_total:.1f} s; AVX-512={'yes' if orc.cpu_has_avx512() else 'no'}",
            "tokens_per_s_equiv": round(gbs * 1e9 / wl.bytes_per_pass, 3)}


TRAFFIC_PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "gemv_mfma_decode7b_pmc.txt")


def profiled_traffic(workload: str):
    """HBM bytes per GEMV launch from the committed FETCH_SIZE / WRITE_SIZE
    summary of this same workload (calibrated against a plain copy), or None."""
    if workload != "decode7b" or not os.path.exists(TRAFFIC_PROFILE):
        return None
    with open(TRAFFIC_PROFILE) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="decode7b", choices=["decode7b", "layer", "gateup"])
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-parity", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the Q4_K GEMV path is built and measured on a "
              "single MI355X in this build (multi-GPU sharding is design-only; see DESIGN.md).",
              file=sys.stderr)
        return 2

    import torch
    from modgrad_amd import q4k, _lib
    _lib.load()
    log(f"device {torch.cuda.get_device_name(0)}; workload {args.workload}")

    if args.workload == "decode7b":
        wl = Workload(torch, decode_step_shapes())
        desc = ("decode7b: 28 x (qkv 4608x3584, o 3584x3584, gate|up 37888x3584, down 3584x18944) "
                "+ lm_head 152064x3584, batch 1, one HIP graph per step")
    elif args.workload == "layer":
        # 7 unfused launches x 10 rotating copies (1.3 GB) so the 256 MB MALL cannot hold them
        wl = Workload(torch, layer_shapes(), copies=10)
        desc = "layer: q,k,v,o,gate,up,down of one 7B layer, unfused, 10 rotating weight copies"
    else:
        wl = Workload(torch, [("gate_up", 2 * INTER, HIDDEN)], copies=16)
        desc = "gateup: 37888x3584 x 16 rotating copies (1.2 GB)"
    torch.cuda.synchronize()
    log(f"{len(wl.launches)} launches, {wl.weight_bytes / 1e9:.3f} GB weights resident")

    ms = time_graph(torch, q4k, wl, args.steps, args.warmup)
    log(f"timed {args.steps} steps: {ms:.4f} ms/step")
    parity = "skipped" if args.no_parity else check_parity(torch, wl)
    log(f"parity: {parity}")
    # The timed region is back-to-back GEMV launches (one graph per step), so
    # the kernel's average launch duration is the step time over its launches.
    nl = len(wl.launches)
    avg_s = ms * 1e-3 / nl
    avg_b = wl.bytes_per_pass / nl
    achieved = avg_b / avg_s / 1e9
    log(f"kernel avg {avg_s * 1e6:.3f} us over {nl} launches, {achieved:.1f} GB/s")

    value = wl.bytes_per_pass / (ms * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": desc, "launches_per_step": len(wl.launches),
                   "bytes_per_step": wl.bytes_per_pass, "weights": "q4_k (144 B / 256 weights)",
                   "batch": 1},
        "tokens_per_s": round(1000.0 / ms, 2) if args.workload == "decode7b" else None,
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "parity": parity,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(args.workload), "kernel": "mgq::gemv_mfma_kernel",
                     "avg_launch_us": round(avg_s * 1e6, 3), "avg_launch_bytes": int(avg_b)},
    }
    if not args.no_cpu:
        threads = min(16, os.cpu_count() or 1)
        log(f"cpu baseline ({threads} threads, ~{args.cpu_seconds:.0f} s)")
        out["cpu_baseline"] = cpu_baseline(torch, wl, args.cpu_seconds, threads)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
