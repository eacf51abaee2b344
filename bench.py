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

The other BASELINE configs have their own workloads (one JSON line each,
measured the same way, not the headline): --workload config1 (4864x896
flattened layout), --workload batched --batch B (config 4) and --workload
prefill (config 5, TFLOP/s against the f16 matrix-core peak). Further rows:
--workload decode7b_dp4a (Q8_1 activations), q5k / q6k (the other K-quants)
decode7b_glue (the step with its RMSNorm/GeGLU glue, fused vs unfused) and
decode7b_q4km (a Q4_K_M-mixed step from one weight arena).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense f16 matrix-core peak
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


def shard_step_shapes(g: int):
    """One GPU's share of the decode step when it is sharded over g GPUs (the
    plan for more than one GPU): q/k/v, gate|up and lm_head split by rows,
    o and down by K at super-block boundaries (the largest share, when the
    blocks do not divide evenly); every GPU then holds a slice of every
    matvec and runs the same 113 launches at these shapes."""
    qkv = NQ * HEAD + 2 * NKV * HEAD
    bo = -(-(NQ * HEAD // BLOCK_ELEMS) // g) * BLOCK_ELEMS
    bd = -(-(INTER // BLOCK_ELEMS) // g) * BLOCK_ELEMS
    shapes = []
    for l in range(LAYERS):
        shapes += [(f"L{l}.qkv", -(-qkv // g), HIDDEN), (f"L{l}.o", HIDDEN, bo),
                   (f"L{l}.gate_up", -(-2 * INTER // g), HIDDEN), (f"L{l}.down", HIDDEN, bd)]
    shapes.append(("lm_head", -(-VOCAB // g), HIDDEN))
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


CHAIN_MODES = {"auto": 0, "graph": 1, "persistent": 2, "eager": 3}


def time_graph(torch, q4k, wl: Workload, steps: int, warmup: int, mode: str = "auto"):
    """ms per step of the workload's matvecs as one mgq_chain (the persistent
    chain kernel, or a HIP graph of the per-matvec launches), the per-step
    spread, and the chain's implementation."""
    chain = q4k.Chain([(w.data_ptr(), x.data_ptr(), y.data_ptr(), n, k // BLOCK_ELEMS)
                       for _, w, x, y, n, k in wl.launches], CHAIN_MODES[mode])
    impl = "persistent" if chain.mode() == CHAIN_MODES["persistent"] else "graph"
    stream = torch.cuda.current_stream()
    _settle(torch, lambda: chain.launch(stream), stream, warmup)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(steps):
        chain.launch(stream)
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    # Spread, in a separate pass after the timed region: each step between its
    # own event pair (the events add a small gap between steps, so these are
    # reported beside the value, never as it).
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(max(1, steps))]
    for a, b in ev:
        a.record(stream)
        chain.launch(stream)
        b.record(stream)
    torch.cuda.synchronize()
    spread = _spread(np.array([a.elapsed_time(b) for a, b in ev]))
    faults = chain.faults()
    chain.close()
    if faults:
        raise RuntimeError("the persistent chain reported a timed-out grid-wide wait")
    return ms, spread, impl


def time_eager(torch, q4k, wl: Workload, steps: int, warmup: int):
    """The reference engine's calling pattern (rocm_gemma.rs:312-345,
    rocm.rs:951-953): every matvec launched by launch_matvec_q4k_ex on the
    null stream (an MGQ_CHAIN_EAGER chain enqueues them one by one, with no
    Python between them), then one device synchronize per step. Returns ms per
    step (host wall clock, the synchronize included), its spread, and the host
    microseconds per launch call (the enqueue loop alone)."""
    chain = q4k.Chain([(w.data_ptr(), x.data_ptr(), y.data_ptr(), n, k // BLOCK_ELEMS)
                       for _, w, x, y, n, k in wl.launches], CHAIN_MODES["eager"])
    assert chain.mode() == CHAIN_MODES["eager"]
    t_end = time.perf_counter() + WARM_MS * 1e-3
    for i in range(max(1, warmup)):
        chain.launch(None)
        torch.cuda.synchronize()
    while time.perf_counter() < t_end:
        chain.launch(None)
        torch.cuda.synchronize()
    host, per = [], []
    t0 = time.perf_counter()
    for _ in range(steps):
        a = time.perf_counter()
        chain.launch(None)
        b = time.perf_counter()
        torch.cuda.synchronize()
        host.append(b - a)
        per.append(time.perf_counter() - a)
    ms = (time.perf_counter() - t0) / steps * 1e3
    chain.close()
    host_us = float(np.median(host)) * 1e6 / len(wl.launches)
    return ms, _spread(np.array(per) * 1e3), host_us


def shape_times(torch, q4k, wl: Workload, reps: int = 20) -> dict:
    """us per launch of each launch shape of the step, measured after the
    timed region: the step's launches of one shape (their own weights and
    activations) as one graph chain, replayed `reps` times between events."""
    groups = {}
    for i, (name, _, _, _, n, k) in enumerate(wl.launches):
        groups.setdefault(name.split(".")[-1].split("#")[0], []).append(i)
    stream = torch.cuda.current_stream()
    out = {}
    for shape, idx in groups.items():
        chain = q4k.Chain([(wl.launches[i][1].data_ptr(), wl.launches[i][2].data_ptr(),
                            wl.launches[i][3].data_ptr(), wl.launches[i][4],
                            wl.launches[i][5] // BLOCK_ELEMS) for i in idx], CHAIN_MODES["graph"])
        for _ in range(3):
            chain.launch(stream)
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(reps):
            chain.launch(stream)
        t1.record(stream)
        torch.cuda.synchronize()
        n, k = wl.launches[idx[0]][4], wl.launches[idx[0]][5]
        us = t0.elapsed_time(t1) * 1e3 / (reps * len(idx))
        out[shape] = {"shape": f"{n}x{k}", "launches": len(idx), "us_per_launch": round(us, 3),
                      "hbm_frac": round(gemv_bytes(n, k) / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        chain.close()
    return out


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


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads() -> int:
    """Threads for the multi-core leg: every core this process may run on
    (its affinity set), capped at OMP_NUM_THREADS when that is set -- the GPU
    boxes allot each GPU a share of the host's cores and set it there."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def cpu_baseline(torch, wl: Workload, target_s: float, threads: int, launches: int = 32,
                 target_1t_s: float = 5.0):
    """The reference CPU GEMV restated (oracle): kfd::llm::matvec
    (llm.rs:468-534, rows in parallel as its rayon pool does, llm.rs:506-511)
    with the AVX-512 dot (llm.rs:748-806). Timed on the first `launches`
    launches of the workload (8 decode layers = 1.05 GB, above any host
    cache, so the CPU streams from DRAM like the GPU streams from HBM), on
    `threads` threads and on one thread."""
    from oracle import oracle as orc
    sample = [(name, w.cpu().numpy(), x.cpu().numpy(), n, k)
              for name, w, x, _, n, k in wl.launches[:launches]]
    nbytes = sum(gemv_bytes(n, k) for _, _, _, n, k in sample)
    ys = [np.empty(n, np.float32) for _, _, _, n, _ in sample]

    def timed(nthreads: int, budget: float):
        for (name, w, x, n, k), y in zip(sample, ys):  # warm-up
            orc.cpu_matvec(w, x, y, n, k // BLOCK_ELEMS, nthreads)
        reps, t_total = 0, 0.0
        while t_total < budget:
            t = time.perf_counter()
            for (name, w, x, n, k), y in zip(sample, ys):
                orc.cpu_matvec(w, x, y, n, k // BLOCK_ELEMS, nthreads)
            t_total += time.perf_counter() - t
            reps += 1
        return nbytes * reps / t_total / 1e9, reps, t_total

    gbs, reps, t_total = timed(threads, target_s)
    gbs1, reps1, t1 = timed(1, target_1t_s) if threads > 1 else (gbs, reps, t_total)
    names = f"{sample[0][0]}..{sample[-1][0]} ({len(sample)} launches)"
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{names}, {nbytes / 1e6:.1f} MB of Q4_K + activations, x {reps} passes, "
                      f"{t_total:.1f} s on {threads} threads; 1 thread: x {reps1} passes, "
                      f"{t1:.1f} s; AVX-512={'yes' if orc.cpu_has_avx512() else 'no'}",
            "value_1thread": round(gbs1, 3),
            "cpu_model": cpu_model(),
            "host_logical_cpus": os.cpu_count(),
            "tokens_per_s_equiv": round(gbs * 1e9 / wl.bytes_per_pass, 3),
            "tokens_per_s_equiv_1thread": round(gbs1 * 1e9 / wl.bytes_per_pass, 4)}


def cpu_jobs_baseline(jobs, units_per_pass: float, unit: str, sample: str, threads: int,
                      target_s: float, target_1t_s: float = 3.0, digits: int = 2):
    """The reference CPU GEMV restated (oracle: kfd::llm::matvec, llm.rs:468-534,
    rows in parallel as its rayon pool does, llm.rs:506-511) on a side
    workload's sample: `jobs` = [(w, x, y, n, bpr)], one pass runs each once
    and is worth `units_per_pass` of the workload's metric (GB as the GPU line
    counts them, or TFLOP); timed on `threads` threads and on one thread."""
    from oracle import oracle as orc

    def timed(nthreads: int, budget: float):
        for w, x, y, n, bpr in jobs:  # warm-up
            orc.cpu_matvec(w, x, y, n, bpr, nthreads)
        reps, t_total = 0, 0.0
        while t_total < budget:
            t = time.perf_counter()
            for w, x, y, n, bpr in jobs:
                orc.cpu_matvec(w, x, y, n, bpr, nthreads)
            t_total += time.perf_counter() - t
            reps += 1
        return units_per_pass * reps / t_total, reps, t_total

    v, reps, t_total = timed(threads, target_s)
    v1, reps1, t1 = timed(1, target_1t_s) if threads > 1 else (v, reps, t_total)
    return {"value": round(v, digits), "unit": unit, "cores": threads, "kind": "port",
            "sample": f"{sample}, x {reps} passes, {t_total:.1f} s on {threads} threads; "
                      f"1 thread: x {reps1} passes, {t1:.1f} s; "
                      f"AVX-512={'yes' if orc.cpu_has_avx512() else 'no'}",
            "value_1thread": round(v1, digits + 1), "cpu_model": cpu_model(),
            "host_logical_cpus": os.cpu_count()}


def cpu_flat_baseline(w, x, n: int, k: int, launch_gb: float, target_s: float = 3.0):
    """Config 1's flattened layout has no CPU path in the reference (the
    LinearResidentQuantized forward is GPU-only, neuron.rs:897-1108); the
    oracle's flat-layout dequant-dot (one thread, f64) stands in, in the
    GPU line's bytes per launch."""
    from oracle import oracle as orc
    orc.gemv_flat(w, x, n, k)
    reps, t_total = 0, 0.0
    while t_total < target_s:
        t = time.perf_counter()
        orc.gemv_flat(w, x, n, k)
        t_total += time.perf_counter() - t
        reps += 1
    return {"value": round(launch_gb * reps / t_total, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "stand_in": "no reference CPU path exists for the flattened layout; this is the oracle's "
                        "f64 flat-layout dequant-dot, not a restatement of a reference CPU kernel",
            "sample": f"oracle flat-layout dequant-dot (f64) on one 4864x896 launch, x {reps} passes, "
                      f"{t_total:.1f} s on 1 thread (the reference has no CPU path for this layout)",
            "cpu_model": cpu_model(), "host_logical_cpus": os.cpu_count()}


WARM_MS = 100.0  # least untimed run time before a timed region (ms)


def _settle(torch, run_once, stream, warmup: int) -> None:
    """`warmup` untimed runs, then more up to ~WARM_MS in all, so that clocks
    and caches are at steady state when the timed region starts (after a
    short warm-up the first timed launches of a heavy kernel run ~10 % slow)."""
    for _ in range(warmup):
        run_once()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    run_once()
    t1.record(stream)
    torch.cuda.synchronize()
    extra = int(min(2000, max(0.0, WARM_MS / max(t0.elapsed_time(t1), 1e-3) - warmup)))
    for _ in range(extra):
        run_once()
    torch.cuda.synchronize()


def time_captured(torch, launch, steps: int, warmup: int) -> float:
    """ms per replay of a HIP graph captured (through torch) from `launch`,
    a callable that enqueues one pass on the stream it is given."""
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        launch(stream)  # eager warm-up: first-use kernel attributes
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        launch(torch.cuda.current_stream())
    cur = torch.cuda.current_stream()
    _settle(torch, g.replay, cur, warmup)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(cur)
    for _ in range(steps):
        g.replay()
    t1.record(cur)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    # per-replay spread, a separate pass after the timed region
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(max(1, steps))]
    for a, b in ev:
        a.record(cur)
        g.replay()
        b.record(cur)
    torch.cuda.synchronize()
    SPREADS.append(_spread(np.array([a.elapsed_time(b) for a, b in ev])))
    return ms


def time_op_chain(torch, q4k, ops, steps: int, warmup: int) -> float:
    """ms per launch of a chain of mgq_op_desc kernels (one HIP graph recorded
    by the library, mgq_chain_create_ops), timed like time_captured."""
    chain = q4k.Chain.from_ops(ops)
    stream = torch.cuda.current_stream()
    _settle(torch, lambda: chain.launch(stream), stream, max(1, warmup))
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(steps):
        chain.launch(stream)
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(max(1, steps))]
    for a, b in ev:
        a.record(stream)
        chain.launch(stream)
        b.record(stream)
    torch.cuda.synchronize()
    SPREADS.append(_spread(np.array([a.elapsed_time(b) for a, b in ev])))
    chain.close()
    return ms


# per-pass (p10, median, p90) ms of every time_captured call, in call order
SPREADS: list = []


def _spread(per) -> dict:
    return {"p10": round(float(np.percentile(per, 10)), 5),
            "median": round(float(np.median(per)), 5),
            "p90": round(float(np.percentile(per, 90)), 5), "n": int(per.size)}


def run_config1(torch, q4k, args):
    """Qwen2.5-0.5B up-projection 4864x896 (896 % 256 != 0,
    so the flattened-tensor layout of LinearResidentQuantized), rotating
    copies past 1 GiB so no cache holds the weights."""
    from oracle import oracle as orc
    n, k = 4864, 896
    nblk = n * k // BLOCK_ELEMS
    wbytes = nblk * BLOCK_BYTES
    copies = -(-(1 << 30) // wbytes)
    # weights from the reference quantizer on seeded N(0, 0.02) (neuron.rs:931-951)
    w_host = orc.seeded_weight(0x514B00 + 5, n, k)
    x_host = orc.normal(0x514B05 ^ 0xA5A5, k)
    w = torch.from_numpy(w_host).cuda().repeat(copies).view(copies, wbytes)
    x = torch.from_numpy(x_host).cuda()
    y = torch.empty((copies, n), device="cuda")

    def launch(st):
        for c in range(copies):
            q4k.kern.matvec_q4k_ex(w[c].data_ptr(), x.data_ptr(), y[c].data_ptr(), n, k,
                                   1, st)  # MGQ_LAYOUT_FLAT
    ms = time_captured(torch, launch, args.steps, args.warmup)
    nbytes = copies * (wbytes + 4 * (n + k))
    y_ref, a = orc.gemv_flat(w_host, x_host, n, k)
    r = np.abs(y[copies - 1].cpu().numpy().astype(np.float64) - y_ref) / np.maximum(a, 1e-300)
    parity = f"ok (max err/absdot {r.max():.2e} <= 1e-4)" if np.all(r <= 1e-4) else \
        f"FAIL: max err/absdot {r.max():.3e}"
    us = ms * 1e3 / copies
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"workload": "config1: 4864x896 flattened Q4_K (LinearResidentQuantized layout), "
                        f"{copies} rotating copies, one graph", "us_per_launch": round(us, 3),
            "gbs": gbs, "bytes_per_launch": nbytes // copies, "parity": parity,
            "kernel": "mgq::gemv_flat_kernel<2>",
            "cpu_flat": (w_host, x_host, n, k, nbytes / copies / 1e9)}


def run_batched(torch, q4k, args):
    """gate/up 18944x3584 and down 3584x18944 at batch B."""
    from oracle import oracle as orc
    B = args.batch
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x514B40 + B)
    shapes = [("gate", INTER, HIDDEN), ("down", HIDDEN, INTER)]
    copies = 16  # 16 x 76 MB: past the 256 MiB MALL
    items = []
    for c in range(copies):
        for name, n, k in shapes:
            bpr = k // BLOCK_ELEMS
            w = make_q4k(torch, n, k, gen)
            X = torch.randn((B, k), device="cuda", generator=gen)
            Y = torch.empty((B, n), device="cuda")
            ws = torch.empty(q4k.kern.batched_workspace_bytes(bpr, B), dtype=torch.uint8, device="cuda")
            items.append((name, w, X, Y, ws, n, bpr))

    def launch(st):
        for name, w, X, Y, ws, n, bpr in items:
            q4k.kern.matvec_q4k_batched(w.data_ptr(), X.data_ptr(), Y.data_ptr(), n, bpr, B, st,
                                        workspace=ws)
    ms = time_captured(torch, launch, args.steps, args.warmup)
    nbytes = sum(n * bpr * BLOCK_BYTES + 4 * B * (bpr * BLOCK_ELEMS + n) for _, _, _, _, _, n, bpr in items)
    worst = 0.0
    parity = None
    for name, w, X, Y, ws, n, bpr in items[-2:]:
        idx = np.sort(np.random.default_rng(n).choice(n, size=128, replace=False))
        wr = w.view(n, bpr * BLOCK_BYTES)[torch.from_numpy(idx).cuda()].cpu().numpy().ravel()
        Xh, Yh = X.cpu().numpy(), Y.cpu().numpy()[:, idx]
        for b in range(B):
            y_ref, a = orc.gemv(wr, Xh[b], idx.size, bpr)
            r = np.abs(Yh[b].astype(np.float64) - y_ref) / np.maximum(a, 1e-300)
            worst = max(worst, float(r.max()))
            if not np.all(r <= 1e-4):
                parity = f"FAIL {name} b={b}: max err/absdot {r.max():.3e}"
    parity = parity or f"ok (max err/absdot {worst:.2e} <= 1e-4)"
    # per shape, and gate|up as one call: in a model gate and up read the
    # same X, so with their rows contiguous (one 37888-row tensor, as the
    # decode workload stores them) one operand table serves both
    per_shape = {}
    for name in ("gate", "down"):
        sub = [it for it in items if it[0] == name]

        def launch_one(st, sub=sub):
            for _, w, X, Y, ws, n, bpr in sub:
                q4k.kern.matvec_q4k_batched(w.data_ptr(), X.data_ptr(), Y.data_ptr(), n, bpr, B, st,
                                            workspace=ws)
        per_shape[f"{name}_us"] = round(time_captured(torch, launch_one, args.steps, args.warmup)
                                        * 1e3 / len(sub), 3)
    gu = []
    for c in range(copies // 2):
        bpr = HIDDEN // BLOCK_ELEMS
        w = make_q4k(torch, 2 * INTER, HIDDEN, gen)
        X = torch.randn((B, HIDDEN), device="cuda", generator=gen)
        Y = torch.empty((B, 2 * INTER), device="cuda")
        ws = torch.empty(q4k.kern.batched_workspace_bytes(bpr, B), dtype=torch.uint8, device="cuda")
        gu.append((w, X, Y, ws, 2 * INTER, bpr))

    def launch_gu(st):
        for w, X, Y, ws, n, bpr in gu:
            q4k.kern.matvec_q4k_batched(w.data_ptr(), X.data_ptr(), Y.data_ptr(), n, bpr, B, st,
                                        workspace=ws)
    us_gu = time_captured(torch, launch_gu, args.steps, args.warmup) * 1e3 / len(gu)
    gu_bytes = 2 * INTER * (HIDDEN // BLOCK_ELEMS) * BLOCK_BYTES + 4 * B * (HIDDEN + 2 * INTER)
    per_shape["gate_up_fused_37888x3584_us"] = round(us_gu, 3)
    per_shape["gate_up_fused_gbs"] = round(gu_bytes / (us_gu * 1e-6) / 1e9, 1)
    # CPU: the reference's CPU GEMV has no batch, so a batched call is B
    # matvecs over the same weights; one pass = the last gate and down calls,
    # worth their bytes as the GPU line counts them
    jobs, pass_bytes = [], 0
    for name, w, X, Y, ws, n, bpr in items[-2:]:
        wh, Xh = w.cpu().numpy(), X.cpu().numpy()
        jobs += [(wh, np.ascontiguousarray(Xh[b]), np.empty(n, np.float32), n, bpr) for b in range(B)]
        pass_bytes += n * bpr * BLOCK_BYTES + 4 * B * (bpr * BLOCK_ELEMS + n)
    return {"workload": f"config4: batched B={B}, gate 18944x3584 + down 3584x18944, "
                        f"{copies} rotating copies, one graph",
            "us_per_launch": round(ms * 1e3 / len(items), 3), "gbs": nbytes / (ms * 1e-3) / 1e9,
            "bytes_per_launch": nbytes // len(items), "parity": parity, "per_shape": per_shape,
            "kernel": "mgq::gemv_batched_wave_kernel (+ batched_table_kernel)",
            "cpu": (jobs, pass_bytes / 1e9, "GB/s",
                    f"one gate and one down call at B={B} as {len(jobs)} CPU matvecs "
                    f"({pass_bytes / 1e6:.1f} MB per pass as the GPU line counts it)", 2)}


def run_prefill(torch, q4k, args):
    """Q4_K W 18944x3584 times f16 A [512 x 3584]."""
    from oracle import oracle as orc
    n, k, m = INTER, HIDDEN, 512
    bpr = k // BLOCK_ELEMS
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0xF16)
    copies = 4
    ws = [make_q4k(torch, n, k, gen) for _ in range(copies)]
    A = torch.randn((m, k), device="cuda", generator=gen).to(torch.float16)
    Cs = [torch.empty((m, n), device="cuda") for _ in range(copies)]

    def launch(st):
        for w, C in zip(ws, Cs):
            q4k.kern.gemm_q4k_f16(w.data_ptr(), A.data_ptr(), C.data_ptr(), n, bpr, m, st)
    ms = time_captured(torch, launch, args.steps, args.warmup)
    s = ms * 1e-3 / copies
    tflops = 2.0 * n * k * m / s / 1e12
    idx = np.sort(np.random.default_rng(5).choice(n, size=64, replace=False))
    wr = ws[-1].view(n, bpr * BLOCK_BYTES)[torch.from_numpy(idx).cuda()].cpu().numpy().ravel()
    a16 = A.cpu().numpy().view(np.uint16).reshape(m, k)
    C_ref, absd = orc.gemm_f16(wr, a16, idx.size, bpr)   # [m][sampled rows]
    C_ref = C_ref.astype(np.float64)
    Cg = Cs[-1].cpu().numpy()[:, idx].astype(np.float64)
    elem_ok = np.all(np.abs(Cg - C_ref) <= 1e-2 * absd / np.sqrt(k))
    frob = float(np.linalg.norm(Cg - C_ref) / max(np.linalg.norm(C_ref), 1e-300))
    parity = (f"ok (frobenius rel {frob:.2e} <= 1e-3, per-element <= 1e-2*sum|w||a|/sqrt(K))"
              if elem_ok and frob <= 1e-3 else f"FAIL: frobenius rel {frob:.3e}, elementwise {elem_ok}")
    # CPU: the reference's prefill is a per-token matvec loop
    # (gemma4_rocm.rs:26-34); on the CPU that is one GEMV per token, timed on
    # 16 of the 512 tokens (f32 activations: the f16 values, exactly)
    wh = ws[-1].cpu().numpy()
    toks = 16
    jobs = [(wh, A[t].float().cpu().numpy(), np.empty(n, np.float32), n, bpr) for t in range(toks)]
    return {"workload": f"config5: prefill 18944x3584 Q4_K x f16 [512x3584], {copies} weight copies",
            "us_per_launch": round(s * 1e6, 3), "tflops": tflops, "parity": parity,
            "kernel": "mgq::gemm_q4k_f16_lds_kernel",
            "cpu": (jobs, 2.0 * n * k * toks / 1e12, "TFLOP/s",
                    f"{toks} of the 512 tokens, one CPU matvec each (2*N*K flops per token)", 5)}


def run_decode_dp4a(torch, q4k, args):
    """The decode step of the default workload on the reference engine's
    default arm (rocm_gemma.rs:298-306): per matvec, launch_quantize_q8_1 on
    its x, then launch_matvec_q4k_dp4a (226 launches); and the same with
    launch_quantize_matvec_q4k_dp4a_ex, which quantizes inside the matvec
    (113 launches, bit-identical y). Accuracy is int8's: the check is the
    reference's RMS-relative error < 0.02 against the f32 dequant-dot."""
    from oracle import oracle as orc
    wl = Workload(torch, decode_step_shapes())
    q8 = []
    for name, w, x, y, n, k in wl.launches:
        nsub = k // 32
        q8.append((torch.empty(k, dtype=torch.int8, device="cuda"),
                   torch.empty(nsub, device="cuda"), torch.empty(nsub, device="cuda")))

    # both recorded by the library as op chains (mgq_chain_create_ops), the
    # way a Rust host keeping the reference's default arm would record them
    two_launch, fused = [], []
    for (name, w, x, y, n, k), (xq, xd, xs) in zip(wl.launches, q8):
        two_launch += [q4k.op_quantize_q8_1(x.data_ptr(), xq.data_ptr(), xd.data_ptr(),
                                            xs.data_ptr(), k),
                       q4k.op_matvec_dp4a(12, w.data_ptr(), xq.data_ptr(), xd.data_ptr(),
                                          xs.data_ptr(), y.data_ptr(), n, k)]
        fused.append(q4k.op_quantize_matvec_dp4a(w.data_ptr(), x.data_ptr(), y.data_ptr(), n, k))
    ms_two = time_op_chain(torch, q4k, two_launch, args.steps, args.warmup)
    ms = time_op_chain(torch, q4k, fused, args.steps, args.warmup)
    worst = 0.0
    for name, w, x, y, n, k in (wl.launches[0], wl.launches[3], wl.launches[-1]):
        bpr = k // BLOCK_ELEMS
        idx = np.sort(np.random.default_rng(n).choice(n, size=min(512, n), replace=False))
        wr = w.view(n, bpr * BLOCK_BYTES)[torch.from_numpy(idx).cuda()].cpu().numpy().ravel()
        y_ref, _ = orc.gemv(wr, x.cpu().numpy(), idx.size, bpr)
        yg = y.cpu().numpy()[idx].astype(np.float64)
        worst = max(worst, float(np.sqrt(np.sum((yg - y_ref) ** 2) / np.sum(y_ref.astype(np.float64) ** 2))))
    parity = (f"ok (RMS_rel vs f32 dequant-dot {worst:.2e} < 0.02)" if worst < 0.02
              else f"FAIL: RMS_rel {worst:.3e}")
    nbytes = wl.bytes_per_pass
    return {"workload": "decode7b_dp4a: the decode7b step on Q8_1 activations, each matvec as "
                        "launch_quantize_matvec_q4k_dp4a_ex (113 launches; the reference's "
                        "quantize_q8_1 + matvec_q4k_dp4a pair, 226 launches, timed beside it), "
                        "each step one op chain (mgq_chain_create_ops)",
            "us_per_launch": round(ms * 1e3 / len(wl.launches), 3), "gbs": nbytes / (ms * 1e-3) / 1e9,
            "bytes_per_launch": nbytes // len(wl.launches), "parity": parity,
            "kernel": "mgq::gemv_mfma_kernel<..., Q8, kFuseQuant>",
            "tokens_per_s": 1000.0 / ms, "ms_per_step": ms,
            "unfused_ms_per_step": ms_two, "unfused_tokens_per_s": 1000.0 / ms_two}


def run_decode_glue(torch, q4k, args):
    """The decode step with its glue, as the reference engine runs it
    (rocm_gemma.rs:439-483, attention itself left out): per layer
    rms_norm -> qkv, o, rms_norm -> gate|up -> geglu -> down, and the final
    rms_norm -> lm_head. Timed twice, each as one captured graph:
      unfused: launch_rms_norm / launch_geglu between the matvecs (198 launches);
      fused:   launch_matvec_q4k_rmsnorm_ex (qkv, lm_head) and
               launch_matvec_q4k_glu_ex (gate, up, geglu) (113 launches).
    value = the fused step's algorithmic GB/s over the same bytes as decode7b."""
    from oracle import oracle as orc
    wl = Workload(torch, decode_step_shapes())
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x6E0)
    eps = 1e-6
    L = wl.launches
    layers = []
    for l in range(LAYERS):
        qkv, o, gu, dn = L[4 * l: 4 * l + 4]
        nw_a = torch.rand(HIDDEN, device="cuda", generator=gen) + 0.5
        nw_f = torch.rand(HIDDEN, device="cuda", generator=gen) + 0.5
        layers.append((qkv, o, gu, dn, nw_a, nw_f, torch.empty(HIDDEN, device="cuda"),
                       torch.empty(HIDDEN, device="cuda"), torch.empty(INTER, device="cuda")))
    lm = L[-1]
    nw_lm = torch.rand(HIDDEN, device="cuda", generator=gen) + 0.5
    xn_lm = torch.empty(HIDDEN, device="cuda")
    bpr_h = HIDDEN // BLOCK_ELEMS
    gu_rows_bytes = INTER * bpr_h * BLOCK_BYTES  # gate rows, then up rows

    def unfused(st):
        k = q4k.kern
        for (qkv, o, gu, dn, nw_a, nw_f, xa, xf, glu) in layers:
            k.rms_norm(qkv[2].data_ptr(), nw_a.data_ptr(), xa.data_ptr(), 1, HIDDEN, eps, st)
            k.matvec_q4k_ex(qkv[1].data_ptr(), xa.data_ptr(), qkv[3].data_ptr(), qkv[4], HIDDEN, stream=st)
            k.matvec_q4k_ex(o[1].data_ptr(), o[2].data_ptr(), o[3].data_ptr(), o[4], o[5], stream=st)
            k.rms_norm(gu[2].data_ptr(), nw_f.data_ptr(), xf.data_ptr(), 1, HIDDEN, eps, st)
            k.matvec_q4k_ex(gu[1].data_ptr(), xf.data_ptr(), gu[3].data_ptr(), gu[4], HIDDEN, stream=st)
            k.glu(gu[3].data_ptr(), gu[3].data_ptr() + 4 * INTER, glu.data_ptr(), INTER, stream=st)
            k.matvec_q4k_ex(dn[1].data_ptr(), glu.data_ptr(), dn[3].data_ptr(), dn[4], dn[5], stream=st)
        k.rms_norm(lm[2].data_ptr(), nw_lm.data_ptr(), xn_lm.data_ptr(), 1, HIDDEN, eps, st)
        k.matvec_q4k_ex(lm[1].data_ptr(), xn_lm.data_ptr(), lm[3].data_ptr(), lm[4], HIDDEN, stream=st)

    def fused(st):
        k = q4k.kern
        for (qkv, o, gu, dn, nw_a, nw_f, xa, xf, glu) in layers:
            k.matvec_q4k_rmsnorm(qkv[1].data_ptr(), qkv[2].data_ptr(), nw_a.data_ptr(), eps,
                                 qkv[3].data_ptr(), qkv[4], bpr_h, st)
            k.matvec_q4k_ex(o[1].data_ptr(), o[2].data_ptr(), o[3].data_ptr(), o[4], o[5], stream=st)
            k.matvec_q4k_glu(gu[1].data_ptr(), gu[1].data_ptr() + gu_rows_bytes, gu[2].data_ptr(),
                             glu.data_ptr(), INTER, bpr_h, nw_f.data_ptr(), eps, stream=st)
            k.matvec_q4k_ex(dn[1].data_ptr(), glu.data_ptr(), dn[3].data_ptr(), dn[4], dn[5], stream=st)
        k.matvec_q4k_rmsnorm(lm[1].data_ptr(), lm[2].data_ptr(), nw_lm.data_ptr(), eps,
                             lm[3].data_ptr(), lm[4], bpr_h, st)

    ms_unfused = time_captured(torch, unfused, args.steps, args.warmup)
    ms = time_captured(torch, fused, args.steps, args.warmup)
    # parity: layer 0's fused qkv and GLU outputs (sampled rows) against the
    # oracle's rms_norm -> f64 matvec (-> gelu_tanh * up)
    qkv, o, gu, dn, nw_a, nw_f, xa, xf, glu = layers[0]
    worst, fail = 0.0, None
    rng = np.random.default_rng(5)
    xn = orc.rms_norm(qkv[2].cpu().numpy(), nw_a.cpu().numpy(), 1, HIDDEN, eps)
    idx = np.sort(rng.choice(qkv[4], size=256, replace=False))
    wr = qkv[1].view(qkv[4], -1)[torch.from_numpy(idx).cuda()].cpu().numpy().ravel()
    y_ref, a = orc.gemv(wr, xn, idx.size, bpr_h)
    r = np.abs(qkv[3].cpu().numpy()[idx].astype(np.float64) - y_ref) / a
    worst = max(worst, float(r.max()))
    if not np.all(r <= 1e-4):
        fail = f"FAIL rmsnorm+qkv: {r.max():.3e}"
    xn = orc.rms_norm(gu[2].cpu().numpy(), nw_f.cpu().numpy(), 1, HIDDEN, eps)
    idx = np.sort(rng.choice(INTER, size=256, replace=False))
    wv = gu[1].view(2 * INTER, -1)
    g, ag = orc.gemv(wv[torch.from_numpy(idx).cuda()].cpu().numpy().ravel(), xn, idx.size, bpr_h)
    u, au = orc.gemv(wv[torch.from_numpy(idx + INTER).cuda()].cpu().numpy().ravel(), xn, idx.size, bpr_h)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    act = 0.5 * g64 * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g64 + 0.044715 * g64 ** 3)))
    ref = act * u64
    bound = 1e-4 * (1.13 * ag * np.abs(u64) + np.abs(act) * au) + 1e-5 * np.abs(ref)
    err = np.abs(glu.cpu().numpy()[idx].astype(np.float64) - ref)
    if not np.all(err <= bound):
        fail = fail or f"FAIL gate/up glu: max err/bound {float((err / bound).max()):.3e}"
    parity = fail or (f"ok (rmsnorm+qkv max err/absdot {worst:.2e} <= 1e-4; gate/up glu within "
                      f"the propagated 1e-4 bound, max err/bound {float((err / bound).max()):.2e})")
    nbytes = wl.bytes_per_pass
    return {"workload": "decode7b_glue: decode7b with its RMSNorm/GeGLU glue; fused "
                        "(rmsnorm+qkv, o, rmsnorm+gate/up+geglu, down; 113 launches) vs unfused "
                        "(198 launches), one graph each",
            "us_per_launch": round(ms * 1e3 / 113, 3), "gbs": nbytes / (ms * 1e-3) / 1e9,
            "bytes_per_launch": nbytes // len(wl.launches), "parity": parity,
            "kernel": "mgq::gemv_mfma_kernel<..., FUSE>", "tokens_per_s": 1000.0 / ms,
            "ms_per_step": ms, "unfused_ms_per_step": ms_unfused,
            "unfused_tokens_per_s": 1000.0 / ms_unfused}


def q4km_more_bits(i: int, n: int) -> bool:
    """llama.cpp's Q4_K_M rule for attn_v / ffn_down: Q6_K on the first and
    last eighth of the layers and every third layer between."""
    return i < n // 8 or i >= 7 * n // 8 or (i - n // 8) % 3 == 2


def run_decode_q4km(torch, q4k, args):
    """A Q4_K_M 7B-class decode step from one weight arena (the GGUF loader's
    layout): Q4_K everywhere except attn_v and ffn_down on the Q4_K_M
    'more bits' layers (Q6_K) and the Q6_K output matrix, as llama.cpp's
    Q4_K_M recipe assigns them. Per layer: RMSNorm fused into q|k and into v
    (Q4_K or Q6_K; an rms_norm launch only where the fused Q6_K kernel cannot
    take the tensor), o, RMSNorm + gate/up + GeGLU fused, down (Q4_K or
    Q6_K); then RMSNorm fused into the Q6_K lm_head. Seeded random weights,
    one captured graph."""
    from oracle import oracle as orc
    from modgrad_amd.arena import WeightArena
    from modgrad_amd.gguf import GgmlType
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x4B4D)
    Q4, Q6 = GgmlType.Q4_K, GgmlType.Q6_K
    kv = NKV * HEAD
    entries = []
    for l in range(LAYERS):
        more = q4km_more_bits(l, LAYERS)
        entries += [(f"blk.{l}.attn_qk.weight", [HIDDEN, HIDDEN + kv], Q4),
                    (f"blk.{l}.attn_v.weight", [HIDDEN, kv], Q6 if more else Q4),
                    (f"blk.{l}.attn_output.weight", [NQ * HEAD, HIDDEN], Q4),
                    (f"blk.{l}.ffn_gate.weight", [HIDDEN, INTER], Q4),
                    (f"blk.{l}.ffn_up.weight", [HIDDEN, INTER], Q4),
                    (f"blk.{l}.ffn_down.weight", [INTER, HIDDEN], Q6 if more else Q4),
                    (f"blk.{l}.attn_norm.weight", [HIDDEN], GgmlType.F32),
                    (f"blk.{l}.ffn_norm.weight", [HIDDEN], GgmlType.F32)]
    entries += [("output_norm.weight", [HIDDEN], GgmlType.F32), ("output.weight", [HIDDEN, VOCAB], Q6)]
    arena = WeightArena(entries)
    for name, dims, t in entries:
        v = arena.tensor(name)
        if t == GgmlType.F32:
            v.view(torch.float32).copy_(torch.rand(dims[0], device="cuda", generator=gen) + 0.5)
            continue
        v.copy_(torch.randint(0, 256, (v.numel(),), dtype=torch.uint8, device="cuda", generator=gen))
        bb = 144 if t == Q4 else 210
        blk = v.view(-1, bb)
        nd = 2 if t == Q4 else 1
        dd = (torch.rand((blk.shape[0], nd), device="cuda", generator=gen) * 2e-3 + 1e-4).to(torch.float16)
        if t == Q4:
            blk[:, 0:4] = dd.view(torch.uint8).view(-1, 4)
        else:
            blk[:, 208:210] = dd.view(torch.uint8).view(-1, 2)
    eps = 1e-6
    f = lambda n: torch.empty(n, device="cuda")
    hs = [torch.randn(HIDDEN, device="cuda", generator=gen) for _ in range(2 * LAYERS + 1)]
    att = [torch.randn(NQ * HEAD, device="cuda", generator=gen) for _ in range(LAYERS)]
    xn, qk, vv, o, glu, dn, logits = f(HIDDEN), f(HIDDEN + kv), f(kv), f(HIDDEN), f(INTER), f(HIDDEN), f(VOCAB)
    # the step as mgq_op_desc descriptors, recorded into one graph through the
    # C ABI (mgq_chain_create_ops): what a Rust host would record
    A, ops = arena, []
    for l in range(LAYERS):
        p = f"blk.{l}."
        h0, h1 = hs[2 * l].data_ptr(), hs[2 * l + 1].data_ptr()
        if A.norm_fusable(p + "attn_v.weight"):
            ops.append(A.op_qmatvec_rmsnorm(p + "attn_qk.weight", h0, p + "attn_norm.weight", eps,
                                            qk.data_ptr()))
            ops.append(A.op_qmatvec_rmsnorm(p + "attn_v.weight", h0, p + "attn_norm.weight", eps,
                                            vv.data_ptr()))
        else:
            ops.append(q4k.op_rms_norm(h0, A.ptr(p + "attn_norm.weight"), xn.data_ptr(), 1, HIDDEN,
                                       eps))
            ops.append(A.op_qmatvec(p + "attn_qk.weight", xn.data_ptr(), qk.data_ptr()))
            ops.append(A.op_qmatvec(p + "attn_v.weight", xn.data_ptr(), vv.data_ptr()))
        ops.append(A.op_qmatvec(p + "attn_output.weight", att[l].data_ptr(), o.data_ptr()))
        ops.append(A.op_qmatvec_glu(p + "ffn_gate.weight", p + "ffn_up.weight", h1, glu.data_ptr(),
                                    norm=p + "ffn_norm.weight", eps=eps))
        ops.append(A.op_qmatvec(p + "ffn_down.weight", glu.data_ptr(), dn.data_ptr()))
    if A.norm_fusable("output.weight"):
        ops.append(A.op_qmatvec_rmsnorm("output.weight", hs[-1].data_ptr(), "output_norm.weight",
                                        eps, logits.data_ptr()))
    else:
        ops.append(q4k.op_rms_norm(hs[-1].data_ptr(), A.ptr("output_norm.weight"), xn.data_ptr(),
                                   1, HIDDEN, eps))
        ops.append(A.op_qmatvec("output.weight", xn.data_ptr(), logits.data_ptr()))
    launches = [len(ops)]
    ms = time_op_chain(torch, q4k, ops, args.steps, args.warmup)
    # parity: the last layer's Q6_K or Q4_K down (its GLU input as produced)
    # and the Q6_K lm_head, sampled rows against the oracle
    worst, fail = 0.0, None
    # lm_head's input: the oracle's rms_norm of the last hidden state (the
    # fused kernel never writes the normalized vector)
    xn_ref = orc.rms_norm(hs[-1].cpu().numpy(), arena.tensor("output_norm.weight").view(torch.float32)
                          .cpu().numpy(), 1, HIDDEN, eps).astype(np.float32)
    checks = [(f"blk.{LAYERS - 1}.ffn_down.weight", glu.cpu().numpy(), dn),
              ("output.weight", xn_ref, logits)]
    rng = np.random.default_rng(9)
    for name, xin, yout in checks:
        nrow, kin = arena.shape(name)
        t = arena.dtype[name]
        bb = 144 if t == Q4 else 210
        idx = np.sort(rng.choice(nrow, size=256, replace=False))
        wv = arena.tensor(name).view(nrow, -1)[torch.from_numpy(idx).cuda()].cpu().numpy().ravel()
        if t == Q4:
            y_ref, a = orc.gemv(wv, xin, idx.size, kin // 256)
        else:
            y_ref, a = orc.gemv_kquant(bb, wv, xin, idx.size, kin // 256)
        r = np.abs(yout.cpu().numpy()[idx].astype(np.float64) - y_ref) / a
        worst = max(worst, float(r.max()))
        if not np.all(r <= 1e-4):
            fail = f"FAIL {name}: max err/absdot {r.max():.3e}"
    parity = fail or f"ok (Q6_K down + Q6_K lm_head sampled rows, max err/absdot {worst:.2e} <= 1e-4)"
    qbytes = sum(arena.nbytes[nm] for nm, _, t in entries if t != GgmlType.F32)
    n6 = sum(1 for nm, _, t in entries if t == Q6)
    return {"workload": f"decode7b_q4km: Q4_K_M 7B-class decode step from one weight arena "
                        f"({n6} Q6_K tensors incl. lm_head, the rest Q4_K; fused RMSNorm/GeGLU; "
                        f"{launches[0]} launches), one mgq_chain_create_ops graph",
            "us_per_launch": round(ms * 1e3 / launches[0], 3), "gbs": qbytes / (ms * 1e-3) / 1e9,
            "bytes_per_launch": qbytes // launches[0], "parity": parity,
            "kernel": "mgq::gemv_wave_kernel / gemv_mfma_kernel + mgq::gemv_q6k_mfma_kernel / _long_kernel",
            "tokens_per_s": 1000.0 / ms, "ms_per_step": ms}


def run_kquant(torch, q4k, args):
    """Q5_K (176 B / 256 weights) on the gate and down shapes, or Q6_K
    (210 B / 256) on the lm_head and ffn_down shapes -- the K-quants real
    GGUFs mix in (Q4_K_M: Q6_K output and half the ffn_down layers). Each
    shape is also timed alone, in a graph of its own copies."""
    from oracle import oracle as orc
    fmt = 176 if args.workload == "q5k" else 210
    shapes = [("gate", INTER, HIDDEN), ("down", HIDDEN, INTER)] if fmt == 176 else \
        [("lm_head", VOCAB, HIDDEN), ("down", HIDDEN, INTER)]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x5150 + fmt)
    per = sum(n * (k // BLOCK_ELEMS) * fmt for _, n, k in shapes)
    copies = max(2, -(-int(1.2e9) // per))
    items = []
    for c in range(copies):
        for name, n, k in shapes:
            nblk = n * (k // BLOCK_ELEMS)
            w = torch.randint(0, 256, (nblk, fmt), dtype=torch.uint8, device="cuda", generator=gen)
            dd = (torch.rand((nblk, 2 if fmt == 176 else 1), device="cuda", generator=gen) * 2e-3
                  + 1e-4).to(torch.float16).view(torch.uint8)
            if fmt == 176:
                w[:, 0:4] = dd.view(nblk, 4)
            else:
                w[:, 208:210] = dd.view(nblk, 2)
            x = torch.randn(k, device="cuda", generator=gen)
            y = torch.empty(n, device="cuda")
            items.append((name, w.view(-1), x, y, n, k))
    fn = q4k.kern.matvec_q5k if fmt == 176 else q4k.kern.matvec_q6k

    def launch(st):
        for name, w, x, y, n, k in items:
            fn(w.data_ptr(), x.data_ptr(), y.data_ptr(), n, k // BLOCK_ELEMS, st)
    ms = time_captured(torch, launch, args.steps, args.warmup)
    nbytes = sum(n * (k // BLOCK_ELEMS) * fmt + 4 * (n + k) for _, _, _, _, n, k in items)
    per_shape = {}
    for sname, n, k in shapes:
        mine = [it for it in items if it[0] == sname]

        def launch_one(st, mine=mine):
            for _, w, x, y, n_, k_ in mine:
                fn(w.data_ptr(), x.data_ptr(), y.data_ptr(), n_, k_ // BLOCK_ELEMS, st)
        us = time_captured(torch, launch_one, args.steps, args.warmup) * 1e3 / len(mine)
        wb = n * (k // BLOCK_ELEMS) * fmt
        per_shape[f"{sname} {n}x{k}"] = {"us": round(us, 2), "gbs": round(wb / (us * 1e-6) / 1e9, 1)}
    worst, parity = 0.0, None
    for name, w, x, y, n, k in items[-len(shapes):]:
        bpr = k // BLOCK_ELEMS
        idx = np.sort(np.random.default_rng(n).choice(n, size=min(256, n), replace=False))
        wr = w.view(n, bpr * fmt)[torch.from_numpy(idx).cuda()].cpu().numpy().ravel()
        y_ref, a = orc.gemv_kquant(fmt, wr, x.cpu().numpy(), idx.size, bpr)
        r = np.abs(y.cpu().numpy()[idx].astype(np.float64) - y_ref) / np.maximum(a, 1e-300)
        worst = max(worst, float(r.max()))
        if not np.all(r <= 1e-4):
            parity = f"FAIL {name}: max err/absdot {r.max():.3e}"
    parity = parity or f"ok (max err/absdot {worst:.2e} <= 1e-4)"
    label = "q5k: Q5_K gate 18944x3584 + down 3584x18944" if fmt == 176 else \
        "q6k: Q6_K lm_head 152064x3584 + down 3584x18944"
    return {"workload": f"{label}, {copies} rotating copies, one graph",
            "us_per_launch": round(ms * 1e3 / len(items), 3), "gbs": nbytes / (ms * 1e-3) / 1e9,
            "bytes_per_launch": nbytes // len(items), "parity": parity, "per_shape": per_shape,
            "kernel": "mgq::gemv_mfma_kernel (Q5_K mode)" if fmt == 176 else
            "mgq::gemv_q6k_mfma_kernel + mgq::gemv_q6k_mfma_long_kernel"}


TRAFFIC_PROFILES = {"decode7b": "gemv_wave_decode7b_pmc.txt",
                    "prefill": "gemm_q4k_f16_prefill_pmc.txt"}


def profiled_traffic(workload: str, impl: str = "graph"):
    """HBM bytes per launch of the workload's dominant kernel from the
    committed FETCH_SIZE / WRITE_SIZE summary of this same workload and
    chain implementation (calibrated against a plain copy), or None."""
    name = TRAFFIC_PROFILES.get(workload if impl == "graph" else f"{workload}/{impl}")
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", name or "")
    if name is None or not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    return None


def other_configs(torch, q4k, steps: int) -> dict:
    """BASELINE configs 1, 2, 4 (B = 8) and 5 measured after the headline's
    timed region, each as its own --workload line measures it (graph
    replays over rotating weight copies, oracle parity on sampled rows) but
    with fewer replays and no CPU baseline, so that the default line records
    every config."""
    ns = argparse.Namespace(steps=steps, warmup=2, batch=8)
    out = {}
    r = run_config1(torch, q4k, ns)
    out["config1"] = {"workload": r["workload"], "kernel": r["kernel"],
                      "us_per_launch": r["us_per_launch"], "gbs": round(r["gbs"], 1),
                      "hbm_frac": round(r["gbs"] / HBM_PEAK_GBS, 4), "parity": r["parity"]}
    del r
    wl = Workload(torch, layer_shapes(), copies=10)
    out["config2"] = {"workload": "layer: q,k,v,o,gate,up,down of one 7B layer, unfused, "
                                  "10 rotating weight copies, one graph per shape",
                      "kernel": "mgq::gemv_wave_kernel (q, k, v, o: direct register loads)",
                      "per_shape": shape_times(torch, q4k, wl),
                      "parity": check_parity(torch, wl)}
    del wl
    r = run_batched(torch, q4k, ns)
    out["config4"] = {"workload": r["workload"], "kernel": r["kernel"],
                      "us_per_launch": r["us_per_launch"], "gbs": round(r["gbs"], 1),
                      "hbm_frac": round(r["gbs"] / HBM_PEAK_GBS, 4), "per_shape": r["per_shape"],
                      "parity": r["parity"]}
    del r
    r = run_prefill(torch, q4k, ns)
    out["config5"] = {"workload": r["workload"], "kernel": r["kernel"],
                      "us_per_launch": r["us_per_launch"], "tflops": round(r["tflops"], 1),
                      "mfma_frac": round(r["tflops"] / MFMA_F16_PEAK_TFLOPS, 4),
                      "parity": r["parity"]}
    del r
    torch.cuda.empty_cache()
    return out


def run_side_workload(torch, q4k, args) -> int:
    """BASELINE configs 1, 4 and 5: one JSON line each, same field layout."""
    fn = {"config1": run_config1, "batched": run_batched, "prefill": run_prefill,
          "decode7b_dp4a": run_decode_dp4a, "q5k": run_kquant, "q6k": run_kquant,
          "decode7b_glue": run_decode_glue, "decode7b_q4km": run_decode_q4km}[args.workload]
    r = fn(torch, q4k, args)
    out = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "warmup_min_ms": WARM_MS,
           # ms per graph replay of the headline measurement (dp4a and glue time
           # their two-launch / unfused baseline first)
           "pass_ms_spread": SPREADS[1 if args.workload in ("decode7b_dp4a", "decode7b_glue")
                                     else 0] if SPREADS else None,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "data": "synthetic",
           "config": {"workload": r["workload"]}, "parity": r["parity"]}
    if "tflops" in r:
        out.update({"value": round(r["tflops"], 2), "unit": "TFLOP/s", "dtype": "f16 x q4_k -> f32",
                    "us_per_launch": r["us_per_launch"],
                    "roofline": {"bound": "mfma", "achieved": round(r["tflops"], 2),
                                 "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                 "frac": round(r["tflops"] / MFMA_F16_PEAK_TFLOPS, 4),
                                 "traffic": profiled_traffic(args.workload),
                                 "kernel": r["kernel"]}})
    else:
        out.update({"value": round(r["gbs"], 2), "unit": "GB/s", "dtype": "f32",
                    "us_per_launch": r["us_per_launch"],
                    "roofline": {"bound": "hbm", "achieved": round(r["gbs"], 2), "peak": HBM_PEAK_GBS,
                                 "unit": "GB/s", "frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
                                 "traffic": None, "kernel": r["kernel"],
                                 "avg_launch_bytes": r["bytes_per_launch"]}})
    for key in ("tokens_per_s", "ms_per_step", "unfused_ms_per_step", "unfused_tokens_per_s"):
        if key in r:
            out[key] = round(r[key], 4)
    if "per_shape" in r:
        out["per_shape"] = r["per_shape"]
    if not args.no_cpu and "cpu" in r:
        jobs, units, unit, sample, digits = r["cpu"]
        threads = cpu_threads()
        secs = min(args.cpu_seconds, 5.0)
        log(f"cpu baseline ({threads} threads, ~{secs:.0f} s, then 1 thread ~3 s)")
        out["cpu_baseline"] = cpu_jobs_baseline(jobs, units, unit, sample, threads, secs, digits=digits)
    elif not args.no_cpu and "cpu_flat" in r:
        out["cpu_baseline"] = cpu_flat_baseline(*r["cpu_flat"])
    log(f"{r['workload']}: {r['us_per_launch']} us per launch; parity {r['parity']}")
    print(json.dumps(out), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="decode7b",
                    choices=["decode7b", "layer", "gateup", "config1", "batched", "prefill",
                             "decode7b_dp4a", "q5k", "q6k", "decode7b_glue", "decode7b_q4km",
                             "shard"])
    ap.add_argument("--shards", type=int, default=8,
                    help="--workload shard: one GPU's share of the decode step over this many GPUs")
    ap.add_argument("--batch", type=int, default=8, help="batch for --workload batched (1..16)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-parity", action="store_true")
    ap.add_argument("--no-shapes", action="store_true",
                    help="decode7b/layer/gateup: skip the per-shape times (and, for decode7b, "
                         "BASELINE configs 1, 2, 4, 5) measured after the timed region")
    ap.add_argument("--chain", default="auto", choices=sorted(CHAIN_MODES),
                    help="decode7b/layer/gateup: the chain's implementation")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the Q4_K GEMV path is built and measured on a "
              "single MI355X in this build (multi-GPU sharding is not implemented).",
              file=sys.stderr)
        return 2

    import torch
    from modgrad_amd import q4k, _lib
    _lib.load()
    log(f"device {torch.cuda.get_device_name(0)}; workload {args.workload}")

    if args.workload in ("config1", "batched", "prefill", "decode7b_dp4a", "q5k", "q6k",
                         "decode7b_glue", "decode7b_q4km"):
        return run_side_workload(torch, q4k, args)
    if args.workload == "decode7b":
        wl = Workload(torch, decode_step_shapes())
        desc = ("decode7b: 28 x (qkv 4608x3584, o 3584x3584, gate|up 37888x3584, down 3584x18944) "
                "+ lm_head 152064x3584, batch 1, one HIP graph per step")
    elif args.workload == "shard":
        g = max(1, args.shards)
        wl = Workload(torch, shard_step_shapes(g))
        qkv = NQ * HEAD + 2 * NKV * HEAD
        desc = (f"shard: one GPU's share of decode7b over {g} GPUs (rows: qkv {-(-qkv // g)}x3584, "
                f"gate|up {-(-2 * INTER // g)}x3584, lm_head {-(-VOCAB // g)}x3584; K: o 3584x"
                f"{-(-14 // g) * 256}, down 3584x{-(-74 // g) * 256}), 113 launches, one HIP graph "
                "per step; collectives not included")
        args.no_cpu = True
    elif args.workload == "layer":
        # 7 unfused launches x 10 rotating copies (1.3 GB) so the 256 MB MALL cannot hold them
        wl = Workload(torch, layer_shapes(), copies=10)
        desc = "layer: q,k,v,o,gate,up,down of one 7B layer, unfused, 10 rotating weight copies"
    else:
        wl = Workload(torch, [("gate_up", 2 * INTER, HIDDEN)], copies=16)
        desc = "gateup: 37888x3584 x 16 rotating copies (1.2 GB)"
    torch.cuda.synchronize()
    log(f"{len(wl.launches)} launches, {wl.weight_bytes / 1e9:.3f} GB weights resident")

    host_us = None
    if args.chain == "eager":
        ms, spread, host_us = time_eager(torch, q4k, wl, args.steps, args.warmup)
        impl = "eager"
        log(f"timed {args.steps} steps (eager, null stream, one device synchronize per step): "
            f"{ms:.4f} ms/step; host {host_us:.3f} us per launch call; per-step {spread}")
    else:
        ms, spread, impl = time_graph(torch, q4k, wl, args.steps, args.warmup, args.chain)
        log(f"timed {args.steps} steps ({impl} chain): {ms:.4f} ms/step; per-step events {spread}")
    shapes = None
    if impl == "graph" and not args.no_shapes:
        shapes = shape_times(torch, q4k, wl)
        log("per shape (graph of that shape's launches, after the timed region): " +
            ", ".join(f"{k} {v['us_per_launch']} us" for k, v in shapes.items()))
    parity = "skipped" if args.no_parity else check_parity(torch, wl)
    log(f"parity: {parity}")
    configs = None
    if args.workload == "decode7b" and not args.no_shapes:
        configs = other_configs(torch, q4k, steps=20)
        for key, c in configs.items():
            log(f"{key}: " + (", ".join(f"{k} {v['us_per_launch']} us" for k, v in
                                        c["per_shape"].items()) if key == "config2"
                              else f"{c['us_per_launch']} us per launch") + f"; parity {c['parity']}")
    nl = len(wl.launches)
    if impl == "persistent":
        # one cooperative launch per step runs all the matvecs: the kernel's
        # launch is the step, its bytes the step's
        kernel, avg_s, avg_b = "mgq::chain_kernel<2>", ms * 1e-3, wl.bytes_per_pass
    else:
        # back-to-back GEMV launches (one graph per step): the kernel's average
        # launch duration is the step time over its launches (every matvec on
        # the wave-private kernel: qkv and o with direct register loads)
        kernel, avg_s, avg_b = ("mgq::gemv_wave_kernel", ms * 1e-3 / nl, wl.bytes_per_pass / nl)
    achieved = avg_b / avg_s / 1e9
    log(f"kernel {kernel} avg {avg_s * 1e6:.3f} us per launch, {achieved:.1f} GB/s")

    value = wl.bytes_per_pass / (ms * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_min_ms": WARM_MS,
        "ms_per_step": round(ms, 5),
        "step_ms_spread": spread,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": desc, "matvecs_per_step": nl, "chain": impl,
                   "launches_per_step": 1 if impl == "persistent" else nl,
                   "stream": "null stream, one hipDeviceSynchronize per step" if impl == "eager"
                   else "one graph launch per step",
                   "bytes_per_step": wl.bytes_per_pass, "weights": "q4_k (144 B / 256 weights)",
                   "batch": 1},
        "tokens_per_s": round(1000.0 / ms, 2) if args.workload == "decode7b" else None,
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "parity": parity,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(args.workload, impl), "kernel": kernel,
                     "avg_launch_us": round(avg_s * 1e6, 3), "avg_launch_bytes": int(avg_b)},
    }
    if host_us is not None:
        out["host_us_per_launch_call"] = round(host_us, 3)
    if shapes is not None:
        out["per_shape"] = shapes
    if configs is not None:
        out["other_configs"] = configs
    if not args.no_cpu:
        threads = cpu_threads()
        log(f"cpu baseline ({threads} threads, ~{args.cpu_seconds:.0f} s, then 1 thread ~5 s)")
        out["cpu_baseline"] = cpu_baseline(torch, wl, args.cpu_seconds, threads)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
