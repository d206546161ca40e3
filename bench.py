#!/usr/bin/env python3
"""Benchmark of the Q4_1 dequant-matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--extras 0,2,3,4|none] [--no-cpu]

Headline: the Llama-3-8B decode weight sweep at
M=1 -- 32 layers of q/k/v/o/gate/up/down plus lm_head, 4.69 GB of Q4_1
weights, synthetic seeded data -- issued as one grouped GEMV launch per step.
`value` = algorithmic bytes (packed weights + bf16 x + f32 y per matrix) /
measured time, inputs resident in HBM. The same JSON line carries:

* roofline     -- that kernel's algorithmic bytes per launch / its mean launch
                  duration from HIP events on its stream, against 8 TB/s;
* cpu_baseline -- the oracle's numpy restatement of the reference CPU path
                  (pool-chunk dequant as q4nx.py:105-126, then an f32 matvec)
                  timed on this host over one Llama layer, 15 passes;
* extras       -- the same sweep issued stage by stage as a decode step would
                  (fused qkv, o, fused gate/up, down per layer, lm_head: 129
                  GEMV calls), config 0 (single GEMV), config 2 (M = 4/8/16),
                  config 3 (prefill GEMM TFLOP/s) and config 4 (routed MoE).
                  Multi-launch extras are captured in a HIP graph and timed
                  over replays (after checking a replay against the eager run),
                  so host launch overhead is not what they measure.

Runs on one GPU only: --gpus above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 / fp16 MFMA, TFLOP/s

LLAMA_LAYER = [  # (name, N, K) per layer of Llama-3-8B
    ("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
    ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336),
]
LM_HEAD = ("lm_head", 128256, 4096)
SEED = 1234


TRAFFIC_SUMMARY = ROOT / "profiles" / "gemv_grouped_llama3_8b_m1.md"


def measured_traffic():
    """HBM bytes per launch of the headline kernel, from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE summary (counter runs cannot happen inside this process)."""
    try:
        for line in TRAFFIC_SUMMARY.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def measured_traffic_ratios():
    """HBM traffic over algorithmic bytes for the decode-step, skinny and MoE workloads,
    from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summaries under profiles/ (lines
    'traffic_over_algorithmic <key>: <ratio>'), with the file each came from."""
    out = {}
    for p in sorted((ROOT / "profiles").glob("*.md")):
        try:
            lines = p.read_text().splitlines()
        except OSError:
            continue
        for line in lines:
            if line.startswith("traffic_over_algorithmic "):
                key, val = line[len("traffic_over_algorithmic "):].split(":", 1)
                out[key.strip()] = {"ratio": float(val), "source": f"profiles/{p.name}"}
    return out


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# --------------------------------------------------------------------------
# synthetic weights, generated on the GPU and packed by the product's packer
# --------------------------------------------------------------------------

def gen_blocks(torch, n: int, k: int, gen, dev):
    """GGUF Q4_1 blocks with the benchmark distribution: q ~ U{0..15},
    d = fp16(|N(0,1)|*0.002 + 1e-4), m = fp16(-8 d U(0.9, 1.1))."""
    nb = k // 32
    d = (torch.randn(n, nb, generator=gen, device=dev).abs() * 0.002 + 1e-4).half()
    u = torch.rand(n, nb, generator=gen, device=dev) * 0.2 + 0.9
    m = (-8.0 * d.float() * u).half()
    blocks = torch.empty(n, nb, 20, dtype=torch.uint8, device=dev)
    blocks[..., 0:2] = d.view(torch.uint8).view(n, nb, 2)
    blocks[..., 2:4] = m.view(torch.uint8).view(n, nb, 2)
    blocks[..., 4:20] = torch.randint(0, 256, (n, nb, 16), generator=gen, device=dev, dtype=torch.uint8)
    return blocks


class Llama:
    """Packed Llama-3-8B weights. q/k/v live in one [6144, 4096] buffer and
    gate/up in one [28672, 4096] buffer: mx row groups are contiguous, so the
    fused matrix and its row slices are the same bytes."""

    def __init__(self, torch, q4, dev, layers: int = 32, scales: str = "bf16"):
        gen = torch.Generator(device=dev)
        gen.manual_seed(SEED)
        self.layers = []
        for _ in range(layers):
            qkv = torch.empty(q4.packed_bytes(6144, 4096), dtype=torch.uint8, device=dev)
            gu = torch.empty(q4.packed_bytes(28672, 4096), dtype=torch.uint8, device=dev)
            parts = {}
            off = {"qkv": 0, "gu": 0}
            for name, n, k in LLAMA_LAYER:
                nb = q4.packed_bytes(n, k)
                if name in ("q", "k", "v", "gate", "up"):
                    buf = qkv if name in ("q", "k", "v") else gu
                    key = "qkv" if name in ("q", "k", "v") else "gu"
                    dst = buf[off[key]:off[key] + nb]
                    off[key] += nb
                else:
                    dst = torch.empty(nb, dtype=torch.uint8, device=dev)
                parts[name] = q4.pack_q4_1(gen_blocks(torch, n, k, gen, dev), dev, out=dst, scales=scales)
            parts["qkv"] = q4.PackedQ4(qkv, 6144, 4096, scales=scales)
            parts["gate_up"] = q4.PackedQ4(gu, 28672, 4096, scales=scales)
            self.layers.append(parts)
        self.head = q4.pack_q4_1(gen_blocks(torch, LM_HEAD[1], LM_HEAD[2], gen, dev), dev, scales=scales)
        torch.cuda.synchronize()
        self.weight_bytes = sum(p[n].nbytes for p in self.layers for n, _, _ in LLAMA_LAYER) + self.head.nbytes
        self.matrices = len(self.layers) * len(LLAMA_LAYER) + 1


def sweep_inputs(torch, model, dev, M: int):
    """Activations of one decode step (q/k/v share x, gate/up share x) and outputs."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED + M)

    def act(k):
        return torch.randn(M, k, generator=gen, device=dev).to(torch.bfloat16)
    per_layer = []
    for _ in model.layers:
        per_layer.append({"in": act(4096), "o": act(4096), "mlp": act(4096), "dn": act(14336)})
    return per_layer, act(4096)


def grouped_sweep(torch, q4, model, acts, xhead, M: int):
    """One GemvGroup over all 225 matrices; returns (group, algorithmic bytes)."""
    dev = model.head.device
    items, nbytes = [], 0
    which = {"q": "in", "k": "in", "v": "in", "o": "o", "gate": "mlp", "up": "mlp", "down": "dn"}
    for parts, xs in zip(model.layers, acts):
        for name, n, k in LLAMA_LAYER:
            y = torch.empty(M, n, dtype=torch.float32, device=dev)
            items.append((parts[name], xs[which[name]], y))
            nbytes += parts[name].nbytes + M * k * 2 + M * n * 4
    y = torch.empty(M, LM_HEAD[1], dtype=torch.float32, device=dev)
    items.append((model.head, xhead, y))
    nbytes += model.head.nbytes + M * 4096 * 2 + M * LM_HEAD[1] * 4
    return q4.GemvGroup(items), nbytes


def time_launches(torch, fn, steps: int, warmup: int):
    """warmup calls, then `steps` calls each bracketed by HIP events on the
    current stream. Returns (total ms between the outer events, mean ms per call)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(st)
    for a, b in ev:
        a.record(st)
        fn()
        b.record(st)
    t1.record(st)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1), sum(a.elapsed_time(b) for a, b in ev) / steps


def graph_time(torch, fn, outputs, replays: int = 20, reset=None) -> float:
    """Capture fn() in a HIP graph, check one replay against the eager run
    (bit for bit: every kernel here is deterministic), replay it untimed for
    about 25 ms (clocks settle under load), then time `replays` replays with
    events (at least ~1 ms of them). Returns mean ms per replay. `reset` restores the state
    of an fn that updates its inputs in place (a residual stream) before the
    eager run and before the checked replay."""
    if reset:
        reset()
    fn()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outputs]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        fn()
    torch.cuda.synchronize()
    if reset:
        reset()
    else:
        for o in outputs:
            o.fill_(float("nan") if o.is_floating_point() else -12345)
    g.replay()
    torch.cuda.synchronize()
    for o, e in zip(outputs, eager):
        if not torch.equal(o, e):
            raise RuntimeError("graph replay differs from the eager run")
    # untimed replays until ~25 ms of load (at least 2): the clocks settle before the timing
    st = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    g.replay()
    b.record(st)
    torch.cuda.synchronize()
    one = max(a.elapsed_time(b), 1e-3)
    for _ in range(max(2, min(2000, int(25.0 / one)))):
        g.replay()
    torch.cuda.synchronize()
    # at least ~1 ms of timed replays: a short graph's mean then does not hang on one late
    # submission (a 5-replay timing of the 8 us activation pre-pass once read 0.24 ms)
    replays = max(replays, min(2000, int(1.0 / one) + 1))
    a.record(st)
    for _ in range(replays):
        g.replay()
    b.record(st)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / replays


# --------------------------------------------------------------------------
# CPU baseline (oracle restatement of the reference CPU path), in a child
# process so the BLAS thread count can be set before numpy loads
# --------------------------------------------------------------------------

def cpu_baseline_child(threads: int, passes: int, runs: int = 5) -> dict:
    """One CPU worker: the oracle's restatement of the reference CPU path over one Llama-3-8B
    layer in pool-chunk form, `runs` timed runs of `passes` passes each (after building the
    layer, untimed). Returns the seconds of each run and the Q4_1 bytes one run streams."""
    import numpy as np
    from oracle import q4_oracle as O
    rng = np.random.default_rng(SEED)
    layer = []
    for name, n, k in LLAMA_LAYER:                       # one layer in pool-chunk form (rs = 1 band order)
        nch = n * k // 8192
        chunks = rng.integers(0, 256, (nch, 5120), dtype=np.uint8)
        d = (np.abs(rng.standard_normal((nch, 256))) * 0.002 + 1e-4).astype(np.float16).astype(np.float32)
        m = (-8 * d * rng.uniform(0.9, 1.1, (nch, 256))).astype(np.float16).astype(np.float32)
        chunks[:, 0:512] = O.f32_to_bf16(d).view(np.uint8).reshape(nch, 512)
        chunks[:, 512:1024] = O.f32_to_bf16(m).view(np.uint8).reshape(nch, 512)
        layer.append((n, k, chunks, rng.standard_normal(k).astype(np.float32)))
    chunk_slice = 2048                                   # 10 MB of chunks -> 64 MB of f32 at a time
    run_bytes = passes * sum(c.nbytes for _, _, c, _ in layer)
    secs = []
    for _ in range(runs):
        t = time.perf_counter()
        for _ in range(passes):
            for n, k, chunks, x in layer:
                per_row = k // 256                       # chunk c: rows 32 (c // per_row), k-tile c % per_row
                xs = x.reshape(per_row, 256)
                y = np.zeros((n // 32, 32), np.float32)
                for c0 in range(0, chunks.shape[0], chunk_slice):
                    c1 = min(chunks.shape[0], c0 + chunk_slice)
                    w = O.dq_chunks_q4_1(chunks[c0:c1]).reshape(c1 - c0, 32, 256)
                    cc = np.arange(c0, c1)
                    part = np.matmul(w, xs[cc % per_row][:, :, None])[..., 0]
                    np.add.at(y, cc // per_row, part)
        secs.append(time.perf_counter() - t)
    return {"run_seconds": secs, "run_bytes": run_bytes, "threads": threads, "passes": passes, "runs": runs}


def cpu_model_name() -> str:
    """The host CPU's model name (lscpu, else /proc/cpuinfo)."""
    try:
        r = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20)
        for line in r.stdout.splitlines():
            if line.strip().lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(workers: int, passes: int, runs: int = 5) -> dict | None:
    """`workers` concurrent single-thread CPU workers (OPENBLAS_NUM_THREADS=1 each, the
    reference harness's setting), each timing `runs` runs of `passes` passes over one layer.
    A worker's rate is its median run; the leg's rate is the sum over workers (they run the
    same work side by side), with the wall time of the whole parallel phase beside it."""
    env = dict(os.environ)
    for v in ("OPENBLAS_NUM_THREADS", "OMP_NUM_THREADS", "MKL_NUM_THREADS"):
        env[v] = "1"
    env["HIP_VISIBLE_DEVICES"] = ""      # the CPU leg never touches the GPU
    cmd = [sys.executable, str(Path(__file__).resolve()), "--cpu-baseline-child", "1", "--cpu-passes", str(passes),
           "--cpu-runs", str(runs)]
    t0 = time.perf_counter()
    try:
        procs = [subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, env=env)
                 for _ in range(workers)]
        outs = []
        for p in procs:
            so, se = p.communicate(timeout=900)
            if p.returncode != 0:
                log(f"cpu baseline worker failed: {se[-500:]}")
                return None
            outs.append(json.loads(so.strip().splitlines()[-1]))
    except Exception as e:  # the baseline is reported, never required
        log(f"cpu baseline skipped: {e}")
        return None
    import statistics
    med = [statistics.median(o["run_seconds"]) for o in outs]
    rates = [o["run_bytes"] / m / 1e9 for o, m in zip(outs, med)]
    return {"gbs": sum(rates), "workers": workers, "median_run_seconds": statistics.median(med),
            "run_bytes": outs[0]["run_bytes"], "passes": passes, "runs": runs,
            "wall_seconds": time.perf_counter() - t0, "worker_gbs_min": min(rates), "worker_gbs_max": max(rates)}


# --------------------------------------------------------------------------
# extras
# --------------------------------------------------------------------------

def extra_staged(torch, q4, model, acts, xhead):
    """The sweep as a decode step issues it: per layer fused qkv, o, fused
    gate/up, down (each its own q4_gemv call, split along K where short), then
    lm_head -- 129 calls, one HIP graph."""
    dev = model.head.device
    calls, outs, nbytes = [], [], 0
    for parts, xs in zip(model.layers, acts):
        for wname, xname in (("qkv", "in"), ("o", "o"), ("gate_up", "mlp"), ("down", "dn")):
            w = parts[wname]
            y = torch.empty(1, w.n, dtype=torch.float32, device=dev)
            calls.append((w, xs[xname], y))
            outs.append(y)
            nbytes += w.nbytes + w.k * 2 + w.n * 4
    y = torch.empty(1, model.head.n, dtype=torch.float32, device=dev)
    calls.append((model.head, xhead, y))
    outs.append(y)
    nbytes += model.head.nbytes + 4096 * 2 + model.head.n * 4
    wsz = max(q4.gemv_workspace_bytes(1, w.n, w.k) for w, _, _ in calls)
    ws = torch.empty(max(wsz, 256), dtype=torch.uint8, device=dev)

    def run():
        for w, x, y in calls:
            q4.gemm_q4(w, x, y, workspace=ws)
    ms = graph_time(torch, run, outs, replays=10)
    return {"ms": ms, "gbs": nbytes / ms / 1e6, "calls": len(calls), "bytes": nbytes}


def extra_decode_step(torch, q4, model, acts, xhead, only=None):
    """A decode step's weight traffic in order with its own epilogues (attention itself
    left out: its output is a fixed bf16 vector): per layer RMSNorm -> fused qkv -> o with
    the residual -> RMSNorm -> SwiGLU gate/up (bf16 h) -> down with the residual; then the
    final RMSNorm and lm_head, one HIP graph. Bytes: the weights streamed (qkv, o, gate, up,
    down per layer, lm_head)."""
    dev = model.head.device
    H, F = 4096, 14336
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED + 29)
    xres0 = torch.randn(1, H, generator=gen, device=dev)
    xres = xres0.clone()
    nw = (1 + 0.1 * torch.randn(H, generator=gen, device=dev)).to(torch.bfloat16)
    xn = torch.empty(1, H, dtype=torch.bfloat16, device=dev)
    qkv = torch.empty(1, 6144, device=dev)
    h = torch.empty(1, F, dtype=torch.bfloat16, device=dev)
    logits = torch.empty(1, model.head.n, device=dev)
    ws = torch.empty(1 << 24, dtype=torch.uint8, device=dev)
    attn = [xs["o"] for xs in acts]
    nbytes = sum(p[n].nbytes for p in model.layers for n in ("qkv", "o", "gate", "up", "down")) + model.head.nbytes

    def step():
        for i, p in enumerate(model.layers):
            q4.rmsnorm_add(xres, nw, xn=xn)
            q4.gemm_q4(p["qkv"], xn, y=qkv, workspace=ws)
            q4.gemm_q4(p["o"], attn[i], y=xres, residual=xres, workspace=ws)
            q4.rmsnorm_add(xres, nw, xn=xn)
            q4.swiglu_q4(p["gate"], p["up"], xn, out_dtype=torch.bfloat16, h=h, workspace=ws)
            q4.gemm_q4(p["down"], h, y=xres, residual=xres, workspace=ws)
        q4.rmsnorm_add(xres, nw, xn=xn)
        q4.gemm_q4(model.head, xn, y=logits, workspace=ws)

    def step_fused():           # the two norms inside the GEMVs that consume them
        for i, p in enumerate(model.layers):
            q4.gemm_q4_rmsnorm(p["qkv"], xres, nw, y=qkv, workspace=ws)
            q4.gemm_q4(p["o"], attn[i], y=xres, residual=xres, workspace=ws)
            q4.swiglu_q4(p["gate"], p["up"], xres, out_dtype=torch.bfloat16, h=h, workspace=ws, norm_w=nw)
            q4.gemm_q4(p["down"], h, y=xres, residual=xres, workspace=ws)
        q4.gemm_q4_rmsnorm(model.head, xres, nw, y=logits, workspace=ws)

    xalt = torch.empty(1, H, device=dev)

    def deferred(so, sd):
        """The norms inside the GEMVs and the o / down K-split sums deferred into them: o and
        down leave partial planes, the next norm GEMV adds them to the residual stream (written
        to the other of two buffers) in its prelude; no reduce launches."""
        po = torch.empty(so, 1, H, device=dev)
        pd = torch.empty(sd, 1, H, device=dev)

        def fn():
            cur, nxt = xres, xalt
            for i, p in enumerate(model.layers):
                if i == 0:
                    q4.gemm_q4_rmsnorm(p["qkv"], cur, nw, y=qkv, workspace=ws)
                else:
                    q4.gemm_q4_rmsnorm_acc(p["qkv"], cur, pd, nw, x_out=nxt, y=qkv, workspace=ws)
                    cur, nxt = nxt, cur
                q4.gemm_q4_partials(p["o"], attn[i], splits=so, part=po)
                q4.swiglu_q4_acc(p["gate"], p["up"], cur, po, nw, out_dtype=torch.bfloat16, x_out=nxt, h=h,
                                 workspace=ws)
                cur, nxt = nxt, cur
                q4.gemm_q4_partials(p["down"], h, splits=sd, part=pd)
            q4.gemm_q4_rmsnorm_acc(model.head, cur, pd, nw, x_out=nxt, y=logits, workspace=ws)
        return fn

    NQ = model.layers[0]["qkv"].n
    sg_o, sg_d, sg_q = q4.decode_segment_splits(H, F, NQ)
    xmid = torch.empty(1, H, device=dev)
    pdg = torch.empty(sg_d, 1, H, device=dev)
    pqg = torch.empty(sg_q, 1, NQ, device=dev)
    wseg = q4.decode_segment_workspace(H, F, NQ, dev)

    def segments():
        """Between two attentions, one launch (decode_segment): o -> norm -> SwiGLU -> down ->
        norm -> the next layer's qkv (its K-split planes, what attention would take). Layer 0's
        norm + qkv and the final norm + lm_head (over the last segment's down planes) are the
        norm GEMVs of the other forms. The residual stream advances in place."""
        q4.gemm_q4_rmsnorm(model.layers[0]["qkv"], xres, nw, y=qkv, workspace=ws)
        last = len(model.layers) - 1
        for i, p in enumerate(model.layers):
            nxt = model.layers[i + 1]["qkv"] if i < last else None
            q4.decode_segment(p["o"], p["gate"], p["up"], p["down"], nxt, attn[i], xres, nw,
                              nw if nxt is not None else None, x_mid=xmid, x_next=xres if nxt is not None else None,
                              down_planes=pdg, qkv_planes=pqg if nxt is not None else None, workspace=wseg)
        q4.gemm_q4_rmsnorm_acc(model.head, xmid, pdg, nw, x_out=xalt, y=logits, workspace=ws)

    l0 = model.layers[0]
    so, sd = q4.gemv_split_count(l0["o"]), q4.gemv_split_count(l0["down"])

    def reset():
        xres.copy_(xres0)
    out = {"bytes": nbytes}
    variants = (("separate_norms", step), ("norms_in_gemv", step_fused),
                (f"deferred_sums_o{so}_d{sd}", deferred(so, sd)), ("deferred_sums_o4_d4", deferred(4, 4)),
                ("segments", segments))
    for name, fn in variants:
        if only and name not in only:
            continue
        ms = graph_time(torch, fn, [logits, xres, xalt], replays=10, reset=reset)
        out[name] = {"ms": ms, "gbs": nbytes / ms / 1e6}
    if only:            # a profiling run of some variants: no cross-variant checks
        return out
    reset()
    step()
    a = logits.clone()
    reset()
    step_fused()
    out["same_logits"] = bool(torch.equal(a, logits))
    reset()
    variants[2][1]()
    out["deferred_same_logits"] = bool(torch.equal(a, logits))
    reset()
    variants[3][1]()
    out["deferred_o4_d4_maxrel"] = float(((logits - a).abs().max() / a.abs().max()).item())
    b = logits.clone()
    reset()
    segments()
    # the segments' residual stream is the o4 / d4 chain's: same splits, tiles, sums and order
    out["segments_same_logits_as_o4_d4"] = bool(torch.equal(b, logits))
    out["segments_timed_out"] = bool(wseg[12544:12548].view(torch.int32).item() != 0)
    out["segment_splits"] = {"o": sg_o, "down": sg_d, "qkv": sg_q}
    return out


def extra_lm_head(torch, q4, dev, head=None, xhead=None):
    """lm_head at vocabulary scale (128256 x 4096, M=1) with its sampling epilogue:
    the GEMV alone, then GEMV + greedy argmax and GEMV + top-40 (the sampler's
    bf16 view), each graph-timed, and the epilogue's own cost beside it (ten epilogues
    per graph replay, so the replay's own submission cost does not count ten times)."""
    if head is None:
        gen = torch.Generator(device=dev)
        gen.manual_seed(SEED + 7)
        head = q4.pack_q4_1(gen_blocks(torch, LM_HEAD[1], LM_HEAD[2], gen, dev), dev)
        xhead = torch.randn(1, LM_HEAD[2], generator=gen, device=dev).to(torch.bfloat16)
    logits = torch.empty(1, head.n, dtype=torch.float32, device=dev)
    ws = torch.empty(max(q4.gemv_workspace_bytes(1, head.n, head.k), 1 << 20), dtype=torch.uint8, device=dev)
    out = {"N": head.n, "K": head.k, "weight_bytes": head.nbytes}
    ms = graph_time(torch, lambda: q4.gemm_q4(head, xhead, logits, workspace=ws), [logits], replays=20)
    out["gemv_us"] = round(ms * 1e3, 2)
    out["gemv_gbs"] = round((head.nbytes + head.k * 2 + head.n * 4) / ms / 1e6, 1)
    for k in (1, 40):
        ids = torch.empty(1, k, dtype=torch.int32, device=dev)
        vals = torch.empty(1, k, dtype=torch.float32, device=dev)

        def full():
            q4.lm_head_topk(head, xhead, k=k, mode="sampler", logits=logits, workspace=ws, ids=ids, vals=vals)
        ms_full = graph_time(torch, full, [logits, ids, vals], replays=20)

        def epi():
            for _ in range(10):
                q4.logits_topk(logits, k, "sampler", workspace=ws, ids=ids, vals=vals)
        ms_epi = graph_time(torch, epi, [ids, vals], replays=20) / 10
        out[f"top{k}_us"] = round(ms_full * 1e3, 2)
        out[f"top{k}_epilogue_us"] = round(ms_epi * 1e3, 2)
    return out


def extra_ffn(torch, q4, model, acts):
    """The decode FFN of all 32 layers at M=1, graph-timed two ways over the same
    weights: fused (q4_rmsnorm_add -> q4_gemv_swiglu with bf16 h -> q4_gemv_residual in
    place) and unfused (torch RMSNorm, the gate/up GEMV, torch silu * up, the down GEMV,
    torch residual add). Bytes: gate/up + down weights + activations per layer."""
    dev = model.head.device
    F, H = 14336, 4096
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED + 11)
    xres = torch.randn(1, H, generator=gen, device=dev)
    nw = (1 + 0.1 * torch.randn(H, generator=gen, device=dev)).to(torch.bfloat16)
    xn = torch.empty(1, H, dtype=torch.bfloat16, device=dev)
    h = torch.empty(1, F, dtype=torch.bfloat16, device=dev)
    gu = torch.empty(1, 2 * F, dtype=torch.float32, device=dev)
    yd = torch.empty(1, H, dtype=torch.float32, device=dev)
    ws = torch.empty(1 << 24, dtype=torch.uint8, device=dev)
    nbytes = sum(p["gate_up"].nbytes + p["down"].nbytes for p in model.layers)

    def fused():
        for p in model.layers:
            q4.rmsnorm_add(xres, nw, xn=xn)
            q4.swiglu_q4(p["gate"], p["up"], xn, out_dtype=torch.bfloat16, h=h, workspace=ws)
            q4.gemm_q4(p["down"], h, y=xres, residual=xres, workspace=ws)

    def unfused():
        for p in model.layers:
            xf = xres * torch.rsqrt(xres.pow(2).mean(-1, keepdim=True) + 1e-6) * nw.to(torch.float32)
            xn.copy_(xf.to(torch.bfloat16))
            q4.gemm_q4(p["gate_up"], xn, y=gu, workspace=ws)
            h.copy_((torch.nn.functional.silu(gu[:, :F]) * gu[:, F:]).to(torch.bfloat16))
            q4.gemm_q4(p["down"], h, y=yd, workspace=ws)
            xres.add_(yd)

    x0 = xres.clone()
    out = {"layers": len(model.layers), "weight_bytes": nbytes}
    results = {}
    for name, fn in (("fused", fused), ("unfused", unfused)):
        ms = graph_time(torch, fn, [xres], replays=5, reset=lambda: xres.copy_(x0))
        results[name] = xres.clone()
        out[f"{name}_ms"] = round(ms, 4)
        out[f"{name}_gbs"] = round(nbytes / ms / 1e6, 1)
    xres.copy_(x0)
    fused()
    a = xres.clone()
    xres.copy_(x0)
    unfused()
    out["fused_vs_unfused_maxrel"] = float(((a - xres).abs().max() / xres.abs().max()).item())
    xres.copy_(x0)
    return out


def extra_q8(torch, q4, dev):
    """The q8 GEMV at M=1 on the Llama-3-8B gate_up and lm_head shapes, graph-timed over
    rotating copies (the set exceeds the caches): the exact hi/lo planes in one launch
    (bytes = both planes + bf16 x + f32 y) and the native mx8 layout (its own bytes), the
    same values s * q either way."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED + 13)
    out = {}
    for name, n, k in (("gate_up", 28672, 4096), ("lm_head", 128256, 4096)):
        nb = n * (k // 32)
        blocks = torch.empty((n, k // 32, 34), dtype=torch.uint8, device=dev)
        d = (torch.randn(n, k // 32, generator=gen, device=dev).abs() * 0.002 + 1e-4).to(torch.float16)
        blocks[..., 0:2] = d.view(torch.uint8).view(n, k // 32, 2)
        blocks[..., 2:] = torch.randint(0, 256, (n, k // 32, 32), generator=gen, device=dev, dtype=torch.uint8)
        copies = 2 if n > 100000 else 8
        ws = [q4.pack_q8(blocks, n, k, "q8_0", device=dev) for _ in range(copies)]
        wn = [q4.pack_q8_native(blocks, n, k, "q8_0", device=dev) for _ in range(copies)]
        del blocks
        x = torch.randn(1, k, generator=gen, device=dev).to(torch.bfloat16)
        y = torch.empty(1, n, dtype=torch.float32, device=dev)
        wsp = torch.empty(max(q4.gemv_workspace_bytes(1, n, k), 256), dtype=torch.uint8, device=dev)

        def run():
            for w in ws:
                q4.gemm_q8(w, x, y, workspace=wsp)

        def run_native():
            for w in wn:
                q4.gemm_q8_native(w, x, y, workspace=wsp)
        ms = graph_time(torch, run, [y], replays=10) / copies
        ms_n = graph_time(torch, run_native, [y], replays=10) / copies
        io = k * 2 + n * 4
        out[name] = {"N": n, "K": k, "us": round(ms * 1e3, 2), "gbs": round((ws[0].nbytes + io) / ms / 1e6, 1),
                     "q8_equivalent_gbs": round((nb * 34 + io) / ms / 1e6, 1),
                     "native_us": round(ms_n * 1e3, 2), "native_gbs": round((wn[0].nbytes + io) / ms_n / 1e6, 1)}
        del ws, wn
        torch.cuda.empty_cache()
    return out


def extra_q40(torch, q4, dev):
    """The Q4_0-native GEMV (mx0, 0.5625 B per weight) against the widened Q4_1 layout of
    the same GGUF Q4_0 blocks (mx, 0.625 B per weight) at M=1 on Llama-3-8B shapes,
    graph-timed over rotating copies; outputs bit-identical."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED + 17)
    out = {}
    for name, n, k in (("o", 4096, 4096), ("down", 4096, 14336), ("gate_up", 28672, 4096),
                       ("lm_head", 128256, 4096)):
        blocks = torch.empty((n, k // 32, 18), dtype=torch.uint8, device=dev)
        d = (torch.randn(n, k // 32, generator=gen, device=dev).abs() * 0.002 + 1e-4).to(torch.float16)
        blocks[..., 0:2] = d.view(torch.uint8).view(n, k // 32, 2)
        blocks[..., 2:] = torch.randint(0, 256, (n, k // 32, 16), generator=gen, device=dev, dtype=torch.uint8)
        copies = max(2, min(32, int(1.2e9 // (n * k))))
        w0 = [q4.pack_q4_0_native(blocks, n, k, "q4_0", device=dev) for _ in range(copies)]
        w1 = [q4.pack_q4_1(blocks, dev) for _ in range(copies)]
        del blocks
        x = torch.randn(1, k, generator=gen, device=dev).to(torch.bfloat16)
        y0 = torch.empty(1, n, dtype=torch.float32, device=dev)
        y1 = torch.empty(1, n, dtype=torch.float32, device=dev)
        wsp = torch.empty(max(q4.gemv_workspace_bytes(1, n, k), 256), dtype=torch.uint8, device=dev)

        def run0():
            for w in w0:
                q4.gemm_q4_0_native(w, x, y0, workspace=wsp)

        def run1():
            for w in w1:
                q4.gemm_q4(w, x, y1, workspace=wsp)
        ms0 = graph_time(torch, run0, [y0], replays=10) / copies
        ms1 = graph_time(torch, run1, [y1], replays=10) / copies
        if not torch.equal(y0, y1):
            raise RuntimeError(f"{name}: the Q4_0-native GEMV differs from the widened layout's")
        io = k * 2 + n * 4
        out[name] = {"N": n, "K": k, "native_us": round(ms0 * 1e3, 2),
                     "native_gbs": round((w0[0].nbytes + io) / ms0 / 1e6, 1),
                     "widened_us": round(ms1 * 1e3, 2), "widened_gbs": round((w1[0].nbytes + io) / ms1 / 1e6, 1)}
        del w0, w1
        torch.cuda.empty_cache()
    return out


def extra_q4k(torch, q4, dev):
    """GGUF Q4_K weights at M=1 on the Llama-3-8B gate_up, down and lm_head shapes: the
    native Q4_K kernel (the super-block's integers, 0.594 B/weight, exact) against the
    same blocks collapsed to the mx q4_1 layout (0.625 B/weight, d sc and m mn rounded
    to bf16), each graph-timed over rotating copies that exceed the caches. GB/s counts
    each layout's own bytes + bf16 x + f32 y; us is the number to compare."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED + 17)
    out = {}
    for name, n, k in (("gate_up", 28672, 4096), ("down", 4096, 14336), ("lm_head", 128256, 4096)):
        ns = k // 256
        blocks = torch.randint(0, 256, (n, ns, 144), generator=gen, device=dev, dtype=torch.uint8)
        d = (torch.rand(n, ns, generator=gen, device=dev) + 0.5) * (0.02 / 600)
        dmin = (torch.rand(n, ns, generator=gen, device=dev) + 0.5) * (0.02 / 40)
        blocks[..., 0:2] = d.to(torch.float16).view(torch.uint8).view(n, ns, 2)
        blocks[..., 2:4] = dmin.to(torch.float16).view(torch.uint8).view(n, ns, 2)
        copies = 1 if n > 100000 else 8
        native = [q4.pack_q4_k_native(blocks, dev) for _ in range(copies)]
        collapsed = [q4.pack_q4_k(blocks, dev) for _ in range(copies)]
        del blocks
        x = torch.randn(1, k, generator=gen, device=dev).to(torch.bfloat16)
        y = torch.empty(1, n, dtype=torch.float32, device=dev)
        wsp = torch.empty(max(q4.gemv_workspace_bytes(1, n, k), 256), dtype=torch.uint8, device=dev)
        wsk = torch.empty(max(q4.load_library().q4_gemv_q4k_workspace_bytes(1, n, k), 256), dtype=torch.uint8,
                          device=dev)

        def run_native():
            for w in native:
                q4.gemm_q4k(w, x, y, workspace=wsk)

        def run_collapsed():
            for w in collapsed:
                q4.gemm_q4(w, x, y, workspace=wsp)
        ms_n = graph_time(torch, run_native, [y], replays=10) / copies
        ms_c = graph_time(torch, run_collapsed, [y], replays=10) / copies
        io = k * 2 + n * 4
        out[name] = {"N": n, "K": k,
                     "native_us": round(ms_n * 1e3, 2), "native_gbs": round((native[0].nbytes + io) / ms_n / 1e6, 1),
                     "collapsed_us": round(ms_c * 1e3, 2),
                     "collapsed_gbs": round((collapsed[0].nbytes + io) / ms_c / 1e6, 1)}
        del native, collapsed
        torch.cuda.empty_cache()
    return out


def extra_peaks(torch, q4, dev):
    """On-box reference points beside the vendor peaks, from the library's own probes
    (q4_probe_stream_read, q4_probe_mfma): the HBM read rate of a plain streaming kernel
    over 4 GiB (16-byte non-temporal loads, past the 256 MB MALL; the best of three grid
    sizes), and the dense fp16 MFMA rate of a loop of independent 16x16x32 MFMAs on register
    operands at 1, 2 and 4 waves per SIMD. The vendor library's dense bf16 GEMM (torch.matmul,
    8192^3, hipBLASLt) is reported as the GEMM a library reaches on this box."""
    lib = q4._lib.load()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    st = lambda: torch.cuda.current_stream(dev).cuda_stream
    nbytes = 1 << 32
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    read = {}
    for per_cu in (2, 4, 8):
        wgs = cus * per_cu
        out = torch.empty(lib.q4_probe_stream_read_out_bytes(wgs) // 4, dtype=torch.int32, device=dev)
        call = lambda: lib.q4_probe_stream_read(buf.data_ptr(), nbytes, wgs, out.data_ptr(), st())
        if call() != 0:
            raise RuntimeError("q4_probe_stream_read failed")
        _, ms = time_launches(torch, call, 10, 3)
        read[f"wg_per_cu_{per_cu}"] = nbytes / ms / 1e6
    del buf
    # random fp16 operand sets (N(0,1), as the prefill's scaled operands toggle their bits)
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED)
    ops = torch.randn(64, 16, 8, generator=gen, device=dev).to(torch.float16)
    mfma, mfma_data = {}, {}
    for waves in (1, 2, 4):
        wgs = cus * waves
        out = torch.empty(wgs * 256, dtype=torch.float32, device=dev)
        for table, operands, iters, per_round in ((mfma, None, 20000, 8), (mfma_data, ops.data_ptr(), 2500, 64)):
            call = lambda: lib.q4_probe_mfma(wgs, iters, operands, out.data_ptr(), st())
            if call() != 0:
                raise RuntimeError("q4_probe_mfma failed")
            _, ms = time_launches(torch, call, 5, 2)
            flops = wgs * 4 * iters * per_round * 16 * 16 * 32 * 2
            table[f"waves_per_simd_{waves}"] = flops / ms / 1e9
    a = torch.randn(8192, 8192, device=dev).to(torch.bfloat16)
    b = torch.randn(8192, 8192, device=dev).to(torch.bfloat16)
    _, ms2 = time_launches(torch, lambda: a @ b, 10, 3)
    return {"hbm_read_gbs": max(read.values()), "hbm_read_gbs_by_grid": read,
            "mfma_f16_tflops": max(mfma.values()), "mfma_f16_tflops_by_waves": mfma,
            "mfma_f16_tflops_random_operands": max(mfma_data.values()),
            "mfma_f16_tflops_random_operands_by_waves": mfma_data,
            "bf16_gemm_tflops_torch_matmul": 2 * 8192 ** 3 / ms2 / 1e9,
            "vendor_hbm_gbs": HBM_PEAK_GBS, "vendor_bf16_tflops": MFMA_PEAK_TFLOPS,
            "how": "hbm_read_gbs: q4_probe_stream_read over 4 GiB, best of 2/4/8 workgroups per CU; "
                   "mfma_f16_tflops: q4_probe_mfma, 8 independent 16x16x32 fp16 MFMA chains per wave on constant "
                   "operands, best of 1/2/4 waves per SIMD; _random_operands: the same with 8 A x 8 B sets of "
                   "N(0,1) fp16 operands paired differently by consecutive MFMAs (the multipliers toggle as on real "
                   "data, and the clock falls under the power limit)"}


def extra_config0(torch, q4, dev):
    """Single GEMV N=K=4096 with fp32 x: the same weights over and over
    (cache-resident) and 32 rotating copies (335 MB, beyond the 256 MB MALL)."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED)
    ws_w = [q4.pack_q4_1(gen_blocks(torch, 4096, 4096, gen, dev), dev) for _ in range(32)]
    x = torch.randn(4096, generator=gen, device=dev)
    ys = [torch.empty(4096, device=dev) for _ in range(32)]
    ws = torch.empty(max(q4.gemv_workspace_bytes(1, 4096, 4096), 256), dtype=torch.uint8, device=dev)
    nbytes = ws_w[0].nbytes + 4096 * 4 + 4096 * 4

    def hot():
        for i in range(32):
            q4.gemv_q4(ws_w[0], x, ys[i], workspace=ws)

    def rot():
        for i in range(32):
            q4.gemv_q4(ws_w[i], x, ys[i], workspace=ws)
    hot_us = graph_time(torch, hot, ys) / 32 * 1e3
    rot_us = graph_time(torch, rot, ys) / 32 * 1e3
    return {"cache_resident_us": hot_us, "cache_resident_gbs": nbytes / hot_us / 1e3,
            "rotated_us": rot_us, "rotated_gbs": nbytes / rot_us / 1e3,
            "splits": q4.gemv_split_count(ws_w[0])}


def extra_fp16_scales(torch, q4, model, acts, xhead, steps, warmup):
    """The headline sweep (M = 1, one grouped launch) over the same synthetic weights packed
    with GGUF's fp16 d and m kept exactly (pack_q4_1(..., scales="fp16"), the opt-in
    exact-scale mode), timed back to back with the bf16-scale model as an A/B on one box."""
    dev = model.head.device
    m16 = Llama(torch, q4, dev, scales="fp16")
    g16, nbytes = grouped_sweep(torch, q4, m16, acts, xhead, 1)
    gb, _ = grouped_sweep(torch, q4, model, acts, xhead, 1)
    out = {}
    for name, grp in (("bf16_scales", gb), ("fp16_scales", g16), ("bf16_scales_again", gb)):
        _, per = time_launches(torch, grp.run, steps, warmup)
        out[name] = {"ms": per, "gbs": nbytes / per / 1e6}
    out["fp16_vs_bf16"] = out["fp16_scales"]["ms"] / (0.5 * (out["bf16_scales"]["ms"] + out["bf16_scales_again"]["ms"]))
    del g16, m16
    return out


def extra_config2(torch, q4, model, steps):
    out = {}
    for M in (4, 8, 16):
        acts, xhead = sweep_inputs(torch, model, model.head.device, M)
        grp, nbytes = grouped_sweep(torch, q4, model, acts, xhead, M)
        _, per = time_launches(torch, grp.run, steps, 5)
        out[f"M{M}"] = {"ms": per, "gbs": nbytes / per / 1e6, "tflops": 2 * M * model.weight_bytes * 1.6 / per / 1e9}
        del grp, acts
    return out


def extra_config3(torch, q4, dev):
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED)
    out = {}
    mats = {"gate_up": (14336, 4096), "down": (4096, 14336)}
    packed = {k: q4.pack_q4_1(gen_blocks(torch, n, kk, gen, dev), dev) for k, (n, kk) in mats.items()}
    for w in packed.values():          # static weights: their fp16 prefill scales are made once
        q4.prefill_scales(w)
    for T in (512, 2048):
        for name, (n, k) in mats.items():
            x = torch.randn(T, k, generator=gen, device=dev).to(torch.bfloat16)
            y = torch.empty(T, n, device=dev)
            ws = torch.empty(q4.prefill_workspace_bytes(T, n, k), dtype=torch.uint8, device=dev)

            def run(prec="fp16"):
                for _ in range(3):
                    q4.gemm_q4_prefill(packed[name], x, y, precision=prec, workspace=ws)
            ms = graph_time(torch, run, [y], replays=5) / 3
            ms_bf16 = graph_time(torch, lambda: run("bf16"), [y], replays=5) / 3
            tf = 2.0 * T * n * k / ms / 1e9
            # the activation pre-pass and the GEMM apart: activations prepared once
            # (q4_prefill_prepare) are what a model hands its projections (gate and up
            # share one; the SwiGLU producer can write down's)
            prep = q4.prefill_prepare(x)
            wsp = torch.empty(max(q4.prefill_workspace_bytes(T, n, k), 256), dtype=torch.uint8, device=dev)

            def run_prepared():
                for _ in range(3):
                    q4.gemm_q4_prefill(packed[name], prep, y, workspace=wsp)

            def run_prepare():
                for _ in range(3):
                    q4.prefill_prepare(x, out=prep.data)
            ms_gemm = graph_time(torch, run_prepared, [y], replays=5) / 3
            ms_prep = graph_time(torch, run_prepare, [], replays=5) / 3   # (padding bytes are not written)
            # the vendor library's dense GEMM on the same shape (fp16 weights already
            # dequantized, [K, N] contiguous): the rate this box sustains for a plain
            # GEMM of this problem, as a yardstick for the dequant GEMM
            xd = x.to(torch.float16)
            wd = (torch.randn(k, n, generator=gen, device=dev) * 0.01).to(torch.float16)
            _, dms = time_launches(torch, lambda: torch.matmul(xd, wd), 10, 3)
            out[f"T{T}_{name}"] = {"ms": ms, "tflops": tf, "frac_of_peak": tf / MFMA_PEAK_TFLOPS,
                                   "prepared_gemm_ms": ms_gemm, "prepared_gemm_tflops": 2.0 * T * n * k / ms_gemm / 1e9,
                                   "prepared_gemm_frac_of_peak": 2.0 * T * n * k / ms_gemm / 1e9 / MFMA_PEAK_TFLOPS,
                                   "prepare_ms": ms_prep,
                                   "bf16_tile_ms": ms_bf16, "bf16_tile_tflops": 2.0 * T * n * k / ms_bf16 / 1e9,
                                   "dense_fp16_matmul_ms": dms,
                                   "dense_fp16_matmul_tflops": 2.0 * T * n * k / dms / 1e9,
                                   "vs_dense_fp16_matmul": dms / ms}
            del xd, wd, prep, wsp
    # Llama-3-8B's gate and up as one [28672, 4096] matrix (row groups concatenated) over
    # one prepared X: the FFN's first GEMM as a model issues it
    gu = q4.pack_q4_1(gen_blocks(torch, 28672, 4096, gen, dev), dev)
    q4.prefill_scales(gu)
    for T in (512, 2048):
        x = torch.randn(T, 4096, generator=gen, device=dev).to(torch.bfloat16)
        prep = q4.prefill_prepare(x)
        y = torch.empty(T, 28672, device=dev)
        wsp = torch.empty(max(q4.prefill_workspace_bytes(T, 28672, 4096), 256), dtype=torch.uint8, device=dev)

        def run_fused():
            for _ in range(3):
                q4.gemm_q4_prefill(gu, prep, y, workspace=wsp)
        msf = graph_time(torch, run_fused, [y], replays=5) / 3
        tff = 2.0 * T * 28672 * 4096 / msf / 1e9
        out[f"T{T}_gate_up_fused_prepared"] = {"N": 28672, "K": 4096, "ms": msf, "tflops": tff,
                                               "frac_of_peak": tff / MFMA_PEAK_TFLOPS}
        # the activation producer in front of gate/up: residual add + RMSNorm writing the
        # prepared activations in one launch, against q4_rmsnorm_add + the pre-pass
        xr = torch.randn(T, 4096, generator=gen, device=dev)
        ad = torch.randn(T, 4096, generator=gen, device=dev)
        nw = (1 + 0.1 * torch.randn(4096, generator=gen, device=dev)).to(torch.bfloat16)
        yb = torch.empty(T, 4096, device=dev)
        xnb = torch.empty(T, 4096, dtype=torch.bfloat16, device=dev)
        p2 = torch.zeros_like(prep.data)

        def run_two():
            for _ in range(3):
                q4.rmsnorm_add(xr, nw, add=ad, y=yb, xn=xnb)
                q4.prefill_prepare(xnb, out=prep.data)

        def run_one():
            for _ in range(3):
                q4.rmsnorm_prepare(xr, nw, add=ad, y=yb, out=p2)
        ms_two = graph_time(torch, run_two, [yb], replays=5) / 3
        ms_one = graph_time(torch, run_one, [yb], replays=5) / 3
        out[f"T{T}_norm_producer_K4096"] = {"norm_then_prepare_ms": ms_two, "rmsnorm_prepare_ms": ms_one,
                                            "same_bytes": bool(torch.equal(prep.data[:T * 4096 * 2],
                                                                           p2[:T * 4096 * 2]))}
        del prep, wsp, y, xr, ad, yb, xnb, p2
    # the prefill FFN block with its producers writing the prepared activations: residual add
    # + RMSNorm -> fused gate/up GEMM -> SwiGLU (bf16 h) -> down GEMM, four launches
    dn = q4.pack_q4_1(gen_blocks(torch, 4096, 14336, gen, dev), dev)
    q4.prefill_scales(dn)
    half = gu.nbytes // 2
    gu_il = q4.interleave_gate_up(q4.PackedQ4(gu.data[:half], 14336, 4096), q4.PackedQ4(gu.data[half:], 14336, 4096))
    q4.prefill_scales(gu_il)
    for T in (512, 2048):
        xr = torch.randn(T, 4096, generator=gen, device=dev)
        ad = torch.randn(T, 4096, generator=gen, device=dev)
        nw = (1 + 0.1 * torch.randn(4096, generator=gen, device=dev)).to(torch.bfloat16)
        yb = torch.empty(T, 4096, device=dev)
        p1 = torch.empty(q4.load_library().q4_prefill_prepared_bytes(T, 4096, 1, 0), dtype=torch.uint8, device=dev)
        p2 = torch.empty(q4.load_library().q4_prefill_prepared_bytes(T, 14336, 1, 0), dtype=torch.uint8, device=dev)
        y1 = torch.empty(T, 28672, device=dev)
        y2 = torch.empty(T, 4096, device=dev)
        w1 = torch.empty(max(q4.prefill_workspace_bytes(T, 28672, 4096), 256), dtype=torch.uint8, device=dev)
        w2 = torch.empty(max(q4.prefill_workspace_bytes(T, 4096, 14336), 256), dtype=torch.uint8, device=dev)

        def block():
            _, a1 = q4.rmsnorm_prepare(xr, nw, add=ad, y=yb, out=p1)
            q4.gemm_q4_prefill(gu, a1, y1, workspace=w1)
            a2 = q4.swiglu_prepare(y1, out=p2)
            q4.gemm_q4_prefill(dn, a2, y2, workspace=w2)
        ms = graph_time(torch, block, [y2, yb], replays=5)
        fl = 2.0 * T * (28672 * 4096 + 4096 * 14336)
        # the same block with SwiGLU in the gate/up GEMM's epilogue (gate and up row groups
        # interleaved): h goes out as bf16 and the f32 gate/up output never reaches memory
        hh = torch.empty(T, 14336, dtype=torch.bfloat16, device=dev)

        def block_epi():
            _, a1 = q4.rmsnorm_prepare(xr, nw, add=ad, y=yb, out=p1)
            q4.gemm_q4_prefill_swiglu(gu_il, a1, h=hh)
            a2 = q4.prefill_prepare(hh, out=p2)
            q4.gemm_q4_prefill(dn, a2, y2, workspace=w2)
        ms_epi = graph_time(torch, block_epi, [y2, yb], replays=5)
        out[f"T{T}_ffn_block"] = {"ms": ms, "gemm_tflops": fl / ms / 1e9, "frac_of_peak": fl / ms / 1e9 / MFMA_PEAK_TFLOPS,
                                  "launches": 4,
                                  "swiglu_epilogue_ms": ms_epi, "swiglu_epilogue_gemm_tflops": fl / ms_epi / 1e9,
                                  "swiglu_epilogue_frac_of_peak": fl / ms_epi / 1e9 / MFMA_PEAK_TFLOPS}
        # two layers back to back, down's K-split sum either reduced by its own launch or left
        # as planes for the next layer's norm producer (no reduce launch): per layer
        yc = torch.empty_like(yb)
        parts = [torch.empty(q4.load_library().q4_prefill_split_count(T, 4096, 14336), T, 4096, device=dev)
                 for _ in range(2)]

        def two_layers(deferred):
            def fn():
                _, a1 = q4.rmsnorm_prepare(xr, nw, add=ad, y=yb, out=p1)
                q4.gemm_q4_prefill_swiglu(gu_il, a1, h=hh)
                a2 = q4.prefill_prepare(hh, out=p2)
                if deferred:
                    q4.gemm_q4_prefill_partials(dn, a2, part=parts[0])
                else:
                    q4.gemm_q4_prefill(dn, a2, y2, workspace=w2)
                _, a1 = q4.rmsnorm_prepare(yb, nw, add=parts[0] if deferred else y2, y=yc, out=p1)
                q4.gemm_q4_prefill_swiglu(gu_il, a1, h=hh)
                a2 = q4.prefill_prepare(hh, out=p2)
                if deferred:
                    q4.gemm_q4_prefill_partials(dn, a2, part=parts[1])
                else:
                    q4.gemm_q4_prefill(dn, a2, y2, workspace=w2)
            return fn
        ms2r = graph_time(torch, two_layers(False), [yc], replays=5)
        yc_r = yc.clone()
        ms2d = graph_time(torch, two_layers(True), [yc], replays=5)
        rec = out[f"T{T}_ffn_block"]
        rec["two_layers_reduce_ms_per_layer"] = ms2r / 2
        rec["two_layers_deferred_sums_ms_per_layer"] = ms2d / 2
        rec["deferred_same_residual"] = bool(torch.equal(yc, yc_r))
        rec["down_splits"] = parts[0].shape[0]
        del xr, ad, yb, yc, yc_r, p1, p2, y1, y2, w1, w2, hh, parts
    return out


def extra_prefill_power(torch, q4, dev):
    """The prepared prefill GEMM at T=2048 on the gate_up shape, same kernel and launch, on
    three operand sets: config 3's (seeded Q4_1 weights, N(0,1) tokens), all-zero weights
    (d = m = 0 and zero codes: every dequantized tile is 0) and all-zero tokens. Only the
    data differ, so a rate gap between them is the MFMA datapath's switching energy under
    the board's power limit, not the instruction stream (run it under rocprofv3 with
    GRBM_GUI_ACTIVE to read each one's clock)."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED)
    n, k, T = 14336, 4096, 2048
    blk = gen_blocks(torch, n, k, gen, dev)
    weights = {"config": q4.pack_q4_1(blk, dev), "zero": q4.pack_q4_1(torch.zeros_like(blk), dev)}
    del blk
    for w in weights.values():
        q4.prefill_scales(w)
    x = torch.randn(T, k, generator=gen, device=dev).to(torch.bfloat16)
    preps = {"config": q4.prefill_prepare(x), "zero": q4.prefill_prepare(torch.zeros_like(x))}
    y = torch.empty(T, n, device=dev)
    wsp = torch.empty(max(q4.prefill_workspace_bytes(T, n, k), 256), dtype=torch.uint8, device=dev)
    out = {}
    for label, (wk, xk) in {"config_data": ("config", "config"), "zero_weights": ("zero", "config"),
                            "zero_tokens": ("config", "zero")}.items():
        def run():
            for _ in range(3):
                q4.gemm_q4_prefill(weights[wk], preps[xk], y, workspace=wsp)
        ms = graph_time(torch, run, [y], replays=5) / 3
        tf = 2.0 * T * n * k / ms / 1e9
        out[label] = {"ms": ms, "tflops": tf, "frac_of_peak": tf / MFMA_PEAK_TFLOPS}
    out["shape"] = {"T": T, "N": n, "K": k}
    return out


def extra_config4(torch, q4, dev):
    """Config 4: the routed block (128 experts, top-8 of 16 tokens, H 2048, F 768) over 4
    rotating expert pools, graph replays; and the block with its residual and a shared expert
    of an expert's size (F 768) as the reference's one-dispatch block runs it
    (moe_experts.py:1-13): the shared expert inside the expert launches
    (q4_moe_gemv_shared) against the two-step form (its own one-expert block, then the
    finish)."""
    import numpy as np
    E, K8, H, F, T, pools = 128, 8, 2048, 768, 16, 4
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED)
    experts = []
    gb, db = q4.packed_bytes(2 * F, H), q4.packed_bytes(H, F)
    for _ in range(pools):             # 4 independent expert pools (4 x 377 MB) defeat the 256 MB MALL
        # an expert's matrix is whole 64-row groups, so the E experts stacked are one mx matrix:
        # one pack per pool and matrix kind, byte-identical to packing expert by expert
        gu = q4.pack_q4_1(gen_blocks(torch, E * 2 * F, H, gen, dev), dev).data
        dn = q4.pack_q4_1(gen_blocks(torch, E * H, F, gen, dev), dev).data
        experts.append((q4.PackedExperts(gu, E, 2 * F, H), q4.PackedExperts(dn, E, H, F)))
    rng = np.random.default_rng(SEED)
    logits = rng.standard_normal((T, E))
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :K8]
    w = np.take_along_axis(p, ids, 1)
    w /= w.sum(1, keepdims=True)
    ids_t = torch.from_numpy(ids.astype(np.int32)).to(dev)
    w_t = torch.from_numpy(w.astype(np.float32)).to(dev)
    x = torch.randn(T, H, generator=gen, device=dev).to(torch.bfloat16)
    outs = [torch.empty(T, H, device=dev) for _ in range(pools)]
    ws = torch.empty(q4.moe_workspace_bytes(T, E, K8, H, F), dtype=torch.uint8, device=dev)
    distinct = len(np.unique(ids))
    nbytes = distinct * (gb + db) + T * H * 2 + T * H * 4

    def run():
        for i, (gu, dn) in enumerate(experts):
            q4.moe_batch(gu, dn, x, ids_t, w_t, outs[i], workspace=ws)
    ms = graph_time(torch, run, outs, replays=10) / pools
    rec = {"ms": ms, "gbs": nbytes / ms / 1e6, "distinct_experts": distinct, "bytes": nbytes,
           "tflops": 2.0 * T * K8 * 3 * H * F / ms / 1e9}
    # the block with the residual and a shared expert (Fs = F), one per pool
    Fs = F
    shared = [(q4.pack_q4_1(gen_blocks(torch, 2 * Fs, H, gen, dev), dev),
               q4.pack_q4_1(gen_blocks(torch, H, Fs, gen, dev), dev)) for _ in range(pools)]
    sgw = (0.05 * torch.randn(H, generator=gen, device=dev)).to(torch.bfloat16)
    res = torch.randn(T, H, generator=gen, device=dev)
    one_id = torch.zeros(T, 1, dtype=torch.int32, device=dev)
    one_w = torch.ones(T, 1, device=dev)
    ys = torch.empty(T, H, device=dev)
    ws_s = torch.empty(q4.moe_shared_workspace_bytes(T, E, K8, H, F, Fs), dtype=torch.uint8, device=dev)
    ws_1 = torch.empty(q4.moe_workspace_bytes(T, 1, 1, H, Fs), dtype=torch.uint8, device=dev)

    def fused():
        for i, (gu, dn) in enumerate(experts):
            q4.moe_batch(gu, dn, x, ids_t, w_t, outs[i], workspace=ws_s, residual=res, shared_gate_w=sgw,
                         shared_expert=shared[i])

    def two_step():
        for i, (gu, dn) in enumerate(experts):
            sgu, sdn = shared[i]
            q4.moe_batch(q4.PackedExperts(sgu.data, 1, 2 * Fs, H), q4.PackedExperts(sdn.data, 1, H, Fs), x, one_id,
                         one_w, ys, workspace=ws_1)
            q4.moe_batch(gu, dn, x, ids_t, w_t, outs[i], workspace=ws, residual=res, shared=ys, shared_gate_w=sgw)
    sbytes = nbytes + shared[0][0].nbytes + shared[0][1].nbytes + T * H * 4
    ms_f = graph_time(torch, fused, outs, replays=10) / pools
    ms_2 = graph_time(torch, two_step, outs, replays=10) / pools
    rec["with_shared_expert"] = {"Fs": Fs, "bytes": sbytes, "fused_ms": ms_f, "fused_gbs": sbytes / ms_f / 1e6,
                                 "two_step_ms": ms_2, "two_step_gbs": sbytes / ms_2 / 1e6}
    return rec


def extra_moe_prefill(torch, q4, dev):
    """Config 4's experts (128 x Qwen3-MoE-style gate/up [1536, 2048] and down [2048, 768],
    top-8 of a seeded softmax) at prefill scale: T = 512 and 2048 tokens through the prefill
    path (q4_moe_prefill, fp16 and bf16 tiles) and, at T = 512 (4096 pairs), the decode path
    beside it. Graph-timed; one expert pool (each expert's weights are read once per token
    tile that routes to it)."""
    import numpy as np
    E, K8, H, F = 128, 8, 2048, 768
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED + 23)
    gb, db = q4.packed_bytes(2 * F, H), q4.packed_bytes(H, F)
    gu = torch.empty(E * gb, dtype=torch.uint8, device=dev)
    dn = torch.empty(E * db, dtype=torch.uint8, device=dev)
    for e in range(E):
        q4.pack_q4_1(gen_blocks(torch, 2 * F, H, gen, dev), dev, out=gu[e * gb:(e + 1) * gb])
        q4.pack_q4_1(gen_blocks(torch, H, F, gen, dev), dev, out=dn[e * db:(e + 1) * db])
    gup, dnp = q4.PackedExperts(gu, E, 2 * F, H), q4.PackedExperts(dn, E, H, F)
    out = {}
    for T in (512, 2048):
        rng = np.random.default_rng(SEED + T)
        logits = rng.standard_normal((T, E))
        pr = np.exp(logits - logits.max(1, keepdims=True))
        pr /= pr.sum(1, keepdims=True)
        ids = np.argsort(-pr, axis=1, kind="stable")[:, :K8]
        w = np.take_along_axis(pr, ids, 1)
        w /= w.sum(1, keepdims=True)
        ids_t = torch.from_numpy(ids.astype(np.int32)).to(dev)
        w_t = torch.from_numpy(w.astype(np.float32)).to(dev)
        x = torch.randn(T, H, generator=gen, device=dev).to(torch.bfloat16)
        y = torch.empty(T, H, device=dev)
        flops = 2.0 * T * K8 * 3 * H * F
        wbytes = len(np.unique(ids)) * (gb + db)
        rec = {"pairs": T * K8, "distinct_experts": int(len(np.unique(ids)))}
        # prefill_fp16_bf16h: the fp16 tile with h rounded to bf16 (the reference kernel's h): one
        # down pass instead of the f32 h's value and remainder passes
        paths = [("prefill_fp16", "prefill", "fp16", False), ("prefill_fp16_bf16h", "prefill", "fp16", True),
                 ("prefill_bf16", "prefill", "bf16", False)]
        if T * K8 <= q4.MOE_DECODE_MAX_PAIRS:
            paths.append(("decode", "decode", "fp16", False))
        for name, path, prec, hb in paths:
            ws = torch.empty(max(q4.moe_prefill_workspace_bytes(T, E, K8, H, F) if path == "prefill"
                                 else q4.moe_workspace_bytes(T, E, K8, H, F), 256), dtype=torch.uint8, device=dev)
            q4.moe_batch(gup, dnp, x, ids_t, w_t, y, workspace=ws, path=path, precision=prec, h_bf16=hb)  # scales
            ms = graph_time(torch, lambda: q4.moe_batch(gup, dnp, x, ids_t, w_t, y, workspace=ws, path=path,
                                                        precision=prec, h_bf16=hb), [y], replays=10)
            rec[name] = {"us": round(ms * 1e3, 1), "tflops": round(flops / ms / 1e9, 1),
                         "weight_gbs": round(wbytes / ms / 1e6, 1)}
            del ws
        out[f"T{T}"] = rec
    return out


# --------------------------------------------------------------------------

def q4nx_decode_harness(model_dir, tensor: str, shape=None, reps: int = 10) -> dict:
    """The reference's decode benchmark (utilities/benchmark-q4-decode.py:37-54) on one q4_1
    tensor of a .q4nx container, with the MI355X path beside its two CPU decoders.

    CPU (restatements in oracle/, the baseline leg): the frozen strided-indexing decode
    (``legacy_seconds``) and the contiguous dq_chunks_q4_1 (``contiguous_seconds``), checked
    byte-identical as the reference checks them. GPU: the same chunks copied to HBM, repacked
    to the mx layout (q4_repack_pool, rs = 1, the file raster) and dequantized there
    (q4_dequant); the device values, put back in chunk order, must equal the legacy decode byte
    for byte. Repack, dequant and the M = 1 GEMV over the matrix are then timed with their
    inputs resident in HBM (HIP events, ``reps`` calls each). The container does not hold the
    logical [out, in]: ``shape`` gives it, else the chunks are read as [32 * chunks, 256] (one
    chunk per 32 rows; the same bytes and values, only the GEMV's shape differs)."""
    import numpy as np
    import torch
    from oracle import q4_oracle as O
    q4 = importlib.import_module("openflowlm-next_amd")
    with q4.Q4NXFile(Path(model_dir) / "model.q4nx") as f:
        fmt = f.quant_format_of(tensor)
        if fmt != "q4_1":
            raise ValueError(f"{tensor}: {fmt or 'not a quantised tensor'}; the decode benchmark reads q4_1 chunks")
        raw = np.array(f.raw(tensor))
    chunks = raw.reshape(-1, 5120)
    nch = chunks.shape[0]
    out_dim, in_dim = (int(shape[0]), int(shape[1])) if shape else (32 * nch, 256)
    if out_dim % 64 or in_dim % 256 or (out_dim // 32) * (in_dim // 256) != nch:
        raise ValueError(f"{tensor}: {nch} chunks do not tile [{out_dim}, {in_dim}] (64-row groups of 256-K chunks)")

    t = time.perf_counter()
    old = O.legacy_decode(chunks)
    legacy_s = time.perf_counter() - t
    t = time.perf_counter()
    new = O.dq_chunks_q4_1(chunks)
    contiguous_s = time.perf_counter() - t
    identical = old.tobytes() == new.tobytes()

    dev = torch.device("cuda", 0)
    src = torch.from_numpy(raw).to(dev)
    w = q4.pack_chunks(src, "q4_1", out_dim, in_dim, rs=1, device=dev)
    deq = q4.dequant(w)
    in_chunk_order = deq.view(out_dim // 32, 32, in_dim // 256, 8, 32).permute(0, 2, 1, 3, 4)
    gpu_identical = in_chunk_order.contiguous().cpu().numpy().tobytes() == old.tobytes()
    x = torch.randn(1, in_dim, device=dev).to(torch.bfloat16)
    y = torch.empty(1, out_dim, device=dev)
    _, repack_ms = time_launches(torch, lambda: q4.pack_chunks(src, "q4_1", out_dim, in_dim, rs=1, device=dev), reps, 2)
    _, dequant_ms = time_launches(torch, lambda: q4.dequant(w, out=deq), reps, 2)
    _, gemv_ms = time_launches(torch, lambda: q4.gemm_q4(w, x, y), reps, 2)
    wb = w.nbytes
    gpu = {"shape": [out_dim, in_dim], "shape_given": bool(shape), "byte_identical": gpu_identical,
           "repack_us": round(repack_ms * 1e3, 2), "repack_gbs": round(2 * raw.nbytes / repack_ms / 1e6, 1),
           "dequant_us": round(dequant_ms * 1e3, 2),
           "dequant_gbs": round((wb + out_dim * in_dim * 4) / dequant_ms / 1e6, 1),
           "gemv_m1_us": round(gemv_ms * 1e3, 2), "gemv_m1_gbs": round((wb + in_dim * 2 + out_dim * 4) / gemv_ms / 1e6, 1),
           "dequant_speedup_vs_contiguous_cpu": round(contiguous_s / (dequant_ms * 1e-3), 1)}
    return {"tensor": tensor, "chunks": nch, "byte_identical": identical, "legacy_seconds": legacy_s,
            "contiguous_seconds": contiguous_s, "speedup": legacy_s / contiguous_s, "gpu": gpu}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # HBM-bound launches reach their steady clocks after ~20 ms of load: the headline launch
    # measured 0.740 ms/step at 5 warmup steps, 0.745 at 5 of 20, 0.697 at 30 (one box)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--extras", default="staged,step,0,2,3,pfpower,4,moe_prefill,lm_head,ffn,q8,q4k,q40,fp16s,peaks",
                    help="comma list (staged,step,0,2,3,pfpower,4,moe_prefill,lm_head,ffn,q8,q4k,q40,fp16s,peaks) "
                         "or 'none'")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-passes", type=int, default=3, help="passes over one layer per timed CPU run")
    ap.add_argument("--cpu-runs", type=int, default=5, help="timed runs per CPU worker (the median is reported)")
    ap.add_argument("--cpu-baseline-child", type=int, default=None, help=argparse.SUPPRESS)
    ap.add_argument("--only-extras", action="store_true",
                    help="skip the headline sweep; run the --extras list and print them (profiling runs)")
    ap.add_argument("--model-dir", default=None,
                    help="decode benchmark on a .q4nx container (model-dir/model.q4nx): the reference "
                         "harness's JSON (benchmark-q4-decode.py) plus the GPU repack, dequant and GEMV")
    ap.add_argument("--tensor", default="model.layers.0.mlp.up_proj.weight", help="the tensor --model-dir decodes")
    ap.add_argument("--shape", type=int, nargs=2, default=None, metavar=("OUT", "IN"),
                    help="the tensor's logical [out, in] for --model-dir (default [32 * chunks, 256])")
    ap.add_argument("--step-variants", default=None,
                    help="decode-step extra: only these variants (comma-separated names), for profiling runs")
    ap.add_argument("--copy-probe", type=int, default=0,
                    help="only copy this many bytes device-to-device 5 times (calibrates HBM traffic counters)")
    a = ap.parse_args()

    if a.cpu_baseline_child is not None:
        print(json.dumps(cpu_baseline_child(a.cpu_baseline_child, a.cpu_passes, a.cpu_runs)))
        return 0
    ws = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or ws != 1:
        print("bench.py measures one GPU only: the Q4_1 path is built and timed on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured configuration).", file=sys.stderr)
        return 2

    import torch
    q4 = importlib.import_module("openflowlm-next_amd")
    q4.load_library()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if a.model_dir:
        r = q4nx_decode_harness(a.model_dir, a.tensor, a.shape)
        print(json.dumps(r, indent=2))
        return 0 if r["byte_identical"] and r["gpu"]["byte_identical"] else 1
    if a.copy_probe:
        src = torch.randint(0, 256, (a.copy_probe,), dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": a.copy_probe, "copies": 5}))
        return 0

    if a.only_extras:
        out = {}
        for cfg in [c.strip() for c in a.extras.split(",") if c.strip()]:
            if cfg == "0":
                out["config0_gemv_4096_f32x"] = extra_config0(torch, q4, dev)
            elif cfg == "3":
                out["config3_prefill"] = extra_config3(torch, q4, dev)
            elif cfg == "4":
                out["config4_moe"] = extra_config4(torch, q4, dev)
            elif cfg == "peaks":
                out["measured_peaks"] = extra_peaks(torch, q4, dev)
            elif cfg == "lm_head":
                out["lm_head_topk"] = extra_lm_head(torch, q4, dev)
            elif cfg == "q8":
                out["q8_gemv"] = extra_q8(torch, q4, dev)
            elif cfg == "q4k":
                out["q4k_native_gemv"] = extra_q4k(torch, q4, dev)
            elif cfg == "q40":
                out["q4_0_native_gemv"] = extra_q40(torch, q4, dev)
            elif cfg == "moe_prefill":
                out["moe_prefill"] = extra_moe_prefill(torch, q4, dev)
            elif cfg == "pfpower":
                out["prefill_power"] = extra_prefill_power(torch, q4, dev)
        print(json.dumps(out), flush=True)
        return 0

    log("packing the Llama-3-8B weights (4.69 GB of Q4_1) ...")
    model = Llama(torch, q4, dev)
    acts, xhead = sweep_inputs(torch, model, dev, 1)
    grp, nbytes = grouped_sweep(torch, q4, model, acts, xhead, 1)
    log(f"{model.matrices} matrices, {model.weight_bytes / 1e9:.3f} GB; timing {a.steps} steps")

    total_ms, per_launch_ms = time_launches(torch, grp.run, a.steps, a.warmup)
    ms_per_step = total_ms / a.steps
    value = nbytes / (ms_per_step * 1e-3) / 1e9            # GB/s, whole job
    achieved = nbytes / (per_launch_ms * 1e-3) / 1e9        # one launch == one step

    extras = {}
    wanted = [] if a.extras == "none" else [s.strip() for s in a.extras.split(",") if s.strip()]
    for cfg in wanted:
        t = time.perf_counter()
        try:
            if cfg == "peaks":
                extras["measured_peaks"] = extra_peaks(torch, q4, dev)
            elif cfg == "fp16s":
                extras["fp16_scales_sweep"] = extra_fp16_scales(torch, q4, model, acts, xhead, a.steps, 10)
            elif cfg == "staged":
                extras["config1_staged_decode_order"] = extra_staged(torch, q4, model, acts, xhead)
            elif cfg == "step":
                extras["config1_decode_step"] = extra_decode_step(torch, q4, model, acts, xhead,
                                                                  a.step_variants.split(",") if a.step_variants else None)
            elif cfg == "0":
                extras["config0_gemv_4096_f32x"] = extra_config0(torch, q4, dev)
            elif cfg == "2":
                extras["config2_skinny"] = extra_config2(torch, q4, model, max(5, a.steps // 2))
            elif cfg == "3":
                extras["config3_prefill"] = extra_config3(torch, q4, dev)
            elif cfg == "4":
                extras["config4_moe"] = extra_config4(torch, q4, dev)
            elif cfg == "lm_head":
                extras["lm_head_topk"] = extra_lm_head(torch, q4, dev, model.head, xhead)
            elif cfg == "ffn":
                extras["ffn_fused_decode"] = extra_ffn(torch, q4, model, acts)
            elif cfg == "q8":
                extras["q8_gemv"] = extra_q8(torch, q4, dev)
            elif cfg == "q4k":
                extras["q4k_native_gemv"] = extra_q4k(torch, q4, dev)
            elif cfg == "q40":
                extras["q4_0_native_gemv"] = extra_q40(torch, q4, dev)
            elif cfg == "moe_prefill":
                extras["moe_prefill"] = extra_moe_prefill(torch, q4, dev)
            elif cfg == "pfpower":
                extras["prefill_power"] = extra_prefill_power(torch, q4, dev)
        except Exception as e:                      # keep the headline line whatever an extra does
            extras[f"config{cfg}_error"] = repr(e)[:300]
        log(f"extra {cfg}: {time.perf_counter() - t:.1f}s")
        torch.cuda.empty_cache()

    cpu = None
    if not a.no_cpu:
        model_name = cpu_model_name()
        log(f"CPU baseline ({model_name}): numpy restatement, 1 worker, {a.cpu_runs} runs of {a.cpu_passes} "
            "passes over one layer ...")
        c1 = cpu_baseline(1, a.cpu_passes, a.cpu_runs)
        cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
        log(f"CPU baseline: {cores} workers, one per core ...")
        call = cpu_baseline(cores, 1, a.cpu_runs)
        if c1:
            cpu = {"value": round(c1["gbs"], 4), "unit": "GB/s", "cores": 1, "kind": "port",
                   "sample": f"median of {c1['runs']} runs, each {c1['passes']} passes over one Llama-3-8B layer "
                             f"(q,k,v,o,gate,up,down; {c1['run_bytes'] / c1['passes'] / 1e6:.1f} MB of Q4_1 per "
                             "pass): pool-chunk dequant (q4nx.dq_chunks_q4_1 restated) + f32 matvec, "
                             "OPENBLAS_NUM_THREADS=1",
                   "seconds_per_run": round(c1["median_run_seconds"], 3), "cpu_model": model_name}
            if call:
                cpu["all_cores"] = {"value": round(call["gbs"], 4), "cores": cores, "workers": call["workers"],
                                    "how": f"{cores} single-thread worker processes side by side, each the median "
                                           f"of {call['runs']} runs of one pass; the sum of their rates",
                                    "worker_gbs_range": [round(call["worker_gbs_min"], 4),
                                                         round(call["worker_gbs_max"], 4)],
                                    "wall_seconds": round(call["wall_seconds"], 2)}

    line = {
        "metric": "Q4_1 decode GEMV HBM GB/s (% of peak) at M=1; prefill GEMM TFLOP/s",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded GGUF Q4_1 weights: q~U{0..15}, d=fp16(|N|*0.002+1e-4), m=fp16(-8dU(0.9,1.1)); "
                "bf16 N(0,1) activations)",
        "config": {"workload": "llama3-8b decode weight sweep, M=1, 32 layers + lm_head, one grouped launch/step",
                   "matrices": model.matrices, "weight_bytes": model.weight_bytes,
                   "algorithmic_bytes_per_step": nbytes, "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "traffic_source": "profiles/gemv_grouped_llama3_8b_m1.md (FETCH_SIZE x2.0 + WRITE_SIZE x1.0, "
                                       "factors from a 1 GiB copy)",
                     "kernel": "gemv_grouped_kernel<1,false>", "mean_launch_ms": round(per_launch_ms, 4)},
        "cpu_baseline": cpu,
        "extras": extras,
    }
    ratios = measured_traffic_ratios()
    if ratios:
        extras["measured_traffic_ratios"] = ratios
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
