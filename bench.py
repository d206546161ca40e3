#!/usr/bin/env python3
"""Benchmark of the Q4_1 dequant-matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--extras 0,2,3,4|none]

Headline: the Llama-3-8B decode weight sweep at
M=1 -- 32 layers of q/k/v/o/gate/up/down plus lm_head, 4.69 GB of Q4_1
weights, synthetic seeded data -- issued as one grouped GEMV launch per step.
`value` = algorithmic bytes (packed weights + bf16 x + f32 y per matrix) /
measured time, inputs resident in HBM. The same JSON line carries:

* roofline     -- that kernel's algorithmic bytes per launch / its mean launch
                  duration from HIP events on its stream, against 8 TB/s;
* cpu_baseline -- the oracle's numpy restatement of the reference CPU path
                  (pool-chunk dequant as q4nx.py:105-126, then an f32 matvec)
                  timed on this host over one Llama layer (136 MB of Q4_1);
* extras       -- configs 0 (single GEMV), 2 (M = 4/8/16), 3 (prefill GEMM
                  TFLOP/s), 4 (routed MoE) and the per-stage decode issue order.

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
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 / fp16 MFMA, TFLOP/s

LLAMA_LAYER = [  # (name, N, K) per layer of Llama-3-8B
    ("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
    ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336),
]
LM_HEAD = ("lm_head", 128256, 4096)
SEED = 1234


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


def build_sweep(torch, q4, dev, M: int = 1, layers: int = 32, weights=None):
    """The Llama-3-8B sweep: (GemvGroup for the whole sweep, staged groups, bytes).

    x inputs follow the decode dataflow: q/k/v share one x, gate/up share one,
    o, down and lm_head have their own; every matrix has its own y."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED + M)
    if weights is None:
        weights = []
        for layer in range(layers):
            for name, n, k in LLAMA_LAYER:
                blocks = gen_blocks(torch, n, k, gen, dev)
                weights.append((f"{name}{layer}", q4.pack_q4_1(blocks, dev)))
                del blocks
        blocks = gen_blocks(torch, LM_HEAD[1], LM_HEAD[2], gen, dev)
        weights.append((LM_HEAD[0], q4.pack_q4_1(blocks, dev)))
        del blocks
        torch.cuda.synchronize()

    def act(k):
        return torch.randn(M, k, generator=gen, device=dev).to(torch.bfloat16)

    items, stages, nbytes = [], [], 0
    wi = iter(weights)
    for layer in range(layers):
        x_in, x_o, x_mlp, x_dn = act(4096), act(4096), act(4096), act(14336)
        xs = {"q": x_in, "k": x_in, "v": x_in, "o": x_o, "gate": x_mlp, "up": x_mlp, "down": x_dn}
        per = {}
        for name, n, k in LLAMA_LAYER:
            _, w = next(wi)
            y = torch.empty(M, n, dtype=torch.float32, device=dev)
            it = (w, xs[name], y)
            items.append(it)
            per[name] = it
            nbytes += w.nbytes + M * k * 2 + M * n * 4
        stages += [[per["q"], per["k"], per["v"]], [per["o"]], [per["gate"], per["up"]], [per["down"]]]
    _, w = next(wi)
    y = torch.empty(M, LM_HEAD[1], dtype=torch.float32, device=dev)
    it = (w, act(4096), y)
    items.append(it)
    stages.append([it])
    nbytes += w.nbytes + M * 4096 * 2 + M * LM_HEAD[1] * 4
    return q4.GemvGroup(items), [q4.GemvGroup(s) for s in stages], nbytes, weights


def time_launches(torch, fn, steps: int, warmup: int):
    """Run fn warmup times, then `steps` timed times bracketed by synchronize;
    each call is bracketed by HIP events on the current stream.
    Returns (total_ms_wall_by_events, mean_ms_per_call)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(st)
    for a, b in ev:
        a.record(st)
        fn()
        b.record(st)
    t1.record(st)
    torch.cuda.synchronize()
    total = t0.elapsed_time(t1)
    per = sum(a.elapsed_time(b) for a, b in ev) / steps
    return total, per


# --------------------------------------------------------------------------
# CPU baseline (oracle restatement of the reference CPU path), in a child
# process so the BLAS thread count can be set before numpy loads
# --------------------------------------------------------------------------

def cpu_baseline_child(threads: int) -> dict:
    import numpy as np
    from oracle import q4_oracle as O
    rng = np.random.default_rng(SEED)
    total_bytes, secs = 0, 0.0
    chunk_slice = 2048                       # 10 MB of chunks -> 64 MB of f32 at a time
    for name, n, k in LLAMA_LAYER:
        nch = n * k // 8192
        chunks = rng.integers(0, 256, (nch, 5120), dtype=np.uint8)
        d = (np.abs(rng.standard_normal((nch, 256))) * 0.002 + 1e-4).astype(np.float16).astype(np.float32)
        m = -8 * d * rng.uniform(0.9, 1.1, (nch, 256)).astype(np.float32)
        chunks[:, 0:512] = O.f32_to_bf16(d).view(np.uint8).reshape(nch, 512)
        chunks[:, 512:1024] = O.f32_to_bf16(m.astype(np.float16).astype(np.float32)).view(np.uint8).reshape(nch, 512)
        x = rng.standard_normal(k).astype(np.float32)
        # rs=1 band order: chunk c covers rows 32*(c // (k/256)), k-tile c % (k/256)
        per_row = k // 256
        y = np.zeros(n, np.float32)
        t = time.perf_counter()
        for c0 in range(0, nch, chunk_slice):
            c1 = min(nch, c0 + chunk_slice)
            w = O.dq_chunks_q4_1(chunks[c0:c1]).reshape(c1 - c0, 32, 256)
            xs = x.reshape(per_row, 256)
            kt = np.arange(c0, c1) % per_row
            part = np.matmul(w, xs[kt][:, :, None])[..., 0]             # [c, 32] f32
            rows = (np.arange(c0, c1) // per_row)
            np.add.at(y.reshape(-1, 32), rows, part)
        secs += time.perf_counter() - t
        total_bytes += nch * 5120
    return {"seconds": secs, "bytes": total_bytes, "gbs": total_bytes / secs / 1e9, "threads": threads}


def cpu_baseline(threads: int) -> dict | None:
    env = dict(os.environ)
    for v in ("OPENBLAS_NUM_THREADS", "OMP_NUM_THREADS", "MKL_NUM_THREADS"):
        env[v] = str(threads)
    env["HIP_VISIBLE_DEVICES"] = ""      # the CPU leg never touches the GPU
    try:
        r = subprocess.run([sys.executable, str(Path(__file__).resolve()), "--cpu-baseline-child", str(threads)],
                           capture_output=True, text=True, env=env, timeout=600)
        if r.returncode != 0:
            log(f"cpu baseline failed: {r.stderr[-500:]}")
            return None
        return json.loads(r.stdout.strip().splitlines()[-1])
    except Exception as e:  # the baseline is reported, never required
        log(f"cpu baseline skipped: {e}")
        return None


# --------------------------------------------------------------------------
# extras
# --------------------------------------------------------------------------

def extra_config0(torch, q4, dev):
    """Single GEMV N=K=4096, fp32 x: cache-resident and over 32 rotated copies (335 MB)."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED)
    ws = [q4.pack_q4_1(gen_blocks(torch, 4096, 4096, gen, dev), dev) for _ in range(32)]
    x = torch.randn(4096, generator=gen, device=dev)
    y = torch.empty(4096, device=dev)
    nbytes = ws[0].nbytes + 4096 * 4 + 4096 * 4
    _, hot = time_launches(torch, lambda: q4.gemv_q4(ws[0], x, y), 50, 10)
    i = [0]

    def rot():
        q4.gemv_q4(ws[i[0] % 32], x, y)
        i[0] += 1
    _, cold = time_launches(torch, rot, 64, 32)
    return {"cache_resident_us": hot * 1e3, "cache_resident_gbs": nbytes / hot / 1e6,
            "rotated_us": cold * 1e3, "rotated_gbs": nbytes / cold / 1e6}


def extra_config2(torch, q4, dev, weights, steps):
    out = {}
    for M in (4, 8, 16):
        grp, _, nbytes, _ = build_sweep(torch, q4, dev, M=M, weights=weights)
        _, per = time_launches(torch, grp.run, steps, 2)
        out[f"M{M}"] = {"ms": per, "gbs": nbytes / per / 1e6, "tflops": 2 * M * 7.505e9 / per / 1e9}
    return out


def extra_config3(torch, q4, dev):
    if not hasattr(q4.load_library(), "q4_gemm_prefill"):
        return None
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED)
    out = {}
    mats = {"gate_up": (14336, 4096), "down": (4096, 14336)}
    packed = {k: q4.pack_q4_1(gen_blocks(torch, n, kk, gen, dev), dev) for k, (n, kk) in mats.items()}
    for T in (512, 2048):
        for name, (n, k) in mats.items():
            x = torch.randn(T, k, generator=gen, device=dev).to(torch.bfloat16)
            y = torch.empty(T, n, device=dev)
            _, per = time_launches(torch, lambda: q4.gemm_q4_prefill(packed[name], x, y), 10, 3)
            out[f"T{T}_{name}"] = {"ms": per, "tflops": 2.0 * T * n * k / per / 1e9}
    return out


def extra_config4(torch, q4, dev):
    if not hasattr(q4.load_library(), "q4_moe_gemv"):
        return None
    import numpy as np
    E, K8, H, F, T, pools = 128, 8, 2048, 768, 16, 4
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED)
    experts = []
    for _ in range(pools):             # 4 independent expert pools (4 x 377 MB) defeat the 256 MB MALL
        gu = torch.empty(E * q4.packed_bytes(2 * F, H), dtype=torch.uint8, device=dev)
        dn = torch.empty(E * q4.packed_bytes(H, F), dtype=torch.uint8, device=dev)
        gb, db = q4.packed_bytes(2 * F, H), q4.packed_bytes(H, F)
        for e in range(E):
            q4.pack_q4_1(gen_blocks(torch, 2 * F, H, gen, dev), dev, out=gu[e * gb:(e + 1) * gb])
            q4.pack_q4_1(gen_blocks(torch, H, F, gen, dev), dev, out=dn[e * db:(e + 1) * db])
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
    out = torch.empty(T, H, device=dev)
    distinct = len(np.unique(ids))
    nbytes = distinct * (q4.packed_bytes(2 * F, H) + q4.packed_bytes(H, F)) + T * H * 2 + T * H * 4
    i = [0]

    def run():
        gu, dn = experts[i[0] % pools]
        q4.moe_batch(gu, dn, x, ids_t, w_t, out)
        i[0] += 1
    _, per = time_launches(torch, run, 40, 8)
    return {"ms": per, "gbs": nbytes / per / 1e6, "distinct_experts": distinct, "bytes": nbytes,
            "tflops": 2.0 * T * K8 * 3 * H * F / per / 1e9}


# --------------------------------------------------------------------------

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--extras", default="0,2,3,4", help="comma list of configs to add, or 'none'")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-baseline-child", type=int, default=None, help=argparse.SUPPRESS)
    a = ap.parse_args()

    if a.cpu_baseline_child is not None:
        print(json.dumps(cpu_baseline_child(a.cpu_baseline_child)))
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

    log("building the Llama-3-8B sweep (4.69 GB of Q4_1 weights) ...")
    grp, stages, nbytes, weights = build_sweep(torch, q4, dev, M=1)
    wbytes = sum(w.nbytes for _, w in weights)
    log(f"{len(weights)} matrices, {wbytes / 1e9:.3f} GB weights; timing {a.steps} steps")

    torch.cuda.synchronize()
    total_ms, per_launch_ms = time_launches(torch, grp.run, a.steps, a.warmup)
    ms_per_step = total_ms / a.steps
    value = nbytes / (ms_per_step * 1e-3) / 1e9            # GB/s, whole job
    achieved = nbytes / (per_launch_ms * 1e-3) / 1e9        # one launch == one step here

    def staged():
        for s in stages:
            s.run()
    _, staged_ms = time_launches(torch, staged, max(3, a.steps // 4), 2)
    extras = {"config1_staged_129_launches": {"ms": staged_ms, "gbs": nbytes / staged_ms / 1e6}}

    wanted = [] if a.extras == "none" else [s.strip() for s in a.extras.split(",") if s.strip()]
    for cfg in wanted:
        t = time.perf_counter()
        try:
            if cfg == "0":
                extras["config0_gemv_4096"] = extra_config0(torch, q4, dev)
            elif cfg == "2":
                extras["config2_skinny"] = extra_config2(torch, q4, dev, weights, max(3, a.steps // 4))
            elif cfg == "3":
                r = extra_config3(torch, q4, dev)
                if r:
                    extras["config3_prefill"] = r
            elif cfg == "4":
                r = extra_config4(torch, q4, dev)
                if r:
                    extras["config4_moe"] = r
        except Exception as e:                      # keep the headline line whatever an extra does
            extras[f"config{cfg}_error"] = repr(e)[:300]
        log(f"extra config {cfg}: {time.perf_counter() - t:.1f}s")

    cpu = None
    if not a.no_cpu:
        log("CPU baseline (numpy restatement, 1 thread) ...")
        c1 = cpu_baseline(1)
        cores = os.cpu_count() or 1
        log(f"CPU baseline (all {cores} cores) ...")
        call = cpu_baseline(cores)
        if c1:
            cpu = {"value": c1["gbs"], "unit": "GB/s", "cores": 1, "kind": "port",
                   "sample": f"one Llama-3-8B layer (q,k,v,o,gate,up,down; {c1['bytes'] / 1e6:.1f} MB Q4_1): "
                             "pool-chunk dequant (q4nx.dq_chunks_q4_1 restated) + f32 matvec, "
                             "OPENBLAS_NUM_THREADS=1",
                   "seconds": c1["seconds"]}
            if call:
                cpu["all_cores"] = {"value": call["gbs"], "cores": cores, "seconds": call["seconds"]}

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
                   "matrices": len(weights), "weight_bytes": wbytes, "algorithmic_bytes_per_step": nbytes,
                   "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "gemv_grouped_kernel<1,bf16>", "mean_launch_ms": round(per_launch_ms, 4)},
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
