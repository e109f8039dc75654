"""Benchmark of nanochat's inference KV-cache path on one MI355X.

Workload ("C2"): d20 shapes -- 20 layers, 10 q /
10 kv heads x 128, bf16 K/V/Q ~ N(0,1); batch 32 rows with cache_seqlens
uniform in [512, 2048] (seed 0), cache length 2304; one step appends one
token per row per layer and runs causal decode attention over the cache
(flash_attn_with_kvcache, window (-1, 0)), then advances the positions.

The timed region replays a HIP graph holding exactly --steps steps
(20 launches of the fused append+split-K decode kernel and one position
advance each), bracketed by synchronisation and HIP events on the stream
the kernels run on.  Inputs are resident in HBM before timing starts.

Prints ONE JSON line (rank 0) with the metric, the roofline of the decode
kernel and a CPU baseline: the oracle (a restatement of the reference's
PyTorch fallback) timed on this host's cores on a bounded sample.

    python bench.py [--steps 256] [--warmup 10] [--gpus 1] [--cpu-seconds 10]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
METRIC = "decode attn+KV-append HBM GB/s (% of peak) and decode tokens/sec, d20 B=32"
HBM_PEAK_GBPS = 8000.0

# C2 shapes
LAYERS, BATCH, HEADS, KV_HEADS, HEAD_DIM = 20, 32, 10, 10, 128
T_MAX = 2304
S_LO, S_HI = 512, 2048
ELEM = 2  # bf16


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def c2_seqlens() -> torch.Tensor:
    g = torch.Generator(device="cpu")
    g.manual_seed(0)
    return torch.randint(S_LO, S_HI + 1, (BATCH,), generator=g, dtype=torch.int32)


def step_bytes(seqlens, layers=LAYERS) -> int:
    """Algorithmic HBM bytes of one decode step (each K/V token counted once).

    Per layer and row: 2*H_kv*D*e bytes per visible key (s_b + 1 keys, the
    new one included), the new K/V token written once (2*H_kv*D*e), q read
    and the output written once (2*H*D*e).  For d20: 5120 * (s_b + 3).
    """
    kv_tok = 2 * KV_HEADS * HEAD_DIM * ELEM
    qo = 2 * HEADS * HEAD_DIM * ELEM
    return layers * sum(kv_tok * (int(s) + 1) + kv_tok + qo for s in seqlens)


def read_traffic():
    """(HBM bytes, algorithmic bytes) per call from the committed rocprofv3 --pmc summary, or None.

    The PMC runs (profiles/attn_decode_d20_pmc.md) measure FETCH_SIZE and WRITE_SIZE per
    dispatch, scaled by the same counters' reading for a 2 GiB copy kernel.
    """
    path = ROOT / "profiles" / "attn_decode_d20_pmc.md"
    if not path.exists():
        return None
    text = path.read_text()
    t = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)\s*$", text, flags=re.M)
    a = re.search(r"^algorithmic_bytes_per_launch:\s*([0-9.eE+]+)\s*$", text, flags=re.M)
    return (float(t.group(1)), float(a.group(1))) if t and a else None


def copy_ceiling(dev, stream, nbytes=1 << 31, reps=10) -> float:
    """Achievable streaming bandwidth on this GPU: torch's device copy of 2 GiB, read + write bytes."""
    with torch.cuda.stream(stream):
        src = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        dst.copy_(src)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            dst.copy_(src)
        e1.record(stream)
        stream.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del src, dst
    return 2 * nbytes / (ms * 1e-3) / 1e9


def cpu_baseline(budget_s: float) -> dict:
    """Time the oracle (reference fallback restated, row by row) on the host cores."""
    sys.path.insert(0, str(ROOT))
    from oracle import kvcache_oracle as orc

    cores = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(cores)
    g = torch.Generator(device="cpu")
    g.manual_seed(0)
    seqlens = c2_seqlens()
    layers = 2
    kc = torch.randn(layers, BATCH, T_MAX, KV_HEADS, HEAD_DIM, generator=g).to(torch.bfloat16)
    vc = torch.randn(layers, BATCH, T_MAX, KV_HEADS, HEAD_DIM, generator=g).to(torch.bfloat16)
    qkv = [torch.randn(BATCH, 1, h, HEAD_DIM, generator=g).to(torch.bfloat16) for h in (HEADS, KV_HEADS, KV_HEADS)]
    done_bytes, layer_steps = 0, 0
    t0 = time.perf_counter()
    while True:
        for layer in range(layers):
            orc.flash_attn_with_kvcache(qkv[0], kc[layer], vc[layer], k=qkv[1], v=qkv[2], cache_seqlens=seqlens,
                                        causal=True, window_size=(-1, 0))
            done_bytes += step_bytes(seqlens, layers=1)
            layer_steps += 1
        seqlens += 1
        if time.perf_counter() - t0 > budget_s or int(seqlens.max()) >= T_MAX - 1:
            break
    dt = time.perf_counter() - t0
    return {
        "value": round(done_bytes / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{layer_steps} layer-steps of C2 decode (2 of 20 layers, B=32, bf16) in {dt:.1f} s "
                  f"through oracle/kvcache_oracle.py (torch CPU SDPA, row by row)",
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--keys-per-split", type=int, default=0)
    ap.add_argument("--eager", action="store_true", help="also time the steps without a graph")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the KV-cache path has no cross-GPU part); "
              "run with --gpus 1", file=sys.stderr)
        return 2
    if args.steps < 1 or args.steps > T_MAX - S_HI:
        print(f"bench.py: --steps must be in [1, {T_MAX - S_HI}] (cache capacity {T_MAX})", file=sys.stderr)
        return 2

    from nanochat_amd import _ext
    from nanochat_amd.flash_attention import flash_attn_with_kvcache
    _ext.lib()  # fail loudly if the HIP library is missing

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(device=dev)
    s0 = c2_seqlens()
    K, W = args.steps, args.warmup
    log(f"[bench] C2 d20 decode: L={LAYERS} B={BATCH} H={HEADS}/{KV_HEADS} D={HEAD_DIM} T_max={T_MAX} "
        f"steps={K} warmup={W} s0 mean={s0.float().mean():.1f}")

    with torch.cuda.stream(stream):
        gd = torch.Generator(device=dev)
        gd.manual_seed(0)
        shape = (LAYERS, BATCH, T_MAX, KV_HEADS, HEAD_DIM)
        k_cache = torch.randn(shape, generator=gd, device=dev, dtype=torch.bfloat16)
        v_cache = torch.randn(shape, generator=gd, device=dev, dtype=torch.bfloat16)
        n_in = max(K, W)
        q_all = torch.randn((n_in, LAYERS, BATCH, 1, HEADS, HEAD_DIM), generator=gd, device=dev, dtype=torch.bfloat16)
        k_all = torch.randn((n_in, LAYERS, BATCH, 1, KV_HEADS, HEAD_DIM), generator=gd, device=dev,
                            dtype=torch.bfloat16)
        v_all = torch.randn_like(k_all)
        seqlens = s0.to(dev)
        s0_dev = s0.to(dev)

        def one_step(i):
            for layer in range(LAYERS):
                flash_attn_with_kvcache(q_all[i, layer], k_cache[layer], v_cache[layer], k=k_all[i, layer],
                                        v=v_all[i, layer], cache_seqlens=seqlens, causal=True,
                                        window_size=(-1, 0), keys_per_split=args.keys_per_split)
            seqlens.add_(1)

        # eager warmup (allocates the split-K workspace on this stream)
        for i in range(W):
            one_step(i)
        eager_ms = None
        if args.eager:
            seqlens.copy_(s0_dev)
            stream.synchronize()
            t0 = time.perf_counter()
            for i in range(K):
                one_step(i)
            stream.synchronize()
            eager_ms = (time.perf_counter() - t0) * 1e3 / K
        seqlens.copy_(s0_dev)
        stream.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(K):
            one_step(i)
    log(f"[bench] captured {K} steps ({K * LAYERS} decode launches) in one HIP graph")

    with torch.cuda.stream(stream):
        # untimed replay, then restore the starting positions
        graph.replay()
        seqlens.copy_(s0_dev)
        stream.synchronize()
        torch.cuda.synchronize()
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        ev0.record(stream)
        graph.replay()
        ev1.record(stream)
        stream.synchronize()
        torch.cuda.synchronize()
        wall_s = time.perf_counter() - t0
        gpu_ms = ev0.elapsed_time(ev1)
        final_seq = seqlens.cpu()
    if not torch.equal(final_seq, s0 + K):
        log(f"[bench] ERROR: positions after the timed region are wrong: {final_seq[:4]} vs {(s0 + K)[:4]}")
        return 1

    total_bytes = sum(step_bytes(s0 + i) for i in range(K))
    t_s = gpu_ms / 1e3
    gbps = total_bytes / t_s / 1e9
    ms_per_step = gpu_ms / K
    launches = K * LAYERS
    avg_launch_us = gpu_ms * 1e3 / launches
    bytes_per_launch = total_bytes / launches
    log(f"[bench] graph replay: {gpu_ms:.3f} ms (HIP events), {wall_s * 1e3:.3f} ms wall; "
        f"{ms_per_step:.4f} ms/step; {gbps:.1f} GB/s; eager {eager_ms} ms/step")

    cpu = None
    if args.cpu_seconds > 0:
        log(f"[bench] CPU baseline: ~{args.cpu_seconds:.0f} s of the oracle on the host cores")
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"[bench] CPU baseline: {cpu}")

    copy_gbps = copy_ceiling(dev, stream)
    log(f"[bench] torch copy_ of 2 GiB: {copy_gbps:.0f} GB/s (read + write)")
    traffic = read_traffic()
    out = {
        "metric": METRIC,
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 caches/q/k/v, cache_seqlens ~ U[512,2048] seed 0)",
        "config": {
            "workload": "C2: d20 decode, flash_attn_with_kvcache append+attention, 20 layers x 10/10 heads x 128, "
                        "B=32, T_max=2304, window (-1,0), one token per row per layer per step",
            "layers": LAYERS, "batch": BATCH, "heads": HEADS, "kv_heads": KV_HEADS, "head_dim": HEAD_DIM,
            "cache_len": T_MAX, "timing": "HIP graph of all steps, HIP events on the launch stream",
        },
        "pct_of_peak": round(100.0 * gbps / HBM_PEAK_GBPS, 2),
        "hbm_copy_gbps": round(copy_gbps, 1),
        "pct_of_copy": round(100.0 * gbps / copy_gbps, 2),
        "tokens_per_s": round(BATCH * K / t_s, 1),
        "wall_ms_per_step": round(wall_s * 1e3 / K, 5),
        "eager_ms_per_step": round(eager_ms, 5) if eager_ms is not None else None,
        "roofline": {
            "bound": "hbm",
            "achieved": round(bytes_per_launch / (avg_launch_us * 1e-6) / 1e9, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(bytes_per_launch / (avg_launch_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
            "traffic": traffic[0] if traffic else None,
            "traffic_over_algorithmic": round(traffic[0] / traffic[1], 4) if traffic else None,
            "kernel": "one flash_attn_with_kvcache decode call: decode_attn_kernel<bf16, packed-q, D=128, GB=1> "
                      "(fused append + split-K) + merge_splits_kernel<128, 1>",
            "avg_launch_us": round(avg_launch_us, 3),
            "algorithmic_bytes_per_launch": round(bytes_per_launch),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
