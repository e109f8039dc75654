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
import ctypes
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
METRIC = "decode attn+KV-append HBM GB/s (% of peak) and decode tokens/sec, d20 B=32"
HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
REPLAYS = 21   # timed graph replays per figure; the median is reported

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
    """torch's device copy of 2 GiB, read + write bytes (a copy ceiling; the decode kernel mostly reads)."""
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


def _probe_lib():
    """nanochat_amd/libnc_probe.so: bench.py's read-bandwidth probes (built with the library)."""
    path = ROOT / "nanochat_amd" / "libnc_probe.so"
    lib = ctypes.CDLL(str(path))
    lib.nc_probe_read_linear.restype = ctypes.c_int
    lib.nc_probe_read_linear.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    lib.nc_probe_read_kv_rows.restype = ctypes.c_int
    lib.nc_probe_read_kv_rows.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                          ctypes.c_void_p, ctypes.c_void_p]
    return lib


def _event_ms(stream, fn, reps):
    """Median ms of `reps` calls of fn(), each bracketed by HIP events on `stream` (after one warm call)."""
    with torch.cuda.stream(stream):
        fn()
        evs = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fn()
            e1.record(stream)
            evs.append((e0, e1))
        stream.synchronize()
    return statistics.median(e0.elapsed_time(e1) for e0, e1 in evs)


def read_ceilings(dev, stream, k_cache, v_cache, seqlens, c2_call_bytes) -> dict:
    """Read-bandwidth ceilings measured on this GPU by libnc_probe.so (read-only kernels):
    - read_linear: one non-temporal pass over a 4 GiB buffer, 32 KiB contiguous per workgroup (the HBM
      streaming read rate);
    - read_c2_shape: the K/V bytes of one C2 decode call (layer 0 of the bench's caches, positions
      [0, s_b] of every row and head) in the decode kernel's access shape (256-byte head rows at the
      2560-byte token stride, 256-position workgroups), with no arithmetic and no output."""
    lib = _probe_lib()
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    nbytes = 1 << 32
    with torch.cuda.stream(stream):
        buf = torch.ones(nbytes // 2, dtype=torch.bfloat16, device=dev)
    sh = stream.cuda_stream

    def lin():
        assert lib.nc_probe_read_linear(buf.data_ptr(), nbytes, sink.data_ptr(), sh) == 0

    ms_lin = _event_ms(stream, lin, 10)
    del buf
    B, T, Hkv, D = k_cache.shape

    def rows():
        assert lib.nc_probe_read_kv_rows(k_cache.data_ptr(), v_cache.data_ptr(), seqlens.data_ptr(), B, Hkv, T,
                                         k_cache.stride(0), k_cache.stride(1), 256, sink.data_ptr(), sh) == 0

    ms_rows = _event_ms(stream, rows, REPLAYS)
    kv_bytes = sum(2 * Hkv * D * 2 * (int(s) + 1) for s in seqlens.tolist())
    return {"read_linear_GBps": round(nbytes / (ms_lin * 1e-3) / 1e9, 1),
            "read_c2_shape_GBps": round(kv_bytes / (ms_rows * 1e-3) / 1e9, 1),
            "read_c2_shape_us": round(ms_rows * 1e3, 2),
            "read_c2_shape_kv_bytes": kv_bytes,
            "note": "libnc_probe.so read-only kernels: read_linear = one non-temporal pass over 4 GiB; "
                    "read_c2_shape = one C2 call's K/V bytes in the decode kernel's access shape, no compute"}


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cgroup_cpus():
    """CPU quota of this process's cgroup in cores (cgroup v2 cpu.max), or None if unlimited/unknown."""
    try:
        quota, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        return None if quota == "max" else round(int(quota) / int(period), 2)
    except (OSError, ValueError):
        return None


def cpu_baseline(budget_s: float) -> dict:
    """Time the oracle (reference fallback restated, row by row) on all the host cores this process may use."""
    sys.path.insert(0, str(ROOT))
    from oracle import kvcache_oracle as orc

    cores = len(os.sched_getaffinity(0))
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
                  f"through oracle/kvcache_oracle.py (torch CPU SDPA, row by row), "
                  f"torch.set_num_threads({cores}) = len(os.sched_getaffinity(0))",
        "cpu_model": _cpu_model(),
        "cgroup_cpu_quota_cores": _cgroup_cpus(),
    }


def _replay_times(stream, graph, reset, reps):
    """Per-replay times (ms) of `reps` replays of `graph`: reset() runs before each replay, outside
    the HIP events on `stream` that bracket the replay itself."""
    evs = []
    with torch.cuda.stream(stream):
        for _ in range(reps):
            reset()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            graph.replay()
            e1.record(stream)
            evs.append((e0, e1))
        stream.synchronize()
    return [e0.elapsed_time(e1) for e0, e1 in evs]


def _graph_time(stream, body, reset, reps=REPLAYS):
    """Capture body() in a HIP graph (after one eager run); median ms of `reps` timed replays."""
    with torch.cuda.stream(stream):
        body()
        reset()
        stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        body()
    with torch.cuda.stream(stream):
        reset()
        graph.replay()
        stream.synchronize()
    ms = statistics.median(_replay_times(stream, graph, reset, reps))
    del graph
    return ms


def _kv_bytes(seqlens, windows, h_kv, h, d, e=2):
    """Decode-step algorithmic bytes (same rule as step_bytes) for per-layer windows."""
    kv_tok, qo = 2 * h_kv * d * e, 2 * h * d * e
    total = 0
    for w in windows:
        for s in seqlens:
            s = int(s)
            n = s + 1 if w < 0 else min(s + 1, w + 1)
            total += kv_tok * n + kv_tok + qo
    return total


def run_c4(dev, stream, steps, kps=0, ckps=0):
    """d26 SSSL decode: 26 layers, 13/13 x 128, S=1024 x19 / L=4096 x7, B=8, s=3072, `steps` tokens."""
    from nanochat_amd.flash_attention import flash_attn_with_kvcache
    from nanochat_amd.gpt import GPTConfig, window_sizes
    L, H, D, B, T, S0 = 26, 13, 128, 8, 4096, 3072
    windows = [w for w, _ in window_sizes(GPTConfig(sequence_len=4096, n_layer=L, window_pattern="SSSL"))]
    with torch.cuda.stream(stream):
        g = torch.Generator(device=dev)
        g.manual_seed(0)
        kc = torch.randn((L, B, T, H, D), generator=g, device=dev, dtype=torch.bfloat16)
        vc = torch.randn_like(kc)
        qs = torch.randn((steps, L, B, 1, H, D), generator=g, device=dev, dtype=torch.bfloat16)
        ks, vs = torch.randn_like(qs), torch.randn_like(qs)
        sl = torch.full((B,), S0, dtype=torch.int32, device=dev)

    def body():
        for i in range(steps):
            for layer in range(L):
                flash_attn_with_kvcache(qs[i, layer], kc[layer], vc[layer], k=ks[i, layer], v=vs[i, layer],
                                        cache_seqlens=sl, causal=True, window_size=(windows[layer], 0),
                                        keys_per_split=kps)
            sl.add_(1)

    ms = _graph_time(stream, body, lambda: sl.fill_(S0))
    total = sum(_kv_bytes([S0 + i] * B, windows, H, H, D) for i in range(steps))
    gbps = total / (ms * 1e-3) / 1e9
    return {"config": "c4", "workload": "d26 SSSL decode, 26 layers (S=1024 x19, L=4096 x7), 13/13 heads x 128, "
                                        f"B=8, s0=3072, {steps} steps", "ms_per_step": round(ms / steps, 5),
            "GB_per_s": round(gbps, 1), "pct_of_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
            "tokens_per_s": round(B * steps / (ms * 1e-3), 1)}


def run_c5(dev, stream, steps, kps=0, ckps=0):
    """GQA mixed batch: 32 layers, 16 q / 4 kv x 128, B=64, Zipf(1.2) lengths; rows 0-47 decode,
    rows 48-63 chunk-append 128 tokens each step: two calls per layer on row-slice views, and the
    same step as one varlen call per layer (cu_seqlens_q over the packed tokens)."""
    import numpy as np
    from nanochat_amd.flash_attention import flash_attn_with_kvcache
    L, H, HKV, D, B, T, C, ND = 32, 16, 4, 128, 64, 16384, 128, 48
    hi = T - C * steps
    rs = np.random.RandomState(0)
    s0 = torch.tensor(np.clip(rs.zipf(1.2, B), 128, hi), dtype=torch.int32)
    with torch.cuda.stream(stream):
        g = torch.Generator(device=dev)
        g.manual_seed(0)
        kc = torch.empty((L, B, T, HKV, D), device=dev, dtype=torch.bfloat16).normal_(generator=g)
        vc = torch.empty_like(kc).normal_(generator=g)
        # packed tokens per (step, layer): 48 decode tokens, then 16 rows x 128 chunk tokens; the
        # two-call legs use views of the same data
        NT = ND + (B - ND) * C
        qp = torch.randn((steps, L, NT, H, D), generator=g, device=dev, dtype=torch.bfloat16)
        kp, vp = (torch.randn((steps, L, NT, HKV, D), generator=g, device=dev, dtype=torch.bfloat16)
                  for _ in range(2))
        qd, kd, vd = (x[:, :, :ND].unflatten(2, (ND, 1)) for x in (qp, kp, vp))
        qc, kch, vch = (x[:, :, ND:].unflatten(2, (B - ND, C)) for x in (qp, kp, vp))
        lens = torch.tensor([1] * ND + [C] * (B - ND), dtype=torch.int32, device=dev)
        cu = torch.cat([torch.zeros(1, dtype=torch.int32, device=dev), lens.cumsum(0).to(torch.int32)])
        sl = s0.to(dev)
        s0d = s0.to(dev)

    def dec_body():
        for i in range(steps):
            for layer in range(L):
                flash_attn_with_kvcache(qd[i, layer], kc[layer, :ND], vc[layer, :ND], k=kd[i, layer], v=vd[i, layer],
                                        cache_seqlens=sl[:ND], causal=True, window_size=(-1, 0), keys_per_split=kps)
            sl[:ND].add_(1)

    def chunk_body():
        for i in range(steps):
            for layer in range(L):
                flash_attn_with_kvcache(qc[i, layer], kc[layer, ND:], vc[layer, ND:], k=kch[i, layer],
                                        v=vch[i, layer], cache_seqlens=sl[ND:], causal=True, window_size=(-1, 0),
                                        keys_per_split=ckps)
            sl[ND:].add_(C)

    def varlen_body():
        for i in range(steps):
            for layer in range(L):
                flash_attn_with_kvcache(qp[i, layer], kc[layer], vc[layer], k=kp[i, layer], v=vp[i, layer],
                                        cache_seqlens=sl, causal=True, window_size=(-1, 0), cu_seqlens_q=cu,
                                        max_seqlen_q=C)
            sl.add_(lens)

    reset = lambda: sl.copy_(s0d)  # noqa: E731
    ms_dec = _graph_time(stream, dec_body, reset)
    ms_chunk = _graph_time(stream, chunk_body, reset)
    ms_varlen = _graph_time(stream, varlen_body, reset)
    dec_bytes = sum(_kv_bytes((s0[:ND] + i).tolist(), [-1] * L, HKV, H, D) for i in range(steps))
    flops = 0
    for i in range(steps):
        for s in (s0[ND:] + C * i).tolist():
            flops += L * 4 * H * D * sum(s + j + 1 for j in range(C))
    gbps = dec_bytes / (ms_dec * 1e-3) / 1e9
    tflops = flops / (ms_chunk * 1e-3) / 1e12
    return {"config": "c5", "workload": f"GQA mixed: 32 layers, 16q/4kv x 128, B=64 (48 decode + 16 x 128-token "
                                        f"chunks), Zipf(1.2) lengths in [128, {hi}], {steps} steps",
            "decode_ms_per_step": round(ms_dec / steps, 4), "decode_GB_per_s": round(gbps, 1),
            "decode_pct_of_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
            "chunk_ms_per_step": round(ms_chunk / steps, 4), "chunk_TFLOP_per_s": round(tflops, 1),
            "chunk_pct_of_bf16_peak": round(100 * tflops / 2500.0, 2),
            "step_ms": round((ms_dec + ms_chunk) / steps, 4),
            "varlen_one_call_step_ms": round(ms_varlen / steps, 4), "seqlens_mean": float(s0.float().mean())}


def run_c3(dev, stream, steps, kps=0, ckps=0):
    """d24 kernel twin: 1024-token chunk prefill into one row (24 layers, SSSL at seq 2048), fan-out to
    16 rows of 1152, then `steps` decode steps of the 16 rows."""
    import ctypes
    from nanochat_amd import _ext
    from nanochat_amd.engine import KVCache
    from nanochat_amd.flash_attention import flash_attn_with_kvcache
    from nanochat_amd.gpt import GPTConfig, window_sizes
    L, H, D, P, N = 24, 12, 128, 1024, 16
    windows = [w for w, _ in window_sizes(GPTConfig(sequence_len=2048, n_layer=L, window_pattern="SSSL"))]
    with torch.cuda.stream(stream):
        g = torch.Generator(device=dev)
        g.manual_seed(0)
        src = KVCache(1, H, P, D, L, dev, torch.bfloat16)
        qp = torch.randn((L, 1, P, H, D), generator=g, device=dev, dtype=torch.bfloat16)
        kp, vp = torch.randn_like(qp), torch.randn_like(qp)
        dst = KVCache(N, H, P + 128, D, L, dev, torch.bfloat16)
        qd = torch.randn((steps, L, N, 1, H, D), generator=g, device=dev, dtype=torch.bfloat16)
        kd, vd = torch.randn_like(qd), torch.randn_like(qd)

    def prefill_body():
        for layer in range(L):
            flash_attn_with_kvcache(qp[layer], src.k_cache[layer], src.v_cache[layer], k=kp[layer], v=vp[layer],
                                    cache_seqlens=src.cache_seqlens, causal=True, window_size=(windows[layer], 0),
                                    keys_per_split=ckps)
        src.cache_seqlens.add_(P)

    ms_prefill = _graph_time(stream, prefill_body, lambda: src.cache_seqlens.zero_())
    a = _ext.FanoutArgs()
    a.k_src, a.v_src = src.k_cache.data_ptr(), src.v_cache.data_ptr()
    a.k_dst, a.v_dst = dst.k_cache.data_ptr(), dst.v_cache.data_ptr()
    a.dst_seqlens = dst.cache_seqlens.data_ptr()
    a.n_layers, a.n_rows, a.prefix_len, a.row_elems = L, N, P, H * D
    a.src_stride_l, a.dst_stride_l, a.dst_stride_b = src.k_cache.stride(0), dst.k_cache.stride(0), dst.k_cache.stride(1)
    a.dtype = 2

    def fanout_body():
        _ext.check(_ext.lib().nc_kv_fanout(ctypes.byref(a), torch.cuda.current_stream().cuda_stream), "fanout")

    ms_fan = _graph_time(stream, fanout_body, lambda: None)

    def decode_body():
        for i in range(steps):
            for layer in range(L):
                flash_attn_with_kvcache(qd[i, layer], dst.k_cache[layer], dst.v_cache[layer], k=kd[i, layer],
                                        v=vd[i, layer], cache_seqlens=dst.cache_seqlens, causal=True,
                                        window_size=(windows[layer], 0), keys_per_split=kps)
            dst.cache_seqlens.add_(1)

    ms_dec = _graph_time(stream, decode_body, lambda: dst.cache_seqlens.fill_(P))
    flops = 0
    for w in windows:
        flops += 4 * H * D * sum(min(i + 1, w + 1) for i in range(P))
    fan_bytes = L * 2 * P * H * D * 2 * (1 + N)
    dec_bytes = sum(_kv_bytes([P + i] * N, windows, H, H, D) for i in range(steps))
    return {"config": "c3", "workload": f"d24: prefill 1024 tokens (24 layers, SSSL S=512/L=2048, 12 heads x 128) "
                                        f"-> fan-out to 16 rows of 1152 -> {steps} decode steps",
            "prefill_ms": round(ms_prefill, 4), "prefill_TFLOP_per_s": round(flops / (ms_prefill * 1e-3) / 1e12, 1),
            "prefill_pct_of_bf16_peak": round(100 * flops / (ms_prefill * 1e-3) / 2.5e15, 2),
            "prefill_GFLOP": round(flops / 1e9, 2),
            "fanout_ms": round(ms_fan, 4), "fanout_GB_per_s": round(fan_bytes / (ms_fan * 1e-3) / 1e9, 1),
            "fanout_pct_of_peak": round(100 * fan_bytes / (ms_fan * 1e-3) / 1e9 / HBM_PEAK_GBPS, 2),
            "decode_ms_per_step": round(ms_dec / steps, 4),
            "decode_GB_per_s": round(dec_bytes / (ms_dec * 1e-3) / 1e9, 1)}


def run_e2e(dev, stream, steps, kps=0, ckps=0):
    """d20 model decode step (random-init weights, bf16, SSSL windows at sequence_len 2048): B=32 rows at
    position 1280, one token per row per step.  Timings of GPT.forward with the cache: the reference's
    op-by-op QK prologue (eager; it needs get_pos(), a host sync), the fused prologue (eager), and the
    fused prologue with one decode step captured in a HIP graph (possible because the fused path has no
    host sync), with torch's logits head and with the fused one (nc_linear + softcap).  Then the
    C3-shaped Engine.generate in the same modes, the last two also sampling with nc_sample, the last one
    with the block projections on nc_linear as well (16 rows).  The d20 step's 32 rows keep F.linear for the
    block projections (nanochat_amd.linear.prefer_for_projection)."""
    from nanochat_amd.engine import KVCache
    from nanochat_amd.gpt import GPTConfig, build_model
    cfg = GPTConfig(sequence_len=2048, vocab_size=32768, n_layer=20, n_head=10, n_kv_head=10, n_embd=1280)
    B, P = 32, 1280
    with torch.cuda.stream(stream):
        model = build_model(cfg, dev, compute_dtype=torch.bfloat16, seed=0)
        g = torch.Generator(device=dev)
        g.manual_seed(0)
        kv = KVCache(B, 10, P + 3 * steps + 16, 128, 20, dev, torch.bfloat16)
        kv.k_cache[:, :, :P].normal_(generator=g)
        kv.v_cache[:, :, :P].normal_(generator=g)
        ids = torch.randint(0, 32768, (B, 1), generator=g, device=dev)

    def timed(fn, n):
        with torch.cuda.stream(stream):
            fn()
            stream.synchronize()
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record(stream)
            for _ in range(n):
                fn()
            ev1.record(stream)
            stream.synchronize()
            return ev0.elapsed_time(ev1) / n

    def step():
        with torch.inference_mode():
            model.forward(ids, kv_cache=kv)

    res = {}
    model.fused_logits_head = False
    for name, fused in (("op_by_op_eager", False), ("fused_eager", True)):
        model.fused_qk_prologue = fused
        kv.cache_seqlens.fill_(P)
        res[name] = timed(step, steps)
    model.fused_qk_prologue = True
    # graph-captured step: separate q/k/v GEMMs and torch's logits head; one qkv GEMM; and with the
    # fused head (nc_linear + softcap) as well
    for name, qkv, head in (("fused_graph_torch_head", False, False), ("fused_graph_qkv", True, False),
                            ("fused_graph", True, True)):
        model.fused_qkv_projection = qkv
        model.fused_logits_head = head
        kv.cache_seqlens.fill_(P)
        with torch.cuda.stream(stream):
            step()  # warm the workspace on this stream
            stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.inference_mode(), torch.cuda.graph(graph, stream=stream):
            model.forward(ids, kv_cache=kv)
        kv.cache_seqlens.fill_(P)
        res[name] = timed(graph.replay, steps)
        del graph
    out = {"config": "e2e", "workload": f"d20 GPT decode step (random init, bf16, SSSL), B={B} at position {P}, "
                                        f"{steps} steps", **{k + "_ms_per_step": round(v, 4) for k, v in res.items()},
           "tokens_per_s_fused_graph": round(B / (res["fused_graph"] * 1e-3), 1)}
    del kv, model
    torch.cuda.empty_cache()

    # C3-shaped Engine.generate: d24, 1024-token prompt, 16 samples, `steps` tokens (wall clock, host loop included)
    from nanochat_amd.engine import Engine

    class _Tok:
        def encode_special(self, s):
            return 32759 + ["<|bos|>", "<|user_start|>", "<|user_end|>", "<|assistant_start|>", "<|assistant_end|>",
                            "<|python_start|>", "<|python_end|>", "<|output_start|>", "<|output_end|>"].index(s)

        def get_bos_token_id(self):
            return 32759

    cfg3 = GPTConfig(sequence_len=2048, vocab_size=32768, n_layer=24, n_head=12, n_kv_head=12, n_embd=1536)
    model3 = build_model(cfg3, dev, compute_dtype=torch.bfloat16, seed=0)
    g3 = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, 32759, (1024,), generator=g3).tolist()
    import nanochat_amd.gpt as gpt_mod
    for name, fused, use_graph, head_smp, proj in (("op_by_op", False, False, False, False),
                                                   ("fused", True, False, False, False),
                                                   ("fused_graph", True, True, False, False),
                                                   ("fused_graph_head_sampler", True, True, True, False),
                                                   ("fused_graph_head_sampler_proj", True, True, True, True)):
        model3.fused_qk_prologue = fused
        model3.fused_logits_head = head_smp
        gpt_mod.SMALL_M_PROJECTIONS = proj   # 16 rows: q/k/v, c_proj and c_fc on nc_linear
        engine = Engine(model3, _Tok(), use_graph=use_graph, fused_sampling=head_smp)
        for _ in engine.generate(prompt, num_samples=16, max_tokens=4, temperature=1.0, seed=0):
            pass  # warm up
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        n = 0
        for _ in engine.generate(prompt, num_samples=16, max_tokens=steps, temperature=1.0, seed=0):
            n += 1
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        out[f"engine_c3_{name}_ms_per_step"] = round(dt * 1e3 / n, 4)
        out[f"engine_c3_{name}_tokens_per_s"] = round(16 * n / dt, 1)
    model3.fused_qk_prologue = True
    model3.fused_logits_head = True
    gpt_mod.SMALL_M_PROJECTIONS = True
    out["engine_c3_workload"] = (f"Engine.generate d24 (random init, bf16), 1024-token prompt, 16 samples, {steps} "
                                 "tokens incl. prefill + fan-out; wall clock")
    return out


def run_paged(dev, stream, steps, kps=0, ckps=0, page=256):
    """C2's decode workload (d20, B=32, 20 layers, lengths U[512, 2048] seed 0) through a paged cache
    (FA3's page_table: `page`-token blocks in a shuffled pool, one table per row) against the same
    workload on the dense cache, in one process: the cost of addressing keys through the table."""
    from nanochat_amd.flash_attention import flash_attn_with_kvcache
    L, B, H, D = LAYERS, BATCH, HEADS, HEAD_DIM
    seq = c2_seqlens()
    nb = (T_MAX + page - 1) // page
    with torch.cuda.stream(stream):
        g = torch.Generator(device=dev)
        g.manual_seed(0)
        kc = torch.randn((L, B, nb * page, KV_HEADS, D), generator=g, device=dev, dtype=torch.bfloat16)
        vc = torch.randn_like(kc)
        qs = torch.randn((steps, L, B, 1, H, D), generator=g, device=dev, dtype=torch.bfloat16)
        ks, vs = torch.randn_like(qs[:, :, :, :, :KV_HEADS]), torch.randn_like(qs[:, :, :, :, :KV_HEADS])
        sl = seq.to(dev)
        # each layer's pool holds the same blocks as its dense cache, shuffled; row b's table names them
        perm = torch.randperm(B * nb, generator=torch.Generator().manual_seed(1))
        table = perm.view(B, nb).to(torch.int32).to(dev)
        inv = torch.argsort(perm).to(dev)
        kp = kc.view(L, B * nb, page, KV_HEADS, D)[:, inv].contiguous()
        vp = vc.view(L, B * nb, page, KV_HEADS, D)[:, inv].contiguous()

    def body(paged):
        def run():
            for i in range(steps):
                for layer in range(L):
                    if paged:
                        flash_attn_with_kvcache(qs[i, layer], kp[layer], vp[layer], k=ks[i, layer], v=vs[i, layer],
                                                cache_seqlens=sl, causal=True, window_size=(-1, 0),
                                                page_table=table, keys_per_split=kps)
                    else:
                        flash_attn_with_kvcache(qs[i, layer], kc[layer], vc[layer], k=ks[i, layer], v=vs[i, layer],
                                                cache_seqlens=sl, causal=True, window_size=(-1, 0),
                                                keys_per_split=kps)
                sl.add_(1)
        return run

    reset = lambda: sl.copy_(seq.to(dev))  # noqa: E731
    ms_dense = _graph_time(stream, body(False), reset)
    ms_paged = _graph_time(stream, body(True), reset)
    total = sum(step_bytes([int(s) + i for s in seq]) for i in range(steps))
    gb_d, gb_p = total / (ms_dense * 1e-3) / 1e9, total / (ms_paged * 1e-3) / 1e9

    # chunked prefill: a 128-token chunk per row into the same caches at the C2 lengths (20 layers, MFMA kernel)
    tc = 128
    with torch.cuda.stream(stream):
        qc = torch.randn((L, B, tc, H, D), generator=g, device=dev, dtype=torch.bfloat16)
        kn, vn = torch.randn_like(qc[:, :, :, :KV_HEADS]), torch.randn_like(qc[:, :, :, :KV_HEADS])

    def chunk_body(paged):
        def run():
            for layer in range(L):
                kcl, vcl = (kp[layer], vp[layer]) if paged else (kc[layer], vc[layer])
                flash_attn_with_kvcache(qc[layer], kcl, vcl, k=kn[layer], v=vn[layer], cache_seqlens=sl,
                                        causal=True, window_size=(-1, 0), page_table=table if paged else None,
                                        keys_per_split=ckps)
        return run

    ms_chunk_dense = _graph_time(stream, chunk_body(False), reset)
    ms_chunk_paged = _graph_time(stream, chunk_body(True), reset)
    return {"config": "paged", "workload": f"C2 decode (d20, B=32, 20 layers) through {page}-token pages of a "
                                           f"shuffled pool vs the dense cache, {steps} steps; and one "
                                           f"{tc}-token chunk per row into the same caches, 20 layers",
            "dense_ms_per_step": round(ms_dense / steps, 5), "paged_ms_per_step": round(ms_paged / steps, 5),
            "dense_GB_per_s": round(gb_d, 1), "paged_GB_per_s": round(gb_p, 1),
            "paged_pct_of_peak": round(100 * gb_p / HBM_PEAK_GBPS, 2),
            "chunk_dense_ms": round(ms_chunk_dense, 5), "chunk_paged_ms": round(ms_chunk_paged, 5)}


def run_head(dev, stream, steps, kps=0, ckps=0):
    """The decode step's tail on d20 shapes (B=32, 1280 -> 32768 vocab, bf16 weights): the logits head
    (lm_head + slice + fp32 + softcap 15, gpt.py:468-472) as one nc_linear call against F.linear + torch's
    ops, and next-token sampling (engine.py:141-156) as one nc_sample call against torch's ops, for greedy,
    whole-row and top-50 draws.  Each leg is captured `steps` times in a HIP graph; us per call."""
    import torch.nn.functional as F
    from nanochat_amd.linear import linear, logits_head
    from nanochat_amd.sampling import sample_with_uniforms
    B, C, V = 32, 1280, 32768
    g = torch.Generator(device=dev)
    g.manual_seed(0)

    def timed(fn):
        with torch.cuda.stream(stream):
            fn()
            stream.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for _ in range(steps):
                    fn()
            graph.replay()
            stream.synchronize()
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record(stream)
            for _ in range(4):
                graph.replay()
            ev1.record(stream)
            stream.synchronize()
            return round(ev0.elapsed_time(ev1) * 1e3 / (4 * steps), 2)

    with torch.cuda.stream(stream), torch.inference_mode():
        x = torch.randn(B, 1, C, device=dev, generator=g).bfloat16()
        w = (torch.randn(V, C, device=dev, generator=g) * 0.05).bfloat16()
        logits = logits_head(x, w, V, 15.0)[:, 0, :].contiguous()
        u = torch.rand(B, device=dev, generator=g)

        def torch_head():
            lg = F.linear(x, w)[..., :V].float()
            return 15 * torch.tanh(lg / 15)

        def torch_top50():
            vals, idx = torch.topk(logits, 50, dim=-1)
            return idx.gather(1, torch.multinomial(F.softmax(vals / 0.8, dim=-1), 1))

        res = {
            "fused_head_us": timed(lambda: logits_head(x, w, V, 15.0)),
            "torch_head_us": timed(torch_head),
            "nc_linear_us": timed(lambda: linear(x, w)),
            "torch_linear_us": timed(lambda: F.linear(x, w)),
            "nc_greedy_us": timed(lambda: sample_with_uniforms(logits, None, 0.0)),
            "torch_greedy_us": timed(lambda: torch.argmax(logits, dim=-1, keepdim=True)),
            "nc_whole_row_us": timed(lambda: sample_with_uniforms(logits, u, 0.8)),
            "torch_whole_row_us": timed(lambda: torch.multinomial(F.softmax(logits / 0.8, dim=-1), 1)),
            "nc_top50_us": timed(lambda: sample_with_uniforms(logits, u, 0.8, 50)),
            "torch_top50_us": timed(torch_top50),
        }
        # block projections (gpt.py:87-89,125,136-138) of d24 at 16 rows (C3's samples) and d20 at 32 rows: one
        # call per layer's weight, 20 distinct weights per graph pass so W streams from HBM; us per call
        for rows, shapes, tag in ((16, ((4608, 1536), (1536, 1536), (6144, 1536), (1536, 6144)), "d24_m16"),
                                  (32, ((3840, 1280), (1280, 1280), (5120, 1280), (1280, 5120)), "d20_m32")):
            for n, k in shapes:
                ws = [(torch.randn(n, k, device=dev, generator=g) * k ** -0.5).bfloat16() for _ in range(20)]
                xp = torch.randn(rows, 1, k, device=dev, generator=g).bfloat16()
                key = f"proj_{tag}_{n}x{k}"
                res[key + "_nc_us"] = round(timed(lambda: [linear(xp, wi) for wi in ws]) / 20, 2)
                res[key + "_torch_us"] = round(timed(lambda: [F.linear(xp, wi) for wi in ws]) / 20, 2)
                del ws
    head_bytes = V * C * 2 + B * C * 2 + B * V * 4
    return {"config": "head", "workload": f"d20 logits head and sampler, B={B}, vocab {V}, K={C}, bf16; "
                                          f"{steps} calls per graph; block projections (m x n x k, 20 weights "
                                          f"per pass)", **res,
            "fused_head_bytes_per_call": head_bytes,
            "fused_head_TBps": round(head_bytes / (res["fused_head_us"] * 1e-6) / 1e12, 3)}


def _profile_value(name: str, key: str):
    """A figure recorded in a committed rocprofv3 summary (profiles/<name>) as a `key: value` line."""
    path = ROOT / "profiles" / name
    if not path.exists():
        return None
    m = re.search(r"^%s:\s*([0-9.eE+-]+)\s*$" % re.escape(key), path.read_text(), flags=re.M)
    return float(m.group(1)) if m else None


def other_configs(dev, stream) -> dict:
    """C3, C4 and C5 figures for the metric line (same kernels and method, bounded step counts)."""
    out = {}
    for name, fn, steps in (("c3", run_c3, 32), ("c4", run_c4, 64), ("c5", run_c5, 8)):
        t0 = time.perf_counter()
        res = fn(dev, stream, steps)
        res.pop("config", None)
        out[name] = res
        torch.cuda.empty_cache()
        log(f"[bench] {name}: {json.dumps(res)} ({time.perf_counter() - t0:.1f} s)")
    out["c3"]["prefill_mfma_busy_pct"] = _profile_value("attn_chunk_d24_prefill_pmc.md", "mfma_busy_pct")
    out["c5"]["chunk_mfma_busy_pct"] = _profile_value("attn_gqa_mixed_c5_pmc.md", "mfma_busy_pct")
    out["mfma_busy_source"] = ("SQ_VALU_MFMA_BUSY_CYCLES / (kernel duration x clock x SIMDs) from the committed "
                               "rocprofv3 --pmc summaries in profiles/ (counters cannot be read inside this run)")
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--replays", type=int, default=REPLAYS, help="timed graph replays (median reported), >= 20")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--keys-per-split", type=int, default=0,
                    help="decode split size (multiple of 64; 0 = library default)")
    ap.add_argument("--chunk-keys-per-split", type=int, default=0,
                    help="c3/c5 chunk-kernel split size (0 = library default)")
    ap.add_argument("--no-eager", action="store_true", help="skip the eager (un-captured) timing of the C2 steps")
    ap.add_argument("--no-configs", action="store_true", help="skip the C3/C4/C5 figures of the metric line")
    ap.add_argument("--config", default="c2", choices=["c2", "c3", "c4", "c5", "e2e", "head", "paged"],
                    help="c2 (default) is the metric line (with C3/C4/C5 figures); c3/c4/c5 print one config's "
                         "figures; e2e times the d20 model's decode step; head the fused logits head and the "
                         "sampler; paged C2 through a page table")
    ap.add_argument("--rope", action="store_true",
                    help="c2 through flash_attn_with_kvcache_rope (QK prologue fused; same bytes + tables)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the KV-cache path has no cross-GPU part); "
              "run with --gpus 1", file=sys.stderr)
        return 2
    if args.config != "c2":
        from nanochat_amd import _ext
        _ext.lib()
        dev = torch.device("cuda", 0)
        torch.cuda.set_device(dev)
        stream = torch.cuda.Stream(device=dev)
        runner = {"c3": run_c3, "c4": run_c4, "c5": run_c5, "e2e": run_e2e, "head": run_head,
                  "paged": run_paged}[args.config]
        steps = {"c3": min(args.steps, 128), "c4": min(args.steps, 256), "c5": min(args.steps, 16),
                 "e2e": min(args.steps, 64), "head": min(args.steps, 50), "paged": min(args.steps, 200)}[args.config]
        print(json.dumps(runner(dev, stream, steps, kps=args.keys_per_split, ckps=args.chunk_keys_per_split)),
              flush=True)
        return 0
    if args.steps < 1 or args.steps > T_MAX - S_HI:
        print(f"bench.py: --steps must be in [1, {T_MAX - S_HI}] (cache capacity {T_MAX})", file=sys.stderr)
        return 2
    reps = max(20, args.replays)

    from nanochat_amd import _ext
    from nanochat_amd.flash_attention import flash_attn_with_kvcache
    _ext.lib()  # fail loudly if the HIP library is missing

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(device=dev)
    s0 = c2_seqlens()
    K, W = args.steps, args.warmup
    log(f"[bench] C2 d20 decode: L={LAYERS} B={BATCH} H={HEADS}/{KV_HEADS} D={HEAD_DIM} T_max={T_MAX} "
        f"steps={K} warmup={W} replays={reps} s0 mean={s0.float().mean():.1f}")

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

        if args.rope:
            from nanochat_amd.flash_attention import flash_attn_with_kvcache_rope
            from nanochat_amd.gpt import rotary_tables
            cos_t, sin_t = rotary_tables(10 * 2048, HEAD_DIM, device=dev, dtype=torch.bfloat16)

        def one_step(i):
            for layer in range(LAYERS):
                if args.rope:
                    flash_attn_with_kvcache_rope(q_all[i, layer], k_cache[layer], v_cache[layer], k_all[i, layer],
                                                 v_all[i, layer], seqlens, cos_t, sin_t, causal=True,
                                                 window_size=(-1, 0), keys_per_split=args.keys_per_split)
                else:
                    flash_attn_with_kvcache(q_all[i, layer], k_cache[layer], v_cache[layer], k=k_all[i, layer],
                                            v=v_all[i, layer], cache_seqlens=seqlens, causal=True,
                                            window_size=(-1, 0), keys_per_split=args.keys_per_split)
            seqlens.add_(1)

        # eager warmup (allocates the split-K workspace on this stream)
        for i in range(W):
            one_step(i)
        eager_ms = None
        if not args.no_eager:
            # the same K steps without a graph: Python dispatch of every call included (wall clock)
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

    reset = lambda: seqlens.copy_(s0_dev)  # noqa: E731
    with torch.cuda.stream(stream):
        # untimed replay; then one replay bracketed by synchronisation on both sides (wall clock)
        reset()
        graph.replay()
        reset()
        stream.synchronize()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        graph.replay()
        stream.synchronize()
        torch.cuda.synchronize()
        wall_s = time.perf_counter() - t0
    # the timed replays: HIP events on the launch stream around each replay; the median is the figure
    times = _replay_times(stream, graph, reset, reps)
    final_seq = seqlens.cpu()
    if not torch.equal(final_seq, s0 + K):
        log(f"[bench] ERROR: positions after the timed region are wrong: {final_seq[:4]} vs {(s0 + K)[:4]}")
        return 1
    gpu_ms = statistics.median(times)

    total_bytes = sum(step_bytes(s0 + i) for i in range(K))
    t_s = gpu_ms / 1e3
    gbps = total_bytes / t_s / 1e9
    ms_per_step = gpu_ms / K
    launches = K * LAYERS
    avg_launch_us = gpu_ms * 1e3 / launches
    bytes_per_launch = total_bytes / launches
    log(f"[bench] graph replays: median {gpu_ms:.3f} ms (min {min(times):.3f}, max {max(times):.3f}, {reps} "
        f"replays, HIP events), one synchronised replay {wall_s * 1e3:.3f} ms wall; {ms_per_step:.4f} ms/step; "
        f"{gbps:.1f} GB/s; eager {eager_ms} ms/step")

    seqlens.copy_(s0_dev)
    ceil = read_ceilings(dev, stream, k_cache[0], v_cache[0], seqlens, bytes_per_launch)
    ceil["copy_rw_GBps"] = round(copy_ceiling(dev, stream), 1)
    log(f"[bench] ceilings: {ceil}")
    del graph, k_cache, v_cache, q_all, k_all, v_all
    torch.cuda.empty_cache()

    configs = None if args.no_configs else other_configs(dev, stream)

    cpu = None
    if args.cpu_seconds > 0:
        log(f"[bench] CPU baseline: ~{args.cpu_seconds:.0f} s of the oracle on the host cores")
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"[bench] CPU baseline: {cpu}")

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
            "cache_len": T_MAX, "s0_mean": round(float(s0.float().mean()), 2),
            "timing": f"HIP graph of all {K} steps; median of {reps} replays timed with HIP events on the launch "
                      f"stream (positions reset between replays, outside the events)",
        },
        "pct_of_peak": round(100.0 * gbps / HBM_PEAK_GBPS, 2),
        "tokens_per_s": round(BATCH * K / t_s, 1),
        "replay_ms": {"median": round(gpu_ms, 4), "min": round(min(times), 4), "max": round(max(times), 4),
                      "replays": reps},
        "wall_ms_per_step": round(wall_s * 1e3 / K, 5),
        "eager_ms_per_step": round(eager_ms, 5) if eager_ms is not None else None,
        "ceilings": ceil,
        "pct_of_read_linear": round(100.0 * gbps / ceil["read_linear_GBps"], 2),
        "pct_of_read_c2_shape": round(100.0 * gbps / ceil["read_c2_shape_GBps"], 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(bytes_per_launch / (avg_launch_us * 1e-6) / 1e9, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(bytes_per_launch / (avg_launch_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
            "traffic": traffic[0] if traffic else None,
            "traffic_over_algorithmic": round(traffic[0] / traffic[1], 4) if traffic else None,
            "kernel": "one flash_attn_with_kvcache decode call (C2 layer): decode_attn_kernel<bf16, packed-q, "
                      "D=128, GB=1> with the fused append and split-K merge",
            "avg_launch_us": round(avg_launch_us, 3),
            "algorithmic_bytes_per_launch": round(bytes_per_launch),
        },
        "configs": configs,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
