"""HIP-graph replay of the attention calls (how bench.py and the Engine counterpart run them).

A captured sequence of calls is replayed several times, with eager work in between and the
caches reset before each replay; every replay must reproduce the eager run exactly (the
kernels are deterministic, so outputs and caches are compared bit for bit).  Covers the split-K
decode with its merge launch, the MFMA chunk path with the fused append, and the fused QK
prologue.
"""
import pytest
import torch

from nanochat_amd.flash_attention import flash_attn
from nanochat_amd.gpt import rotary_tables
from tests.helpers import bits, gen, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _state(seed, B, T_max, H_kv, D, seqlens):
    g = gen(seed)
    kc = torch.zeros(B, T_max, H_kv, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    for b, s in enumerate(seqlens):
        kc[b, :s] = randn((s, H_kv, D), g, torch.bfloat16)
        vc[b, :s] = randn((s, H_kv, D), g, torch.bfloat16)
    return kc.to(DEV), vc.to(DEV), torch.tensor(seqlens, dtype=torch.int32, device=DEV)


def _inputs(seed, steps, B, T_new, H, H_kv, D):
    g = gen(seed)
    return [(randn((B, T_new, H, D), g, torch.bfloat16).to(DEV), randn((B, T_new, H_kv, D), g, torch.bfloat16).to(DEV),
             randn((B, T_new, H_kv, D), g, torch.bfloat16).to(DEV)) for _ in range(steps)]


@pytest.mark.parametrize("mode", ["decode", "chunk", "rope_decode", "rope_chunk"])
def test_graph_replays_equal_eager(mode):
    B, H, H_kv, D, T_max = 3, 8, 4, 128, 1400
    seqlens = [0, 700, 1200]
    T_new = 16 if "chunk" in mode else 1
    steps = 3
    ins = _inputs(400, steps, B, T_new, H, H_kv, D)
    cos_t, sin_t = rotary_tables(4096, D, device=DEV, dtype=torch.bfloat16)
    kc0, vc0, sl0 = _state(401, B, T_max, H_kv, D, seqlens)

    def run(kc, vc, sl):
        outs = []
        for q, k, v in ins:
            if mode.startswith("rope"):
                outs.append(flash_attn.flash_attn_with_kvcache_rope(q, kc, vc, k, v, sl, cos_t, sin_t,
                                                                    window_size=(-1, 0), keys_per_split=256))
            else:
                outs.append(flash_attn.flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=sl, causal=True,
                                                               window_size=(-1, 0), keys_per_split=256))
            sl.add_(T_new)
        return outs

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        kc, vc, sl = kc0.clone(), vc0.clone(), sl0.clone()
        ref_outs = [o.clone() for o in run(kc, vc, sl)]   # eager, also warms this stream's workspace
        ref_kc, ref_vc, ref_sl = kc.clone(), vc.clone(), sl.clone()
        kc.copy_(kc0); vc.copy_(vc0); sl.copy_(sl0)
        stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        g_outs = run(kc, vc, sl)
    for rep in range(3):
        with torch.cuda.stream(stream):
            kc.copy_(kc0); vc.copy_(vc0); sl.copy_(sl0)
            graph.replay()
            stream.synchronize()
        for a, b in zip(g_outs, ref_outs):
            assert torch.equal(bits(a), bits(b)), f"replay {rep}: output differs"
        assert torch.equal(bits(kc), bits(ref_kc)) and torch.equal(bits(vc), bits(ref_vc)), f"replay {rep}: cache"
        assert torch.equal(sl, ref_sl)
        # unrelated eager work on the default stream between replays
        x = torch.randn(64, 128, device=DEV, dtype=torch.bfloat16)
        y = flash_attn.flash_attn_with_kvcache(x.view(1, 64, 1, 128), x.view(1, 64, 1, 128).clone(),
                                               x.view(1, 64, 1, 128).clone(),
                                               cache_seqlens=torch.full((1,), 64, dtype=torch.int32, device=DEV))
        torch.cuda.synchronize()
        assert torch.isfinite(y.float()).all()
