"""GPU parity of the online softmax of the chunk and decode kernels when the row maxima move.

Both kernels keep an exponent base per query row (the decode kernel: per key
group of a wave) and move it to the running max only when that max outgrows it
by more than 2^8 (the output accumulators are rescaled then).  N(0,1) inputs
barely exercise that: here the
keys carry a component along the row's query direction whose weight depends on
the key position, so the scores
- ramp: grow by tens of log2 units per 64-key tile (a rebase on every tile),
- spike: are N(0,1) except one key far above the rest (one rebase mid-row,
  with the earlier tiles' weight underflowing to zero),
- drift: grow by a few log2 units over the whole row (no rebase after the
  first tile: P reaches up to 2^5 before normalisation),
on the chunk kernel's 64-row form (small calls), its 128-row form (>= 512 row
units) and a split-K call (key span > 2048), and on single-token decode: the
split plan with in-kernel merge (MHA), length-balanced pieces (GQA 16/4, skewed
rows), 8-wave workgroups without split, and explicit 64-key splits.

Reference: the oracle (nanochat/flash_attention.py:155-177 + :69-102 row by
row) in float32 on the CPU, from the same inputs.  Tolerance as the other
bf16/fp16 parity tests: max rel err <= 2e-2 and allclose(atol=rtol=1e-2)
(nanochat tests/test_attention_fallback.py:39); caches bit-exact.
"""
import math

import pytest
import torch

from nanochat_amd.flash_attention import flash_attn
from oracle import kvcache_oracle as orc
from tests.helpers import bits, gen, max_rel_err, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _weight(mode, j, n):
    """Weight of the query direction in key j (of n positions)."""
    if mode == "ramp":
        return 3.0 * j / 64.0
    if mode == "spike":
        return 12.0 if j == (2 * n) // 3 else 0.0
    return 0.2 * j / max(n, 1)  # drift


def _inputs(seed, mode, B, T_new, H, H_kv, D, T_max, seqlens, dtype):
    g = gen(seed)
    G = H // H_kv
    # one query direction per (row, kv head), shared by that kv head's q heads (plus noise)
    u = randn((B, H_kv, D), g)
    u = u / u.norm(dim=-1, keepdim=True)
    q = (u.repeat_interleave(G, dim=1)[:, None] * math.sqrt(D) + 0.3 * randn((B, T_new, H, D), g)).to(dtype)
    kc = torch.zeros(B, T_max, H_kv, D, dtype=dtype)
    vc = torch.zeros(B, T_max, H_kv, D, dtype=dtype)
    k = torch.empty(B, T_new, H_kv, D, dtype=dtype)
    v = randn((B, T_new, H_kv, D), g, dtype)
    for b, s in enumerate(seqlens):
        n = int(s) + T_new
        w = torch.tensor([_weight(mode, j, n) for j in range(n)], dtype=torch.float32)
        keys = randn((n, H_kv, D), g) + w[:, None, None] * u[b][None] * math.sqrt(D)
        kc[b, :s] = keys[:s].to(dtype)
        vc[b, :s] = randn((int(s), H_kv, D), g, dtype)
        k[b] = keys[s:].to(dtype)
    return q, k, v, kc, vc, torch.as_tensor(seqlens, dtype=torch.int32)


SHAPES = {
    # (B, T_new, H, H_kv, D, T_max, seqlens, keys_per_split)
    "rows64": (1, 256, 4, 4, 128, 1024, [0], 0),            # 64-row kernel, prefill into an empty cache
    "rows128": (16, 128, 16, 4, 128, 512, [300] * 16, 0),   # 16 x 128 / 16 x 4 = 512 units: 128-row kernel
    "split": (1, 64, 4, 1, 128, 4096, [3000], 1024),        # key span 3064 in 1024-key splits
    "dec_mha": (4, 1, 8, 8, 128, 4096, [3000, 100, 2000, 4000], 0),     # 16 splits, merged in-kernel
    "dec_gqa_bal": (24, 1, 16, 4, 128, 12288,                           # 96 groups, 42 splits: pieces
                    [8000, 128, 300, 7000, 129, 1, 0, 5000] + [128 + 37 * i for i in range(16)], 0),
    "dec_wide": (16, 1, 12, 12, 128, 2048, [1000 + 61 * i for i in range(16)], 0),  # 192 groups, no split
    "dec_split64": (2, 1, 4, 4, 128, 4096, [4000, 300], 64),           # explicit 64-key splits (63 on row 0)
}


@pytest.mark.parametrize("mode", ["ramp", "spike", "drift"])
@pytest.mark.parametrize("shape", list(SHAPES))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_chunk_softmax_rebase(mode, shape, dtype):
    B, T_new, H, H_kv, D, T_max, seqlens, kps = SHAPES[shape]
    q, k, v, kc, vc, sl = _inputs(7, mode, B, T_new, H, H_kv, D, T_max, seqlens, dtype)
    kc_d, vc_d, sl_d = kc.to(DEV), vc.to(DEV), sl.to(DEV)
    out = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc_d, vc_d, k=k.to(DEV), v=v.to(DEV), cache_seqlens=sl_d,
                                             causal=True, window_size=(-1, 0), keys_per_split=kps)
    ref = orc.flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=sl, causal=True, window_size=(-1, 0),
                                      compute_dtype=torch.float32)
    assert torch.isfinite(out.float()).all()
    err = max_rel_err(out, ref.float())
    assert err <= 2e-2, f"{shape}/{mode}: max rel err {err:.3e}"
    assert torch.allclose(out.float().cpu(), ref.float(), atol=1e-2, rtol=1e-2)
    assert torch.equal(bits(kc_d), bits(kc)), "k_cache bytes differ from the oracle"
    assert torch.equal(bits(vc_d), bits(vc)), "v_cache bytes differ from the oracle"
