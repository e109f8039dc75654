"""GPU parity at the full per-layer workloads of two BASELINE configs, on the library's default plans.

- C4, d26 SSSL decode: B=8, 13/13 heads x 128, cache 4096, every row at s=3072, the short
  window 1024 and the long window 4096 of _compute_window_sizes(4096, "SSSL") (nanochat/gpt.py:285-312);
  two consecutive decode steps, so the second runs on the cache the first appended to.
- C5, GQA 16/4 mixed batch: B=64, cache 16384, Zipf(1.2) lengths (numpy RandomState(0), clipped to
  [128, 14336]); rows 0-47 decode one token and rows 48-63 append a 128-token chunk (causal inside
  the chunk).  Once as two calls on row-slice views of the cache (the reference's call shape) and
  once as one varlen call (cu_seqlens_q over the packed tokens).

Reference: the oracle (nanochat/flash_attention.py:155-177 + :69-102 applied row by row) in fp32 on
the CPU from the same seeded inputs.  Tolerance: bf16 caches, max rel err <= 2e-2 against fp32 and
torch.allclose(atol=1e-2, rtol=1e-2).  Caches are compared bit for bit as whole tensors after every
call, so a stray or missing write anywhere in the 1 GB of C5 cache fails.
"""
import numpy as np
import pytest
import torch

from nanochat_amd import _ext
from nanochat_amd.flash_attention import flash_attn
from oracle import kvcache_oracle as orc
from tests.helpers import bits, gen, max_rel_err, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF16 = torch.bfloat16


def _filled(g, B, T_max, H_kv, D, seqlens):
    kc = torch.zeros(B, T_max, H_kv, D, dtype=BF16)
    vc = torch.zeros_like(kc)
    for b, s in enumerate(seqlens):
        kc[b, :s] = randn((s, H_kv, D), g, BF16)
        vc[b, :s] = randn((s, H_kv, D), g, BF16)
    return kc, vc


def _close(out, ref):
    err = max_rel_err(out, ref.float())
    assert err <= 2e-2, f"max rel err {err:.3e}"
    assert torch.allclose(out.float().cpu(), ref.float(), atol=1e-2, rtol=1e-2)


def _sync_region_is_zero():
    torch.cuda.synchronize()
    for buf in list(_ext._workspaces.values()):
        assert int(buf[:_ext.NC_WORKSPACE_SYNC_BYTES].count_nonzero()) == 0


@pytest.mark.parametrize("window", [1024, 4096])
def test_c4_d26_sssl_decode_layer(window):
    B, H, D, T_max, s0 = 8, 13, 128, 4096, 3072
    g = gen(4000 + window)
    kc, vc = _filled(g, B, T_max, H, D, [s0] * B)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    sl = torch.full((B,), s0, dtype=torch.int32)
    sl_d = sl.to(DEV)
    for step in range(2):
        q, k, v = (randn((B, 1, H, D), g, BF16) for _ in range(3))
        out = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc_d, vc_d, k=k.to(DEV), v=v.to(DEV), cache_seqlens=sl_d,
                                                 causal=True, window_size=(window, 0))
        ref = orc.flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=sl, causal=True,
                                          window_size=(window, 0), compute_dtype=torch.float32)
        _close(out, ref)
        assert torch.equal(bits(kc_d), bits(kc)) and torch.equal(bits(vc_d), bits(vc)), f"step {step}: caches"
        assert torch.equal(sl_d.cpu(), sl)
        _sync_region_is_zero()
        sl += 1
        sl_d += 1


C5_B, C5_H, C5_HKV, C5_D, C5_T, C5_C, C5_ND = 64, 16, 4, 128, 16384, 128, 48


def _c5_inputs():
    rs = np.random.RandomState(0)
    seqlens = np.clip(rs.zipf(1.2, C5_B), 128, C5_T - 16 * C5_C).astype(np.int32)
    g = gen(5000)
    kc, vc = _filled(g, C5_B, C5_T, C5_HKV, C5_D, seqlens.tolist())
    n_tok = C5_ND + (C5_B - C5_ND) * C5_C
    q = randn((n_tok, C5_H, C5_D), g, BF16)       # packed: 48 decode tokens, then 16 rows x 128
    k = randn((n_tok, C5_HKV, C5_D), g, BF16)
    v = randn((n_tok, C5_HKV, C5_D), g, BF16)
    return torch.from_numpy(seqlens), kc, vc, q, k, v


def _c5_oracle(sl, kc, vc, q, k, v):
    """The reference's two calls (decode rows, chunk rows) on row slices of the CPU caches."""
    nd = C5_ND
    dec = orc.flash_attn_with_kvcache(q[:nd, None], kc[:nd], vc[:nd], k=k[:nd, None], v=v[:nd, None],
                                      cache_seqlens=sl[:nd], causal=True, window_size=(-1, 0),
                                      compute_dtype=torch.float32)
    rows = C5_B - nd
    chk = orc.flash_attn_with_kvcache(q[nd:].view(rows, C5_C, C5_H, C5_D), kc[nd:], vc[nd:],
                                      k=k[nd:].view(rows, C5_C, C5_HKV, C5_D),
                                      v=v[nd:].view(rows, C5_C, C5_HKV, C5_D), cache_seqlens=sl[nd:],
                                      causal=True, window_size=(-1, 0), compute_dtype=torch.float32)
    return dec, chk


@pytest.fixture(scope="module")
def c5_case():
    sl, kc, vc, q, k, v = _c5_inputs()
    kc_ref, vc_ref = kc.clone(), vc.clone()
    dec, chk = _c5_oracle(sl, kc_ref, vc_ref, q, k, v)
    return sl, kc, vc, q, k, v, kc_ref, vc_ref, dec, chk


def test_c5_gqa_mixed_batch_two_calls(c5_case):
    sl, kc, vc, q, k, v, kc_ref, vc_ref, dec_ref, chk_ref = c5_case
    nd, rows = C5_ND, C5_B - C5_ND
    kc_d, vc_d, sl_d = kc.to(DEV), vc.to(DEV), sl.to(DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    dec = flash_attn.flash_attn_with_kvcache(qd[:nd, None], kc_d[:nd], vc_d[:nd], k=kd[:nd, None],
                                             v=vd[:nd, None], cache_seqlens=sl_d[:nd], causal=True,
                                             window_size=(-1, 0))
    chk = flash_attn.flash_attn_with_kvcache(qd[nd:].view(rows, C5_C, C5_H, C5_D), kc_d[nd:], vc_d[nd:],
                                             k=kd[nd:].view(rows, C5_C, C5_HKV, C5_D),
                                             v=vd[nd:].view(rows, C5_C, C5_HKV, C5_D), cache_seqlens=sl_d[nd:],
                                             causal=True, window_size=(-1, 0))
    _close(dec, dec_ref)
    _close(chk, chk_ref)
    assert torch.equal(bits(kc_d), bits(kc_ref)) and torch.equal(bits(vc_d), bits(vc_ref))
    assert torch.equal(sl_d.cpu(), sl)
    _sync_region_is_zero()


def test_c5_gqa_mixed_batch_one_varlen_call(c5_case):
    sl, kc, vc, q, k, v, kc_ref, vc_ref, dec_ref, chk_ref = c5_case
    nd = C5_ND
    lens = torch.tensor([1] * nd + [C5_C] * (C5_B - nd), dtype=torch.int32)
    cu = torch.cat([torch.zeros(1, dtype=torch.int32), lens.cumsum(0).to(torch.int32)])
    kc_d, vc_d, sl_d = kc.to(DEV), vc.to(DEV), sl.to(DEV)
    out = flash_attn.flash_attn_with_kvcache(q.to(DEV), kc_d, vc_d, k=k.to(DEV), v=v.to(DEV), cache_seqlens=sl_d,
                                             causal=True, window_size=(-1, 0), cu_seqlens_q=cu.to(DEV),
                                             max_seqlen_q=C5_C)
    assert out.shape == q.shape
    _close(out[:nd], dec_ref[:, 0])
    _close(out[nd:], chk_ref.reshape(-1, C5_H, C5_D))
    assert torch.equal(bits(kc_d), bits(kc_ref)) and torch.equal(bits(vc_d), bits(vc_ref))
    _sync_region_is_zero()
