"""Pins of the CPU oracle (oracle/kvcache_oracle.py), CPU only.

Every oracle function is checked against something that does not retype its
formula: an fp64 key-by-key brute force, closed forms, the reference's own
known-answer test (tests/test_engine.py:124-155 of nanochat), and invariants.
A planted-mistake test shows the brute-force check catches an off-by-one.
"""
import math

import numpy as np
import pytest
import torch

from oracle import kvcache_oracle as orc
from tests.helpers import brute_attention, gen, randn


def _case(seed, B, T_new, H, H_kv, D, T_max, seqlens, dtype=torch.float64):
    g = gen(seed)
    q = randn((B, T_new, H, D), g, dtype)
    k = randn((B, T_new, H_kv, D), g, dtype)
    v = randn((B, T_new, H_kv, D), g, dtype)
    kc = torch.zeros(B, T_max, H_kv, D, dtype=dtype)
    vc = torch.zeros(B, T_max, H_kv, D, dtype=dtype)
    for b, s in enumerate(seqlens):
        kc[b, :s] = randn((s, H_kv, D), g, dtype)
        vc[b, :s] = randn((s, H_kv, D), g, dtype)
    sl = torch.tensor(seqlens, dtype=torch.int32)
    return q, k, v, kc, vc, sl


CASES = [
    # (B, T_new, H, H_kv, D, T_max, seqlens, window)
    (2, 1, 4, 4, 8, 40, [16, 16], -1),          # decode, uniform
    (3, 1, 4, 2, 8, 40, [0, 7, 31], -1),        # decode, ragged, GQA 2:1, empty row
    (3, 1, 4, 4, 8, 40, [5, 20, 33], 8),        # decode, window < Tk
    (2, 5, 6, 2, 8, 40, [0, 11], -1),           # chunk into empty and non-empty cache
    (2, 5, 4, 4, 8, 40, [3, 17], 4),            # chunk with window
    (1, 6, 4, 1, 8, 16, [0], 40),               # Tq == Tk, window >= Tq: plain causal branch
    (1, 6, 2, 2, 8, 16, [0], 2),                # Tq == Tk, window < Tq: explicit mask branch
]


@pytest.mark.parametrize("B,T_new,H,H_kv,D,T_max,seqlens,window", CASES)
def test_oracle_matches_fp64_brute_force(B, T_new, H, H_kv, D, T_max, seqlens, window):
    q, k, v, kc, vc, sl = _case(1, B, T_new, H, H_kv, D, T_max, seqlens)
    out = orc.flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=sl, causal=True,
                                      window_size=(window, 0))
    ref = brute_attention(q.numpy(), kc.numpy(), vc.numpy(), seqlens, window)
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-10, atol=1e-10)


def test_oracle_append_closed_form():
    """Appended tokens land at [s_b, s_b + T_new) of their row; nothing else changes."""
    B, T_new, H_kv, D, T_max = 3, 4, 2, 4, 16
    seqlens = [0, 5, 12]
    kc = torch.full((B, T_max, H_kv, D), -1.0)
    vc = torch.full((B, T_max, H_kv, D), -2.0)
    # code(b, t, h, d) makes every appended element distinct
    code = torch.arange(B * T_new * H_kv * D, dtype=torch.float32).view(B, T_new, H_kv, D)
    orc.kv_append(kc, vc, code, code + 1000, torch.tensor(seqlens, dtype=torch.int32))
    for b in range(B):
        for pos in range(T_max):
            t = pos - seqlens[b]
            if 0 <= t < T_new:
                assert torch.equal(kc[b, pos], code[b, t])
                assert torch.equal(vc[b, pos], code[b, t] + 1000)
            else:
                assert (kc[b, pos] == -1.0).all() and (vc[b, pos] == -2.0).all()


def test_oracle_cache_written_by_attention_call():
    q, k, v, kc, vc, sl = _case(2, 2, 3, 4, 2, 8, 20, [4, 9])
    kc0, vc0 = kc.clone(), vc.clone()
    orc.flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=sl, window_size=(-1, 0))
    for b, s in enumerate([4, 9]):
        assert torch.equal(kc[b, s:s + 3], k[b]) and torch.equal(vc[b, s:s + 3], v[b])
        assert torch.equal(kc[b, :s], kc0[b, :s]) and torch.equal(kc[b, s + 3:], kc0[b, s + 3:])
    assert torch.equal(sl, torch.tensor([4, 9], dtype=torch.int32)), "cache_seqlens must not move"


def test_single_key_returns_v_exactly():
    """s = 0, T_new = 1: softmax over one key is 1, so the output is v itself."""
    q, k, v, kc, vc, sl = _case(3, 2, 1, 4, 2, 8, 8, [0, 0], dtype=torch.float32)
    out = orc.flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=sl)
    expect = v.repeat_interleave(2, dim=2)
    assert torch.equal(out, expect)


def test_constant_keys_average_values():
    """All keys equal: the weights are uniform over the visible window."""
    B, H, D, T_max, s, w = 1, 2, 8, 32, 20, 5
    g = gen(4)
    q = randn((B, 1, H, D), g, torch.float64)
    kc = torch.ones(B, T_max, H, D, dtype=torch.float64)
    vc = randn((B, T_max, H, D), g, torch.float64)
    k = torch.ones(B, 1, H, D, dtype=torch.float64)
    v = randn((B, 1, H, D), g, torch.float64)
    out = orc.flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=torch.tensor([s], dtype=torch.int32),
                                      window_size=(w, 0))
    expect = vc[0, s - w:s + 1].mean(dim=0)
    torch.testing.assert_close(out[0, 0], expect, rtol=1e-12, atol=1e-12)


def test_window_covering_everything_equals_full():
    q, k, v, kc, vc, sl = _case(5, 2, 3, 4, 4, 8, 30, [10, 20])
    a = orc.flash_attn_with_kvcache(q, kc.clone(), vc.clone(), k=k, v=v, cache_seqlens=sl, window_size=(-1, 0))
    b = orc.flash_attn_with_kvcache(q, kc.clone(), vc.clone(), k=k, v=v, cache_seqlens=sl, window_size=(10_000, 0))
    torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)


def test_gqa_equals_repeated_mha():
    q, k, v, kc, vc, sl = _case(6, 2, 2, 8, 2, 8, 24, [3, 15])
    gqa = orc.flash_attn_with_kvcache(q, kc.clone(), vc.clone(), k=k, v=v, cache_seqlens=sl, window_size=(6, 0))
    rep = lambda t: t.repeat_interleave(4, dim=2)
    mha = orc.flash_attn_with_kvcache(q, rep(kc), rep(vc), k=rep(k), v=rep(v), cache_seqlens=sl, window_size=(6, 0))
    torch.testing.assert_close(gqa, mha, rtol=1e-12, atol=1e-12)


def test_chunk_equals_sequential_decode():
    """Appending T tokens at once equals appending them one at a time."""
    q, k, v, kc, vc, sl = _case(7, 2, 6, 4, 2, 8, 30, [4, 9])
    kc2, vc2 = kc.clone(), vc.clone()
    chunk = orc.flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=sl, window_size=(5, 0))
    steps = []
    pos = sl.clone()
    for t in range(6):
        steps.append(orc.flash_attn_with_kvcache(q[:, t:t + 1], kc2, vc2, k=k[:, t:t + 1], v=v[:, t:t + 1],
                                                 cache_seqlens=pos, window_size=(5, 0)))
        pos = pos + 1
    torch.testing.assert_close(chunk, torch.cat(steps, dim=1), rtol=1e-12, atol=1e-12)
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)


def test_uniform_batch_matches_reference_fallback_shape_of_computation():
    """For a uniform batch the row-by-row oracle equals one batched fallback call."""
    q, k, v, kc, vc, sl = _case(8, 3, 4, 4, 2, 8, 24, [7, 7, 7])
    per_row = orc.flash_attn_with_kvcache(q, kc.clone(), vc.clone(), k=k, v=v, cache_seqlens=sl,
                                          window_size=(3, 0))
    # the reference's batched form: one position for all rows (flash_attention.py:157-177)
    kb, vb = kc.clone(), vc.clone()
    kb[:, 7:11] = k
    vb[:, 7:11] = v
    y = orc.sdpa_attention(q.transpose(1, 2), kb[:, :11].transpose(1, 2), vb[:, :11].transpose(1, 2), (3, 0), True)
    torch.testing.assert_close(per_row, y.transpose(1, 2), rtol=1e-12, atol=1e-12)


def test_mixed_dtype_rounds_on_store():
    """fp32 k/v into a bf16 cache: stored values are torch's RNE casts."""
    q, k, v, kc, vc, sl = _case(9, 2, 1, 2, 2, 8, 8, [2, 5], dtype=torch.float32)
    kcb, vcb = kc.to(torch.bfloat16), vc.to(torch.bfloat16)
    orc.flash_attn_with_kvcache(q, kcb, vcb, k=k, v=v, cache_seqlens=sl)
    assert torch.equal(kcb[0, 2], k[0, 0].to(torch.bfloat16))
    assert torch.equal(vcb[1, 5], v[1, 0].to(torch.bfloat16))


def test_brute_force_detects_planted_window_off_by_one(monkeypatch):
    """Plant an off-by-one (window+2 keys) in the oracle; the brute-force pin must fail."""
    orig = orc.sdpa_attention

    def planted(q, k, v, window_size, enable_gqa):
        w = window_size[0]
        return orig(q, k, v, (w + 1 if w >= 0 else w, 0), enable_gqa)

    monkeypatch.setattr(orc, "sdpa_attention", planted)
    q, k, v, kc, vc, sl = _case(10, 2, 1, 4, 4, 8, 40, [20, 30])
    out = orc.flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=sl, window_size=(6, 0))
    ref = brute_attention(q.numpy(), kc.numpy(), vc.numpy(), [20, 30], 6)
    assert not np.allclose(out.numpy(), ref, rtol=1e-6, atol=1e-6)


def test_brute_force_detects_planted_gqa_mapping(monkeypatch):
    """Plant a wrong GQA head map (h -> h % H_kv instead of h // G); the pin must fail."""
    orig = orc.sdpa_attention

    def planted(q, k, v, window_size, enable_gqa):
        if enable_gqa:
            G = q.size(1) // k.size(1)
            k, v = k.repeat(1, G, 1, 1), v.repeat(1, G, 1, 1)
        return orig(q, k, v, window_size, False)

    q, k, v, kc, vc, sl = _case(11, 1, 1, 4, 2, 8, 16, [9])
    kc_ref, vc_ref = kc.clone(), vc.clone()
    orc.kv_append(kc_ref, vc_ref, k, v, sl)
    ref = brute_attention(q.numpy(), kc_ref.numpy(), vc_ref.numpy(), [9], -1)
    good = orc.flash_attn_with_kvcache(q, kc.clone(), vc.clone(), k=k, v=v, cache_seqlens=sl)
    np.testing.assert_allclose(good.numpy(), ref, rtol=1e-10, atol=1e-10)
    monkeypatch.setattr(orc, "sdpa_attention", planted)
    wrong = orc.flash_attn_with_kvcache(q, kc.clone(), vc.clone(), k=k, v=v, cache_seqlens=sl)
    assert not np.allclose(wrong.numpy(), ref, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------------------
# KVCache: nanochat's own tests (tests/test_engine.py:84-155) on the oracle cache
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("T_new,with_kv", [(1, True), (5, True), (3, False)])
def test_cache_batch_idx_is_a_row_permutation_of_the_cache(T_new, with_kv):
    """FA3's cache_batch_idx: attending batch row b on cache row idx[b] equals attending on the
    gathered cache C[idx] without indices; appends land in rows idx[b]; other rows are untouched."""
    g = gen(401 + T_new)
    Bc, B, T_max, H, H_kv, D = 5, 3, 24, 4, 2, 16
    idx = torch.tensor([4, 0, 2], dtype=torch.int32)
    kc = randn((Bc, T_max, H_kv, D), g, torch.float32)
    vc = randn((Bc, T_max, H_kv, D), g, torch.float32)
    q = randn((B, T_new, H, D), g, torch.float32)
    k = randn((B, T_new, H_kv, D), g, torch.float32) if with_kv else None
    v = randn((B, T_new, H_kv, D), g, torch.float32) if with_kv else None
    sl = torch.tensor([7, 0, 19], dtype=torch.int32)
    kc1, vc1 = kc.clone(), vc.clone()
    out1 = orc.flash_attn_with_kvcache(q, kc1, vc1, k=k, v=v, cache_seqlens=sl, causal=True,
                                       window_size=(6, 0), cache_batch_idx=idx)
    kc2, vc2 = kc[idx.long()].clone(), vc[idx.long()].clone()
    out2 = orc.flash_attn_with_kvcache(q, kc2, vc2, k=k, v=v, cache_seqlens=sl, causal=True, window_size=(6, 0))
    assert torch.equal(out1, out2)
    assert torch.equal(kc1[idx.long()], kc2) and torch.equal(vc1[idx.long()], vc2)
    for r in (1, 3):
        assert torch.equal(kc1[r], kc[r]) and torch.equal(vc1[r], vc[r])


def test_varlen_uniform_lengths_equal_the_fixed_length_call():
    """cu_seqlens_q with every row holding T tokens is the (B, T, ...) call on flattened tokens."""
    g = gen(410)
    B, T, T_max, H, H_kv, D = 3, 4, 30, 4, 2, 16
    q, k, v = (randn((B, T, h, D), g, torch.float32) for h in (H, H_kv, H_kv))
    kc, vc = randn((B, T_max, H_kv, D), g, torch.float32), randn((B, T_max, H_kv, D), g, torch.float32)
    sl = torch.tensor([3, 0, 20], dtype=torch.int32)
    cu = torch.arange(0, (B + 1) * T, T, dtype=torch.int32)
    kc1, vc1, kc2, vc2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    o1 = orc.flash_attn_with_kvcache(q.reshape(B * T, H, D), kc1, vc1, k=k.reshape(B * T, H_kv, D),
                                     v=v.reshape(B * T, H_kv, D), cache_seqlens=sl, causal=True,
                                     window_size=(5, 0), cu_seqlens_q=cu)
    o2 = orc.flash_attn_with_kvcache(q, kc2, vc2, k=k, v=v, cache_seqlens=sl, causal=True, window_size=(5, 0))
    assert torch.equal(o1, o2.reshape(B * T, H, D))
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)


def test_varlen_mixed_lengths_equal_one_call_per_row():
    """Rows of 0, 1 and several tokens: each row's output and appends equal a B=1 call of its own."""
    g = gen(411)
    lens, T_max, H, H_kv, D = [2, 0, 1, 5], 40, 4, 4, 8
    cu = torch.tensor([0, 2, 2, 3, 8], dtype=torch.int32)
    total = int(cu[-1])
    q, k, v = (randn((total, h, D), g, torch.float32) for h in (H, H_kv, H_kv))
    kc, vc = randn((4, T_max, H_kv, D), g, torch.float32), randn((4, T_max, H_kv, D), g, torch.float32)
    sl = torch.tensor([7, 30, 0, 11], dtype=torch.int32)
    kc1, vc1 = kc.clone(), vc.clone()
    out = orc.flash_attn_with_kvcache(q, kc1, vc1, k=k, v=v, cache_seqlens=sl, causal=True, cu_seqlens_q=cu)
    assert out.shape == (total, H, D)
    for b, n in enumerate(lens):
        a = int(cu[b])
        kb, vb = kc[b:b + 1].clone(), vc[b:b + 1].clone()
        if n:
            ob = orc.flash_attn_with_kvcache(q[a:a + n][None], kb, vb, k=k[a:a + n][None], v=v[a:a + n][None],
                                             cache_seqlens=sl[b:b + 1], causal=True)
            assert torch.equal(out[a:a + n], ob[0])
        assert torch.equal(kc1[b], kb[0]) and torch.equal(vc1[b], vb[0])


def test_oracle_kv_cache_basic():
    c = orc.KVCache(batch_size=2, num_heads=3, seq_len=64, head_dim=5, num_layers=6, device="cpu", dtype=torch.float32)
    assert c.get_pos() == 0
    assert c.k_cache.shape == (6, 2, 64, 3, 5) and c.v_cache.shape == (6, 2, 64, 3, 5)
    c.advance(10)
    assert c.get_pos() == 10
    c.advance(5)
    assert c.get_pos() == 15
    c.reset()
    assert c.get_pos() == 0
    k0, v0 = c.get_layer_cache(0)
    assert k0.shape == (2, 64, 3, 5) and v0.shape == (2, 64, 3, 5)


def test_oracle_kv_cache_prefill_known_answer():
    """nanochat tests/test_engine.py:124-155: 1.0 / 2.0 fill copied through prefill."""
    src = orc.KVCache(batch_size=1, num_heads=4, seq_len=32, head_dim=8, num_layers=2, device="cpu", dtype=torch.float32)
    src.k_cache[0, 0, :16, :, :] = 1.0
    src.v_cache[0, 0, :16, :, :] = 2.0
    src.advance(16)
    dst = orc.KVCache(batch_size=1, num_heads=4, seq_len=64, head_dim=8, num_layers=2, device="cpu", dtype=torch.float32)
    dst.prefill(src)
    assert dst.get_pos() == 16
    assert (dst.k_cache[0, 0, :16] == 1.0).all() and (dst.v_cache[0, 0, :16] == 2.0).all()
    assert (dst.k_cache[:, :, 16:] == 0).all() and (dst.k_cache[1] == 0).all()


def test_oracle_prefill_preconditions():
    a = orc.KVCache(1, 2, 8, 4, 1, "cpu", torch.float32)
    b = orc.KVCache(1, 2, 4, 4, 1, "cpu", torch.float32)
    with pytest.raises(AssertionError):
        b.prefill(a)  # destination shorter than source
    a.advance(1)
    with pytest.raises(AssertionError):
        a.prefill(b)  # destination not empty


# ---------------------------------------------------------------------------
# Window sizes (nanochat/gpt.py:285-312) against closed forms
# ---------------------------------------------------------------------------
def test_window_sizes_closed_form():
    # short window = ceil(seq / 4 / 128) * 128; the last layer is always long
    w = orc.compute_window_sizes(2048, "SSSL", 24)
    assert [x[0] for x in w] == ([512, 512, 512, 2048] * 6)
    w = orc.compute_window_sizes(4096, "SSSL", 26)
    assert sum(1 for x in w if x[0] == 1024) == 19 and sum(1 for x in w if x[0] == 4096) == 7
    assert w[-1] == (4096, 0) and w[-2] == (1024, 0)
    assert orc.compute_window_sizes(1024, "L", 12) == [(1024, 0)] * 12
    assert orc.compute_window_sizes(1000, "S", 3) == [(256, 0), (256, 0), (1000, 0)]
    assert orc.compute_window_sizes(2048, "SL", 4) == [(512, 0), (2048, 0), (512, 0), (2048, 0)]


def test_decode_bytes_closed_form():
    # 20 layers x sum_b 5120 (s_b + 3) for d20 shapes (10/10 heads x 128, bf16)
    s = [512, 1000, 2047]
    assert orc.decode_bytes(s, 20, 10, 10, 128, 2) == 20 * sum(5120 * (x + 3) for x in s)
    # a window caps the keys at w + 1
    assert orc.decode_bytes([100], 1, 1, 1, 128, 2, windows=[9]) == 512 * 10 + 512 + 512
    assert math.isclose(orc.softmax_scale(128), 128 ** -0.5)


# ---- the QK prologue (rotary, RMS norm, x1.2): nanochat/gpt.py:42-43,57-63,98-102,268-283 ----
def _complex_rotary(x, cos, sin):
    """Closed form: (x1 + i x2) * exp(-i theta) with cos/sin of theta."""
    d = x.shape[3] // 2
    z = torch.complex(x[..., :d].double(), x[..., d:].double()) * torch.complex(cos.double(), -sin.double())
    return torch.cat([z.real, z.imag], 3)


def test_rotary_tables_closed_form():
    cos, sin = orc.rotary_tables(64, 16, dtype=torch.float64)
    assert cos.shape == (64, 8)
    assert torch.equal(cos[0], torch.ones(8, dtype=torch.float64)) and torch.equal(sin[0], torch.zeros(8, dtype=torch.float64))
    t, i = 37, 3
    theta = t * 100000.0 ** (-(2 * i) / 16)
    assert abs(cos[t, i].item() - math.cos(theta)) < 1e-6 and abs(sin[t, i].item() - math.sin(theta)) < 1e-6


def test_rotary_equals_complex_rotation_and_preserves_pair_norms():
    g = gen(60)
    x = torch.randn(2, 5, 3, 16, generator=g, dtype=torch.float64)
    cos_t, sin_t = orc.rotary_tables(40, 16, dtype=torch.float64)
    pos = torch.tensor([0, 31])
    idx = pos[:, None] + torch.arange(5)[None, :]
    cos, sin = cos_t[idx][:, :, None, :], sin_t[idx][:, :, None, :]
    y = orc.rotary(x, cos, sin)
    assert torch.allclose(y, _complex_rotary(x, cos, sin), atol=1e-12)
    pair = lambda z: z[..., :8] ** 2 + z[..., 8:] ** 2  # noqa: E731
    assert torch.allclose(pair(y), pair(x), atol=1e-12)
    assert torch.allclose(y[0, 0], x[0, 0])  # position 0 is the identity
    # rotations compose: angle a then angle b equals angle a + b (tables are built in fp32, as the reference's)
    a, b = 3, 11
    ya = orc.rotary(x, cos_t[a], sin_t[a])
    assert torch.allclose(orc.rotary(ya, cos_t[b], sin_t[b]), orc.rotary(x, cos_t[a + b], sin_t[a + b]), atol=1e-5)


def test_qk_prologue_normalises_and_scales():
    g = gen(61)
    x = torch.randn(3, 4, 2, 32, generator=g, dtype=torch.float64) * 3.0
    cos_t, sin_t = orc.rotary_tables(64, 32, dtype=torch.float64)
    pos = torch.tensor([0, 5, 40])
    eps = 1e-3
    y = orc.qk_prologue(x, cos_t, sin_t, pos, scale=1.2, eps=eps)
    idx = pos[:, None] + torch.arange(4)[None, :]
    r = _complex_rotary(x, cos_t[idx][:, :, None, :], sin_t[idx][:, :, None, :])
    ms = (r ** 2).mean(-1, keepdim=True)
    assert torch.allclose(y, 1.2 * r / torch.sqrt(ms + eps), atol=1e-12)
    assert torch.allclose((y / 1.2).pow(2).mean(-1), (ms / (ms + eps)).squeeze(-1), atol=1e-12)


def test_qk_prologue_detects_planted_sign_mistake(monkeypatch):
    g = gen(62)
    x = torch.randn(1, 3, 1, 8, generator=g, dtype=torch.float64)
    cos_t, sin_t = orc.rotary_tables(16, 8, dtype=torch.float64)
    pos = torch.tensor([4])
    idx = pos[:, None] + torch.arange(3)[None, :]
    ref = _complex_rotary(x, cos_t[idx][:, :, None, :], sin_t[idx][:, :, None, :])

    def wrong(x, cos, sin):
        d = x.shape[3] // 2
        x1, x2 = x[..., :d], x[..., d:]
        return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], 3)  # rotation the other way

    monkeypatch.setattr(orc, "rotary", wrong)
    out = orc.rotary(x, cos_t[idx][:, :, None, :], sin_t[idx][:, :, None, :])
    assert not torch.allclose(out, ref, atol=1e-6)


@pytest.mark.parametrize("T_new,with_kv,P", [(1, True, 16), (5, True, 32), (3, False, 16)])
def test_paged_cache_is_a_block_shuffle_of_the_dense_cache(T_new, with_kv, P):
    """A dense (B, T, H_kv, D) cache cut into P-token blocks and stored in a shuffled pool (with
    spare blocks) gives the dense call's outputs, and the pool read back through the table
    equals the dense cache after the call (append included)."""
    g = gen(50 + T_new + P)
    B, H, H_kv, D, nb = 3, 4, 2, 16, 4
    T = nb * P
    q = randn((B, T_new, H, D), g)
    kd = randn((B, T, H_kv, D), g)
    vd = randn((B, T, H_kv, D), g)
    k = randn((B, T_new, H_kv, D), g) if with_kv else None
    v = randn((B, T_new, H_kv, D), g) if with_kv else None
    seqlens = torch.tensor([0, 17, T - T_new], dtype=torch.int32)
    perm = torch.randperm(B * nb + 5, generator=g)[:B * nb]          # 5 spare blocks never named
    table = perm.view(B, nb).to(torch.int32)
    kp = torch.full((B * nb + 5, P, H_kv, D), float("nan"))
    vp = torch.full((B * nb + 5, P, H_kv, D), float("nan"))
    orc.dense_to_paged(kd, kp, table)
    orc.dense_to_paged(vd, vp, table)
    y_dense = orc.flash_attn_with_kvcache(q, kd, vd, k=k, v=v, cache_seqlens=seqlens, window_size=(-1, 0))
    y_paged = orc.flash_attn_with_kvcache(q, kp, vp, k=k, v=v, cache_seqlens=seqlens, window_size=(-1, 0),
                                          page_table=table)
    assert torch.equal(y_dense, y_paged)
    assert torch.equal(orc.paged_to_dense(kp, table), kd) and torch.equal(orc.paged_to_dense(vp, table), vd)
    spare = [i for i in range(B * nb + 5) if i not in set(perm.tolist())]
    assert torch.isnan(kp[spare]).all()                                # blocks outside the table untouched
