"""GPU parity of the sampling kernel (nc_sample) with oracle/sampling_oracle.py.

- Greedy: bit-exact token ids with torch.argmax on the GPU (ties, NaN, -0/+0).
- Draws: for the same uniform, the token equals the oracle's float64 inverse-CDF token wherever
  u lies more than 1e-5 from a CDF boundary (closer draws may round either way; at least 95% of
  draws are compared).  Top-k ties at the cut keep lower indices, as the oracle does.
- Distribution: a grid of 4096 uniforms over one row reproduces the reference's probabilities
  (topk + softmax of logits / T, engine.py:146-156) within 2/4096 per token.
"""
import pytest
import torch

from nanochat_amd import _ext
from nanochat_amd.sampling import sample_next_token, sample_with_uniforms
from oracle import sampling_oracle as so
from tests.helpers import gen

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _logits(seed, B, V, scale=3.0):
    g = gen(seed)
    return (torch.randn(B, V, generator=g) * scale).float()


def test_greedy_equals_torch_argmax():
    x = _logits(1, 32, 32768)
    x[3, [100, 2000, 30000]] = 50.0                 # tie of the maximum: first index
    x[4, 777] = float("nan")                        # NaN wins
    x[5, [9, 4000]] = float("nan")                  # first NaN
    x[6] = 0.0
    x[6, 5] = -0.0                                  # -0 == +0: index 0
    x[7, :] = float("-inf")
    xd = x.to(DEV)
    got = sample_with_uniforms(xd, None, 0.0)
    assert torch.equal(got.cpu(), torch.argmax(xd, dim=-1, keepdim=True).cpu())


@pytest.mark.parametrize("V", [1, 50, 1000, 32768, 50257])
def test_greedy_odd_sizes(V):
    x = _logits(2, 5, V).to(DEV)
    assert torch.equal(sample_with_uniforms(x, None, 0.0), torch.argmax(x, dim=-1, keepdim=True))


def _compare_draws(x, u, T, top_k):
    got = sample_with_uniforms(x.to(DEV), u.to(DEV), T, top_k).cpu()[:, 0]
    compared = 0
    for b in range(x.shape[0]):
        row = x[b].numpy()
        if so.boundary_margin(row, float(u[b]), T, top_k) < 3e-6:
            continue
        assert int(got[b]) == so.sample_inverse_cdf(row, float(u[b]), T, top_k), (b, float(u[b]))
        compared += 1
    assert compared >= 0.75 * x.shape[0]


@pytest.mark.parametrize("V,k,T", [(32768, None, 1.0), (50257, None, 0.7), (32768, 200, 1.0), (32768, 1024, 1.5),
                                   (65536, 100, 0.9)])
def test_draws_at_category_midpoints_pick_that_category(V, k, T):
    # u at the middle of a chosen category's CDF interval (float64): the kernel must return it
    x = _logits(30 + V, 32, V)
    g = torch.Generator().manual_seed(V)
    us, want = [], []
    for b in range(32):
        ids, probs = so.reference_probabilities(x[b], T, k)
        c = torch.cumsum(torch.tensor(probs, dtype=torch.float64), 0)
        j = int(torch.multinomial(torch.tensor(probs), 1, generator=g))
        lo = float(c[j - 1]) if j > 0 else 0.0
        us.append((lo + float(c[j])) / 2)
        want.append(int(ids[j]))
    got = sample_with_uniforms(x.to(DEV), torch.tensor(us, dtype=torch.float32).to(DEV), T, k).cpu()[:, 0]
    for b in range(32):
        ids, probs = so.reference_probabilities(x[b], T, k)
        if probs[list(ids).index(want[b])] > 1e-5:   # wide enough for fp32 sums
            assert int(got[b]) == want[b], b


@pytest.mark.parametrize("V,T", [(50, 1.0), (1000, 0.6), (32768, 1.0), (32768, 2.0), (50257, 0.8)])
def test_whole_row_draws_match_oracle(V, T):
    x = _logits(10 + V, 48, V)
    u = torch.rand(48, generator=gen(V))
    _compare_draws(x, u, T, None)


def test_whole_row_draw_at_segment_boundaries():
    """u planted at the boundaries of the kernel's 1024 per-thread segments (32 logits each at
    V = 32768), and one float32 ulp either side: the fp32 segment sums need not tile [0, total)
    exactly, and a target between two segments must still draw a category next to the boundary
    (the last of segment t or the first of segment t + 1), never a far one.  Logits are flat
    enough (N(0, 0.3^2)) that each of those two categories is wider than the fp32 rounding."""
    V, seg = 32768, 32
    row = _logits(12, 1, V, scale=0.3)[0]
    p = torch.softmax(row.double(), 0)
    cum = torch.cumsum(p.view(-1, seg).sum(1), 0)[:-1]        # mass through segment t, t < 1023
    us, seg_of = [], []
    for t, c in enumerate(cum.tolist()):
        for f in (1 - 2 ** -23, 1.0, 1 + 2 ** -23):
            us.append(min(c * f, 1 - 2 ** -24))
            seg_of.append(t)
    u = torch.tensor(us, dtype=torch.float32)
    x = row.to(DEV).expand(len(us), -1)                       # one row, stride 0
    got = sample_with_uniforms(x, u.to(DEV), 1.0, None).cpu()[:, 0]
    for i, t in enumerate(seg_of):
        assert int(got[i]) in (seg * t + seg - 1, seg * (t + 1)), (t, us[i], int(got[i]))


@pytest.mark.parametrize("V,k,T", [(32768, 1, 1.0), (32768, 5, 1.0), (32768, 50, 0.7), (32768, 200, 1.0),
                                   (32768, 1024, 1.3), (1000, 999, 1.0), (300, 64, 0.9), (50257, 50, 1.0),
                                   (65536, 1024, 0.8)])
def test_top_k_draws_match_oracle(V, k, T):
    x = _logits(20 + k, 40, V)
    u = torch.rand(40, generator=gen(k))
    _compare_draws(x, u, T, k)


@pytest.mark.parametrize("V", [4096, 40000])
def test_top_k_ties_at_the_cut_keep_lower_indices(V):
    x = torch.zeros(64, V)
    x[:, [5, 700, 701, 3000, V - 1]] = 2.0          # 5 equal maxima, k = 3: indices 5, 700, 701
    u = (torch.arange(64, dtype=torch.float32) + 0.5) / 64
    got = sample_with_uniforms(x.to(DEV), u.to(DEV), 1.0, 3).cpu()[:, 0]
    assert set(got.tolist()) == {5, 700, 701}
    for b in range(64):
        assert int(got[b]) == so.sample_inverse_cdf(x[b].numpy(), float(u[b]), 1.0, 3)


@pytest.mark.parametrize("T,top_k", [(1.0, None), (0.7, 20)])
def test_grid_of_uniforms_reproduces_reference_distribution(T, top_k):
    n = 4096
    row = _logits(7, 1, 300, scale=1.5)[0]
    x = row.expand(n, -1).contiguous()
    u = (torch.arange(n, dtype=torch.float32) + 0.5) / n
    got = sample_with_uniforms(x.to(DEV), u.to(DEV), T, top_k).cpu()[:, 0]
    ids, probs = so.reference_probabilities(row, T, top_k)
    counts = torch.bincount(got, minlength=300)
    assert set(torch.nonzero(counts)[:, 0].tolist()) <= set(int(i) for i in ids)
    for i, p in zip(ids, probs):
        assert abs(int(counts[int(i)]) / n - p) <= 2.0 / n, (int(i), p)


def test_nan_never_drawn_and_all_inf_row_flags():
    _ext.read_and_clear_device_errors(torch.device(DEV, 0))
    x = _logits(8, 64, 500)
    x[:, ::3] = float("nan")
    x[63, :] = float("-inf")
    u = torch.rand(64, generator=gen(8))
    xd = x.to(DEV)
    got = sample_with_uniforms(xd, u.to(DEV), 1.0, None).cpu()[:, 0]
    assert all(int(t) % 3 != 0 for t in got[:63])
    assert int(got[63]) == 0
    got_k = sample_with_uniforms(xd, u.to(DEV), 1.0, 10).cpu()[:, 0]
    assert all(int(t) % 3 != 0 for t in got_k[:63])
    assert _ext.read_and_clear_device_errors(xd.device) & _ext.NC_DEVERR_SAMPLE


def test_expanded_logits_broadcast_one_row():
    row = _logits(11, 1, 32768)
    x = row.to(DEV).expand(16, -1)                 # row stride 0, as Engine.generate's first step
    u = torch.rand(16, generator=gen(11))
    got = sample_with_uniforms(x, u.to(DEV), 1.0, 50).cpu()[:, 0]
    want = sample_with_uniforms(x.contiguous(), u.to(DEV), 1.0, 50).cpu()[:, 0]
    assert torch.equal(got, want)


def test_sample_next_token_api_and_graph_replay():
    x = _logits(9, 16, 32768).to(DEV)
    rng = torch.Generator(device=DEV)
    rng.manual_seed(0)
    t = sample_next_token(x, rng, temperature=0.0)
    assert t.shape == (16, 1) and t.dtype == torch.int64
    assert torch.equal(t, torch.argmax(x, dim=-1, keepdim=True))
    # captured with a uniforms buffer refilled between replays: every replay equals the eager call
    u = torch.empty(16, device=DEV)
    out = torch.empty((16, 1), dtype=torch.int64, device=DEV)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        u.uniform_()
        sample_with_uniforms(x, u, 1.0, 50, out=out)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            sample_with_uniforms(x, u, 1.0, 50, out=out)
        for i in range(4):
            u.copy_(torch.rand(16, generator=gen(100 + i)).to(DEV))
            g.replay()
            s.synchronize()
            assert torch.equal(out, sample_with_uniforms(x, u, 1.0, 50))
