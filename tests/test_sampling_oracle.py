"""Pins of oracle/sampling_oracle.py (CPU): the restated sampler against the reference's own
distribution (engine.py:141-156: topk, softmax of logits / T), closed forms, and planted mistakes.

A grid of N evenly spaced uniforms u_i = (i + 0.5) / N through an inverse CDF gives every
category a count within 1 of N * p: the grid test compares those counts with the reference's
probabilities, so a sampler that ignores the temperature, skips the top-k cut or is off by one
category fails it.
"""
import numpy as np
import pytest
import torch

from oracle import sampling_oracle as so
from tests.helpers import gen

N_GRID = 20000


def _grid_counts(row, T, top_k, sampler=so.sample_inverse_cdf):
    counts = {}
    for i in range(N_GRID):
        t = sampler(row, (i + 0.5) / N_GRID, T, top_k)
        counts[t] = counts.get(t, 0) + 1
    return counts


def _check_grid(row, T, top_k, sampler=so.sample_inverse_cdf):
    ids, probs = so.reference_probabilities(torch.as_tensor(row), T, top_k)
    counts = _grid_counts(row, T, top_k, sampler)
    assert set(counts) <= set(int(i) for i in ids)
    for i, p in zip(ids, probs):
        assert abs(counts.get(int(i), 0) / N_GRID - p) <= 1.0 / N_GRID + 1e-12, (int(i), p)


@pytest.mark.parametrize("T,top_k", [(1.0, None), (0.7, None), (1.6, None), (1.0, 5), (0.6, 12), (1.0, 1), (1.0, 60)])
def test_inverse_cdf_grid_reproduces_reference_distribution(T, top_k):
    g = gen(3)
    row = (torch.randn(40, generator=g) * 2.0).numpy().astype(np.float32)
    _check_grid(row, T, top_k)


def test_top_k_of_one_is_argmax_and_top_k_past_vocab_is_whole_row():
    g = gen(4)
    row = torch.randn(100, generator=g).numpy().astype(np.float32)
    for u in (0.0, 0.3, 0.999):
        assert so.sample_inverse_cdf(row, u, 0.8, 1) == int(np.argmax(row))
        assert so.sample_inverse_cdf(row, u, 0.8, 100) == so.sample_inverse_cdf(row, u, 0.8, None)
        assert so.sample_inverse_cdf(row, u, 0.8, 1000) == so.sample_inverse_cdf(row, u, 0.8, None)


def test_closed_forms():
    V = 64
    flat = np.zeros(V, dtype=np.float32)
    for u in (0.01, 0.26, 0.5, 0.77, 0.99):
        assert so.sample_inverse_cdf(flat, u, 1.0) == int(u * V)
    spike = np.zeros(V, dtype=np.float32)
    spike[17] = 100.0
    for u in (1e-6, 0.5, 0.999999):   # the other 63 tokens hold 63 * e^-100 of the mass
        assert so.sample_inverse_cdf(spike, u, 1.0) == 17
    # equal logits at the top-k cut: lower indices are kept (value descending, then index)
    tie = np.zeros(V, dtype=np.float32)
    tie[[3, 9, 40]] = 1.0
    assert {so.sample_inverse_cdf(tie, (i + 0.5) / 8, 1.0, 2) for i in range(8)} == {3, 9}


def test_greedy_matches_torch_argmax_on_ties_and_nan():
    rows = [
        [0.0, 2.0, 2.0, 1.0],                       # tie: first index
        [-1.0, float("nan"), 3.0, float("nan")],    # NaN counts as the maximum, first NaN
        [float("-inf")] * 4,
        [-0.0, 0.0, -0.0, 0.0],
    ]
    for r in rows:
        t = torch.tensor([r], dtype=torch.float32)
        assert int(so.greedy(t)[0, 0]) == so.sample_inverse_cdf(np.array(r, np.float32), 0.5, 0.0)
        assert int(torch.argmax(t, dim=-1)) == int(so.greedy(t)[0, 0])


def test_multinomial_draws_follow_the_oracle_distribution():
    from scipy.stats import chisquare
    g = gen(5)
    row = torch.randn(12, generator=g) * 1.5
    ids, probs = so.reference_probabilities(row, 0.9, None)
    gen_t = torch.Generator().manual_seed(0)
    draws = torch.multinomial(torch.tensor(probs), 40000, replacement=True, generator=gen_t).numpy()
    observed = np.bincount(draws, minlength=len(probs))
    counts = _grid_counts(row.numpy(), 0.9, None)
    expected = np.array([counts.get(i, 0) for i in range(len(probs))], dtype=np.float64) / N_GRID * 40000
    assert chisquare(observed, expected * observed.sum() / expected.sum()).pvalue > 1e-4


def test_nan_and_inf_logits_are_never_drawn():
    row = np.array([np.nan, 1.0, -np.inf, 2.0, np.nan], dtype=np.float32)
    drawn = {so.sample_inverse_cdf(row, (i + 0.5) / 200, 1.0) for i in range(200)}
    assert drawn == {1, 3}
    assert so.sample_inverse_cdf(np.full(5, -np.inf, np.float32), 0.3, 1.0) == 0


def test_softcap_closed_form():
    x = torch.tensor([0.0, 1e-3, -1e-3, 15.0, 300.0, -300.0], dtype=torch.bfloat16)
    y = so.softcap_logits(x)
    assert y.dtype == torch.float32
    assert y[0] == 0 and abs(float(y[1]) - float(x[1])) < 1e-8 and float(y[2]) == -float(y[1])
    assert abs(float(y[3]) - 15 * np.tanh(1.0)) < 1e-5
    assert float(y[4]) == 15.0 and float(y[5]) == -15.0


def _ignores_temperature(row, u, T, top_k=None):
    return so.sample_inverse_cdf(row, u, 1.0, top_k)


def _no_top_k(row, u, T, top_k=None):
    return so.sample_inverse_cdf(row, u, T, None)


def _off_by_one(row, u, T, top_k=None):
    ids, v = so._order(np.asarray(row, np.float64), top_k)
    w = np.exp(v / T - (v / T).max())
    c = np.cumsum(w)
    j = min(int(np.searchsorted(c, u * c[-1], side="right")) + 1, len(c) - 1)
    return int(ids[j])


@pytest.mark.parametrize("mistake,T,top_k", [(_ignores_temperature, 0.5, None), (_no_top_k, 1.0, 5),
                                             (_off_by_one, 1.0, None)])
def test_grid_detects_planted_mistakes(mistake, T, top_k):
    g = gen(6)
    row = (torch.randn(30, generator=g) * 2.0).numpy().astype(np.float32)
    with pytest.raises(AssertionError):
        _check_grid(row, T, top_k, sampler=mistake)
