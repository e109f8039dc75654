"""CPU restatement of nanochat's next-token sampling -- TEST INFRASTRUCTURE.

Only tests/ may import this module, as the checker of the HIP sampling kernel
(nc_sample); the product never imports it.

  - reference_probabilities   nanochat/engine.py:141-156 sample_next_token up to the
                              draw, with the reference's own torch ops (topk, softmax
                              of logits / temperature): the categorical distribution the
                              reference's torch.multinomial samples from, as
                              (token ids, probabilities) in torch.topk's order.
  - sample_inverse_cdf        the draw as an inverse-CDF lookup at a given uniform u, in
                              float64: the first category, in the order above, whose
                              running probability exceeds u.  Same distribution as
                              torch.multinomial; torch's own stream of draws is internal
                              to its generator and is not restated.
  - greedy                    engine.py:145 (torch.argmax).
  - softcap_logits            nanochat/gpt.py:468-472, the logits the sampler receives.

Pins (tests/test_sampling_oracle.py): greedy equals torch.argmax on ties and NaN; a grid of uniforms
reproduces reference_probabilities exactly (frequencies within 1/N); top_k = 1 is argmax and
top_k >= vocab is the whole row; closed forms (uniform logits -> floor(u * V), one dominant
logit); torch.multinomial draws with a fixed seed match the distribution by a chi-square test;
planted mistakes (temperature ignored, top-k cut skipped, off by one category) fail the grid
test.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def softcap_logits(logits_lowp: torch.Tensor, softcap: float = 15.0) -> torch.Tensor:
    """gpt.py:470-471: logits.float(), then softcap * tanh(logits / softcap)."""
    x = logits_lowp.float()
    return softcap * torch.tanh(x / softcap)


def greedy(logits: torch.Tensor) -> torch.Tensor:
    """engine.py:145: argmax over the last dim, (B, 1)."""
    return torch.argmax(logits, dim=-1, keepdim=True)


def reference_probabilities(logits_row: torch.Tensor, temperature: float, top_k: int | None):
    """(ids, probs) of the categorical the reference samples from (engine.py:146-156), one row."""
    row = logits_row.float().unsqueeze(0)
    if top_k is not None and top_k > 0:
        k = min(top_k, row.size(-1))
        vals, idx = torch.topk(row, k, dim=-1)
        probs = F.softmax(vals / temperature, dim=-1)
        return idx[0].numpy(), probs[0].double().numpy()
    probs = F.softmax(row / temperature, dim=-1)
    return np.arange(row.size(-1)), probs[0].double().numpy()


def _order(values: np.ndarray, top_k: int | None):
    """Category order of the draw: value descending with ties by index (top-k), else index order."""
    v = values.astype(np.float64)
    v = np.where(np.isnan(v), -np.inf, v)
    n = v.shape[0]
    if top_k is not None and 0 < top_k < n:
        order = np.lexsort((np.arange(n), -v))[:top_k]
        return order, v[order]
    return np.arange(n), v


def sample_inverse_cdf(logits_row, u: float, temperature: float, top_k: int | None = None):
    """Token drawn at uniform u (float64): first category whose running probability exceeds u."""
    values = np.asarray(logits_row, dtype=np.float64)
    if temperature == 0.0:
        return int(np.argmax(values))   # numpy, like torch, takes the first NaN / first maximum
    ids, v = _order(values, top_k)
    finite = np.isfinite(v)
    if not finite.any():
        return 0
    x = v / temperature
    w = np.where(finite, np.exp(x - x[finite].max()), 0.0)
    c = np.cumsum(w)
    j = int(np.searchsorted(c, u * c[-1], side="right"))
    if j >= len(c):
        j = int(np.nonzero(w > 0)[0][-1])
    return int(ids[j])


def boundary_margin(logits_row, u: float, temperature: float, top_k: int | None = None) -> float:
    """Distance of u from the nearest CDF boundary (float64): draws closer than rounding may differ."""
    values = np.asarray(logits_row, dtype=np.float64)
    ids, v = _order(values, top_k)
    finite = np.isfinite(v)
    x = v / temperature
    w = np.where(finite, np.exp(x - x[finite].max()), 0.0)
    c = np.cumsum(w) / w.sum()
    return float(np.min(np.abs(c - u)))
