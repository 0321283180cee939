"""Oracle for token sampling — TEST INFRASTRUCTURE ONLY.

Restates the rule of the reference's sample_tokens (qwen3/sampling.py:234-270)
as an exact distribution instead of a draw, in float64 on the CPU:
  temperature <= 0: the argmax (:256-258, logits.argmax);
  otherwise x = logits / temperature; the top_k largest (all when top_k <= 0,
  :86-93), sorted descending; position j kept when the softmax mass of the
  list before it is <= top_p, position 0 always (:95-102 torch path, and the
  c_prev <= top_p rule of the Triton kernel :161-166); probabilities
  proportional to exp(x) over the kept positions (:103-105, the Gumbel-max
  draw of :168-174 has the same law).
Ties in value are ordered by token index (lower first): the reference leaves
their order to torch.topk; this build fixes it.
"""
from __future__ import annotations

import numpy as np
import torch


def sampling_distribution(logits_row, temperature: float, top_k: int = 0,
                          top_p: float = 1.0) -> np.ndarray:
    """Probability of drawing each token of one row (float64, sums to 1)."""
    x = torch.as_tensor(logits_row).double().numpy()
    V = x.shape[0]
    if temperature <= 0:
        out = np.zeros(V)
        out[int(np.argmax(x))] = 1.0  # first index of the maximum
        return out
    x = x / temperature
    order = np.lexsort((np.arange(V), -x))  # value descending, index ascending
    k = V if top_k <= 0 or top_k > V else top_k
    cand = order[:k]
    xc = x[cand]
    e = np.exp(xc - xc.max())
    p = e / e.sum()
    before = np.cumsum(p) - p
    keep = before <= top_p
    keep[0] = True
    w = np.where(keep, e, 0.0)
    out = np.zeros(V)
    out[cand] = w / w.sum()
    return out


def kept_set(logits_row, temperature: float, top_k: int = 0, top_p: float = 1.0) -> set:
    return set(np.nonzero(sampling_distribution(logits_row, temperature, top_k, top_p))[0].tolist())
