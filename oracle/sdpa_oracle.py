"""CPU oracle of scaled dot-product self-attention (test infrastructure only).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` use this module, as the
checker; the product path never imports it.  It restates the reference's explicit fp32 evaluation
(src/radeon_kernels/ops/sdpa/reference.py:13-38) in numpy:

* ``expand_kv``: query head h reads KV head h // (Hq // Hkv) (reference.py:6-10, repeat_interleave);
* ``sdpa_numpy``: scores q k^T * scale (reference.py:28-30), causal mask keeping key j <= query i
  (the ``tril`` of a square of ones, :31-36), softmax over keys (:37), P V (:38), in the chosen
  accumulation dtype (float64 by default: a tighter reference than the reference's own fp32);
* ``sdpa_bruteforce``: the same definition as explicit Python loops for tiny shapes;
* ``fallback_restated``: the reference's torch fp32 path verbatim in torch ops (for cross-checks
  with torch's own scaled_dot_product_attention, the declared fallback, :41-58).

Pinned in tests/test_sdpa_oracle.py against torch's scaled_dot_product_attention (a library
routine) and the brute force, and by closed forms: a causal first row equals V[0]; equal scores give
the mean of V; a noncausal result is invariant under permuting keys with their values; GQA equals
MHA with the KV heads duplicated.
"""

from __future__ import annotations

import math
from typing import Any

import numpy as np


def expand_kv(query: np.ndarray, tensor: np.ndarray) -> np.ndarray:
    group = query.shape[1] // tensor.shape[1]
    return tensor if group == 1 else np.repeat(tensor, group, axis=1)


def sdpa_numpy(query: np.ndarray, key: np.ndarray, value: np.ndarray, is_causal: bool, scale: float | None = None,
               accum: Any = np.float64) -> np.ndarray:
    """[B, Hq, S, D] attention output in ``accum`` (inputs converted from their stored values)."""

    d = query.shape[-1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    q = query.astype(accum)
    k = expand_kv(query, key).astype(accum)
    v = expand_kv(query, value).astype(accum)
    scores = np.einsum("bhsd,bhtd->bhst", q, k) * accum(scale)
    if is_causal:
        s = query.shape[2]
        scores = np.where(np.tril(np.ones((s, s), dtype=bool)), scores, -np.inf)
    scores = scores - scores.max(axis=-1, keepdims=True)
    weights = np.exp(scores)
    weights = weights / weights.sum(axis=-1, keepdims=True)
    return np.einsum("bhst,bhtd->bhsd", weights, v)


def sdpa_bruteforce(query: np.ndarray, key: np.ndarray, value: np.ndarray, is_causal: bool,
                    scale: float | None = None) -> np.ndarray:
    b_, hq, s_, d = query.shape
    hkv = key.shape[1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    out = np.zeros((b_, hq, s_, d))
    for b in range(b_):
        for h in range(hq):
            kv = h // (hq // hkv)
            for i in range(s_):
                keys = range(i + 1) if is_causal else range(s_)
                logits = [sum(float(query[b, h, i, c]) * float(key[b, kv, j, c]) for c in range(d)) * scale
                          for j in keys]
                top = max(logits)
                weights = [math.exp(x - top) for x in logits]
                total = sum(weights)
                for c in range(d):
                    out[b, h, i, c] = sum(w * float(value[b, kv, j, c]) for w, j in zip(weights, keys)) / total
    return out


def fallback_restated(torch: Any, query: Any, key: Any, value: Any, is_causal: bool, scale: float) -> Any:
    group = int(query.shape[1]) // int(key.shape[1])
    keys = key.repeat_interleave(group, dim=1).float() if group > 1 else key.float()
    values = value.repeat_interleave(group, dim=1).float() if group > 1 else value.float()
    scores = torch.matmul(query.float(), keys.transpose(-2, -1)) * scale
    if is_causal:
        s = int(query.shape[2])
        scores = scores.masked_fill(~torch.ones((s, s), dtype=torch.bool).tril(), float("-inf"))
    return torch.matmul(torch.softmax(scores, dim=-1, dtype=torch.float32), values)


def as_numpy_f32(tensor: Any) -> np.ndarray:
    return tensor.detach().float().cpu().numpy()
