"""Reference and declared fallback of scaled dot-product self-attention (prefill).

Both restate src/radeon_kernels/ops/sdpa/reference.py:6-58 in the reference:

* ``sdpa_reference`` -- the explicit fp32 evaluation the contract names as its reference
  (contracts/sdpa-1.0.json:24): expand KV heads to query heads with ``repeat_interleave`` over the
  group, scores ``q k^T * scale`` in fp32, the causal mask ``tril`` of a square of ones, fp32
  softmax, ``P V``, cast to the query dtype;
* ``sdpa_fallback`` -- the operator's general path: torch's ``scaled_dot_product_attention`` with
  ``enable_gqa`` when the head counts differ.

Neither is the oracle the kernels are tested against (that lives in ``oracle/``); the fallback is
the product's own path for requests no dispatch entry covers.
"""

from __future__ import annotations

from typing import Any


def _expanded_kv(torch_module: Any, query: Any, tensor: Any) -> Any:
    group = int(query.shape[1]) // int(tensor.shape[1])
    return tensor if group == 1 else tensor.repeat_interleave(group, dim=1)


def sdpa_reference(torch_module: Any, query: Any, key: Any, value: Any, is_causal: bool, scale: float) -> Any:
    torch = torch_module
    keys = _expanded_kv(torch, query, key).float()
    values = _expanded_kv(torch, query, value).float()
    scores = torch.matmul(query.float(), keys.transpose(-2, -1)) * scale
    if is_causal:
        sequence = int(query.shape[2])
        keep = torch.ones((sequence, sequence), device=query.device, dtype=torch.bool).tril()
        scores = scores.masked_fill(~keep, float("-inf"))
    weights = torch.softmax(scores, dim=-1, dtype=torch.float32)
    return torch.matmul(weights, values).to(dtype=query.dtype)


def sdpa_fallback(torch_module: Any, query: Any, key: Any, value: Any, is_causal: bool, scale: float) -> Any:
    return torch_module.nn.functional.scaled_dot_product_attention(
        query, key, value, attn_mask=None, dropout_p=0.0, is_causal=is_causal, scale=scale,
        enable_gqa=int(query.shape[1]) != int(key.shape[1]))
