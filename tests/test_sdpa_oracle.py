"""Pinning the self-attention oracle (oracle/sdpa_oracle.py) before trusting it as the checker.

The reference holds no numeric vectors for sdpa.  What pins the oracle:

* torch's ``scaled_dot_product_attention`` (a library routine, the reference's declared fallback,
  src/radeon_kernels/ops/sdpa/reference.py:41-58) in float64 on CPU, causal and not, with GQA;
* the explicit-loop brute force on tiny shapes;
* closed forms and invariants: a causal first row is V[0]; equal scores give the mean of V; a
  noncausal result is invariant when keys and values are permuted together; GQA equals MHA with
  the KV heads duplicated; the restated torch fp32 path (``fallback_restated``) agrees;
* planted mistakes in copies of the oracle (an off-by-one causal mask, the wrong KV head mapping,
  a missing scale, keys and values swapped) each fail one of these checks.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import sdpa_oracle


def tensors(seed, b=2, hq=8, hkv=2, s=13, d=16):
    gen = np.random.default_rng(seed)
    return (gen.standard_normal((b, hq, s, d)), gen.standard_normal((b, hkv, s, d)),
            gen.standard_normal((b, hkv, s, d)))


def torch_sdpa(q, k, v, causal, scale=None):
    return torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), is_causal=causal, scale=scale,
        enable_gqa=q.shape[1] != k.shape[1]).numpy()


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", [(2, 8, 2, 13, 16), (1, 4, 4, 33, 64), (3, 6, 1, 7, 8)])
def test_matches_torch_sdpa_in_float64(shape, causal):
    b, hq, hkv, s, d = shape
    q, k, v = tensors(sum(shape), b, hq, hkv, s, d)
    np.testing.assert_allclose(sdpa_oracle.sdpa_numpy(q, k, v, causal), torch_sdpa(q, k, v, causal),
                               rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(sdpa_oracle.sdpa_numpy(q, k, v, causal, 0.3), torch_sdpa(q, k, v, causal, 0.3),
                               rtol=1e-12, atol=1e-12)


def test_matches_bruteforce():
    for causal in (True, False):
        q, k, v = tensors(5, b=1, hq=4, hkv=2, s=6, d=4)
        np.testing.assert_allclose(sdpa_oracle.sdpa_numpy(q, k, v, causal), sdpa_oracle.sdpa_bruteforce(q, k, v, causal),
                                   rtol=1e-12, atol=1e-12)


def test_closed_forms_and_invariants():
    q, k, v = tensors(7)
    out = sdpa_oracle.sdpa_numpy(q, k, v, True)
    for h in range(8):
        np.testing.assert_array_equal(out[:, h, 0], v[:, h // 4, 0])
    same = sdpa_oracle.sdpa_numpy(q, np.zeros_like(k), v, False)
    np.testing.assert_allclose(same, np.repeat(v.mean(axis=2, keepdims=True), 4, axis=1).repeat(13, axis=2),
                               rtol=1e-12)
    perm = np.random.default_rng(1).permutation(13)
    np.testing.assert_allclose(sdpa_oracle.sdpa_numpy(q, k[:, :, perm], v[:, :, perm], False),
                               sdpa_oracle.sdpa_numpy(q, k, v, False), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(sdpa_oracle.sdpa_numpy(q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1), True),
                               out, rtol=1e-12, atol=1e-12)
    restated = sdpa_oracle.fallback_restated(torch, torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
                                             True, 1 / math.sqrt(16)).numpy()
    np.testing.assert_allclose(restated, out, rtol=1e-5, atol=1e-5)


def _mutant(kind):
    def attend(q, k, v, causal, scale=None):
        d = q.shape[-1]
        scale = 1 / math.sqrt(d) if scale is None else scale
        group = q.shape[1] // k.shape[1]
        kk = np.tile(k, (1, group, 1, 1)) if kind == "tiled_heads" else np.repeat(k, group, axis=1)
        vv = np.tile(v, (1, group, 1, 1)) if kind == "tiled_heads" else np.repeat(v, group, axis=1)
        if kind == "kv_swapped":
            kk, vv = vv, kk
        scores = np.einsum("bhsd,bhtd->bhst", q, kk) * (1.0 if kind == "no_scale" else scale)
        if causal:
            s = q.shape[2]
            keep = np.tril(np.ones((s, s), dtype=bool), k=1 if kind == "mask_off_by_one" else 0)
            scores = np.where(keep, scores, -np.inf)
        weights = np.exp(scores - scores.max(-1, keepdims=True))
        return np.einsum("bhst,bhtd->bhsd", weights / weights.sum(-1, keepdims=True), vv)
    return attend


def _pinning_checks(attend):
    q, k, v = tensors(11)
    failures = []
    for causal in (True, False):
        if not np.allclose(attend(q, k, v, causal), torch_sdpa(q, k, v, causal), rtol=1e-10, atol=1e-10):
            failures.append(f"torch sdpa causal={causal}")
    return failures


@pytest.mark.parametrize("kind", ["mask_off_by_one", "tiled_heads", "no_scale", "kv_swapped"])
def test_planted_mistakes_are_caught(kind):
    assert _pinning_checks(_mutant(kind)), f"mutant {kind} passed every pinning check"


def test_unmutated_restatement_passes_the_same_checks():
    assert _pinning_checks(_mutant("none")) == []
