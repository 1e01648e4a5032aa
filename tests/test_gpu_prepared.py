"""Prepared launches (arguments converted once, one foreign call per launch) repeat exactly the launch
the per-call wrappers make: bench.py times them, so they must compute the same bits.

Each check runs the wrapper once and the prepared callable twice (the second call proves a prepared
launch can be repeated: the fused merge's arrival counters are left zero by every call) and compares
all outputs bit for bit.
"""

from __future__ import annotations

import pytest

from _helpers import announce

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("key, partition, phase", [("c1", 128, "all"), ("c2", 256, "fused"), ("c3", 512, "all"),
                                                   ("c4", 128, "fused")])
def test_decode_prepared_matches_wrapper(gpu, palib, key, partition, phase):
    import torch

    from benchmarks.workloads import make_inputs

    data = make_inputs(key, device=gpu)
    q, kc, vc, bt, cl = (data[n] for n in ("query", "key_cache", "value_cache", "block_tables", "context_lengths"))
    announce(f"prepared decode {key} P={partition} {phase}")
    expected = palib.decode(q, kc, vc, bt, cl, partition_tokens=partition, phase=phase)
    out = torch.empty_like(q)
    need = palib.workspace_bytes(q.shape[0], q.shape[1], q.shape[2], kc.shape[1], bt.shape[1], partition)
    workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=gpu)
    counters = torch.zeros(palib.counter_words(q.shape[0], q.shape[1], kc.shape[2]), dtype=torch.int32, device=gpu)
    launch = palib.prepare(q, kc, vc, bt, cl, partition_tokens=partition, out=out, workspace=workspace,
                           phase=phase, counters=counters)
    for _ in range(2):
        out.fill_(0)
        launch()
        torch.cuda.synchronize()
        assert torch.equal(out, expected)
    assert int(counters.abs().sum()) == 0


@pytest.mark.parametrize("case", ["decode-t8-gqa8-d128-p16", "prefill-t128-mha32-d128-p32"])
def test_append_prepared_matches_wrapper(gpu, kvlib, case):
    import torch

    from benchmarks.workloads import make_append_inputs

    data = make_append_inputs(case, dtype="bf16", index_dtype="int64", device=gpu)
    announce(f"prepared append {case}")
    reference = [data["key_cache"].clone(), data["value_cache"].clone()]
    kvlib.append(data["key"], data["value"], *reference, data["slot_mapping"])
    caches = [data["key_cache"].clone(), data["value_cache"].clone()]
    launch = kvlib.prepare_append(data["key"], data["value"], *caches, data["slot_mapping"])
    for _ in range(2):
        launch()
        torch.cuda.synchronize()
        assert torch.equal(caches[0], reference[0]) and torch.equal(caches[1], reference[1])


@pytest.mark.parametrize("case", ["beam-pairs8-gqa8-d128-p16", "beam-pairs64-gqa8-d256-p16"])
def test_copy_prepared_matches_wrapper(gpu, kvlib, case):
    import torch

    from benchmarks.workloads import make_copy_inputs

    data = make_copy_inputs(case, dtype="fp16", index_dtype="int32", device=gpu)
    announce(f"prepared copy {case}")
    reference = [data["key_cache"].clone(), data["value_cache"].clone()]
    kvlib.copy(*reference, data["block_mapping"])
    caches = [data["key_cache"].clone(), data["value_cache"].clone()]
    launch = kvlib.prepare_copy(*caches, data["block_mapping"])
    for _ in range(2):
        launch()
        torch.cuda.synchronize()
        assert torch.equal(caches[0], reference[0]) and torch.equal(caches[1], reference[1])


@pytest.mark.parametrize("case", ["b1-gqa32x8-s512-d128-causal", "b1-mha16-s256-d64-noncausal",
                                  "b2-gqa16x4-s256-d256-causal"])
def test_sdpa_prepared_matches_wrapper(gpu, case):
    import torch

    from radeon_kernels.cabi import sdpa_library
    from benchmarks.workloads import make_sdpa_inputs

    lib = sdpa_library()
    data = make_sdpa_inputs(case, dtype="fp16", device=gpu)
    q, k, v, c = data["query"], data["key"], data["value"], data["case"]
    announce(f"prepared sdpa {case}")
    expected = lib.forward(q, k, v, is_causal=c.causal)
    out = torch.empty_like(q)
    launch = lib.prepare_forward(q, k, v, is_causal=c.causal, out=out)
    for _ in range(2):
        out.fill_(0)
        launch()
        torch.cuda.synchronize()
        assert torch.equal(out, expected)
