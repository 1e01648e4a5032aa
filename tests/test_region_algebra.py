"""Dispatch value sets and manifest selection against brute-force enumeration.

The manifest rules (reference src/radeon_kernels/runtime/registry.py:60-401) are defined on the sets
of values a constraint admits.  These tests enumerate those sets over a small finite universe that
contains every endpoint the generators can produce, and check membership, intersection, inclusion
and the manifest's priority/shadowing validation and selection against that definition, including
the reference's one exception: a multi-valued integer range is never covered by an enumeration.
"""

from __future__ import annotations

import itertools
import random

import pytest

from radeon_kernels.errors import ConfigError
from radeon_kernels.runtime.fingerprint import EnvironmentFingerprint
from radeon_kernels.runtime.registry import DispatchManifest, ValueConstraint

UNIVERSE = [*range(1, 9), "a", "b", 1.0, 2.5, True, False]
ENV = {"architecture": "gfx950", "wavefront_size": 64, "rocm_abi": "7.0", "python_abi": "cp310",
       "pytorch_version": "2.10.0+rocm7.0"}


def random_raw(rng: random.Random):
    form = rng.choice(("eq", "range", "one_of"))
    if form == "range":
        low = rng.randint(1, 8)
        return [low, rng.randint(low, 8)]
    if form == "eq":
        return rng.choice(UNIVERSE)
    pool = list(range(1, 9)) + ["a", "b", 1.0, 2.5, True]
    choices = rng.sample(pool, rng.randint(1, 4))
    typed = {(type(item), item) for item in choices}
    return {"one_of": choices} if len(typed) == len(choices) else {"one_of": choices[:1]}


def members(constraint: ValueConstraint) -> set:
    return {(type(item), item) for item in UNIVERSE if constraint.matches(item)}


def multi_range(raw) -> bool:
    return isinstance(raw, list) and raw[0] < raw[1]


def test_value_sets_agree_with_enumeration():
    rng = random.Random(7)
    raws = [random_raw(rng) for _ in range(160)]
    constraints = [ValueConstraint.from_raw(raw, "x") for raw in raws]
    for raw, constraint in zip(raws, constraints):
        admitted = members(constraint)
        if isinstance(raw, list):
            assert admitted == {(int, v) for v in range(raw[0], raw[1] + 1)}
        elif isinstance(raw, dict):
            assert admitted == {(type(v), v) for v in raw["one_of"]}
        else:
            assert admitted == {(type(raw), raw)}
    for (raw_a, a), (raw_b, b) in itertools.product(zip(raws, constraints), repeat=2):
        ma, mb = members(a), members(b)
        assert a.overlaps(b) == bool(ma & mb)
        covered = ma <= mb and not (multi_range(raw_a) and not isinstance(raw_b, list))
        assert a.is_subset_of(b) == covered, (raw_a, raw_b)


def entry(identifier, priority, workload, features=()):
    environment = dict(ENV, features=list(features)) if features else dict(ENV)
    return {"id": identifier, "priority": priority, "environment": environment, "workload": workload,
            "winner": {"provider": "native", "artifact": f"lib/{identifier}.so", "entrypoint": "run",
                       "sha256": "0" * 64},
            "launch": {}, "fallbacks": ["torch"], "evidence_id": f"ev-{identifier}"}


def typed(signature):
    """A signature point with its values' types, so that 1, 1.0 and True stay apart in sets."""

    return tuple((key, type(value), value) for key, value in signature)


def region(raw_entry, signature_space, feature_space):
    """The (features, signature) points an entry matches, by enumeration."""

    manifest = DispatchManifest.from_mapping({"schema_version": "1.0", "operator": "op", "semantic_version": "1.0",
                                              "default_fallbacks": ["torch"], "entries": [raw_entry]})
    parsed = manifest.entries[0]
    points = set()
    for features in feature_space:
        fp = EnvironmentFingerprint(**ENV, features=features)
        for signature in signature_space:
            if parsed.matches(fp, dict(signature)):
                points.add((features, typed(signature)))
    return points, parsed


def enumerated_within(inner, outer) -> bool:
    """Region inclusion by enumeration, with the reference's range-versus-enumeration exception."""

    (inner_points, inner_raw), (outer_points, outer_raw) = inner, outer
    uncovered_range = any(multi_range(inner_raw["workload"][key]) and not isinstance(bound, list)
                          for key, bound in outer_raw["workload"].items() if key in inner_raw["workload"])
    return inner_points <= outer_points and not uncovered_range


@pytest.mark.parametrize("seed", range(6))
def test_manifest_validation_and_selection_agree_with_enumeration(seed):
    rng = random.Random(seed)
    keys = ("batch", "dtype")
    signature_space = [tuple(zip(keys, values)) for values in itertools.product(UNIVERSE, repeat=2)]
    feature_space = [(), ("mfma",), ("lds_dma", "mfma")]
    accepted = rejected = 0
    for trial in range(40):
        raw_entries = []
        for position in range(rng.randint(2, 4)):
            workload = {key: random_raw(rng) for key in rng.sample(keys, rng.randint(1, 2))}
            features = rng.choice([(), ("mfma",)])
            raw_entries.append(entry(f"e{position}", rng.choice((1, 2, 3)), workload, features))
        regions = [(region(raw, signature_space, feature_space)[0], raw) for raw in raw_entries]
        # The rule on enumerated regions: two regions that share a point differ in priority, and
        # the higher-priority one lies inside the lower one without being equal to it.
        violation = False
        for a, b in itertools.combinations(regions, 2):
            if not a[0] & b[0]:
                continue
            if a[1]["priority"] == b[1]["priority"]:
                violation = True
                continue
            high, low = (a, b) if a[1]["priority"] > b[1]["priority"] else (b, a)
            if not enumerated_within(high, low) or enumerated_within(low, high):
                violation = True
        document = {"schema_version": "1.0", "operator": "op", "semantic_version": "1.0",
                    "default_fallbacks": ["torch"], "entries": raw_entries}
        if violation:
            with pytest.raises(ConfigError, match="ambiguous overlapping|must be a strict subset"):
                DispatchManifest.from_mapping(document)
            rejected += 1
            continue
        manifest = DispatchManifest.from_mapping(document)
        accepted += 1
        for features in feature_space:
            fp = EnvironmentFingerprint(**ENV, features=features)
            for signature in signature_space:
                hits = [raw for points, raw in regions if (features, typed(signature)) in points]
                chosen = manifest.select(fp, dict(signature))
                if not hits:
                    assert chosen is None
                    continue
                best = max(hits, key=lambda raw: raw["priority"])
                assert sum(raw["priority"] == best["priority"] for raw in hits) == 1
                assert chosen is not None and chosen.id == best["id"]
    assert accepted and rejected


def test_other_environment_keys_never_meet():
    document = {"schema_version": "1.0", "operator": "op", "semantic_version": "1.0", "default_fallbacks": ["torch"],
                "entries": [entry("here", 5, {"batch": [1, 8]}),
                            dict(entry("there", 5, {"batch": [1, 8]}), environment=dict(ENV, rocm_abi="7.1"))]}
    manifest = DispatchManifest.from_mapping(document)
    assert manifest.select(EnvironmentFingerprint(**ENV), {"batch": 3}).id == "here"
    assert manifest.select(EnvironmentFingerprint(**dict(ENV, rocm_abi="7.1")), {"batch": 3}).id == "there"
    assert manifest.select(EnvironmentFingerprint(**dict(ENV, rocm_abi="7.2")), {"batch": 3}) is None


def manifest_of(*entries):
    return {"schema_version": "1.0", "operator": "op", "semantic_version": "1.0", "default_fallbacks": ["torch"],
            "entries": list(entries)}


@pytest.mark.parametrize("high_batch", [[128, 128], 128, {"one_of": [128]}])
def test_equal_regions_at_different_priorities_are_rejected(high_batch):
    # [128, 128], 128 and one_of [128] all admit exactly {128}: the high entry would shadow the
    # low one completely, which is not a proper subset.
    with pytest.raises(ConfigError, match="must be a strict subset"):
        DispatchManifest.from_mapping(manifest_of(entry("low", 1, {"batch": 128}), entry("high", 2, {"batch": high_batch})))


def test_feature_or_key_narrowing_makes_a_proper_subset():
    narrower_by_feature = manifest_of(entry("low", 1, {"batch": 128}), entry("high", 2, {"batch": 128}, ("mfma",)))
    narrower_by_key = manifest_of(entry("low", 1, {"batch": 128}), entry("high", 2, {"batch": 128, "dtype": "a"}))
    for document in (narrower_by_feature, narrower_by_key):
        manifest = DispatchManifest.from_mapping(document)
        assert manifest.select(EnvironmentFingerprint(**ENV, features=("mfma",)), {"batch": 128, "dtype": "a"}).id == "high"
        assert manifest.select(EnvironmentFingerprint(**ENV), {"batch": 128, "dtype": "b"}).id == "low"
