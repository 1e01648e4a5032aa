"""CPU tests of the static-dispatch runtime: fingerprint, manifest algebra, dispatcher, explain, loader.

The cases follow the reference's own runtime unit tests (tests/test_runtime.py:96-311 there):
strict-subset priority accepted, same-priority overlap and partial shadows rejected, unknown fields /
non-scalar launch parameters / unknown schema versions rejected, most-specific match wins, declared
fallbacks without search, and loader path-escape / digest / format checks.
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path
from types import SimpleNamespace

import pytest

from radeon_kernels.errors import ConfigError
from radeon_kernels.runtime.compatibility import EnvironmentConstraint
from radeon_kernels.runtime.dispatcher import DispatchRequest, Dispatcher
from radeon_kernels.runtime.explain import clear_last_dispatch, explain_last_dispatch, get_last_dispatch, record_dispatch
from radeon_kernels.runtime.fingerprint import EnvironmentFingerprint, FingerprintError, normalize_rocm_abi
from radeon_kernels.runtime.loader import (
    ArtifactIntegrityError,
    ArtifactLoadError,
    PrecompiledArtifactLoader,
    module_name_for,
)
from radeon_kernels.runtime.registry import ArtifactSpec, DispatchManifest, DispatchRegistry, ValueConstraint

ENV = {"architecture": "gfx950", "wavefront_size": 64, "rocm_abi": "7.0", "python_abi": "cp310",
       "pytorch_version": "2.10.0+rocm7.0"}


def fingerprint(**overrides) -> EnvironmentFingerprint:
    values = dict(ENV)
    values.update(overrides)
    return EnvironmentFingerprint(**values)


def entry(identifier, *, priority, batch, dtype="bf16", env=None, launch=None):
    return {
        "id": identifier,
        "priority": priority,
        "environment": dict(env or ENV),
        "workload": {"dtype": dtype, "batch": batch, "head_dim": 128},
        "winner": {"provider": "native", "artifact": f"lib/{identifier}.so", "entrypoint": "decode_mfma",
                   "sha256": "a" * 64},
        "launch": launch if launch is not None else {"partition_tokens": 512},
        "fallbacks": ["torch"],
        "evidence_id": f"evidence-{identifier}",
    }


def manifest(*entries):
    return {"schema_version": "1.0", "operator": "paged_attention_decode", "semantic_version": "1.0",
            "default_fallbacks": ["torch"], "entries": list(entries)}


# ---------------------------------------------------------------------------------------------
def test_fingerprint_normalises_rocm_abi_and_features():
    value = fingerprint(rocm_abi="7.02.51831-rc1", features=("mfma", "mfma", "lds_dma"))
    assert value.rocm_abi == "7.2"
    assert value.features == ("lds_dma", "mfma")
    assert normalize_rocm_abi("7.0.51831") == "7.0"
    with pytest.raises(FingerprintError):
        normalize_rocm_abi("rocm")
    with pytest.raises(FingerprintError, match="wavefront"):
        fingerprint(wavefront_size=48)
    with pytest.raises(FingerprintError, match="architecture"):
        fingerprint(architecture="sm_90")


def test_fingerprint_detects_gfx950_from_torch_without_a_gpu():
    fake = SimpleNamespace(
        __version__="2.10.0+rocm7.0",
        version=SimpleNamespace(hip="7.0.51831"),
        cuda=SimpleNamespace(is_available=lambda: True,
                             get_device_properties=lambda index: SimpleNamespace(
                                 gcnArchName="gfx950:sramecc+:xnack-", warp_size=64)),
    )
    value = EnvironmentFingerprint.detect(torch_module=fake)
    assert (value.architecture, value.wavefront_size, value.rocm_abi) == ("gfx950", 64, "7.0")
    assert value.python_abi == f"cp{sys.version_info.major}{sys.version_info.minor}"
    no_hip = SimpleNamespace(__version__="2.10", version=SimpleNamespace(hip=None),
                             cuda=SimpleNamespace(is_available=lambda: True))
    with pytest.raises(FingerprintError, match="does not report a ROCm"):
        EnvironmentFingerprint.detect(torch_module=no_hip)
    no_gpu = SimpleNamespace(__version__="2.10", version=SimpleNamespace(hip="7.0"),
                             cuda=SimpleNamespace(is_available=lambda: False))
    with pytest.raises(FingerprintError, match="no visible ROCm GPU"):
        EnvironmentFingerprint.detect(torch_module=no_gpu)


def test_fingerprint_round_trips_through_mapping():
    value = fingerprint(features=("mfma",))
    assert EnvironmentFingerprint.from_mapping(value.to_dict()) == value
    with pytest.raises(FingerprintError, match="unknown fingerprint fields"):
        EnvironmentFingerprint.from_mapping({**value.to_dict(), "vendor": "amd"})


def test_environment_constraint_matching_and_features():
    constraint = EnvironmentConstraint.from_mapping({**ENV, "features": ["mfma"]}, "env")
    assert constraint.matches(fingerprint(features=("mfma", "lds_dma")))
    assert not constraint.matches(fingerprint())
    assert not constraint.matches(fingerprint(pytorch_version="2.10.0+rocm7.1"))
    broad = EnvironmentConstraint.from_mapping(ENV, "env")
    assert constraint.is_strict_subset_of(broad) and not broad.is_subset_of(constraint)
    for bad, message in (({**ENV, "wavefront_size": True}, "32 or 64"), ({**ENV, "python_abi": "py3"}, "cpXY"),
                         ({**ENV, "rocm_abi": "x"}, "MAJOR.MINOR"), ({**ENV, "extra": 1}, "unknown fields")):
        with pytest.raises(ConfigError, match=message):
            EnvironmentConstraint.from_mapping(bad, "env")


# ---------------------------------------------------------------------------------------------
def test_value_constraints_use_type_identity():
    eq = ValueConstraint.from_raw(16, "x")
    assert eq.matches(16) and not eq.matches(16.0) and not eq.matches(True)
    rng = ValueConstraint.from_raw([1, 1024], "x")
    assert rng.matches(1024) and not rng.matches(0) and not rng.matches(True)
    one = ValueConstraint.from_raw({"one_of": ["int32", "int64"]}, "x")
    assert one.matches("int64") and not one.matches("int16")
    for bad in ([0, 5], [5, 1], [1.0, 2], {"one_of": []}, {"one_of": [1, 1]}, None, [1]):
        with pytest.raises(ConfigError):
            ValueConstraint.from_raw(bad, "x")


def test_accepts_fallback_only_manifest():
    value = DispatchManifest.from_mapping(manifest())
    assert value.entries == () and value.default_fallbacks == ("torch",)


def test_accepts_strict_higher_priority_subset():
    value = DispatchManifest.from_mapping(manifest(entry("broad", priority=10, batch=[1, 512]),
                                                   entry("exact", priority=100, batch=[128, 128])))
    assert len(value.entries) == 2


def test_rejects_same_priority_overlap():
    with pytest.raises(ConfigError, match="ambiguous overlapping"):
        DispatchManifest.from_mapping(manifest(entry("first", priority=10, batch=[1, 512]),
                                               entry("second", priority=10, batch=[128, 128])))


def test_rejects_partial_high_priority_shadow():
    with pytest.raises(ConfigError, match="must be a strict subset"):
        DispatchManifest.from_mapping(manifest(entry("broad", priority=10, batch=[1, 512]),
                                               entry("partial", priority=100, batch=[256, 768])))


def test_non_overlapping_entries_need_no_priority_order():
    value = DispatchManifest.from_mapping(manifest(entry("bf16", priority=10, batch=[1, 512]),
                                                   entry("fp16", priority=10, batch=[1, 512], dtype="fp16"),
                                                   entry("other-gpu", priority=10, batch=[1, 512],
                                                         env={**ENV, "architecture": "gfx942"})))
    assert len(value.entries) == 3


@pytest.mark.parametrize(
    "mutate, message",
    [
        (lambda m: m.update(search_on_user_machine=True), "unknown fields"),
        (lambda m: m["entries"][0].update(launch={"partition_tokens": [512]}), "expected a string, number or boolean"),
        (lambda m: m.update(schema_version="2.0"), "unsupported dispatch schema"),
        (lambda m: m["entries"][0]["winner"].update(sha256="A" * 64), "lowercase SHA-256"),
        (lambda m: m["entries"][0]["winner"].update(artifact="../escape.so"), "normalized relative path"),
        (lambda m: m["entries"][0]["winner"].update(entrypoint="decode-mfma"), "identifier"),
        (lambda m: m["entries"][0]["winner"].update(format="elf"), "python_extension or hsaco"),
        (lambda m: m["entries"][0].update(priority=-1), "non-negative"),
        (lambda m: m["entries"][0].update(fallbacks=["torch", "torch"]), "duplicates"),
        (lambda m: m.update(default_fallbacks=[]), "non-empty"),
        (lambda m: m["entries"].append(dict(m["entries"][0])), "unique"),
    ],
)
def test_rejects_malformed_manifests(mutate, message):
    payload = manifest(entry("exact", priority=100, batch=[128, 128]))
    mutate(payload)
    with pytest.raises(ConfigError, match=message):
        DispatchManifest.from_mapping(payload)


def test_manifest_round_trips_and_loads_from_directory(tmp_path):
    payload = manifest(entry("exact", priority=100, batch=[128, 128]))
    parsed = DispatchManifest.from_mapping(payload)
    assert DispatchManifest.from_mapping(parsed.to_dict()) == parsed
    (tmp_path / "pa.json").write_text(json.dumps(payload), encoding="utf-8")
    registry = DispatchRegistry.from_directory(tmp_path)
    assert registry.keys() == (("paged_attention_decode", "1.0"),)
    with pytest.raises(ConfigError, match="no manifest"):
        registry.get("sdpa", "1.0")
    with pytest.raises(ConfigError, match="duplicate manifest"):
        registry.add(parsed)
    (tmp_path / "bad.json").write_text("{", encoding="utf-8")
    with pytest.raises(ConfigError, match="invalid JSON"):
        DispatchRegistry.from_directory(tmp_path)


# ---------------------------------------------------------------------------------------------
@pytest.fixture()
def dispatcher():
    clear_last_dispatch()
    registry = DispatchRegistry([DispatchManifest.from_mapping(manifest(
        entry("broad", priority=10, batch=[1, 512]),
        entry("exact", priority=100, batch=[128, 128], launch={"partition_tokens": 2048})))])
    return Dispatcher(registry)


def request(batch, dtype="bf16"):
    return DispatchRequest("paged_attention_decode", "1.0", {"dtype": dtype, "batch": batch, "head_dim": 128})


def test_selects_most_specific_matching_entry(dispatcher):
    decision = dispatcher.select(request(128), fingerprint())
    assert decision.matched and decision.entry_id == "exact"
    assert dict(decision.launch) == {"partition_tokens": 2048}
    assert decision.winner.artifact == "lib/exact.so"
    record = get_last_dispatch()
    assert record["selected"] == "native/decode_mfma" and record["entry_id"] == "exact"
    assert "entry 'exact'" in explain_last_dispatch()


def test_selects_broad_region_outside_exact_shape(dispatcher):
    assert dispatcher.select(request(64), fingerprint()).entry_id == "broad"


def test_returns_declared_fallback_without_search(dispatcher):
    decision = dispatcher.select(request(128, dtype="fp16"), fingerprint())
    assert not decision.matched
    assert decision.fallbacks == ("torch",)
    assert "no compatible" in decision.reason
    assert get_last_dispatch()["selected"] is None
    other = dispatcher.select(request(128), fingerprint(architecture="gfx942"))
    assert not other.matched


def test_decisions_are_memoised_and_still_recorded(dispatcher):
    first = dispatcher.select(request(128), fingerprint())
    clear_last_dispatch()
    again = dispatcher.select(request(128), fingerprint())
    assert again is first  # same (operator, version, fingerprint, signature) -> the same decision
    assert get_last_dispatch()["entry_id"] == "exact"  # every select still writes the record
    assert dispatcher.select(request(64), fingerprint()).entry_id == "broad"  # other keys decide afresh
    assert dispatcher.select(request(128), fingerprint(architecture="gfx942")).matched is False
    clear_last_dispatch()
    assert dispatcher.select(request(128), fingerprint(), record=False) is first
    assert get_last_dispatch() is None
    # An unhashable signature value (keys no entry constrains are ignored by matching) is decided
    # without memoising, with the same result.
    odd = DispatchRequest("paged_attention_decode", "1.0", {"dtype": "bf16", "batch": 128, "head_dim": 128,
                                                            "extra": ["unhashable"]})
    decided = dispatcher.select(odd, fingerprint())
    assert decided.entry_id == "exact" and decided is not first


def test_owned_records_skip_the_inbound_copy_but_reads_still_copy():
    clear_last_dispatch()
    value = {"operator": "x", "architecture": "gfx950", "reason": "r", "launch": {"partition_tokens": 64}}
    record_dispatch(value, owned=True)
    out = get_last_dispatch()
    out["launch"]["partition_tokens"] = 1
    assert get_last_dispatch()["launch"] == {"partition_tokens": 64}
    shared = {"operator": "x", "architecture": "gfx950", "reason": "r", "launch": {"partition_tokens": 64}}
    record_dispatch(shared)  # not owned: copied on the way in
    shared["launch"]["partition_tokens"] = 2
    assert get_last_dispatch()["launch"] == {"partition_tokens": 64}


def test_explain_text_and_isolation():
    clear_last_dispatch()
    assert explain_last_dispatch() == "No Radeon kernel dispatch has been performed in this context."
    record_dispatch({"operator": "paged_attention_decode", "architecture": "gfx950", "selected": "native/decode_mfma",
                     "artifact": "lib/rk_pa_gfx950.so", "evidence_id": "e1", "fallbacks": ["torch"], "reason": "r"})
    text = explain_last_dispatch().splitlines()
    assert text == ["operator: paged_attention_decode", "architecture: gfx950", "selected: native/decode_mfma",
                    "artifact: lib/rk_pa_gfx950.so", "evidence: e1", "fallbacks: torch", "reason: r"]
    copy = get_last_dispatch()
    copy["selected"] = "tampered"
    assert get_last_dispatch()["selected"] == "native/decode_mfma"


def test_explain_record_is_per_thread():
    import threading

    clear_last_dispatch()
    record_dispatch({"operator": "x", "architecture": "gfx950", "reason": "main"})
    seen = {}

    def worker():
        seen["before"] = get_last_dispatch()
        record_dispatch({"operator": "y", "architecture": "gfx950", "reason": "thread"})

    thread = threading.Thread(target=worker)
    thread.start()
    thread.join()
    assert seen["before"] is None
    assert get_last_dispatch()["reason"] == "main"


# ---------------------------------------------------------------------------------------------
@pytest.fixture()
def pack_root(tmp_path):
    (tmp_path / "lib").mkdir()
    path = tmp_path / "lib" / "kernel.so"
    path.write_bytes(b"not a real extension")
    return tmp_path, hashlib.sha256(path.read_bytes()).hexdigest()


def spec(digest, artifact="lib/kernel.so", fmt="python_extension"):
    return ArtifactSpec(provider="native", artifact=artifact, entrypoint="decode_mfma", sha256=digest, format=fmt)


def test_loader_verifies_artifact_inside_pack(pack_root):
    root, digest = pack_root
    loader = PrecompiledArtifactLoader(root)
    assert loader.resolve_and_verify(spec(digest)) == (root / "lib" / "kernel.so").resolve()
    with pytest.raises(ArtifactIntegrityError, match="SHA-256 mismatch"):
        loader.resolve_and_verify(spec("0" * 64))
    with pytest.raises(ArtifactIntegrityError, match="missing"):
        loader.resolve_and_verify(spec(digest, artifact="lib/absent.so"))


def test_loader_rejects_path_escape(pack_root):
    root, _ = pack_root
    outside = root.parent / "outside.so"
    outside.write_bytes(b"outside")
    loader = PrecompiledArtifactLoader(root)
    escaped = ArtifactSpec("native", "../outside.so", "decode_mfma", hashlib.sha256(b"outside").hexdigest())
    with pytest.raises(ArtifactIntegrityError, match="escapes"):
        loader.resolve_and_verify(escaped)


def test_loader_hsaco_needs_provider_launcher_and_broken_extension_fails_cleanly(pack_root):
    root, digest = pack_root
    loader = PrecompiledArtifactLoader(root)
    with pytest.raises(ArtifactLoadError, match="provider-specific"):
        loader.load_module(spec(digest, fmt="hsaco"))
    with pytest.raises(ArtifactLoadError, match="failed to load"):
        loader.load_module(spec(digest))


def test_module_name_comes_from_the_file_stem():
    assert module_name_for(Path("lib/rk_pa_gfx950.so")) == "rk_pa_gfx950"
    assert module_name_for(Path("lib/rk_pa_gfx950.cpython-310-x86_64-linux-gnu.so")) == "rk_pa_gfx950"
    with pytest.raises(ArtifactLoadError):
        module_name_for(Path("lib/rk-pa.so"))


def test_loader_imports_python_extension_and_caches_entrypoint(tmp_path):
    """A pure-Python module stands in for the extension: the import and lookup path are identical."""

    (tmp_path / "lib").mkdir()
    module = tmp_path / "lib" / "fake_pa_ext.py"
    module.write_text("calls = []\ndef decode_mfma(*a, **k):\n    calls.append(k)\n    return 'out'\n")
    digest = hashlib.sha256(module.read_bytes()).hexdigest()
    artifact = ArtifactSpec("native", "lib/fake_pa_ext.py", "decode_mfma", digest)
    loader = PrecompiledArtifactLoader(tmp_path)
    first = loader.load_entrypoint(artifact)
    assert first.callable(partition_tokens=64) == "out"
    assert loader.load_entrypoint(artifact) is first  # verified once, then cached
    missing = ArtifactSpec("native", "lib/fake_pa_ext.py", "decode_valu", digest)
    with pytest.raises(ArtifactLoadError, match="does not export"):
        loader.load_entrypoint(missing)
