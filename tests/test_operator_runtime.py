"""CPU tests of the operator runtime and kernel-pack resolution, with injected fakes.

Follows the reference's tests/test_operator_runtime.py:97-131 (fallback-only manifest runs the
fallback without touching packs; a matching entry runs the native callable) and the fault injections
of its tests/test_gemm_dispatch.py:214-286 (missing pack, ABI mismatch, corrupted digest, native
errors -> declared fallback with the reason recorded).
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path
from types import SimpleNamespace

import pytest

from radeon_kernels.ops._runtime import NativeDemotionWarning, OperatorDispatchError, OperatorRuntime
from radeon_kernels.providers.native import NativeProviderError
from radeon_kernels.runtime.explain import clear_last_dispatch, get_last_dispatch
from radeon_kernels.runtime.fingerprint import EnvironmentFingerprint
from radeon_kernels.runtime.packs import KernelPackRegistry, PackResolutionError, default_pack_roots
from radeon_kernels.runtime.ed25519 import Ed25519PrivateKey
from radeon_kernels.runtime.signing import TrustedKey, TrustedKeyring, signature_document

TEST_KEY = Ed25519PrivateKey.from_private_bytes(hashlib.sha256(b"rk-test-pack-key").digest())
TEST_KEYRING = TrustedKeyring([TrustedKey("rk-test", TEST_KEY.public_key().public_bytes(), "active",
                                          "2026-12-01T00:00:00+00:00")])
from radeon_kernels.runtime.registry import ArtifactSpec, DispatchManifest, DispatchRegistry

ENV = {"architecture": "gfx950", "wavefront_size": 64, "rocm_abi": "7.0", "python_abi": "cp310",
       "pytorch_version": "2.10.0+rocm7.0"}
SIGNATURE = {"dtype": "bf16", "batch": 128, "head_dim": 128}


def fingerprint(**overrides):
    return EnvironmentFingerprint(**{**ENV, **overrides})


def manifest(*, winner: bool, fallbacks=("torch",), digest="a" * 64):
    entries = []
    if winner:
        entries.append({
            "id": "pa-gfx950-b128", "priority": 100, "environment": dict(ENV),
            "workload": {"dtype": "bf16", "batch": [128, 128], "head_dim": 128},
            "winner": {"provider": "native", "artifact": "lib/pa.py", "entrypoint": "decode_mfma",
                       "sha256": digest, "format": "python_extension"},
            "launch": {"partition_tokens": 2048}, "fallbacks": list(fallbacks), "evidence_id": "evidence-pa",
        })
    return DispatchManifest.from_mapping({"schema_version": "1.0", "operator": "paged_attention_decode",
                                          "semantic_version": "1.0", "default_fallbacks": list(fallbacks) or ["torch"],
                                          "entries": entries})


class FakePacks:
    def __init__(self, root: Path, fail: Exception | None = None):
        self.root, self.fail, self.calls = root, fail, 0

    def resolve(self, **_):
        self.calls += 1
        if self.fail is not None:
            raise self.fail
        return SimpleNamespace(pack=SimpleNamespace(root=self.root, pack_id="pack", pack_version="1.0.0"))


class FakeLoader:
    behaviour = "ok"

    def __init__(self, _root):
        pass

    def load_entrypoint(self, _artifact):
        def call(*args, **launch):
            if FakeLoader.behaviour == "raise":
                raise ValueError("kernel rejected the shape")
            if FakeLoader.behaviour == "none":
                return None
            return ("native", args, launch)

        return SimpleNamespace(callable=call)


def run(runtime, fallback=lambda: "torch-result"):
    return runtime.execute(operator="paged_attention_decode", semantic_version="1.0", signature=SIGNATURE,
                           device_index=0, torch_module=object(), native_arguments=("q", "k"), fallback=fallback,
                           fallback_selected="torch/paged_attention")


def make(tmp_path, *, winner=True, packs=None, strict=False, fallbacks=("torch",)):
    clear_last_dispatch()
    FakeLoader.behaviour = "ok"
    packs = packs or FakePacks(tmp_path)
    runtime = OperatorRuntime(registry=DispatchRegistry([manifest(winner=winner, fallbacks=fallbacks)]),
                              pack_registry=packs, loader_factory=FakeLoader,
                              fingerprint_detector=lambda **_: fingerprint(), strict_native=strict)
    return runtime, packs


def test_fallback_only_manifest_executes_declared_fallback(tmp_path):
    runtime, packs = make(tmp_path, winner=False)
    assert run(runtime) == "torch-result"
    assert packs.calls == 0
    record = get_last_dispatch()
    assert record["selected"] == "torch/paged_attention"
    assert record["reason"].endswith("executed declared torch fallback")


def test_matching_entry_runs_native_winner_with_launch_parameters(tmp_path):
    runtime, packs = make(tmp_path)
    assert run(runtime) == ("native", ("q", "k"), {"partition_tokens": 2048})
    record = get_last_dispatch()
    assert record["selected"] == "native/decode_mfma"
    assert record["entry_id"] == "pa-gfx950-b128"
    assert record["evidence_id"] == "evidence-pa"
    assert "loaded pack pack 1.0.0" in record["reason"]


@pytest.mark.parametrize("behaviour, error", [("raise", "kernel rejected the shape"),
                                               ("none", "returned no output")])
def test_native_failure_demotes_to_fallback_with_warning(tmp_path, behaviour, error):
    runtime, _ = make(tmp_path)
    FakeLoader.behaviour = behaviour
    with pytest.warns(NativeDemotionWarning, match="decode_mfma unavailable"):
        assert run(runtime) == "torch-result"
    record = get_last_dispatch()
    assert record["selected"] == "torch/paged_attention"
    assert f"winner unavailable: {error}" in record["reason"] or error in record["reason"]


def test_missing_pack_demotes(tmp_path):
    runtime, _ = make(tmp_path, packs=FakePacks(tmp_path, fail=PackResolutionError("no installed kernel pack")))
    with pytest.warns(NativeDemotionWarning):
        assert run(runtime) == "torch-result"
    assert "no installed kernel pack" in get_last_dispatch()["reason"]


def test_strict_native_mode_raises_instead_of_demoting(tmp_path):
    runtime, _ = make(tmp_path, strict=True)
    FakeLoader.behaviour = "raise"
    with pytest.raises(OperatorDispatchError, match="native winner"):
        run(runtime)
    assert get_last_dispatch()["selected"] == "none"


def test_no_fallback_declared_raises(tmp_path):
    runtime, _ = make(tmp_path, fallbacks=("hipblaslt",))
    FakeLoader.behaviour = "raise"
    with pytest.warns(NativeDemotionWarning), pytest.raises(OperatorDispatchError, match="no approved implementation"):
        run(runtime)
    assert get_last_dispatch()["reason"].endswith("no supported fallback is available")


def test_fallback_failure_is_recorded_and_reraised(tmp_path):
    runtime, _ = make(tmp_path, winner=False)

    def broken():
        raise RuntimeError("out of memory")

    with pytest.raises(RuntimeError, match="out of memory"):
        run(runtime, broken)
    assert get_last_dispatch()["reason"] == "torch fallback failed: out of memory"


def test_fingerprint_is_detected_once_per_device(tmp_path):
    calls = []

    def detect(**kwargs):
        calls.append(kwargs["device_index"])
        return fingerprint()

    runtime = OperatorRuntime(registry=DispatchRegistry([manifest(winner=False)]), pack_registry=FakePacks(tmp_path),
                              fingerprint_detector=detect)
    for _ in range(3):
        run(runtime)
    assert calls == [0]


# ---------------------------------------------------------------------------------------------
def write_pack(root: Path, *, env=None, digest=None, evidence="evidence-pa", extra=None):
    (root / "lib").mkdir(parents=True, exist_ok=True)
    artifact = root / "lib" / "pa.py"
    artifact.write_text("def decode_mfma(*a, **k):\n    return ('pack', a, k)\n")
    document = {
        "schema_version": "1.0", "pack_id": "rk-pa-test", "pack_version": "1.0.0", "environment": env or dict(ENV),
        "artifacts": [{"operator": "paged_attention_decode", "semantic_version": "1.0", "provider": "native",
                       "artifact": "lib/pa.py", "entrypoint": "decode_mfma",
                       "sha256": digest or hashlib.sha256(artifact.read_bytes()).hexdigest(),
                       "format": "python_extension", "evidence_id": evidence}],
    }
    if extra:
        document.update(extra)
    (root / "manifest.json").write_text(json.dumps(document), encoding="utf-8")
    sign_manifest(root)
    return hashlib.sha256(artifact.read_bytes()).hexdigest()


def sign_manifest(root: Path, key=TEST_KEY, key_id="rk-test"):
    digest = hashlib.sha256((root / "manifest.json").read_bytes()).hexdigest()
    envelope = signature_document(private_key=key, key_id=key_id, signed_file="manifest.json", signed_sha256=digest)
    (root / "manifest.sig.json").write_text(json.dumps(envelope), encoding="utf-8")


def test_pack_discovery_resolution_and_end_to_end(tmp_path):
    digest = write_pack(tmp_path / "packs" / "gfx950")
    write_pack(tmp_path / "packs" / "broken", extra={"unexpected": 1})
    registry = KernelPackRegistry.discover([tmp_path / "packs"], trusted_keys=TEST_KEYRING)
    assert [p.pack_id for p in registry.packs] == ["rk-pa-test"]
    assert len(registry.rejected) == 1 and "unknown fields" in registry.rejected[0]
    spec = ArtifactSpec("native", "lib/pa.py", "decode_mfma", digest)
    resolved = registry.resolve(fingerprint=fingerprint(), operator="paged_attention_decode", semantic_version="1.0",
                                artifact=spec, evidence_id="evidence-pa")
    assert resolved.pack.pack_id == "rk-pa-test"
    with pytest.raises(PackResolutionError, match="1 invalid pack"):
        registry.resolve(fingerprint=fingerprint(rocm_abi="7.1"), operator="paged_attention_decode",
                         semantic_version="1.0", artifact=spec, evidence_id="evidence-pa")
    with pytest.raises(PackResolutionError):
        registry.resolve(fingerprint=fingerprint(), operator="paged_attention_decode", semantic_version="1.0",
                         artifact=spec, evidence_id="other-evidence")
    clear_last_dispatch()
    runtime = OperatorRuntime(registry=DispatchRegistry([manifest(winner=True, digest=digest)]),
                              pack_registry=registry, fingerprint_detector=lambda **_: fingerprint())
    assert run(runtime) == ("pack", ("q", "k"), {"partition_tokens": 2048})
    assert get_last_dispatch()["selected"] == "native/decode_mfma"


def test_corrupted_artifact_demotes(tmp_path):
    digest = write_pack(tmp_path / "packs" / "gfx950")
    (tmp_path / "packs" / "gfx950" / "lib" / "pa.py").write_text("def decode_mfma(*a, **k):\n    return 'tampered'\n")
    registry = KernelPackRegistry.discover([tmp_path / "packs"], trusted_keys=TEST_KEYRING)
    clear_last_dispatch()
    runtime = OperatorRuntime(registry=DispatchRegistry([manifest(winner=True, digest=digest)]),
                              pack_registry=registry, fingerprint_detector=lambda **_: fingerprint())
    with pytest.warns(NativeDemotionWarning):
        assert run(runtime) == "torch-result"
    assert "SHA-256 mismatch" in get_last_dispatch()["reason"]


def test_packs_load_only_with_a_valid_manifest_signature(tmp_path):
    """The registry verifies manifest.sig.json before reading a pack (reference packs.py:88-113)."""

    root = tmp_path / "packs"
    write_pack(root / "signed")
    write_pack(root / "unsigned")
    (root / "unsigned" / "manifest.sig.json").unlink()
    write_pack(root / "tampered")
    manifest = root / "tampered" / "manifest.json"
    manifest.write_text(manifest.read_text().replace("rk-pa-test", "rk-pa-test-2"))
    write_pack(root / "other-key")
    sign_manifest(root / "other-key", key=Ed25519PrivateKey.from_private_bytes(b"\1" * 32))
    write_pack(root / "unknown-key")
    sign_manifest(root / "unknown-key", key_id="rk-unknown")
    registry = KernelPackRegistry.discover([root], trusted_keys=TEST_KEYRING)
    assert [p.root.name for p in registry.packs] == ["signed"]
    reasons = {Path(line.split(":", 1)[0]).name: line for line in registry.rejected}
    assert "cannot read detached signature" in reasons["unsigned"]
    assert "SHA-256 mismatch" in reasons["tampered"]
    assert "invalid Ed25519 signature" in reasons["other-key"]
    assert "unknown key 'rk-unknown'" in reasons["unknown-key"]
    revoked = TrustedKeyring([TrustedKey("rk-test", TEST_KEY.public_key().public_bytes(), "revoked",
                                         "2026-12-01T00:00:00+00:00", "test")])
    assert KernelPackRegistry.discover([root / "signed"], trusted_keys=revoked).packs == ()
    assert len(KernelPackRegistry.discover([root], require_signatures=False).packs) == 5


def test_in_tree_pack_is_signed_by_a_key_of_the_builtin_keyring():
    from radeon_kernels.runtime.packs import IN_TREE_PACK_ROOT

    if not (IN_TREE_PACK_ROOT / "gfx950" / "manifest.json").is_file():
        pytest.fail("the kernel pack is not built; run __graft_entry__.build()")
    registry = KernelPackRegistry.discover([IN_TREE_PACK_ROOT])
    assert [p.pack_id for p in registry.packs] == ["rk-paged-attention-gfx950"] and registry.rejected == ()


def test_default_pack_roots_order(tmp_path):
    roots = default_pack_roots(environ={"RADEON_KERNELS_PACK_PATH": f"{tmp_path}/a:{tmp_path}/b"},
                               home=tmp_path / "home", prefix=tmp_path / "prefix")
    assert roots[:2] == ((tmp_path / "a").absolute(), (tmp_path / "b").absolute())
    assert roots[2] == (tmp_path / "home" / ".local" / "share" / "radeon-kernels" / "packs").absolute()
    assert roots[3] == (tmp_path / "prefix" / "share" / "radeon-kernels" / "packs").absolute()
    assert roots[4].name == "packs" and roots[4].parent.name == "radeon-kernels_amd"
    assert len(default_pack_roots(environ={}, include_in_tree=False)) == 2
