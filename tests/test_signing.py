"""Ed25519 signing, detached signatures, the keyring and this build's signed promotion records.

What pins the pure-Python Ed25519 (radeon_kernels/runtime/ed25519.py, RFC 8032 section 5.1):

* the RFC's own test vectors 1-3 (section 7.1): public key, signature and verification;
* every detached signature the reference publishes -- 164 envelopes over its evidence, approval,
  pack-index and compatibility records (tests/golden/reference_signing/signatures.json, made by
  tests/golden/make_golden.py) -- verifies under the reference's keyring, produced there by the
  ``cryptography`` package the reference imports (runtime/signing.py:14-18);
* altered envelopes, altered content, a non-canonical S and foreign keys are all rejected.

The envelope, payload and keyring rules follow the reference's runtime/signing.py:21-279.  The
schema checks use tests/_schema.py against the reference's own schemas (fixtures), pinned first on
the reference's signed records.
"""

from __future__ import annotations

import base64
import hashlib
import json
import os
import tarfile
from pathlib import Path

import pytest

import _schema
from radeon_kernels.errors import ConfigError
from radeon_kernels.runtime import ed25519
from radeon_kernels.runtime.signing import (
    DetachedSignature,
    SignatureVerificationError,
    TrustedKey,
    TrustedKeyring,
    builtin_trusted_keyring,
    signature_document,
    signature_payload,
    verify_detached_content,
    verify_detached_file,
)

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_signing"
PACKAGE = Path(__file__).resolve().parents[1] / "radeon-kernels_amd"

# RFC 8032 section 7.1, TEST 1-3: (secret key, public key, message, signature), hex.
RFC8032 = [
    ("9d61b19deffd5a60ba844af492ec2cc44449c5697b326919703bac031cae7f60",
     "d75a980182b10ab7d54bfed3c964073a0ee172f3daa62325af021a68f707511a", "",
     "e5564300c360ac729086e2cc806e828a84877f1eb8e5d974d873e065224901555fb8821590a33bacc61e39701cf9b46bd25bf5f0595bbe2465"
     "5141438e7a100b"),
    ("4ccd089b28ff96da9db6c346ec114e0f5b8a319f35aba624da8cf6ed4fb8a6fb",
     "3d4017c3e843895a92b70aa74d1b7ebc9c982ccf2ec4968cc0cd55f12af4660c", "72",
     "92a009a9f0d4cab8720e820b5f642540a2b27b5416503f8fb3762223ebdb69da085ac1e43e15996e458f3613d0f11d8c387b2eaeb4302aeeb0"
     "0d291612bb0c00"),
    ("c5aa8df43f9f837bedb7442f31dcb7b166d38535076f094b85ce3a2e0b4458f7",
     "fc51cd8e6218a1a38da47ed00230f0580816ed13ba3303ac5deb911548908025", "af82",
     "6291d657deec24024827e69c3abe01a30ce548a284743a445e3680d7db5ac3ac18ff9b538d16f290ae67f760984dc6594a7c15e9716ed28dc0"
     "27beceea1ec40a"),
]


def reference_keyring() -> TrustedKeyring:
    return TrustedKeyring.from_file(GOLDEN / "trusted-keys.json")


def reference_envelopes() -> list[dict]:
    return [item["envelope"] for item in json.loads((GOLDEN / "signatures.json").read_text())]


def schema(name: str) -> dict:
    return json.loads((GOLDEN / "schemas" / f"{name}.schema.json").read_text())


@pytest.mark.parametrize("vector", RFC8032, ids=["test1", "test2", "test3"])
def test_rfc8032_vectors(vector):
    secret, public, message, signature = (bytes.fromhex(x) for x in vector)
    assert ed25519.public_key(secret) == public
    assert ed25519.sign(secret, message) == signature
    assert ed25519.verify(public, message, signature)
    assert not ed25519.verify(public, message + b"\0", signature)


def test_every_reference_signature_verifies():
    keyring = reference_keyring()
    envelopes = reference_envelopes()
    assert len(envelopes) == 164
    for raw in envelopes:
        envelope = DetachedSignature.from_mapping(raw)
        keyring.active_public_key(envelope.key_id).verify(
            envelope.signature, signature_payload(envelope.signed_file, envelope.signed_sha256))


def test_altered_reference_signatures_are_rejected():
    keyring = reference_keyring()
    for raw in reference_envelopes()[:12]:
        envelope = DetachedSignature.from_mapping(raw)
        key = keyring.active_public_key(envelope.key_id)
        payload = signature_payload(envelope.signed_file, envelope.signed_sha256)
        flipped = bytearray(envelope.signature)
        flipped[5] ^= 0x10
        digit = "0" if envelope.signed_sha256[0] != "0" else "1"
        for signature, message in ((bytes(flipped), payload),
                                   (envelope.signature, signature_payload(envelope.signed_file,
                                                                          digit + envelope.signed_sha256[1:])),
                                   (envelope.signature, signature_payload("x" + envelope.signed_file,
                                                                          envelope.signed_sha256))):
            with pytest.raises(ed25519.InvalidSignature):
                key.verify(signature, message)
        # S + L encodes the same scalar but is not canonical: RFC 8032 requires rejecting it.
        s = int.from_bytes(envelope.signature[32:], "little") + ed25519.L
        if s < 2**256:
            assert not ed25519.verify(key.public_bytes(), payload, envelope.signature[:32] + s.to_bytes(32, "little"))


def test_signed_reference_documents_and_tampered_copies(tmp_path):
    keyring = reference_keyring()
    for signature in sorted(GOLDEN.glob("*.sig.json")):
        document = signature.with_name(signature.name.replace(".sig.json", ".json"))
        envelope = verify_detached_file(document, signature, keyring)
        assert envelope.signed_file == document.name
        altered = tmp_path / document.name
        altered.write_bytes(document.read_bytes().replace(b"gfx", b"gfy", 1))
        with pytest.raises(SignatureVerificationError, match="SHA-256 mismatch"):
            verify_detached_file(altered, signature, keyring)
        with pytest.raises(SignatureVerificationError, match="signature names"):
            verify_detached_file(document, signature, keyring, signed_file="other.json")


def test_keyring_rules():
    keyring = reference_keyring()
    (key,) = keyring.keys
    revoked = TrustedKeyring([TrustedKey(key.key_id, key.public_key, "revoked", key.created_at, "rotated")])
    with pytest.raises(SignatureVerificationError, match="not active"):
        revoked.active_public_key(key.key_id)
    with pytest.raises(SignatureVerificationError, match="unknown key"):
        keyring.active_public_key("rk-other")
    with pytest.raises(ConfigError, match="unique"):
        TrustedKeyring([key, key])
    raw = json.loads((GOLDEN / "trusted-keys.json").read_text())
    for mutate, message in ((lambda k: k.update(algorithm="rsa"), "ed25519"),
                            (lambda k: k.update(status="retired"), "active or revoked"),
                            (lambda k: k.update(comment="x"), "unknown"),
                            (lambda k: k.update(public_key=base64.b64encode(b"\0" * 31).decode()), "32 decoded")):
        bad = json.loads(json.dumps(raw))
        mutate(bad["keys"][0])
        with pytest.raises(ConfigError, match=message):
            TrustedKeyring.from_mapping(bad)


def test_envelope_strictness():
    raw = reference_envelopes()[0]
    for mutate, message in ((lambda e: e.update(extra=1), "expected exactly"),
                            (lambda e: e.update(algorithm="ed448"), "unsupported"),
                            (lambda e: e.update(signed_sha256=e["signed_sha256"].upper()), "lowercase SHA-256"),
                            (lambda e: e.update(signed_file="../x.json"), "normalized relative"),
                            (lambda e: e.update(signature=e["signature"][:-4]), "decoded bytes")):
        bad = dict(raw)
        mutate(bad)
        with pytest.raises(ConfigError, match=message):
            DetachedSignature.from_mapping(bad)


def test_sign_and_verify_round_trip():
    key = ed25519.Ed25519PrivateKey.generate()
    keyring = TrustedKeyring([TrustedKey("rk-test", key.public_key().public_bytes(), "active", "2026-12-01")])
    content = b'{"hello": "gfx950"}\n'
    document = signature_document(private_key=key, key_id="rk-test", signed_file="hello.json",
                                  signed_sha256=hashlib.sha256(content).hexdigest())
    assert document == signature_document(private_key=key, key_id="rk-test", signed_file="hello.json",
                                          signed_sha256=hashlib.sha256(content).hexdigest())  # deterministic
    assert not _schema.errors(document, schema("signature"))
    verify_detached_content(content, document, keyring, signed_file="hello.json")
    with pytest.raises(SignatureVerificationError):
        verify_detached_content(content, document, reference_keyring(), signed_file="hello.json")


# ---------------------------------------------------------------------------------------------
# The schema checker, pinned on the reference's records.
SIGNED_EXAMPLES = {"evidence": "m6-20260918-paged_attention_decode-gfx1201-b1-gqa32x8-c128-d128-p16-bf16.json",
                   "approval": "approval-proposal-m6-20260918-paged_attention_decode-gfx1201-b1-gqa32x8-c128-d128-p16-"
                               "bf16-3b9165d37c22d4c4-approved.json",
                   "pack-index": "paged_attention_decode-1.0.json"}


def test_reference_records_satisfy_reference_schemas():
    for name, file in SIGNED_EXAMPLES.items():
        assert _schema.errors(json.loads((GOLDEN / file).read_text()), schema(name)) == [], name
    assert _schema.errors(json.loads((GOLDEN / "trusted-keys.json").read_text()), schema("trusted-keys")) == []
    for envelope in reference_envelopes():
        assert _schema.errors(envelope, schema("signature")) == []


@pytest.mark.parametrize("mutation, fragment", [
    (lambda d: d.pop("guarantee_boundary"), "missing 'guarantee_boundary'"),
    (lambda d: d.update(extra=1), "unexpected property 'extra'"),
    (lambda d: d.update(candidate_content_hash="ABC"), "does not match"),
    (lambda d: d["correctness"]["cases"][0].update(max_absolute_error=-1.0), "below 0"),
    (lambda d: d["timing"].update(candidate_samples_ms=[1.0]), "fewer than 2 items"),
    (lambda d: d["timing"].update(candidate_median_ms=0), "not above 0"),
    (lambda d: d.update(decision="ship"), "not in"),
    (lambda d: d["environment"].update(wavefront_size=16), "not in"),
    (lambda d: d.update(schema_version="2.0"), "expected '1.0'"),
    (lambda d: d["workload"].update({"Bad Key": 1}), "does not match"),
    (lambda d: d["correctness"].update(passed="yes"), "expected type boolean"),
])
def test_schema_checker_catches_planted_violations(mutation, fragment):
    document = json.loads((GOLDEN / SIGNED_EXAMPLES["evidence"]).read_text())
    mutation(document)
    found = _schema.errors(document, schema("evidence"))
    assert any(fragment in item for item in found), found


# ---------------------------------------------------------------------------------------------
# This build's keyring and signed records.
def test_builtin_keyring_holds_release_keys_only():
    """The shipped trust root: the reference's release key and the gfx950 release key, nothing else
    (no development key of any build machine)."""

    keyring = builtin_trusted_keyring()
    assert not _schema.errors(keyring.to_dict(), schema("trusted-keys"))
    keys = {key.key_id: key for key in keyring.keys}
    assert sorted(keys) == ["rk-gfx950-release-2026-12", "rk-release-2026-09"]
    assert keys["rk-release-2026-09"].public_key == reference_keyring().keys[0].public_key
    assert keys["rk-gfx950-release-2026-12"].status == "active"
    assert all("development" not in (key.reason or "") for key in keys.values())


def _dev_keyring_file(tmp_path, key_id="rk-dev-test"):
    key = ed25519.Ed25519PrivateKey.from_private_bytes(bytes(range(32)))
    ring = TrustedKeyring([TrustedKey(key_id, key.public_key().public_bytes(), "active", "2026-12-02")])
    path = tmp_path / "dev-trusted-keys.json"
    path.write_text(json.dumps(ring.to_dict()))
    return path, key


def test_development_keyring_is_trusted_only_on_opt_in(tmp_path):
    from radeon_kernels.runtime.signing import DEV_KEYRING_ENV, default_trusted_keyring

    path, key = _dev_keyring_file(tmp_path)
    assert {k.key_id for k in default_trusted_keyring(environ={}).keys} == \
        {k.key_id for k in builtin_trusted_keyring().keys}
    merged = default_trusted_keyring(environ={DEV_KEYRING_ENV: str(path)})
    assert merged.active_public_key("rk-dev-test").public_bytes() == key.public_key().public_bytes()
    assert merged.active_public_key("rk-release-2026-09")  # built-in keys stay
    (tmp_path / "clash").mkdir()
    clash, _ = _dev_keyring_file(tmp_path / "clash", key_id="rk-release-2026-09")
    with pytest.raises(ConfigError, match="redefines built-in key ids"):
        default_trusted_keyring(environ={DEV_KEYRING_ENV: str(clash)})


def test_a_build_without_the_release_key_never_touches_the_builtin_keyring(tmp_path, monkeypatch):
    """publish.signing_key() on a machine without the release key: a development key signs, its public
    half goes to the machine's own dev keyring, and the shipped keyring's bytes are unchanged."""

    import importlib.util

    spec = importlib.util.spec_from_file_location("rk_publish_under_test", PACKAGE / "promotion" / "publish.py")
    publish = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(publish)
    before = publish.BUILTIN_KEYRING.read_bytes()
    monkeypatch.setattr(publish, "KEY_DIR", tmp_path / "signing")
    monkeypatch.setattr(publish, "DEV_KEYRING", tmp_path / "signing" / "dev-trusted-keys.json")
    key_id, key = publish.signing_key()
    assert key_id == "rk-gfx950-dev"
    assert publish.BUILTIN_KEYRING.read_bytes() == before
    dev = TrustedKeyring.from_file(tmp_path / "signing" / "dev-trusted-keys.json")
    assert dev.active_public_key(key_id).public_bytes() == key.public_key().public_bytes()
    with pytest.raises(SignatureVerificationError, match="unknown key"):
        builtin_trusted_keyring().active_public_key(key_id)
    with pytest.raises(ConfigError, match="already exists"):
        monkeypatch.setattr(publish, "KEY_DIR", tmp_path / "other")
        (tmp_path / "other").mkdir()
        publish.create_release_key()  # the shipped keyring already holds the release key id
    assert publish.BUILTIN_KEYRING.read_bytes() == before


def _records(directory: str) -> list[Path]:
    return sorted(p for p in (PACKAGE / directory).glob("*.json") if not p.name.endswith(".sig.json"))


def test_pack_manifest_signature_verifies():
    pack = PACKAGE / "packs" / "gfx950"
    verify_detached_file(pack / "manifest.json", pack / "manifest.sig.json", builtin_trusted_keyring())


def test_promotion_records_are_schema_valid_signed_and_consistent():
    evidence = _records("evidence")
    if not evidence:
        pytest.skip("no promoted operator: no GPU evaluation under radeon-kernels_amd/evaluations matches this build")
    keyring = builtin_trusted_keyring()
    approvals = {json.loads(p.read_text())["approval_id"]: p for p in _records("approvals")}
    proposals = {json.loads(p.read_text())["proposal_id"]: p for p in _records("proposals")}
    for kind, files in (("evidence", evidence), ("approval", list(approvals.values())),
                        ("pack-index", _records("pack-index"))):
        for path in files:
            document = json.loads(path.read_text())
            assert _schema.errors(document, schema(kind)) == [], path.name
            verify_detached_file(path, path.with_name(path.name[:-5] + ".sig.json"), keyring)
    manifest = PACKAGE / "packs" / "gfx950" / "manifest.json"
    for path in evidence:
        record = json.loads(path.read_text())
        approval = json.loads(approvals[record["approval_id"]].read_text())
        proposal_path = proposals[approval["proposal_id"]]
        assert approval["proposal_sha256"] == hashlib.sha256(proposal_path.read_bytes()).hexdigest()
        proposal = json.loads(proposal_path.read_text())
        assert all(proposal["gates"].values()) and record["decision"] == "promote"
        assert record["source_evidence_hashes"]["manifest"] == hashlib.sha256(manifest.read_bytes()).hexdigest()
        timing = record["timing"]
        import statistics

        reduction = (1 - statistics.median(timing["candidate_samples_ms"])
                     / statistics.median(timing["baseline_samples_ms"])) * 100
        assert abs(reduction - timing["latency_reduction_pct"]) < 1e-9
        assert timing["confidence_interval_pct"][0] >= 3.0 and timing["stable"]
        assert all(case["runtime_ok"] and case["finite"] for case in record["correctness"]["cases"])


def test_every_promoting_evaluation_is_published():
    """An evaluation whose promotion gates all pass for the built pack has its evidence and pack-index
    records in the tree.  The build publishes whatever promotes, so a missing record means the
    evaluation was installed without publishing (or a stale one withdrew the records)."""

    import importlib.util

    spec = importlib.util.spec_from_file_location("rk_publish_gates", PACKAGE / "promotion" / "publish.py")
    publish = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(publish)
    evidence_ids = {json.loads(p.read_text())["evidence_id"] for p in _records("evidence")}
    checked = 0
    for path in sorted((PACKAGE / "evaluations").glob("*-gfx950.json")):
        operator = json.loads(path.read_text())["operator"]
        proposal = publish.proposal_for(operator, path)
        if proposal["recommended_decision"] != "promote":
            continue
        checked += 1
        assert (PACKAGE / "pack-index" / f"{operator}-1.0.json").is_file(), operator
        assert proposal["public_evidence"]["evidence_id"] in evidence_ids, operator
        assert {record["evidence_id"] for record in proposal["entry_evidence"]} <= evidence_ids, operator
    if not checked:
        pytest.skip("no committed evaluation promotes this build")


def test_pack_index_records_name_this_pack_and_its_release_archive():
    records = _records("pack-index")
    if not records:
        pytest.skip("no promoted operator: no GPU evaluation under radeon-kernels_amd/evaluations matches this build")
    pack = PACKAGE / "packs" / "gfx950"
    manifest = json.loads((pack / "manifest.json").read_text())
    for path in records:
        (entry,) = json.loads(path.read_text())["packs"]
        assert entry["manifest_sha256"] == hashlib.sha256((pack / "manifest.json").read_bytes()).hexdigest()
        assert entry["manifest_signature"] == json.loads((pack / "manifest.sig.json").read_text())
        assert entry["artifacts"] == manifest["artifacts"] and entry["environment"] == manifest["environment"]
        archive = PACKAGE / "releases" / entry["release_file"]
        if not archive.is_file():
            continue  # release archives are build outputs, not committed
        data = archive.read_bytes()
        assert len(data) == entry["release_size"] and hashlib.sha256(data).hexdigest() == entry["release_sha256"]
        # The reference installer's payload rule (installer.py:187-220): exactly these regular files.
        expected = {f"{entry['pack_id']}/manifest.json", f"{entry['pack_id']}/manifest.sig.json",
                    *(f"{entry['pack_id']}/{a['artifact']}" for a in entry["artifacts"])}
        with tarfile.open(archive, "r:gz") as handle:
            members = handle.getmembers()
            assert {m.name for m in members if m.isfile()} == expected and all(m.isfile() for m in members)
            for member in members:
                assert handle.extractfile(member).read() == (pack / member.name.split("/", 1)[1]).read_bytes()


def test_signing_keys_stay_out_of_the_repository_history():
    ignore = (PACKAGE.parent / ".gitignore").read_text()
    assert "radeon-kernels_amd/.signing/" in ignore
    key_dir = PACKAGE / ".signing"
    if key_dir.is_dir():
        for path in key_dir.iterdir():
            assert os.stat(path).st_mode & 0o077 == 0, f"{path} must be private (0600)"
