"""Detached Ed25519 signatures over release files, and the trusted keyring.

Format and semantics of src/radeon_kernels/runtime/signing.py:21-279 in the reference, so that
signatures written here verify there and the reference's published signatures verify here:

* the signed message is ``b"radeon-kernels-ed25519-v1\\0" + signed_file + b"\\0" + sha256_hex`` --
  a domain-separated statement "file <name> has SHA-256 <digest>", not the file bytes themselves
  (signing.py:24,66-70);
* a signature is a ``*.sig.json`` envelope with exactly the fields schema_version "1.0", algorithm
  "ed25519", key_id, signed_file (normalized relative path), signed_sha256 (lowercase hex) and the
  base64 signature (schemas/signature.schema.json);
* a keyring (schemas/trusted-keys.schema.json) lists keys as active or revoked; verification
  refuses unknown and revoked keys, a file name other than the one signed, and content whose
  SHA-256 differs from the envelope's.

The Ed25519 arithmetic is radeon_kernels.runtime.ed25519 (RFC 8032, pure Python), standing in for
the ``cryptography`` package the reference imports.

The built-in keyring (radeon_kernels/keys/trusted-keys.json) holds release keys only: the reference's
release key (public data from its keys/trusted-keys.json, so its signed packs verify) and the gfx950
pack's release key.  A development key is trusted only through a separate keyring that
RADEON_KERNELS_DEV_TRUSTED_KEYS names, and never shadows a built-in key id.
"""

from __future__ import annotations

import base64
import hashlib
import hmac
import json
import os
import re
from collections.abc import Mapping, Sequence
from dataclasses import dataclass
from pathlib import Path, PurePosixPath
from typing import Any

from radeon_kernels.errors import ConfigError, RadeonKernelsError
from radeon_kernels.runtime.ed25519 import Ed25519PrivateKey, Ed25519PublicKey, InvalidSignature

SIGNATURE_DOMAIN = b"radeon-kernels-ed25519-v1\x00"
BUILTIN_KEYRING = Path(__file__).resolve().parents[1] / "keys" / "trusted-keys.json"

_IDENTIFIER = re.compile(r"^[a-z][a-z0-9_.-]*$")
_SHA256 = re.compile(r"^[0-9a-f]{64}$")
_KEY_FIELDS = {"key_id", "algorithm", "public_key", "status", "created_at", "reason"}
_ENVELOPE_FIELDS = {"schema_version", "algorithm", "key_id", "signed_file", "signed_sha256", "signature"}


class SignatureVerificationError(RadeonKernelsError):
    """A signature, or the file it covers, cannot be trusted."""


def sha256_file(path: Path) -> str:
    digest = hashlib.sha256()
    with path.open("rb") as handle:
        for block in iter(lambda: handle.read(1 << 20), b""):
            digest.update(block)
    return digest.hexdigest()


def _identifier(value: Any, where: str) -> str:
    if not isinstance(value, str) or not _IDENTIFIER.fullmatch(value):
        raise ConfigError(where, "expected a lowercase identifier")
    return value


def _relative_path(value: Any, where: str) -> str:
    if not isinstance(value, str) or not value:
        raise ConfigError(where, "expected a relative file path")
    parsed = PurePosixPath(value)
    if parsed.is_absolute() or ".." in parsed.parts or parsed.as_posix() != value:
        raise ConfigError(where, "expected a normalized relative file path")
    return value


def _base64(value: Any, where: str, length: int) -> bytes:
    if not isinstance(value, str):
        raise ConfigError(where, "expected base64 text")
    try:
        decoded = base64.b64decode(value, validate=True)
    except ValueError as error:
        raise ConfigError(where, "invalid base64 text") from error
    if len(decoded) != length:
        raise ConfigError(where, f"expected {length} decoded bytes")
    return decoded


def signature_payload(signed_file: str, signed_sha256: str) -> bytes:
    """The exact bytes an Ed25519 signature covers."""

    name = _relative_path(signed_file, "signature.signed_file")
    if not isinstance(signed_sha256, str) or not _SHA256.fullmatch(signed_sha256):
        raise ConfigError("signature.signed_sha256", "expected a lowercase SHA-256")
    return SIGNATURE_DOMAIN + name.encode("utf-8") + b"\x00" + signed_sha256.encode("ascii")


@dataclass(frozen=True)
class TrustedKey:
    key_id: str
    public_key: bytes
    status: str
    created_at: str
    reason: str | None = None

    def to_dict(self) -> dict[str, Any]:
        value = {"key_id": self.key_id, "algorithm": "ed25519",
                 "public_key": base64.b64encode(self.public_key).decode("ascii"), "status": self.status,
                 "created_at": self.created_at}
        if self.reason is not None:
            value["reason"] = self.reason
        return value


class TrustedKeyring:
    def __init__(self, keys: Sequence[TrustedKey]) -> None:
        if not keys:
            raise ConfigError("trusted-keys.keys", "expected at least one key")
        ids = [key.key_id for key in keys]
        if len(set(ids)) != len(ids):
            raise ConfigError("trusted-keys.keys", "key ids must be unique")
        self._keys = {key.key_id: key for key in keys}

    @property
    def keys(self) -> tuple[TrustedKey, ...]:
        return tuple(self._keys.values())

    @classmethod
    def from_mapping(cls, value: Any, where: str = "trusted-keys") -> TrustedKeyring:
        if not isinstance(value, Mapping) or set(value) != {"schema_version", "keys"}:
            raise ConfigError(where, "expected exactly ['keys', 'schema_version']")
        if value["schema_version"] != "1.0":
            raise ConfigError(f"{where}.schema_version", "unsupported version")
        raw = value["keys"]
        if not isinstance(raw, list):
            raise ConfigError(f"{where}.keys", "expected a list")
        keys = []
        for index, item in enumerate(raw):
            at = f"{where}.keys[{index}]"
            if not isinstance(item, Mapping):
                raise ConfigError(at, "expected a mapping")
            unknown, missing = set(item) - _KEY_FIELDS, (_KEY_FIELDS - {"reason"}) - set(item)
            if unknown or missing:
                raise ConfigError(at, f"unknown={sorted(unknown)}, missing={sorted(missing)}")
            if item["algorithm"] != "ed25519":
                raise ConfigError(f"{at}.algorithm", "expected ed25519")
            if item["status"] not in ("active", "revoked"):
                raise ConfigError(f"{at}.status", "expected active or revoked")
            if not isinstance(item["created_at"], str) or not item["created_at"]:
                raise ConfigError(f"{at}.created_at", "expected a timestamp")
            reason = item.get("reason")
            if reason is not None and (not isinstance(reason, str) or not reason):
                raise ConfigError(f"{at}.reason", "expected non-empty text")
            keys.append(TrustedKey(_identifier(item["key_id"], f"{at}.key_id"),
                                   _base64(item["public_key"], f"{at}.public_key", 32), item["status"],
                                   item["created_at"], reason))
        return cls(keys)

    @classmethod
    def from_file(cls, path: Path) -> TrustedKeyring:
        try:
            value = json.loads(Path(path).read_text(encoding="utf-8"))
        except (OSError, json.JSONDecodeError) as error:
            raise ConfigError(str(path), f"cannot read trusted keys: {error}") from error
        return cls.from_mapping(value, str(path))

    def to_dict(self) -> dict[str, Any]:
        return {"schema_version": "1.0", "keys": [key.to_dict() for key in self._keys.values()]}

    def active_public_key(self, key_id: str) -> Ed25519PublicKey:
        key = self._keys.get(key_id)
        if key is None:
            raise SignatureVerificationError(f"signature uses unknown key {key_id!r}")
        if key.status != "active":
            raise SignatureVerificationError(f"signature key {key_id!r} is not active")
        try:
            return Ed25519PublicKey.from_public_bytes(key.public_key)
        except ValueError as error:
            raise SignatureVerificationError(f"key {key_id!r} is not an Ed25519 public key") from error


@dataclass(frozen=True)
class DetachedSignature:
    key_id: str
    signed_file: str
    signed_sha256: str
    signature: bytes

    @classmethod
    def from_mapping(cls, value: Any, where: str = "signature") -> DetachedSignature:
        if not isinstance(value, Mapping) or set(value) != _ENVELOPE_FIELDS:
            raise ConfigError(where, f"expected exactly {sorted(_ENVELOPE_FIELDS)}")
        if value["schema_version"] != "1.0" or value["algorithm"] != "ed25519":
            raise ConfigError(where, "unsupported signature version or algorithm")
        digest = value["signed_sha256"]
        if not isinstance(digest, str) or not _SHA256.fullmatch(digest):
            raise ConfigError(f"{where}.signed_sha256", "expected a lowercase SHA-256")
        return cls(_identifier(value["key_id"], f"{where}.key_id"),
                   _relative_path(value["signed_file"], f"{where}.signed_file"), digest,
                   _base64(value["signature"], f"{where}.signature", 64))

    @classmethod
    def from_file(cls, path: Path) -> DetachedSignature:
        try:
            value = json.loads(Path(path).read_text(encoding="utf-8"))
        except (OSError, json.JSONDecodeError) as error:
            raise SignatureVerificationError(f"cannot read detached signature {path}: {error}") from error
        try:
            return cls.from_mapping(value, str(path))
        except ConfigError as error:
            raise SignatureVerificationError(str(error)) from error

    def to_dict(self) -> dict[str, str]:
        return {"schema_version": "1.0", "algorithm": "ed25519", "key_id": self.key_id,
                "signed_file": self.signed_file, "signed_sha256": self.signed_sha256,
                "signature": base64.b64encode(self.signature).decode("ascii")}


def signature_document(*, private_key: Ed25519PrivateKey, key_id: str, signed_file: str,
                       signed_sha256: str) -> dict[str, str]:
    """The ``*.sig.json`` envelope for ``signed_file`` with content hash ``signed_sha256``."""

    _identifier(key_id, "signature.key_id")
    signature = private_key.sign(signature_payload(signed_file, signed_sha256))
    return DetachedSignature(key_id, signed_file, signed_sha256, signature).to_dict()


def verify_detached_content(content: bytes, signature: DetachedSignature | Mapping[str, Any],
                            keyring: TrustedKeyring, *, signed_file: str) -> DetachedSignature:
    envelope = signature if isinstance(signature, DetachedSignature) else DetachedSignature.from_mapping(signature)
    expected = _relative_path(signed_file, "signed_file")
    if envelope.signed_file != expected:
        raise SignatureVerificationError(f"signature names {envelope.signed_file!r}, expected {expected!r}")
    actual = hashlib.sha256(content).hexdigest()
    if not hmac.compare_digest(actual, envelope.signed_sha256):
        raise SignatureVerificationError(
            f"signed file SHA-256 mismatch: expected {envelope.signed_sha256}, got {actual}")
    public = keyring.active_public_key(envelope.key_id)
    try:
        public.verify(envelope.signature, signature_payload(envelope.signed_file, envelope.signed_sha256))
    except InvalidSignature as error:
        raise SignatureVerificationError("invalid Ed25519 signature") from error
    return envelope


def verify_detached_file(file_path: Path, signature_path: Path, keyring: TrustedKeyring, *,
                         signed_file: str | None = None) -> DetachedSignature:
    try:
        content = Path(file_path).read_bytes()
    except OSError as error:
        raise SignatureVerificationError(f"cannot read signed file {file_path}: {error}") from error
    return verify_detached_content(content, DetachedSignature.from_file(signature_path), keyring,
                                   signed_file=signed_file or Path(file_path).name)


def builtin_trusted_keyring() -> TrustedKeyring:
    """The release keys shipped with the package (never rewritten by a build)."""

    return TrustedKeyring.from_file(BUILTIN_KEYRING)


# A keyring file of development keys, trusted in addition to the built-in release keys only when this
# environment variable names it: packs signed on a build machine without a release key load only for a
# process that opts in.
DEV_KEYRING_ENV = "RADEON_KERNELS_DEV_TRUSTED_KEYS"


def default_trusted_keyring(environ: Mapping[str, str] | None = None) -> TrustedKeyring:
    """The built-in keyring, plus the development keyring named by ``RADEON_KERNELS_DEV_TRUSTED_KEYS``.

    A development keyring may add keys but never replace or shadow a built-in key id.
    """

    builtin = builtin_trusted_keyring()
    path = (os.environ if environ is None else environ).get(DEV_KEYRING_ENV, "")
    if not path:
        return builtin
    extra = TrustedKeyring.from_file(Path(path))
    clash = sorted({key.key_id for key in builtin.keys} & {key.key_id for key in extra.keys})
    if clash:
        raise ConfigError(f"{DEV_KEYRING_ENV}={path}", f"development keyring redefines built-in key ids {clash}")
    return TrustedKeyring([*builtin.keys, *extra.keys])
