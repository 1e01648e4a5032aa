"""Ed25519 signatures (RFC 8032, section 5.1) in pure Python.

The reference verifies release signatures with the ``cryptography`` package
(src/radeon_kernels/runtime/signing.py:14-18), which is not installed in this environment.  This
module is the same published algorithm written from the RFC's mathematics: the twisted Edwards
curve -x^2 + y^2 = 1 + d x^2 y^2 over GF(2^255 - 19), extended coordinates, SHA-512 from hashlib.
Signatures are deterministic, so anything it signs verifies under any conforming implementation
and vice versa.

It is used to verify pack manifests and promotion records and to sign this build's own records.
It is not constant-time: fine for verification and for signing with a development key on a build
machine, not for a long-lived release key on a shared host.
"""

from __future__ import annotations

import hashlib

P = 2**255 - 19
L = 2**252 + 27742317777372353535851937790883648493  # order of the base point
D = -121665 * pow(121666, P - 2, P) % P
SQRT_M1 = pow(2, (P - 1) // 4, P)

PUBLIC_KEY_BYTES = 32
SEED_BYTES = 32
SIGNATURE_BYTES = 64


class InvalidSignature(Exception):
    """The signature does not verify under the given public key."""


def _inverse(x: int) -> int:
    return pow(x, P - 2, P)


def _recover_x(y: int, sign: int) -> int | None:
    """x with x^2 = (y^2 - 1) / (d y^2 + 1) and the given low bit, or None when there is none."""

    if y >= P:
        return None
    x2 = (y * y - 1) * _inverse(D * y * y + 1) % P
    if x2 == 0:
        return None if sign else 0
    x = pow(x2, (P + 3) // 8, P)
    if (x * x - x2) % P:
        x = x * SQRT_M1 % P
    if (x * x - x2) % P:
        return None
    if (x & 1) != sign:
        x = P - x
    return x


# Points are (X, Y, Z, T) with x = X/Z, y = Y/Z and x*y = T/Z.
_IDENTITY = (0, 1, 1, 0)


def _add(p1: tuple[int, int, int, int], p2: tuple[int, int, int, int]) -> tuple[int, int, int, int]:
    x1, y1, z1, t1 = p1
    x2, y2, z2, t2 = p2
    a = (y1 - x1) * (y2 - x2) % P
    b = (y1 + x1) * (y2 + x2) % P
    c = 2 * D * t1 * t2 % P
    d = 2 * z1 * z2 % P
    e, f, g, h = b - a, d - c, d + c, b + a
    return e * f % P, g * h % P, f * g % P, e * h % P


def _multiply(scalar: int, point: tuple[int, int, int, int]) -> tuple[int, int, int, int]:
    result = _IDENTITY
    while scalar:
        if scalar & 1:
            result = _add(result, point)
        point = _add(point, point)
        scalar >>= 1
    return result


def _equal(p1: tuple[int, int, int, int], p2: tuple[int, int, int, int]) -> bool:
    x1, y1, z1, _ = p1
    x2, y2, z2, _ = p2
    return (x1 * z2 - x2 * z1) % P == 0 and (y1 * z2 - y2 * z1) % P == 0


def _encode(point: tuple[int, int, int, int]) -> bytes:
    x, y, z, _ = point
    zi = _inverse(z)
    x, y = x * zi % P, y * zi % P
    return int.to_bytes(y | ((x & 1) << 255), 32, "little")


def _decode(data: bytes) -> tuple[int, int, int, int] | None:
    if len(data) != 32:
        return None
    value = int.from_bytes(data, "little")
    y = value & ((1 << 255) - 1)
    x = _recover_x(y, value >> 255)
    if x is None:
        return None
    return x, y, 1, x * y % P


_BASE_Y = 4 * _inverse(5) % P
_BASE = (_recover_x(_BASE_Y, 0), _BASE_Y, 1, _recover_x(_BASE_Y, 0) * _BASE_Y % P)


def _hash_int(*parts: bytes) -> int:
    return int.from_bytes(hashlib.sha512(b"".join(parts)).digest(), "little")


def _expand(seed: bytes) -> tuple[int, bytes]:
    if len(seed) != SEED_BYTES:
        raise ValueError(f"an Ed25519 private key seed is {SEED_BYTES} bytes")
    digest = hashlib.sha512(seed).digest()
    scalar = int.from_bytes(digest[:32], "little")
    scalar &= (1 << 254) - 8  # clear the three low bits and bit 255
    scalar |= 1 << 254
    return scalar, digest[32:]


def public_key(seed: bytes) -> bytes:
    """The 32-byte public key of a 32-byte private key seed."""

    scalar, _ = _expand(seed)
    return _encode(_multiply(scalar, _BASE))


def sign(seed: bytes, message: bytes) -> bytes:
    """The 64-byte signature R || S of ``message`` under the private key ``seed``."""

    scalar, prefix = _expand(seed)
    encoded_public = _encode(_multiply(scalar, _BASE))
    r = _hash_int(prefix, message) % L
    encoded_r = _encode(_multiply(r, _BASE))
    h = _hash_int(encoded_r, encoded_public, message) % L
    s = (r + h * scalar) % L
    return encoded_r + int.to_bytes(s, 32, "little")


def verify(public: bytes, message: bytes, signature: bytes) -> bool:
    """True when ``signature`` is a valid signature of ``message`` under ``public``.

    Checks [S]B = R + [k]A with k = SHA-512(R || A || M) mod L; rejects S >= L and encodings that
    are not points of the curve.
    """

    if len(public) != PUBLIC_KEY_BYTES or len(signature) != SIGNATURE_BYTES:
        return False
    a_point = _decode(public)
    r_point = _decode(signature[:32])
    if a_point is None or r_point is None:
        return False
    s = int.from_bytes(signature[32:], "little")
    if s >= L:
        return False
    k = _hash_int(signature[:32], public, message) % L
    return _equal(_multiply(s, _BASE), _add(r_point, _multiply(k, a_point)))


class Ed25519PublicKey:
    """A verification key (32 bytes, RFC 8032 encoding)."""

    def __init__(self, data: bytes) -> None:
        if len(data) != PUBLIC_KEY_BYTES or _decode(data) is None:
            raise ValueError("not an Ed25519 public key")
        self._data = bytes(data)

    @classmethod
    def from_public_bytes(cls, data: bytes) -> Ed25519PublicKey:
        return cls(data)

    def public_bytes(self) -> bytes:
        return self._data

    def verify(self, signature: bytes, message: bytes) -> None:
        if not verify(self._data, message, signature):
            raise InvalidSignature("Ed25519 signature does not verify")


class Ed25519PrivateKey:
    """A signing key held as its 32-byte seed."""

    def __init__(self, seed: bytes) -> None:
        _expand(seed)  # validates the length
        self._seed = bytes(seed)

    @classmethod
    def generate(cls) -> Ed25519PrivateKey:
        import os

        return cls(os.urandom(SEED_BYTES))

    @classmethod
    def from_private_bytes(cls, seed: bytes) -> Ed25519PrivateKey:
        return cls(seed)

    def private_bytes(self) -> bytes:
        return self._seed

    def public_key(self) -> Ed25519PublicKey:
        return Ed25519PublicKey(public_key(self._seed))

    def sign(self, message: bytes) -> bytes:
        return sign(self._seed, message)
