"""Count sketches of gradient tensors: a fixed-size linear summary from which the relative L2 distance
between two tensors can be estimated without keeping either whole.

Element i of a tensor goes to bucket h(i) with sign s(i) (both from a SplitMix64 hash of i and the
tensor's name); the sketch is S(g)[b] = Σ_{h(i)=b} s(i)·g[i]. S is linear and E‖S(x)‖² = ‖x‖², so
‖S(a) − S(b)‖ / ‖S(b)‖ estimates rel-L2(a, b) with a relative spread of about √(2/B) (3 % at
B = 2048 buckets). Tensors of at most B elements are kept exactly instead.

Test infrastructure: used by the full-size parity tests and by the script that writes their fixtures
(tests/golden/make_fullsize_fixtures.py)."""
from __future__ import annotations

import zlib

import numpy as np

BUCKETS = 2048
_CHUNK = 1 << 22
_M1, _M2, _PHI = np.uint64(0xBF58476D1CE4E5B9), np.uint64(0x94D049BB133111EB), np.uint64(0x9E3779B97F4A7C15)


def _hash(idx: np.ndarray, salt: int) -> np.ndarray:
    z = idx * _PHI + np.uint64(salt)
    z ^= z >> np.uint64(30)
    z *= _M1
    z ^= z >> np.uint64(27)
    z *= _M2
    z ^= z >> np.uint64(31)
    return z


def salt_of(name: str) -> int:
    return zlib.crc32(name.encode()) * 0x100000001


def sketch(name: str, values: np.ndarray, buckets: int = BUCKETS) -> np.ndarray:
    """S(values) in float64: the exact values when they have at most `buckets` elements."""
    v = np.asarray(values).reshape(-1)
    if v.size <= buckets:
        return v.astype(np.float64)
    out = np.zeros(buckets, np.float64)
    salt = salt_of(name)
    with np.errstate(over="ignore"):
        for b in range(0, v.size, _CHUNK):
            chunk = v[b:b + _CHUNK].astype(np.float64)
            z = _hash(np.arange(b, b + chunk.size, dtype=np.uint64), salt)
            sign = 1.0 - 2.0 * (z >> np.uint64(63)).astype(np.float64)
            out += np.bincount((z % np.uint64(buckets)).astype(np.int64), weights=sign * chunk, minlength=buckets)
    return out


def rel_l2(sk_expected: np.ndarray, sk_actual: np.ndarray) -> float:
    e = np.asarray(sk_expected, np.float64)
    a = np.asarray(sk_actual, np.float64)
    return float(np.linalg.norm(e - a) / max(np.linalg.norm(e), 1e-30))


def top_entries(values: np.ndarray, k: int = 64):
    """Indices and values of the k largest-magnitude elements (for the reference's max|Δ|/max|g|)."""
    v = np.asarray(values).reshape(-1)
    k = min(k, v.size)
    idx = np.argpartition(np.abs(v), v.size - k)[v.size - k:]
    return idx.astype(np.int64), v[idx].astype(np.float64)
