"""Seeded synthetic inputs shared by the tests, the bench and the oracle runs.

SplitMix64 (Steele, Lea & Flood 2014) gives 64-bit words; the top 53 bits
make doubles in (0, 1]; the Box-Muller transform turns pairs of them into
standard normals in float64, which are rounded once to float32.  Element i of
a stream depends only on (seed, i), so any slice of a stream can be produced
without producing the rest, and the same numbers come out on every host.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, start: int, count: int) -> np.ndarray:
    """Words start..start+count-1 of the SplitMix64 stream for `seed`."""
    idx = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def uniform(seed: int, count: int, start: int = 0) -> np.ndarray:
    """float64 uniforms in (0, 1]."""
    words = splitmix64(seed, start, count)
    return ((words >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)


def normal(seed: int, count: int, sigma: float = 1.0, mean: float = 0.0,
           chunk: int = 1 << 22) -> np.ndarray:
    """`count` float32 draws of N(mean, sigma^2): Box-Muller over word pairs."""
    out = np.empty(count, dtype=np.float32)
    pairs_total = (count + 1) // 2
    done = 0
    while done < pairs_total:
        n = min(chunk, pairs_total - done)
        u = uniform(seed, 2 * n, start=2 * done)
        r = np.sqrt(-2.0 * np.log(u[0::2]))
        t = 2.0 * np.pi * u[1::2]
        z = np.empty(2 * n, dtype=np.float64)
        z[0::2] = r * np.cos(t)
        z[1::2] = r * np.sin(t)
        lo = 2 * done
        hi = min(count, lo + 2 * n)
        out[lo:hi] = (z[: hi - lo] * sigma + mean).astype(np.float32)
        done += n
    return out


def l2_normalise_heads(x: np.ndarray, head_dim: int) -> np.ndarray:
    """Per-head L2 normalisation in float64, rounded to float32."""
    h = x.astype(np.float64).reshape(-1, head_dim)
    h = h / np.maximum(np.sqrt((h * h).sum(axis=1, keepdims=True)), 1e-6)
    return h.reshape(x.shape).astype(np.float32)


def sigmoid64(x: np.ndarray) -> np.ndarray:
    return (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)


def neg_softplus64(x: np.ndarray) -> np.ndarray:
    """-softplus(x), the log of the decay exp(-softplus(x))."""
    x64 = x.astype(np.float64)
    return (-np.where(x64 > 20.0, x64, np.log1p(np.exp(np.minimum(x64, 20.0))))).astype(np.float32)


# Stream ids: every tensor of a config draws from its own seed so that resizing
# one tensor never shifts another.
def stream_seed(base: int, tensor: int) -> int:
    return (base * 0x100000001B3 + tensor * 0x9E3779B1) & 0xFFFFFFFFFFFFFFFF


class GdnStepInputs:
    """Per-step inputs of a Gated-DeltaNet decode run: q, k ~N(0,1) then L2
    normalised per 128-wide head, v ~N(0,1), beta = sigmoid(N(0,1)) and the
    log-decay g = -softplus(N(0,1))."""

    def __init__(self, seed: int, n_seq: int = 1):
        self.seed = seed
        self.n_seq = n_seq

    def step(self, t: int):
        n = self.n_seq
        s = stream_seed(self.seed, 1000 + t)
        q = l2_normalise_heads(normal(stream_seed(s, 1), n * 2048), 128)
        k = l2_normalise_heads(normal(stream_seed(s, 2), n * 2048), 128)
        v = normal(stream_seed(s, 3), n * 6144)
        beta = sigmoid64(normal(stream_seed(s, 4), n * 48))
        g = neg_softplus64(normal(stream_seed(s, 5), n * 48))
        return q, k, v, beta, g

    def steps(self, t0: int, count: int):
        parts = [self.step(t) for t in range(t0, t0 + count)]
        return tuple(np.stack([p[i] for p in parts]) for i in range(5))
