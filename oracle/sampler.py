"""Restatement of the reference's sampler (src/sampler.rs) and of its random stream.

TEST INFRASTRUCTURE ONLY: imported by tests/, never by the shipped library.

Sampler::distribution (:98-141): penalties on the logits, greedy argmax at temperature <= 1e-5,
otherwise the top-k candidates (value descending, index ascending on ties, as top_k_small keeps
them), their temperature softmax, min-p, top-p and renormalisation.  Sampler::draw (:143-158),
Sampler::sample (:55-60) and Sampler::verify (:62-75).  Arithmetic on probabilities is float32 in
the reference's order.

The random stream is rand 0.10.3's StdRng (Cargo.lock): ChaCha12 (chacha20 0.10.2; 64-bit block
counter in words 12-13, stream 0 in words 14-15) keyed by rand_core 0.10.1's seed_from_u64
(eight PCG32 outputs as little-endian words), and random::<f32>() = (next_u32 >> 8) * 2^-24.

Parity: the ChaCha block function is pinned by RFC 7539's block test vector and the zero-key
keystream (tests/test_sampler.py); the distribution, draw and verify by hand-worked cases and an
exact integration of verify's output distribution.  The seed expansion's PCG32 arithmetic (the
LCG multiplier and the XSH-RR output) is pinned by the PCG reference implementation's demo outputs
(pcg32_srandom_r(42, 54)); its increment and its advance-then-output order follow rand_core's
published source, and the f32 conversion rand's: with no Rust here nothing checks those against
the crates' own output, so parity is unpinned for those two.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Tuple

import numpy as np

M32 = 0xFFFFFFFF
F32 = np.float32


def _rotl(x: int, n: int) -> int:
    return ((x << n) | (x >> (32 - n))) & M32


def chacha_block(state: List[int], rounds: int) -> List[int]:
    x = list(state)

    def q(a, b, c, d):
        x[a] = (x[a] + x[b]) & M32
        x[d] = _rotl(x[d] ^ x[a], 16)
        x[c] = (x[c] + x[d]) & M32
        x[b] = _rotl(x[b] ^ x[c], 12)
        x[a] = (x[a] + x[b]) & M32
        x[d] = _rotl(x[d] ^ x[a], 8)
        x[c] = (x[c] + x[d]) & M32
        x[b] = _rotl(x[b] ^ x[c], 7)

    for _ in range(rounds // 2):
        q(0, 4, 8, 12)
        q(1, 5, 9, 13)
        q(2, 6, 10, 14)
        q(3, 7, 11, 15)
        q(0, 5, 10, 15)
        q(1, 6, 11, 12)
        q(2, 7, 8, 13)
        q(3, 4, 9, 14)
    return [(x[i] + state[i]) & M32 for i in range(16)]


PCG_MUL = 6364136223846793005
SEED_INC = 11634580027462260723  # the increment of rand_core's seed_from_u64


def lcg(state: int, inc: int = SEED_INC) -> int:
    """PCG32's state step."""
    return (state * PCG_MUL + inc) & ((1 << 64) - 1)


def xsh_rr(state: int) -> int:
    """PCG32's output function (xorshift high, random rotation right)."""
    xorshifted = (((state >> 18) ^ state) >> 27) & M32
    rot = state >> 59
    return ((xorshifted >> rot) | (xorshifted << ((32 - rot) & 31))) & M32


def pcg32(state: int) -> Tuple[int, int]:
    """One word of rand_core's seed_from_u64: the state advances first, then the new state's output."""
    state = lcg(state)
    return state, xsh_rr(state)


class StdRng:
    CONST = [0x61707865, 0x3320646E, 0x79622D32, 0x6B206574]

    def __init__(self, seed: int):
        st = seed & ((1 << 64) - 1)
        self.key = []
        for _ in range(8):
            st, w = pcg32(st)
            self.key.append(w)
        self.counter = 0
        self.buf: List[int] = []

    def u32(self) -> int:
        if not self.buf:
            state = self.CONST + self.key + [self.counter & M32, self.counter >> 32, 0, 0]
            self.buf = chacha_block(state, 12)
            self.counter += 1
        return self.buf.pop(0)

    def f32(self) -> float:
        return float(F32(self.u32() >> 8) * F32(1.0 / 16777216.0))


def penalise(logits: np.ndarray, counts: Dict[int, int], rep: float, presence: float, frequency: float) -> np.ndarray:
    """src/sampler.rs:99-106 on a float32 copy."""
    out = logits.astype(np.float32).copy()
    for t, c in counts.items():
        v = out[t]
        if rep != 1.0:
            v = v / F32(rep) if v > 0 else v * F32(rep)
        out[t] = F32(v) - (F32(presence) + F32(frequency) * F32(c))
    return out


def top_k(logits: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest values, value descending and index ascending on ties."""
    order = np.lexsort((np.arange(len(logits)), -logits.astype(np.float64)))
    return order[:k]


def finish(vals: np.ndarray, temperature: float, min_p: float, top_p: float) -> np.ndarray:
    """src/sampler.rs:111-140 over candidate logits in descending order: the kept probabilities."""
    vals = vals.astype(np.float32)
    mx = vals[0]
    probs = [F32(np.exp(F32(F32(v - mx) / F32(temperature)))) for v in vals]
    s = F32(0.0)
    for p in probs:
        s = F32(s + p)
    probs = [F32(p / s) for p in probs]
    keep = len(probs)
    if min_p > 0.0:
        thresh = F32(probs[0] * F32(min_p))
        c = 0
        while c < len(probs) and probs[c] >= thresh:
            c += 1
        keep = max(c, 1)
    if top_p < 1.0:
        cum = F32(0.0)
        for i in range(keep):
            cum = F32(cum + probs[i])
            if cum >= F32(top_p):
                keep = i + 1
                break
    total = F32(0.0)
    for p in probs[:keep]:
        total = F32(total + p)
    return np.array([F32(p / total) for p in probs[:keep]], np.float32)


def distribution(logits: np.ndarray, counts: Dict[int, int], p: dict):
    """(greedy, tokens, probs) of Sampler::distribution."""
    lg = penalise(logits, counts, p["repetition_penalty"], p["presence_penalty"], p["frequency_penalty"])
    if p["temperature"] <= 1e-5:
        return True, np.array([int(np.argmax(lg))]), np.array([1.0], np.float32)
    k = len(lg) if p["top_k"] == 0 else min(p["top_k"], len(lg))
    idx = top_k(lg, k)
    probs = finish(lg[idx], p["temperature"], p["min_p"], p["top_p"])
    return False, idx[:len(probs)], probs


def draw(tokens, probs, exclude: Optional[int], u: float) -> int:
    total = F32(0.0)
    for t, q in zip(tokens, probs):
        if t != exclude:
            total = F32(total + F32(q))
    r = F32(F32(u) * total)
    last = int(tokens[0])
    for t, q in zip(tokens, probs):
        if t == exclude:
            continue
        r = F32(r - F32(q))
        last = int(t)
        if r <= 0.0:
            return int(t)
    return last


def verify(greedy: bool, tokens, probs, draft: int, rng) -> Tuple[bool, int]:
    if greedy:
        return int(tokens[0]) == draft, int(tokens[0])
    p_draft = 0.0
    for t, q in zip(tokens, probs):
        if int(t) == draft:
            p_draft = float(q)
            break
    if p_draft > 0.0 and rng.f32() < p_draft:
        return True, draft
    return False, draw(tokens, probs, draft, rng.f32())
