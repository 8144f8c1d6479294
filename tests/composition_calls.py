"""The oracle side of the composition pin (test infrastructure, no transformers import).

The oracle runs a short prompt the way the reference's worker drives the engine
(src/worker.rs:291-323 for the feed, :197-255 for the decode step): prefill in chunks of 5 with
the MTP catch-up after each, the first draft, a checkpointed verify [t, d] left accepted, then the
draft over the 2 pairs that follows an accept.  The independent side, the same model composed
from transformers' Qwen3.5 modules, was run once on the same weights and tokens by
tests/golden/make_composition.py; its outputs are the fixture tests/golden/composition.npz.
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

PROMPT_LEN = 11
CHUNK = 5
K_MHC_ATTN, K_MHC_FFN = 11, 12


def cfgs():
    """The three model shapes of the pin: the tiny config without mHC or loop, with the loop, and
    with both (the configuration the GPU tests use)."""
    import snl.config as C

    tiny = C.tiny_config()
    plain = dataclasses.replace(tiny, mhc=None, loop_count=1)
    looped = dataclasses.replace(tiny, mhc=None)
    return {"mhc_loop": tiny, "plain": plain, "loop": looped}


def prompt_for(seed: int, vocab: int):
    return np.random.default_rng(seed).integers(0, vocab, PROMPT_LEN).tolist()


def run_oracle(oracle, cfg, seed, quant, prompt, setup=None):
    """The oracle engine after the calls, and their outputs: prefill / draft1 / verify / draft2
    logits and the tokens t (prefill pick), d (first draft), t2 (verify row 1 pick)."""
    o = oracle.Engine(cfg, seed=seed, quant=quant, ctx=64, max_m=CHUNK)
    if setup:
        setup(o)
    n = len(prompt)
    pos = [[i] * 3 for i in range(n)]
    lg = None
    for c0 in range(0, n, CHUNK):
        c1 = min(c0 + CHUNK, n)
        lg = o.forward(prompt[c0:c1], pos[c0:c1], logit_rows=1 if c1 == n else 0)
        r0 = 1 if c0 == 0 else 0
        o.mtp(r0, prompt[c0 + r0:c1], pos[c0 + r0 - 1:c1 - 1], c0 + r0 - 1, False)
    out = {"prefill": lg[0]}
    t = int(np.argmax(lg[0]))
    d, dl = o.mtp(o.hid_rows, [t], [[n - 1] * 3], n - 1, True)
    out["draft1"] = dl
    out["t"], out["d"] = t, d
    v = o.forward([t, d], [[n] * 3, [n + 1] * 3], logit_rows=2, ckpt=True)
    out["verify"] = v
    t2 = int(np.argmax(v[1]))
    out["t2"] = t2
    _, dl2 = o.mtp(1, [d, t2], [[n] * 3, [n + 1] * 3], n, True)
    out["draft2"] = dl2
    return o, out


def closed_form_coef(b):
    """Coefficients of a zero router with biases b (src/shaders/layers.wgsl:94-126): sigmoid gates
    and the Sinkhorn limit of exp([[b4, b5], [b6, b7]]), p = sigmoid((b4 + b7 - b5 - b6) / 2),
    since the iteration keeps the cross ratio."""
    s = lambda v: 1.0 / (1.0 + math.exp(-v))  # noqa: E731
    p = s((b[4] + b[7] - b[5] - b[6]) / 2.0)
    return [s(b[0]), s(b[1]), 2 * s(b[2]), 2 * s(b[3]), p, 1 - p, 1 - p, p]


def zero_router(cfg, seed=3):
    """Biases per mHC site (router weights zero), the closed-form coefficients they fix, and the
    oracle set-up that installs them."""
    h = cfg.hidden
    r = np.random.default_rng(seed)
    biases, override = {}, {}
    for l in range(cfg.mhc[0], cfg.mhc[1]):
        for which, kind in (("attn", K_MHC_ATTN), ("ffn", K_MHC_FFN)):
            b = np.concatenate([r.uniform(-1.5, 1.5, 4), r.uniform(-0.6, 0.6, 4)]).astype(np.float32)
            biases[(l, kind)] = b
            override[(l, which)] = closed_form_coef([float(v) for v in b])

    def setup(o):
        for (l, kind), b in biases.items():
            o.set_vector(l, kind, np.concatenate([np.zeros(16 * h, np.float32), b]))

    return override, setup


# (case name, model shape, seed, quant, zero router): the composition fixture holds, per case,
# the independent side's logits for the oracle calls above
CASES = [(f"{name}_{'q8' if q == 0 else 'q4'}", name, 7 + q, q, False)
         for name in ("plain", "loop", "mhc_loop") for q in (0, 1)] + [("zero_router", "mhc_loop", 11, 0, True)]
# the planted mistakes of the independent side (mhc_loop, seed 5, Q8_0)
PLANTED_SEED = 5
