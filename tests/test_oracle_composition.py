"""Pins the oracle's model composition (oracle/snl_oracle_engine.inc: run_layers, orc_forward,
orc_mtp) against an independent composition built from transformers' Qwen3.5 modules.

The independent side (tests/qwen35_compose.py) takes the oracle's dequantised weights and maps
them through the converter's fused layouts (src/convert.rs:203-311) onto `Qwen3_5Attention`,
`Qwen3_5GatedDeltaNet`, `Qwen3_5MLP` and `Qwen3_5RMSNorm`.  It then composes them in the order of
src/engine.rs:383-493 and :495-570, over the whole token sequence at once from empty caches.
The oracle runs the same tokens the way the engine does: in chunks, with a verify pass, the
MTP catch-up, the first draft and the draft after an accepted verify.

What a mistake would break:
* (1 + w) versus w in any norm;
* fc_e and fc_h swapped;
* the z / b / a rows of in_proj or the q / gate interleave mixed up;
* a wrong merge mode at the end of the mHC range;
* the loop plan, or the hidden-row bookkeeping of the MTP head (r0, slots, rotary positions).

The mHC router has no transformers counterpart.  Two checks cover it:
* the router fixed to W = 0 with chosen biases, whose coefficients follow in closed form
  (sigmoids, and the 2x2 Sinkhorn limit p = sigmoid((b4 + b7 - b5 - b6) / 2), since the
  iteration keeps the cross ratio);
* the seeded router, restated from src/shaders/layers.wgsl:75-126 in float64.
"""
import dataclasses
import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")

import qwen35_compose as QC  # noqa: E402

TOL = 3e-4  # relative to the largest |logit|: the oracle is f32, the composition f64 (measured 3e-5..1e-4)


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / np.abs(b).max())


def _cfgs():
    import snl.config as C

    tiny = C.tiny_config()
    plain = dataclasses.replace(tiny, mhc=None, loop_count=1)
    looped = dataclasses.replace(tiny, mhc=None)
    return {"mhc_loop": tiny, "plain": plain, "loop": looped}


def _run_oracle(oracle, cfg, seed, quant, prompt, setup=None):
    """Oracle calls as the worker makes them: prefill in chunks of 5, the MTP catch-up, the
    first draft, a checkpointed verify [t, d] left accepted, the next draft over 2 pairs."""
    o = oracle.Engine(cfg, seed=seed, quant=quant, ctx=64, max_m=5)
    if setup:
        setup(o)
    n = len(prompt)
    pos = [[i] * 3 for i in range(n)]
    lg = None
    for c0 in range(0, n, 5):  # Worker::feed (src/worker.rs:291-323): each chunk, then its MTP pairs
        c1 = min(c0 + 5, n)
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


def _check(oracle, cfg, seed, quant, setup=None, coef_override=None):
    prompt = np.random.default_rng(seed).integers(0, cfg.vocab, 11).tolist()
    o, ref = _run_oracle(oracle, cfg, seed, quant, prompt, setup)
    comp = QC.Composed(o, cfg, oracle.dequant, coef_override)
    n = len(prompt)
    t, d, t2 = ref["t"], ref["d"], ref["t2"]
    logits, hid = comp.forward(prompt + [t, d])
    errs = {"prefill": _rel(ref["prefill"], logits[n - 1]), "verify0": _rel(ref["verify"][0], logits[n]),
            "verify1": _rel(ref["verify"][1], logits[n + 1])}
    # MTP pairs: (hidden of token i, token i + 1) at slot and rotary position i; then the draft pair
    # (hidden of token n - 1, t), and after the accepted verify (hidden of t, d), (hidden of d, t2)
    toks = prompt[1:] + [t]
    errs["draft1"] = _rel(ref["draft1"], comp.mtp(hid[:n], toks, list(range(n))))
    errs["draft2"] = _rel(ref["draft2"], comp.mtp(hid[:n + 2], toks + [d, t2], list(range(n + 2))))
    o.close()
    return errs


@pytest.mark.parametrize("quant", [0, 1], ids=["q8", "q4"])
@pytest.mark.parametrize("name", ["plain", "loop", "mhc_loop"])
def test_oracle_composition_matches_transformers(oracle, name, quant):
    cfg = _cfgs()[name]
    errs = _check(oracle, cfg, seed=7 + quant, quant=quant)
    assert max(errs.values()) < TOL, errs


def _closed_form_coef(b):
    """Coefficients of a zero router with biases b (layers.wgsl:94-126): sigmoid gates and the
    Sinkhorn limit of exp([[b4, b5], [b6, b7]])."""
    s = lambda v: 1.0 / (1.0 + math.exp(-v))  # noqa: E731
    p = s((b[4] + b[7] - b[5] - b[6]) / 2.0)
    return [s(b[0]), s(b[1]), 2 * s(b[2]), 2 * s(b[3]), p, 1 - p, 1 - p, p]


def test_oracle_mhc_zero_router_closed_form(oracle):
    """A zero router makes every mHC coefficient a constant known in closed form, so each site's
    pre-mix, post scale, mixing and the mode-2 collapse at the range end are checked with no
    restated router arithmetic."""
    cfg = _cfgs()["mhc_loop"]
    h = cfg.hidden
    r = np.random.default_rng(3)
    biases, override = {}, {}
    for l in range(cfg.mhc[0], cfg.mhc[1]):
        for which, kind in (("attn", QC.K_MHC_ATTN), ("ffn", QC.K_MHC_FFN)):
            b = np.concatenate([r.uniform(-1.5, 1.5, 4), r.uniform(-0.6, 0.6, 4)]).astype(np.float32)
            biases[(l, kind)] = b
            override[(l, which)] = _closed_form_coef([float(v) for v in b])
    # the limit is reached well inside the configured iterations at these cross ratios
    assert cfg.mhc[3] >= 20

    def setup(o):
        for (l, kind), b in biases.items():
            o.set_vector(l, kind, np.concatenate([np.zeros(16 * h, np.float32), b]))

    errs = _check(oracle, cfg, seed=11, quant=0, setup=setup, coef_override=override)
    assert max(errs.values()) < TOL, errs


def test_composition_detects_planted_mistakes(oracle):
    """The comparison has teeth: the composition with one plausible mistake planted disagrees by
    far more than the tolerance (measured 0.4 and more): the final norm as w instead of 1 + w,
    mode 1 instead of mode 2 at the end of the mHC range, fc_e and fc_h swapped."""
    cfg = _cfgs()["mhc_loop"]
    prompt = np.random.default_rng(5).integers(0, cfg.vocab, 11).tolist()
    o, ref = _run_oracle(oracle, cfg, 5, 0, prompt)
    comp = QC.Composed(o, cfg, oracle.dequant)
    n = len(prompt)
    good, _ = comp.forward(prompt + [ref["t"], ref["d"]])
    assert _rel(ref["prefill"], good[n - 1]) < TOL
    with torch.no_grad():
        comp.final_norm.weight -= 1.0  # (1 + w) -> w
    bad, _ = comp.forward(prompt + [ref["t"], ref["d"]])
    assert _rel(ref["prefill"], bad[n - 1]) > 0.05
    with torch.no_grad():
        comp.final_norm.weight += 1.0
    orig = QC.merge

    def wrong_merge(x0, x1, br, coef, mode):
        return orig(x0, x1, br, coef, 1 if mode == 2 else mode)

    QC.merge = wrong_merge
    try:
        bad2, _ = comp.forward(prompt + [ref["t"], ref["d"]])
    finally:
        QC.merge = orig
    assert _rel(ref["prefill"], bad2[n - 1]) > 0.05
    h = cfg.hidden
    _, hid = comp.forward(prompt + [ref["t"], ref["d"]])
    toks = prompt[1:] + [ref["t"]]
    assert _rel(ref["draft1"], comp.mtp(hid[:n], toks, list(range(n)))) < TOL
    comp.fc = torch.cat([comp.fc[:, h:], comp.fc[:, :h]], dim=1)
    assert _rel(ref["draft1"], comp.mtp(hid[:n], toks, list(range(n)))) > 0.05
    o.close()
