"""Pins the oracle's model composition (oracle/snl_oracle_engine.inc: run_layers, orc_forward,
orc_mtp) against an independent composition built from transformers' Qwen3.5 modules.

The independent side (tests/golden/qwen35_compose.py, run once by
tests/golden/make_composition.py into tests/golden/composition.npz) took the oracle's dequantised
weights through the converter's fused layouts (src/convert.rs:203-311) onto `Qwen3_5Attention`,
`Qwen3_5GatedDeltaNet`, `Qwen3_5MLP` and `Qwen3_5RMSNorm`, composed in the order of
src/engine.rs:383-493 and :495-570 over the whole token sequence at once from empty caches, in
float64.  Here the oracle runs the same tokens the way the engine does (tests/composition_calls.py):
in chunks, with a verify pass, the MTP catch-up, the first draft and the draft after an accepted
verify, and its logits are compared with the stored ones.

What a mistake would break:
* (1 + w) versus w in any norm;
* fc_e and fc_h swapped;
* the z / b / a rows of in_proj or the q / gate interleave mixed up;
* a wrong merge mode at the end of the mHC range;
* the loop plan, or the hidden-row bookkeeping of the MTP head (r0, slots, rotary positions).

The mHC router has no transformers counterpart.  Two checks cover it:
* the router fixed to W = 0 with chosen biases, whose coefficients follow in closed form
  (sigmoids, and the 2x2 Sinkhorn limit), the `zero_router` case;
* the seeded router, restated from src/shaders/layers.wgsl:75-126 in float64 on the independent
  side.
"""
import os

import numpy as np
import pytest

import composition_calls as CC

TOL = 3e-4  # relative to the largest |logit|: the oracle is f32, the composition f64 (measured 3e-5..1e-4)
FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "composition.npz")


@pytest.fixture(scope="module")
def comp():
    with np.load(FIXTURE) as z:
        return {k: z[k] for k in z.files}


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / np.abs(b).max())


def _errors(comp, case, ref):
    # the stored logits were computed for the tokens the oracle picked then: they must still be its picks
    assert [ref["t"], ref["d"], ref["t2"]] == comp[f"{case}_tokens"].tolist(), case
    return {"prefill": _rel(ref["prefill"], comp[f"{case}_prefill"]),
            "verify0": _rel(ref["verify"][0], comp[f"{case}_verify0"]),
            "verify1": _rel(ref["verify"][1], comp[f"{case}_verify1"]),
            "draft1": _rel(ref["draft1"], comp[f"{case}_draft1"]),
            "draft2": _rel(ref["draft2"], comp[f"{case}_draft2"])}


@pytest.mark.parametrize("case,shape,seed,quant,zero", CC.CASES, ids=[c[0] for c in CC.CASES])
def test_oracle_composition_matches_transformers(oracle, comp, case, shape, seed, quant, zero):
    """plain / loop / mhc_loop x Q8_0 / Q4_0, and the zero-router case: the mHC coefficients of
    every site fixed in closed form, so each site's pre-mix, post scale, mixing and the mode-2
    collapse at the range end are checked with no restated router arithmetic."""
    cfg = CC.cfgs()[shape]
    setup = None
    if zero:
        assert cfg.mhc[3] >= 20  # the limit is reached well inside the configured iterations
        _, setup = CC.zero_router(cfg)
    o, ref = CC.run_oracle(oracle, cfg, seed, quant, CC.prompt_for(seed, cfg.vocab), setup)
    o.close()
    errs = _errors(comp, case, ref)
    assert max(errs.values()) < TOL, errs


def test_composition_detects_planted_mistakes(oracle, comp):
    """The comparison has teeth: the composition with one plausible mistake planted disagrees with
    the oracle by far more than the tolerance (measured 0.4 and more): the final norm as w instead of
    1 + w, mode 1 instead of mode 2 at the end of the mHC range, fc_e and fc_h swapped."""
    cfg = CC.cfgs()["mhc_loop"]
    o, ref = CC.run_oracle(oracle, cfg, CC.PLANTED_SEED, 0, CC.prompt_for(CC.PLANTED_SEED, cfg.vocab))
    o.close()
    assert [ref["t"], ref["d"], ref["t2"]] == comp["planted_tokens"].tolist()
    assert _rel(ref["prefill"], comp["planted_norm_prefill"]) > 0.05
    assert _rel(ref["prefill"], comp["planted_merge_prefill"]) > 0.05
    assert _rel(ref["draft1"], comp["planted_fc_draft1"]) > 0.05
