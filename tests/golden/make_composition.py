"""Writes tests/golden/composition.npz: the independent side of the oracle's composition pin.

    python tests/golden/make_composition.py      (from the repository root, on the CPU)

For each case of tests/composition_calls.py the oracle runs its calls (prefill in chunks, MTP
catch-up, first draft, accepted verify, 2-pair draft), and the same model composed from
transformers' Qwen3.5 modules (qwen35_compose.py, float64, whole sequence from empty caches) runs
the same tokens.  The composition's logits are stored with the tokens they were computed for:

* <case>_prefill, _verify0, _verify1: main-model logits of the prompt's last token, t and d;
* <case>_draft1, _draft2: MTP draft logits after the prompt and after the accepted verify;
* <case>_tokens: [t, d, t2], the oracle's picks that fixed the sequence.

Plus three planted mistakes in the composition (mhc_loop, seed 5, Q8_0), each of which the pin
must reject: planted_norm_prefill (final norm w instead of 1 + w), planted_merge_prefill (mode 1
instead of mode 2 at the end of the mHC range), planted_fc_draft1 (fc_e and fc_h swapped), with
planted_tokens.  transformers 5.15.0 is imported here only; the tests read the data.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(REPO, "oracle"), os.path.join(REPO, "sense-nova-server_amd"), os.path.dirname(HERE), HERE):
    sys.path.insert(0, p)

import torch  # noqa: E402

import composition_calls as CC  # noqa: E402
import oracle as O  # noqa: E402
import qwen35_compose as QC  # noqa: E402


def composed_outputs(o, cfg, ref, prompt, override=None):
    comp = QC.Composed(o, cfg, O.dequant, override)
    n = len(prompt)
    t, d, t2 = ref["t"], ref["d"], ref["t2"]
    logits, hid = comp.forward(prompt + [t, d])
    toks = prompt[1:] + [t]
    return comp, {"prefill": logits[n - 1], "verify0": logits[n], "verify1": logits[n + 1],
                  "draft1": comp.mtp(hid[:n], toks, list(range(n))),
                  "draft2": comp.mtp(hid[:n + 2], toks + [d, t2], list(range(n + 2)))}


def main():
    O.lib()
    out = {}
    shapes = CC.cfgs()
    for case, shape, seed, quant, zero in CC.CASES:
        cfg = shapes[shape]
        override, setup = CC.zero_router(cfg) if zero else (None, None)
        prompt = CC.prompt_for(seed, cfg.vocab)
        o, ref = CC.run_oracle(O, cfg, seed, quant, prompt, setup)
        _, res = composed_outputs(o, cfg, ref, prompt, override)
        for k, v in res.items():
            out[f"{case}_{k}"] = np.asarray(v, np.float32)
        out[f"{case}_tokens"] = np.array([ref["t"], ref["d"], ref["t2"]], np.int64)
        o.close()
        print(case, "done", flush=True)
    # planted mistakes
    cfg = shapes["mhc_loop"]
    prompt = CC.prompt_for(CC.PLANTED_SEED, cfg.vocab)
    o, ref = CC.run_oracle(O, cfg, CC.PLANTED_SEED, 0, prompt)
    comp, _ = composed_outputs(o, cfg, ref, prompt)
    n, h = len(prompt), cfg.hidden
    seq = prompt + [ref["t"], ref["d"]]
    with torch.no_grad():
        comp.final_norm.weight -= 1.0  # (1 + w) -> w
    out["planted_norm_prefill"] = np.asarray(comp.forward(seq)[0][n - 1], np.float32)
    with torch.no_grad():
        comp.final_norm.weight += 1.0
    orig = QC.merge
    QC.merge = lambda x0, x1, br, coef, mode: orig(x0, x1, br, coef, 1 if mode == 2 else mode)
    try:
        out["planted_merge_prefill"] = np.asarray(comp.forward(seq)[0][n - 1], np.float32)
    finally:
        QC.merge = orig
    _, hid = comp.forward(seq)
    comp.fc = torch.cat([comp.fc[:, h:], comp.fc[:, :h]], dim=1)
    out["planted_fc_draft1"] = np.asarray(comp.mtp(hid[:n], prompt[1:] + [ref["t"]], list(range(n))), np.float32)
    out["planted_tokens"] = np.array([ref["t"], ref["d"], ref["t2"]], np.int64)
    o.close()
    path = os.path.join(HERE, "composition.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
