"""The HIP engine and GEMV against the committed golden fixtures (tests/golden/make_golden.py).

Token ids must match except at an oracle near-tie (top-2 logit gap below 1e-3); logits within
1e-3 relative to the largest magnitude; GEMV within 1e-5 of the sum of |terms| of the float64
product."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TIE = 1e-3


@pytest.fixture(scope="module")
def snl_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import snl

    snl.lib()
    return snl


def _load(name):
    return np.load(os.path.join(GOLDEN, name))


@pytest.mark.parametrize("tag", ["q0_64x256", "q0_48x512", "q1_64x256", "q1_48x512"])
def test_gemv_golden(snl_mod, tag):
    import torch

    g = _load("gemv_small.npz")
    quant = int(tag[1])
    n, k = (int(v) for v in tag.split("_")[1].split("x"))
    print(f"gemv golden {tag}", flush=True)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    y = torch.zeros((2, n), dtype=torch.float32, device="cuda")
    snl_mod.kernels.gemv(quant, dev(g[tag + "_q"]), dev(g[tag + "_s"]), dev(g[tag + "_x"]), y, 2, n, k, k, n)
    torch.cuda.synchronize()
    assert np.all(np.abs(y.cpu().numpy() - g[tag + "_y64"]) <= 1e-5 * g[tag + "_abs"] + 1e-7)


@pytest.mark.parametrize("quant", [0, 1], ids=["q8", "q4"])
def test_tiny_engine_golden(snl_mod, quant):
    fx = _load(f"tiny_stream_q{'8' if quant == 0 else '4'}.npz")
    cfg = snl_mod.tiny_config()
    prompt = fx["prompt"].tolist()
    print(f"tiny engine golden quant={quant}", flush=True)
    e = snl_mod.Engine(cfg, seed=int(fx["seed"]), quant=quant, ctx=256)
    try:
        lg = e.forward(prompt, logit_rows=1)[0]
        assert np.abs(lg - fx["logits"]).max() <= 1e-3 * np.abs(fx["logits"]).max()
        for spec, key, gaps in ((True, "tokens_spec", "gaps_spec"), (False, "tokens_plain", "gaps_plain")):
            e.reset()
            got = e.generate(prompt, len(fx[key]), spec)["tokens"]
            ref = fx[key].tolist()
            for i, (a, b) in enumerate(zip(got, ref)):
                if a != b:
                    assert fx[gaps][i] < TIE, f"token {i} differs at oracle gap {fx[gaps][i]}"
                    break
            else:
                assert len(got) == len(ref)
    finally:
        e.close()
