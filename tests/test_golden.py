"""The oracle against the committed golden fixtures (tests/golden/make_golden.py says where each
comes from): quantisation known answers, float64 products, and the tiny model's recorded greedy
streams (MTP on and off) and prompt logits."""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLDEN, name))


def test_quant_known_answers(oracle):
    kat = _load("quant_kat.npz")
    q, s = oracle.quantize(kat["q8_x"], 0)
    assert np.array_equal(q.view(np.int8), kat["q8_q"])
    assert np.array_equal(s.reshape(-1), kat["q8_s"])
    q, s = oracle.quantize(kat["q4_x"], 1)
    assert np.array_equal(q, kat["q4_bytes"])
    assert np.array_equal(s.reshape(-1), kat["q4_s"])


@pytest.mark.parametrize("tag", ["q0_64x256", "q0_48x512", "q1_64x256", "q1_48x512"])
def test_gemv_against_float64(oracle, tag):
    g = _load("gemv_small.npz")
    quant = int(tag[1])
    n, k = (int(v) for v in tag.split("_")[1].split("x"))
    y = oracle.gemv(quant, g[tag + "_q"], g[tag + "_s"], g[tag + "_x"], n, k)
    assert np.all(np.abs(y - g[tag + "_y64"]) <= 1e-5 * g[tag + "_abs"] + 1e-7)


@pytest.mark.parametrize("quant", [0, 1], ids=["q8", "q4"])
def test_tiny_streams_reproduce(oracle, quant):
    import snl.config as C

    fx = _load(f"tiny_stream_q{'8' if quant == 0 else '4'}.npz")
    cfg = C.tiny_config()
    prompt = fx["prompt"].tolist()
    e = oracle.Engine(cfg, seed=int(fx["seed"]), quant=quant, ctx=256, max_m=2)
    lg = e.forward(prompt, logit_rows=1)[0]
    e.close()
    assert np.allclose(lg, fx["logits"], rtol=1e-6, atol=1e-7)
    for spec, key in ((True, "tokens_spec"), (False, "tokens_plain")):
        e = oracle.Engine(cfg, seed=int(fx["seed"]), quant=quant, ctx=256, max_m=2)
        r = e.generate(prompt, len(fx[key]), spec)
        e.close()
        assert r["tokens"] == fx[key].tolist()
        if spec:
            assert (r["drafted"], r["accepted"]) == (int(fx["drafted"]), int(fx["accepted"]))
    # greedy output is the same with and without speculative drafting
    assert np.array_equal(fx["tokens_spec"], fx["tokens_plain"])
