"""The sampler (src/sampler.rs) over the engine's logits on the GPU, against oracle/sampler.py.

The device applies the penalties and keeps the top-k candidates; the kept token lists must equal
the restatement's over the same logits read back to the host, and the probabilities agree within
1e-5 relative (expf on the host against numpy's float32 exp).  With the library's random stream,
sample and verify must pick the restatement's tokens.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def snl_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import snl

    snl.lib()
    return snl


@pytest.fixture(scope="module")
def eng(snl_mod):
    cfg = snl_mod.tiny_config()
    e = snl_mod.Engine(cfg, seed=11, quant=0, ctx=256)
    yield cfg, e
    e.close()


def _logits(e, cfg, seed, rows=1):
    prompt = np.random.default_rng(seed).integers(0, cfg.vocab, 12).tolist()
    e.reset()
    lg, _ = e.forward(prompt, [[i] * 3 for i in range(12)], logit_rows=rows)
    return lg


PARAMS = [
    dict(temperature=1.0, top_p=0.95, top_k=20, min_p=0.0, presence_penalty=0.0, frequency_penalty=0.0,
         repetition_penalty=1.0),
    dict(temperature=0.7, top_p=0.9, top_k=0, min_p=0.0, presence_penalty=0.0, frequency_penalty=0.0,
         repetition_penalty=1.0),
    dict(temperature=1.3, top_p=1.0, top_k=2000, min_p=0.05, presence_penalty=0.0, frequency_penalty=0.0,
         repetition_penalty=1.0),
    dict(temperature=0.8, top_p=0.95, top_k=50, min_p=0.0, presence_penalty=0.2, frequency_penalty=0.1,
         repetition_penalty=1.3),
    dict(temperature=0.0, top_p=1.0, top_k=20, min_p=0.0, presence_penalty=0.5, frequency_penalty=0.3,
         repetition_penalty=1.5),
]


@pytest.mark.parametrize("pi", range(len(PARAMS)))
def test_distribution_matches_oracle(snl_mod, eng, pi):
    import sampler as S

    cfg, e = eng
    p = PARAMS[pi]
    print(f"distribution params {pi}", flush=True)
    lg = _logits(e, cfg, 100 + pi)[0]
    counts = {}
    smp = snl_mod.Sampler(e, snl_mod.Sampling(**p), seed=1)
    for t in np.argsort(-lg)[:6].tolist() + [int(np.argmax(lg))]:  # penalise the current favourites
        smp.accept(t)
        counts[t] = counts.get(t, 0) + 1
    toks, probs = smp.distribution(0)
    greedy, rt, rp = S.distribution(lg, counts, p)
    assert toks.tolist() == [int(t) for t in rt]
    assert np.allclose(probs, rp, rtol=1e-5, atol=1e-7)
    smp.close()


def test_sample_and_verify_follow_the_stream(snl_mod, eng):
    import sampler as S

    cfg, e = eng
    p = PARAMS[0]
    for seed in (3, 4, 5, 6):
        lg = _logits(e, cfg, 200 + seed, rows=2)
        smp = snl_mod.Sampler(e, snl_mod.Sampling(**p), seed=seed)
        rng = snl_mod.Rng(seed)
        draft = int(np.argsort(-lg[0])[1])  # a plausible draft
        ok, tok = smp.verify(0, draft)
        _, rt, rp = S.distribution(lg[0], {}, p)
        assert (ok, tok) == S.verify(False, rt, rp, draft, rng)
        smp.accept(tok)
        t1 = smp.sample(1)
        _, rt1, rp1 = S.distribution(lg[1], {tok: 1} if p["presence_penalty"] else {}, p)
        assert t1 == S.draw(rt1, rp1, None, rng.f32())
        smp.close()


def test_worker_sampled(snl_mod, eng):
    cfg, e = eng
    w = snl_mod.Worker(e, self_pause=False)
    prompt = np.random.default_rng(9).integers(0, cfg.vocab, 20).tolist()
    sp = snl_mod.Sampling(temperature=1.0, top_p=0.95, top_k=20)
    a = w.run_sampled(prompt, 24, sp, seed=77)
    b = w.run_sampled(prompt, 24, sp, seed=77)
    assert a["tokens"] == b["tokens"] and len(a["tokens"]) == 24
    # top_k = 1 leaves the argmax with probability 1: the greedy stream, drafts accepted as greedy
    one = snl_mod.Sampling(temperature=1.0, top_p=1.0, top_k=1)
    g = w.run(prompt, 24)
    for spec in (True, False):
        s = w.run_sampled(prompt, 24, one, seed=1, spec=spec)
        assert s["tokens"] == g["tokens"]
    # greedy parameters take the greedy path
    z = w.run_sampled(prompt, 24, snl_mod.Sampling(temperature=0.0), seed=1)
    assert z["tokens"] == g["tokens"]
    w.close()
