"""Size-independent properties of the MTP decode step at the full SenseNova-Loop-9B shape.

The oracle would take minutes per token at this size, so these tests check what must hold
whatever the weights (random-init, drawn on the device) and whatever the size:
  * greedy output is byte-identical with and without MTP drafting (src/worker.rs decode loop);
  * a verify pass [t, d] gives, row by row, bitwise the logits of feeding t and then d alone
    (the GEMVs, attention and DeltaNet results do not depend on M);
  * verify + rollback leaves the engine exactly where feeding t alone leaves it.
The prompts cross the 512-row prefill chunk, so the prefill path runs at full size too.
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


def _prompt(n, vocab, seed):
    return np.random.default_rng(seed).integers(0, vocab, n).tolist()


@pytest.fixture(scope="module", params=[0, 1], ids=["q8", "q4"])
def big(request, snl_mod):
    cfg = snl_mod.nine_b_config()
    print(f"9B engine quant={request.param}", flush=True)
    e = snl_mod.Engine(cfg, seed=5, quant=request.param, ctx=2048)
    yield cfg, e
    e.close()


def test_mtp_on_off_identical_full_size(big):
    cfg, e = big
    prompt = _prompt(600, cfg.vocab, seed=4)
    a = e.generate(prompt, 24, False)
    b = e.generate(prompt, 24, True)
    assert a["tokens"] == b["tokens"]
    assert b["drafted"] > 0


def test_verify_rows_equal_single_token_feeds_full_size(big):
    cfg, e = big
    n = 530
    prompt = _prompt(n, cfg.vocab, seed=6)
    pos = [[i] * 3 for i in range(n)]
    t, d = 5, 6
    e.reset()
    e.forward(prompt, pos, logit_rows=1)
    both, pk2 = e.forward([t, d], [[n] * 3, [n + 1] * 3], logit_rows=2)
    e.reset()
    e.forward(prompt, pos, logit_rows=1)
    one, pk_t = e.forward([t], [[n] * 3], logit_rows=1)
    two, pk_d = e.forward([d], [[n + 1] * 3], logit_rows=1)
    assert np.array_equal(both[0], one[0])
    assert np.array_equal(both[1], two[0])
    assert pk2[0].token == pk_t[0].token and pk2[1].token == pk_d[0].token


def test_rollback_equals_never_run_full_size(big):
    cfg, e = big
    n = 520
    prompt = _prompt(n, cfg.vocab, seed=8)
    pos = [[i] * 3 for i in range(n)]
    e.reset()
    e.forward(prompt, pos, logit_rows=1)
    e.forward([5, 6], [[n] * 3, [n + 1] * 3], logit_rows=2, ckpt=True)
    e.rollback()
    s1, c1, h1 = e.buffer(3), e.buffer(4), e.buffer(2)
    l1, _ = e.forward([7], [[n + 1] * 3], logit_rows=1)
    e.reset()
    e.forward(prompt, pos, logit_rows=1)
    e.forward([5], [[n] * 3], logit_rows=1)
    s2, c2, h2 = e.buffer(3), e.buffer(4), e.buffer(2)
    l2, _ = e.forward([7], [[n + 1] * 3], logit_rows=1)
    assert np.array_equal(s1, s2) and np.array_equal(c1, c2) and np.array_equal(h1, h2)
    assert np.array_equal(l1, l2)
