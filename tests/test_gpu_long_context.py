"""The 9B model in Q4_0 at 32K context: prefill in 512-row passes, decode with attention over
the whole f16 KV cache, and a second turn served from a prefix snapshot (src/worker.rs:139-174,
src/engine.rs:663-683, decode attention parts src/engine.rs:827).

* Engine level: restoring the recurrent-state snapshot taken after 30720 tokens and feeding the
  1024-token tail gives the logits of a cold feed of all 31744 tokens, and so does the verify
  pass that follows (decode attention over 31.7K keys, 496 key parts).
* Worker level: a 32768-token prompt with a snapshot at 30720, then a second prompt sharing those
  30720 tokens; the second turn reuses them and produces the tokens of a cold run, and MTP on and
  off give the same tokens at this context.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TIE = 1e-3


@pytest.fixture(scope="module")
def snl_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import snl

    snl.lib()
    return snl


@pytest.fixture(scope="module")
def q4_32k(snl_mod):
    cfg = snl_mod.nine_b_config()
    print("9B Q4_0 engine, ctx 34000", flush=True)
    e = snl_mod.Engine(cfg, seed=9, quant=1, ctx=34000)
    yield cfg, e
    e.close()


def _rel(a, b):
    return float(np.abs(np.asarray(a) - np.asarray(b)).max() / np.abs(np.asarray(b)).max())


def test_snapshot_restore_at_30k_equals_cold_feed(q4_32k):
    cfg, e = q4_32k
    snap, tail = 30720, 1024
    n = snap + tail
    r = np.random.default_rng(17)
    prompt = r.integers(0, cfg.vocab, n).tolist()
    other = r.integers(0, cfg.vocab, tail).tolist()
    pos = [[i] * 3 for i in range(n)]
    print("cold feed of 31744 tokens", flush=True)
    e.reset()
    lg_c, pk_c = e.forward(prompt, pos, logit_rows=1)
    t = pk_c[0].token
    v_c, _ = e.forward([t, 7], [[n] * 3, [n + 1] * 3], logit_rows=2, ckpt=True)
    e.rollback()
    one_c, _ = e.forward([7], [[n + 1] * 3], logit_rows=1)
    print("snapshot at 30720, another tail, restore, the same tail", flush=True)
    e.reset()
    e.forward(prompt[:snap], pos[:snap], logit_rows=0)
    e.snapshot(0)
    e.forward(other, pos[snap:], logit_rows=0)
    e.restore(0, snap)
    assert e.pos == snap
    lg_w, pk_w = e.forward(prompt[snap:], pos[snap:], logit_rows=1)
    v_w, _ = e.forward([t, 7], [[n] * 3, [n + 1] * 3], logit_rows=2, ckpt=True)
    e.rollback()
    one_w, _ = e.forward([7], [[n + 1] * 3], logit_rows=1)
    print(f"bitwise: prefill {np.array_equal(lg_c, lg_w)} verify {np.array_equal(v_c, v_w)}", flush=True)
    assert _rel(lg_w, lg_c) < 1e-3
    assert _rel(v_w, v_c) < 1e-3
    assert _rel(one_w, one_c) < 1e-3
    # the verify rows are the single-token feeds (the decode kernels at 31.7K keys do not depend on M)
    assert np.array_equal(v_w[1], v_c[1]) or _rel(v_w[1], v_c[1]) < 1e-3


def test_worker_32k_prefix_reuse_and_mtp_identity(snl_mod, q4_32k):
    cfg, e = q4_32k
    n, snap, new, gen = 32768, 30720, 1024, 48
    r = np.random.default_rng(23)
    prompt = r.integers(0, cfg.vocab, n).tolist()
    p2 = prompt[:snap] + r.integers(0, cfg.vocab, new).tolist()
    w = snl_mod.Worker(e, self_pause=False)
    try:
        print("worker turn 1: 32768 tokens, snapshot at 30720", flush=True)
        r1 = w.run(prompt, gen, snapshot_at=snap)
        assert r1["completion_tokens"] == gen and r1["cached_tokens"] == 0 and r1["drafted"] > 0
        print("worker turn 2: 30720 shared + 1024 new", flush=True)
        r2 = w.run(p2, gen)
        assert r2["cached_tokens"] == snap
        print(f"turn 2 prefill {r2['prefill_s']:.3f}s; cold runs with and without MTP", flush=True)
    finally:
        w.close()
    cold = e.generate(p2, gen, True)
    off = e.generate(p2, gen, False)
    assert off["tokens"] == cold["tokens"]
    for i, (a, b) in enumerate(zip(r2["tokens"], cold["tokens"])):
        if a != b:
            assert cold["gaps"][i] < TIE, f"turn 2 diverges from the cold run at {i} (gap {cold['gaps'][i]})"
            break
    else:
        assert len(r2["tokens"]) == len(cold["tokens"])
