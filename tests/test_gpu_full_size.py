"""The MTP decode step at the full SenseNova-Loop-9B shape (hidden 4096, FFN 12288, vocab 248320,
32 layers with layers 4-27 run twice, 2-stream mHC, 1-layer MTP head), Q8_0 and Q4_0.

Parity with the oracle at this size (a 40-token prompt costs the oracle seconds on the host):
prefill logits and DeltaNet state, the first MTP draft, a checkpointed verify pass, the MTP draft
over 2 pairs that follows an accepted draft, a rollback, and a few greedy speculative steps.
These run the 9B-only kernel instances: the K = 4096 / 12288 GEMVs with four quant blocks per
lane group, their fused norm, mHC, SwiGLU and head-norm prologues and epilogues, and the
tile-major vocabulary head with the fused final norm of the draft.

Then the size-independent properties, at prompts that cross the 512-row prefill chunk:
  * greedy output is byte-identical with and without MTP drafting (src/worker.rs decode loop);
  * a verify pass [t, d] gives, row by row, bitwise the logits of feeding t and then d alone
    (the GEMVs, attention and DeltaNet results do not depend on M);
  * verify + rollback leaves the engine exactly where feeding t alone leaves it.
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


TIE = 1e-3


@pytest.fixture(scope="module", params=[0, 1], ids=["q8", "q4"])
def big(request, snl_mod):
    cfg = snl_mod.nine_b_config()
    print(f"9B engine quant={request.param}", flush=True)
    e = snl_mod.Engine(cfg, seed=5, quant=request.param, ctx=2048)
    yield cfg, e, request.param
    e.close()


def _rel(a, b):
    return float(np.abs(np.asarray(a) - np.asarray(b)).max() / np.abs(np.asarray(b)).max())


def _check_pick(got, ref, ref_logits):
    top = np.sort(ref_logits)[-2:]
    assert got == ref or top[1] - top[0] < TIE, (got, ref, top[1] - top[0])


def test_nine_b_matches_oracle(big, oracle):
    cfg, g, quant = big
    print(f"9B oracle quant={quant}", flush=True)
    o = oracle.Engine(cfg, seed=5, quant=quant, ctx=128, max_m=64)
    try:
        n = 40
        prompt = _prompt(n, cfg.vocab, seed=12)
        pos = [[i] * 3 for i in range(n)]
        g.reset()
        lg_g, pk = g.forward(prompt, pos, logit_rows=1)
        lg_o = o.forward(prompt, pos, logit_rows=1)
        assert _rel(lg_g, lg_o) < 1e-3
        _check_pick(pk[0].token, int(np.argmax(lg_o[0])), lg_o[0])
        st_g = g.buffer(3)
        assert _rel(st_g, o.buf(3, st_g.size)) < 1e-2
        print("9B prefill ok", flush=True)
        # the worker's MTP catch-up over the prompt, then the first draft from hidden row n
        for e in (g, o):
            e.mtp(1, prompt[1:], pos[:n - 1], 0, False)
        t = int(np.argmax(lg_o[0]))
        d_g, _, dl_g = g.mtp(g.hid_rows, [t], [[n - 1] * 3], n - 1, True, want_logits=True)
        d_o, dl_o = o.mtp(o.hid_rows, [t], [[n - 1] * 3], n - 1, True)
        assert _rel(dl_g, dl_o) < 1e-3
        _check_pick(d_g, d_o, dl_o)
        print("9B draft ok", flush=True)
        # checkpointed verify [t, d]
        d = d_o
        p2 = [[n] * 3, [n + 1] * 3]
        v_g, pk2 = g.forward([t, d], p2, logit_rows=2, ckpt=True)
        v_o = o.forward([t, d], p2, logit_rows=2, ckpt=True)
        assert _rel(v_g, v_o) < 1e-3
        for r in range(2):
            _check_pick(pk2[r].token, int(np.argmax(v_o[r])), v_o[r])
        st_g = g.buffer(3)
        assert _rel(st_g, o.buf(3, st_g.size)) < 1e-2
        # the draft after an accepted verify: 2 pairs from hidden rows 1 and 2, slot n
        t2 = int(np.argmax(v_o[1]))
        d2_g, _, dl2_g = g.mtp(1, [d, t2], p2, n, True, want_logits=True)
        d2_o, dl2_o = o.mtp(1, [d, t2], p2, n, True)
        assert _rel(dl2_g, dl2_o) < 1e-3
        _check_pick(d2_g, d2_o, dl2_o)
        print("9B verify and second draft ok", flush=True)
        # reject instead: roll back, then feed the token after t
        g.rollback()
        o.rollback()
        assert g.pos == o.pos == n + 1
        st_g = g.buffer(3)
        assert _rel(st_g, o.buf(3, st_g.size)) < 1e-2
        l3_g, _ = g.forward([t2], [[n + 1] * 3], logit_rows=1)
        l3_o = o.forward([t2], [[n + 1] * 3], logit_rows=1)
        assert _rel(l3_g, l3_o) < 1e-3
        # greedy speculative decoding, as the worker runs it
        rg = g.generate(prompt, 6, True)
        ro = o.generate(prompt, 6, True)
        m = min(len(rg["tokens"]), len(ro["tokens"]))
        for i in range(m):
            if rg["tokens"][i] != ro["tokens"][i]:
                assert ro["gaps"][i] < TIE, f"divergence at {i} with oracle gap {ro['gaps'][i]}"
                break
        else:
            assert len(rg["tokens"]) == len(ro["tokens"])
            assert (rg["drafted"], rg["accepted"]) == (ro["drafted"], ro["accepted"])
        print(f"9B generate: {rg['tokens']} vs {ro['tokens']}, drafted {rg['drafted']}/{ro['drafted']} "
              f"accepted {rg['accepted']}/{ro['accepted']}", flush=True)
    finally:
        o.close()


@pytest.mark.parametrize("quant", [0, 1], ids=["q8", "q4"])
def test_nine_b_accept_branch_matches_oracle(snl_mod, oracle, quant):
    """The accept branch of the decode loop at 9B (src/worker.rs:236-246).  Random weights never
    accept a draft, so the LM head (shared by the main model and the MTP head) is confined to its
    first rows on both sides: block scales zeroed from row 4 on, so those logits are exactly 0 and
    the first of them wins whenever rows 0-3 are all negative.  Greedy speculative decoding through
    the captured step graph (its device-side accept decision, the 2-pair draft over the verify's
    hidden rows, the rotary and slot bookkeeping), once step by step and once with every step
    queued ahead from the records the previous step wrote on the device: tokens, drafted and
    accepted counts and the DeltaNet state after equal the oracle's (ties aside)."""
    cfg = snl_mod.nine_b_config()
    print(f"9B accept branch quant={quant}", flush=True)
    g = snl_mod.Engine(cfg, seed=17, quant=quant, ctx=256)
    o = oracle.Engine(cfg, seed=17, quant=quant, ctx=256, max_m=64)
    try:
        g.zero_rows(-1, snl_mod.engine.K_LM_HEAD, 4)
        o.zero_rows(-1, oracle.K_LM_HEAD, 4)
        n, steps = 40, 12
        prompt = _prompt(n, cfg.vocab, seed=19)
        ro = o.generate(prompt, steps, True)
        st_o = o.buf(3, g.buffer(3).size)
        print(f"9B accept oracle: {ro['tokens']} drafted {ro['drafted']} accepted {ro['accepted']}", flush=True)
        assert ro["accepted"] > 0
        rg = g.generate(prompt, steps, True)
        st_g = g.buffer(3)
        print(f"9B accept gpu: {rg['tokens']} drafted {rg['drafted']} accepted {rg['accepted']}", flush=True)
        matched = n_match = min(len(rg["tokens"]), len(ro["tokens"]))
        for i in range(n_match):
            if rg["tokens"][i] != ro["tokens"][i]:
                assert ro["gaps"][i] < TIE, f"divergence at {i} with oracle gap {ro['gaps'][i]}"
                matched = i
                break
        if matched == n_match:
            assert len(rg["tokens"]) == len(ro["tokens"])
            assert (rg["drafted"], rg["accepted"]) == (ro["drafted"], ro["accepted"])
            assert _rel(st_g, st_o) < 1e-2
        assert rg["accepted"] > 0
        # the same loop with every step queued ahead equals single steps: tokens, counts, state
        res = []
        for many in (False, True):
            d = g.decoder(prompt, spec=True)
            toks = []
            for k in (1, 4, 3):
                if many:
                    toks += d.steps(k)
                else:
                    for _ in range(k):
                        toks += d.step()
            st = d.stats()
            res.append((toks, st["drafted"], st["accepted"], g.pos, g.buffer(2), g.buffer(3)))
            d.close()
        one, queued = res
        print(f"9B accept steps: {one[0]} drafted {one[1]} accepted {one[2]}", flush=True)
        assert one[2] > 0
        assert queued[:4] == one[:4]
        assert np.array_equal(queued[4], one[4]) and np.array_equal(queued[5], one[5])
    finally:
        g.close()
        o.close()


def test_mtp_on_off_identical_full_size(big):
    """The 9B workload itself: a 1024-token prompt (two prefill chunks), 512 greedy tokens with the
    MTP head drafting and without it, byte-identical."""
    cfg, e, _ = big
    prompt = _prompt(1024, cfg.vocab, seed=4)
    a = e.generate(prompt, 512, False)
    b = e.generate(prompt, 512, True)
    # (an end-of-sequence pick would stop both runs at the same token)
    assert 0 < len(a["tokens"]) == len(b["tokens"]) <= 512
    assert a["tokens"] == b["tokens"]
    assert b["drafted"] > 0 and 0 <= b["accepted"] <= b["drafted"]
    print(f"9B 1024 + {len(b['tokens'])}: drafted {b['drafted']} accepted {b['accepted']}", flush=True)


def test_verify_rows_equal_single_token_feeds_full_size(big):
    cfg, e, _ = big
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
    cfg, e, _ = big
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
