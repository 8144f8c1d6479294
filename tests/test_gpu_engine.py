"""End-to-end parity of the engine (C ABI) on the tiny SenseNova-Loop-style model.

hidden 256, FFN 768, vocab 4096, 8 layers (DeltaNet : attention = 3 : 1), layers 2-5 looped
twice, 2-stream mHC over the loop, 1-layer MTP head; seeded Q8_0 / Q4_0 weights drawn on the
device and, independently, by the oracle on the CPU.

Bars: weights bit-exact; token ids and acceptance decisions bit-exact except at
argmax near-ties (top-2 gap < 1e-3 in the oracle's logits); logits and DeltaNet state within
1e-2 relative; greedy output byte-identical with and without MTP.
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


def _prompt(n, vocab, seed=1):
    return np.random.default_rng(seed).integers(0, vocab, n).tolist()


@pytest.fixture(scope="module", params=[0, 1], ids=["q8", "q4"])
def pair(request, snl_mod, oracle):
    cfg = snl_mod.tiny_config()
    quant = request.param
    print(f"engine pair quant={quant}", flush=True)
    g = snl_mod.Engine(cfg, seed=3, quant=quant, ctx=256)
    o = oracle.Engine(cfg, seed=3, quant=quant, ctx=256, max_m=g.prefill_chunk)
    yield cfg, g, o
    g.close()
    o.close()


def test_weights_bit_exact(pair, oracle):
    cfg, g, o = pair
    import snl

    kinds = [(-1, snl.engine.K_EMBED), (-1, snl.engine.K_LM_HEAD), (-1, snl.engine.K_NORM)]
    for l in range(cfg.n_layers):
        ks = [1, 2, 9, 10] + ([3, 5, 6] if cfg.full_attention[l] else [4, 7, 8])
        if cfg.is_mhc(l):
            ks += [11, 12]
        kinds += [(l, k) for k in ks]
    kinds += [(snl.engine.MTP_LAYER, k) for k in (20, 21, 22, 23, 24, 1, 2, 3, 5, 6, 9, 10)]
    for layer, kind in kinds:
        gt, gq, gs = g.tensor(layer, kind)
        ot, oq, os_ = o.tensor(layer, kind)
        assert gt == ot, (layer, kind)
        if gt == 2:
            assert np.array_equal(gq.view(np.uint32), oq.view(np.uint32)), (layer, kind)
        else:
            assert np.array_equal(gq, oq), (layer, kind)
            assert np.array_equal(gs.view(np.uint32), os_.view(np.uint32)), (layer, kind)


def test_forward_logits_match_oracle(pair):
    cfg, g, o = pair
    g.reset()
    o.reset()
    prompt = _prompt(9, cfg.vocab, seed=4)
    pos = [[i] * 3 for i in range(len(prompt))]
    lg_g, picks = g.forward(prompt, pos, logit_rows=1)
    lg_o = o.forward(prompt, pos, logit_rows=1)
    rel = np.abs(lg_g - lg_o).max() / np.abs(lg_o).max()
    assert rel < 1e-3, rel
    assert picks[0].token == int(np.argmax(lg_g[0]))
    # a verify step: two rows, checkpointed
    t = [int(np.argmax(lg_o[0])), 17]
    p2 = [[9] * 3, [10] * 3]
    lg_g2, picks2 = g.forward(t, p2, logit_rows=2, ckpt=True)
    lg_o2 = o.forward(t, p2, logit_rows=2, ckpt=True)
    rel = np.abs(lg_g2 - lg_o2).max() / np.abs(lg_o2).max()
    assert rel < 1e-3, rel
    for r in range(2):
        srt = np.sort(lg_o2[r])
        if srt[-1] - srt[-2] >= TIE:
            assert picks2[r].token == int(np.argmax(lg_o2[r]))
    # DeltaNet state after the verify step, current slot
    st_g = g.buffer(3)
    st_o = o.buf(3, st_g.size)
    assert np.abs(st_g - st_o).max() / np.abs(st_o).max() < 1e-2
    # rollback then compare again
    g.rollback()
    o.rollback()
    assert g.pos == o.pos == 10 and g.hid_rows == o.hid_rows == 1
    st_g = g.buffer(3)
    st_o = o.buf(3, st_g.size)
    assert np.abs(st_g - st_o).max() / np.abs(st_o).max() < 1e-2
    hl_g, hl_o = g.buffer(2), o.buf(2, cfg.hidden)
    assert np.abs(hl_g - hl_o).max() / np.abs(hl_o).max() < 1e-2


def test_mtp_draft_matches_oracle(pair):
    cfg, g, o = pair
    for e in (g, o):
        e.reset()
    prompt = _prompt(12, cfg.vocab, seed=5)
    pos = [[i] * 3 for i in range(12)]
    g.forward(prompt, pos, logit_rows=1)
    o.forward(prompt, pos, logit_rows=1)
    d_g, pk, lg_g = g.mtp(1, [33], [[11] * 3], 11, True, want_logits=True)
    d_o, lg_o = o.mtp(1, [33], [[11] * 3], 11, True)
    rel = np.abs(lg_g - lg_o).max() / np.abs(lg_o).max()
    assert rel < 1e-3, rel
    srt = np.sort(lg_o)
    if srt[-1] - srt[-2] >= TIE:
        assert d_g == d_o


def _compare_streams(a, ref_tokens, ref_gaps):
    """Tokens equal up to the first divergence, which must sit at an oracle near-tie."""
    n = min(len(a), len(ref_tokens))
    for i in range(n):
        if a[i] != ref_tokens[i]:
            assert ref_gaps[i] < TIE, f"divergence at {i} with oracle gap {ref_gaps[i]}"
            return i
    assert len(a) == len(ref_tokens)
    return n


@pytest.mark.parametrize("spec", [False, True])
def test_generate_matches_oracle(pair, spec):
    cfg, g, o = pair
    prompt = _prompt(32, cfg.vocab, seed=1)
    rg = g.generate(prompt, 64, spec)
    ro = o.generate(prompt, 64, spec)
    matched = _compare_streams(rg["tokens"], ro["tokens"], ro["gaps"])
    print(f"spec={spec} matched {matched}/64 drafted {rg['drafted']}/{ro['drafted']} "
          f"accepted {rg['accepted']}/{ro['accepted']}", flush=True)
    if matched == 64 and spec:
        assert (rg["drafted"], rg["accepted"]) == (ro["drafted"], ro["accepted"])


def test_accept_path_matches_oracle(pair):
    """The calls the decode loop makes after an accepted draft (src/worker.rs:236-246): the verify
    [t, d] stays committed and the MTP head then drafts over 2 pairs (hidden rows 1 and 2 of the
    verify, tokens d and t2) at cache slot `pos before the verify`; then the next verify."""
    cfg, g, o = pair
    n = 12
    prompt = _prompt(n, cfg.vocab, seed=15)
    pos = [[i] * 3 for i in range(n)]
    for e in (g, o):
        e.reset()
    g.forward(prompt, pos, logit_rows=1)
    lg_o = o.forward(prompt, pos, logit_rows=1)
    for e in (g, o):
        e.mtp(1, prompt[1:], pos[:n - 1], 0, False)
    t = int(np.argmax(lg_o[0]))
    d_g, _, dl_g = g.mtp(g.hid_rows, [t], [[n - 1] * 3], n - 1, True, want_logits=True)
    d_o, dl_o = o.mtp(o.hid_rows, [t], [[n - 1] * 3], n - 1, True)
    assert np.abs(dl_g - dl_o).max() / np.abs(dl_o).max() < 1e-3
    _check_pick(d_g, d_o, dl_o)
    d = d_o
    p2 = [[n] * 3, [n + 1] * 3]
    v_g, _ = g.forward([t, d], p2, logit_rows=2, ckpt=True)
    v_o = o.forward([t, d], p2, logit_rows=2, ckpt=True)
    assert np.abs(v_g - v_o).max() / np.abs(v_o).max() < 1e-3
    t2 = int(np.argmax(v_o[1]))
    d2_g, _, dl2_g = g.mtp(1, [d, t2], p2, n, True, want_logits=True)
    d2_o, dl2_o = o.mtp(1, [d, t2], p2, n, True)
    assert np.abs(dl2_g - dl2_o).max() / np.abs(dl2_o).max() < 1e-3
    _check_pick(d2_g, d2_o, dl2_o)
    p3 = [[n + 2] * 3, [n + 3] * 3]
    v3_g, _ = g.forward([t2, d2_o], p3, logit_rows=2, ckpt=True)
    v3_o = o.forward([t2, d2_o], p3, logit_rows=2, ckpt=True)
    assert np.abs(v3_g - v3_o).max() / np.abs(v3_o).max() < 1e-3
    st_g = g.buffer(3)
    st_o = o.buf(3, st_g.size)
    assert np.abs(st_g - st_o).max() / np.abs(st_o).max() < 1e-2


def _check_pick(got, ref, ref_logits):
    """Token ids equal unless the oracle's top-2 gap is a near-tie."""
    top = np.sort(ref_logits)[-2:]
    assert got == ref or top[1] - top[0] < TIE, (got, ref, top[1] - top[0])


@pytest.mark.parametrize("quant", [0, 1], ids=["q8", "q4"])
def test_forced_acceptance_matches_oracle(snl_mod, oracle, quant, tmp_path):
    """Random weights never accept a draft, so the accept branch of the decode loop is driven
    with a head that confines every argmax to 5 tokens: the LM head's block scales are zeroed
    from row 4 on (those logits are exactly 0, the first of them wins when the live rows are
    all negative).  The same weights go to the oracle and, through a `.snl` file, to the GPU.
    Streams, drafted and accepted counts must agree, with MTP on and off."""
    import snl_format as F

    cfg = snl_mod.tiny_config()
    o = oracle.Engine(cfg, seed=13, quant=quant, ctx=256, max_m=512)
    o.zero_rows(-1, oracle.K_LM_HEAD, 4)
    main, mtp = str(tmp_path / "model.snl"), str(tmp_path / "mtp.snl")
    F.write_engine_files(o, cfg, quant, main, mtp)
    g = snl_mod.Engine.load(main, mtp, ctx=256)
    try:
        for seed in (1, 2):
            prompt = _prompt(24, cfg.vocab, seed=seed)
            ro = o.generate(prompt, 64, True)
            rg = g.generate(prompt, 64, True)
            off = g.generate(prompt, 64, False)
            matched = _compare_streams(rg["tokens"], ro["tokens"], ro["gaps"])
            print(f"forced acceptance quant={quant} seed={seed}: matched {matched}/64 drafted "
                  f"{rg['drafted']}/{ro['drafted']} accepted {rg['accepted']}/{ro['accepted']}", flush=True)
            assert ro["accepted"] > 0 and rg["accepted"] > 0
            assert off["tokens"] == rg["tokens"]
            if matched == 64:
                assert (rg["drafted"], rg["accepted"]) == (ro["drafted"], ro["accepted"])
    finally:
        g.close()
        o.close()


def _decode_both(g, prompt, counts):
    """The greedy speculative loop once through snl_decoder_step and once through
    snl_decoder_steps (calls of `counts` steps each): tokens, stats and the engine state after."""
    res = []
    for many in (False, True):
        d = g.decoder(prompt, spec=True)
        toks = []
        for k in counts:
            if many:
                toks += d.steps(k)
            else:
                for _ in range(k):
                    toks += d.step()
        st = d.stats()
        res.append((toks, st["drafted"], st["accepted"], g.pos, g.hid_rows, g.buffer(2), g.buffer(3), g.buffer(4)))
        d.close()
    return res


@pytest.mark.parametrize("quant", [0, 1], ids=["q8", "q4"])
def test_decoder_steps_match_single_steps(snl_mod, oracle, quant, tmp_path):
    """snl_decoder_steps queues each speculative step before the host reads the one before it, the
    step's records being written on the device by the previous step's control kernel (accept
    decision, state slots, positions, rotary table, the rollback's carried row).  Its tokens,
    drafted / accepted counts and the engine state it leaves (position, hidden rows, carried hidden
    row, recurrent and conv state of the current slot) must equal those of as many
    snl_decoder_step calls, which the oracle tests pin: on random weights (every draft rejected), on
    a head that confines the argmax to 5 tokens (drafts accepted), and up to the end of a short
    context, where the loop stops queueing ahead."""
    import snl_format as F

    cfg = snl_mod.tiny_config()
    o = oracle.Engine(cfg, seed=13, quant=quant, ctx=256, max_m=512)
    o.zero_rows(-1, oracle.K_LM_HEAD, 4)
    main, mtp = str(tmp_path / "model.snl"), str(tmp_path / "mtp.snl")
    F.write_engine_files(o, cfg, quant, main, mtp)
    o.close()
    cases = [("random", snl_mod.Engine(cfg, seed=3, quant=quant, ctx=256), [1, 17, 23]),
             ("forced", snl_mod.Engine.load(main, mtp, ctx=256), [2, 30, 9]),
             ("context end", snl_mod.Engine(cfg, seed=3, quant=quant, ctx=48), [23])]
    try:
        for name, g, counts in cases:
            prompt = _prompt(24, cfg.vocab, seed=5)
            one, many = _decode_both(g, prompt, counts)
            print(f"decoder steps quant={quant} {name}: {len(one[0])} tokens, drafted {one[1]} accepted {one[2]}, "
                  f"pos {one[3]}", flush=True)
            assert many[0] == one[0], name
            assert many[1:5] == one[1:5], name
            for a, b in zip(one[5:], many[5:]):
                assert np.array_equal(a, b), name
            if name == "forced":
                assert one[2] > 0
    finally:
        for _, g, _ in cases:
            g.close()


def test_mtp_on_off_identical(pair):
    cfg, g, o = pair
    for seed in (1, 2, 3):
        prompt = _prompt(32, cfg.vocab, seed=seed)
        a = g.generate(prompt, 64, False)
        b = g.generate(prompt, 64, True)
        assert a["tokens"] == b["tokens"]
        assert b["drafted"] > 0


def test_rollback_equals_never_run(pair):
    """verify([t, d]) + rollback leaves exactly the state of forward([t])."""
    cfg, g, o = pair
    prompt = _prompt(10, cfg.vocab, seed=8)
    pos = [[i] * 3 for i in range(10)]
    g.reset()
    g.forward(prompt, pos, logit_rows=1)
    g.forward([5, 6], [[10] * 3, [11] * 3], logit_rows=2, ckpt=True)
    g.rollback()
    s1, c1, h1 = g.buffer(3), g.buffer(4), g.buffer(2)
    _, pk1 = g.forward([7], [[11] * 3], logit_rows=1)
    g.reset()
    g.forward(prompt, pos, logit_rows=1)
    g.forward([5], [[10] * 3], logit_rows=1)
    s2, c2, h2 = g.buffer(3), g.buffer(4), g.buffer(2)
    _, pk2 = g.forward([7], [[11] * 3], logit_rows=1)
    assert np.array_equal(s1, s2) and np.array_equal(c1, c2) and np.array_equal(h1, h2)
    assert pk1[0].token == pk2[0].token and pk1[0].top1 == pk2[0].top1


def test_carried_hidden_row(pair):
    """forward_mm (src/engine.rs:801-936) starts a pass with hlast in hid row 0 and ends it with the
    last token's normalized hidden in hlast; both copies ride in the embed and final-norm launches."""
    cfg, g, o = pair
    h = cfg.hidden
    n = 6
    g.reset()
    g.forward(_prompt(n, cfg.vocab, seed=11), [[i] * 3 for i in range(n)], logit_rows=1)
    g.forward([5, 6], [[n] * 3, [n + 1] * 3], logit_rows=2)
    hid = g.buffer(1)[: 3 * h].reshape(3, h)
    carried = g.buffer(2)[:h]
    assert np.array_equal(carried, hid[2])
    g.forward([7], [[n + 2] * 3], logit_rows=1)
    hid2 = g.buffer(1)[: 2 * h].reshape(2, h)
    assert np.array_equal(hid2[0], carried)
    assert np.array_equal(g.buffer(2)[:h], hid2[1])
    assert not np.array_equal(hid2[1], carried)


def test_snapshot_restore(pair):
    cfg, g, o = pair
    prompt = _prompt(20, cfg.vocab, seed=9)
    pos = [[i] * 3 for i in range(20)]
    g.reset()
    g.forward(prompt[:12], pos[:12], logit_rows=0)
    g.snapshot(2)
    lg_a, _ = g.forward(prompt[12:], pos[12:], logit_rows=1)
    g.forward([1, 2, 3], [[20] * 3, [21] * 3, [22] * 3], logit_rows=1)
    g.restore(2, 12)
    assert g.pos == 12
    lg_b, _ = g.forward(prompt[12:], pos[12:], logit_rows=1)
    assert np.array_equal(lg_a, lg_b)


def test_error_paths(pair):
    cfg, g, o = pair
    import snl
    from snl.engine import SnlError

    g.reset()
    with pytest.raises(SnlError) as ei:
        g.forward([cfg.vocab], None, 1)
    assert ei.value.code == snl.engine.SNL_ETOKEN
    with pytest.raises(SnlError) as ei:
        g.forward([1, 2, 3], None, 3)
    assert ei.value.code == snl.engine.SNL_EARG
    with pytest.raises(SnlError) as ei:
        g.forward([1], None, 1, ckpt=True)
    assert ei.value.code == snl.engine.SNL_EARG
    with pytest.raises(SnlError) as ei:
        g.forward([], None, 1)
    assert ei.value.code == snl.engine.SNL_EARG
    with pytest.raises(SnlError) as ei:
        g.rollback()
    assert ei.value.code == snl.engine.SNL_ESTATE
    with pytest.raises(SnlError) as ei:
        g.forward([1] * (g.ctx + 1), None, 1)
    assert ei.value.code == snl.engine.SNL_ECTX
    g.forward([1, 2], None, 1)
    with pytest.raises(SnlError) as ei:
        g.mtp(2, [1, 2], [[0] * 3, [1] * 3], 0, True)
    assert ei.value.code == snl.engine.SNL_EARG
    g.reset()
    assert g.pos == 0


@pytest.mark.parametrize("quant", [0, 1], ids=["q8", "q4"])
def test_prompt_across_prefill_chunks(snl_mod, oracle, quant):
    """1100 prompt tokens run as prefill passes of 512, 512 and 76 rows (and the MTP catch-up
    after each): logits, greedy streams and acceptance decisions against the oracle."""
    cfg = snl_mod.tiny_config()
    print(f"long prompt quant={quant}", flush=True)
    g = snl_mod.Engine(cfg, seed=21, quant=quant, ctx=1400)
    o = oracle.Engine(cfg, seed=21, quant=quant, ctx=1400, max_m=g.prefill_chunk)
    try:
        prompt = _prompt(1100, cfg.vocab, seed=31)
        pos = [[i] * 3 for i in range(1100)]
        lg_g, _ = g.forward(prompt, pos, logit_rows=2)
        lg_o = o.forward(prompt, pos, logit_rows=2)
        assert np.abs(lg_g - lg_o).max() / np.abs(lg_o).max() < 1e-3
        st_g = g.buffer(3)
        st_o = o.buf(3, st_g.size)
        assert np.abs(st_g - st_o).max() / np.abs(st_o).max() < 1e-2
        # the worker's feed (src/worker.rs:291-323): each 512-row chunk, then the MTP head over its
        # pairs; then the first draft from hidden row hid_rows (the last chunk's last row)
        chunk = g.prefill_chunk
        for e in (g, o):
            e.reset()
            for c0 in range(0, 1100, chunk):
                c1 = min(c0 + chunk, 1100)
                e.forward(prompt[c0:c1], pos[c0:c1], logit_rows=1 if c1 == 1100 else 0)
                r0 = 1 if c0 == 0 else 0
                e.mtp(r0, prompt[c0 + r0:c1], pos[c0 + r0 - 1:c1 - 1], c0 + r0 - 1, False)
        assert g.hid_rows == o.hid_rows == 1100 - 2 * chunk
        t = int(np.argmax(lg_o[1]))
        d_g, _, dl_g = g.mtp(g.hid_rows, [t], [[1099] * 3], 1099, True, want_logits=True)
        d_o, dl_o = o.mtp(o.hid_rows, [t], [[1099] * 3], 1099, True)
        assert np.abs(dl_g - dl_o).max() / np.abs(dl_o).max() < 1e-3
        _check_pick(d_g, d_o, dl_o)
        for spec in (True, False):
            g.reset()
            o.reset()
            rg = g.generate(prompt, 32, spec)
            ro = o.generate(prompt, 32, spec)
            matched = _compare_streams(rg["tokens"], ro["tokens"], ro["gaps"])
            print(f"spec={spec} matched {matched}/32 drafted {rg['drafted']}/{ro['drafted']} "
                  f"accepted {rg['accepted']}/{ro['accepted']}", flush=True)
            if matched == 32 and spec:
                assert (rg["drafted"], rg["accepted"]) == (ro["drafted"], ro["accepted"])
    finally:
        g.close()
        o.close()


def test_long_prefill_matches_decode_feed(snl_mod):
    """4600 prompt tokens: the prefill passes past 4096 keys split attention into key parts and
    merge them; the same prompt fed two tokens at a time through the decode kernels (held against
    the oracle above) must give the same logits and DeltaNet state within the tolerances."""
    cfg = snl_mod.tiny_config()
    e = snl_mod.Engine(cfg, seed=23, quant=0, ctx=4700)
    try:
        n = 4600
        prompt = _prompt(n, cfg.vocab, seed=41)
        pos = [[i] * 3 for i in range(n)]
        print("long prefill: one call", flush=True)
        lg_a, _ = e.forward(prompt, pos, logit_rows=2)
        st_a = e.buffer(3)
        e.reset()
        print("long prefill: two tokens per pass", flush=True)
        for i in range(0, n, 2):
            lg_b, _ = e.forward(prompt[i:i + 2], pos[i:i + 2], logit_rows=2 if i + 2 >= n else 0)
        st_b = e.buffer(3)
        assert np.abs(lg_a - lg_b).max() / np.abs(lg_b).max() < 1e-3
        assert np.abs(st_a - st_b).max() / np.abs(st_b).max() < 1e-2
    finally:
        e.close()


@pytest.mark.parametrize("n", [512, 1024])
def test_draft_after_full_prefill_chunk(snl_mod, oracle, n):
    """A prompt whose last prefill pass is a full 512 rows leaves the first draft at hidden row 512;
    the two-row draft pass then also reads row 513 (its padding row), which the hidden buffer holds.
    The speculative stream must equal the oracle's and the stream without MTP."""
    cfg = snl_mod.tiny_config()
    print(f"draft after a full chunk: prompt {n}", flush=True)
    g = snl_mod.Engine(cfg, seed=29, quant=0, ctx=n + 80)
    o = oracle.Engine(cfg, seed=29, quant=0, ctx=n + 80, max_m=g.prefill_chunk)
    try:
        prompt = _prompt(n, cfg.vocab, seed=n)
        rg = g.generate(prompt, 24, True)
        off = g.generate(prompt, 24, False)
        ro = o.generate(prompt, 24, True)
        assert rg["tokens"] == off["tokens"]
        matched = _compare_streams(rg["tokens"], ro["tokens"], ro["gaps"])
        if matched == 24:
            assert (rg["drafted"], rg["accepted"]) == (ro["drafted"], ro["accepted"])
    finally:
        g.close()
        o.close()


def test_decode_cost_follows_position(snl_mod):
    """Decode passes size their attention launches by the context bucket of the live position
    (2048 * 2^k keys, capped at the allocated context), not by the allocated context.  An engine
    sized for 16384 positions and one sized for 2200 must give bitwise the same tokens, counts,
    logits and recurrent state across the 2048-key bucket edge (2048 -> 4096 keys on one, 2048 ->
    2200 on the other), with MTP on."""
    cfg = snl_mod.tiny_config()
    n = 2030
    prompt = _prompt(n, cfg.vocab, seed=43)
    res = []
    for ctx in (16384, 2200):
        print(f"position-sized attention: ctx {ctx}", flush=True)
        e = snl_mod.Engine(cfg, seed=31, quant=0, ctx=ctx)
        try:
            r = e.generate(prompt, 40, True)
            pos = e.pos
            lg, _ = e.forward([5, 6], [[pos] * 3, [pos + 1] * 3], logit_rows=2)
            res.append((r["tokens"], r["drafted"], r["accepted"], pos, lg, e.buffer(3)))
        finally:
            e.close()
    a, b = res
    assert a[3] > 2048 + 4
    assert a[0] == b[0] and a[1:4] == b[1:4]
    assert np.array_equal(a[4], b[4])
    assert np.array_equal(a[5], b[5])


def test_decoder_steps_across_a_context_bucket(snl_mod):
    """Steps queued ahead of the host across the 2048-key bucket edge: the next bucket's step graphs
    are captured while a step is still queued.  Tokens, counts and the engine state after equal
    those of single steps."""
    cfg = snl_mod.tiny_config()
    e = snl_mod.Engine(cfg, seed=37, quant=0, ctx=4200)
    try:
        prompt = _prompt(2030, cfg.vocab, seed=47)
        one, many = _decode_both(e, prompt, [3, 25, 12])
        print(f"queued across the bucket edge: {len(one[0])} tokens, pos {one[3]}", flush=True)
        assert one[3] > 2048 + 4
        assert many[0] == one[0]
        assert many[1:5] == one[1:5]
        for a, b in zip(one[5:], many[5:]):
            assert np.array_equal(a, b)
    finally:
        e.close()
