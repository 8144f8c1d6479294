"""The generation worker's prefix cache (src/worker.rs:115-174) on the tiny model, through the C ABI.

A request served from the live state or a restored snapshot must give the token stream of the
same prompt run cold (reset, prefill from position 0) on a second engine with the same weights,
up to a divergence at a near-tie of the cold run (top-2 gap < 1e-3), with top-2 margins within
1e-3; the cold stream is the one the engine tests hold against the oracle.  (Not bit for bit:
the cold run feeds the earlier answer through the prefill GEMM, the warm one decoded it through
the GEMV, and the two sum in different orders.)  The worker's bookkeeping (cached tokens, live length, slot contents and
clocks) must follow the restatement in oracle/prefix_cache.py request by request, with the
tokens fed during decoding read from the engine's position.
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


@pytest.fixture(scope="module", params=[0, 1], ids=["q8", "q4"])
def engines(request, snl_mod):
    cfg = snl_mod.tiny_config()
    print(f"worker engines quant={request.param}", flush=True)
    warm = snl_mod.Engine(cfg, seed=5, quant=request.param, ctx=512)
    cold = snl_mod.Engine(cfg, seed=5, quant=request.param, ctx=512)
    yield cfg, warm, cold
    warm.close()
    cold.close()


def _rand(n, vocab, seed):
    return np.random.default_rng(seed).integers(0, vocab, n).tolist()


class Checked:
    """Runs requests on a worker and checks each against a cold run and the cache restatement."""

    def __init__(self, snl_mod, warm, cold, spec):
        from prefix_cache import PrefixCache

        self.w = snl_mod.Worker(warm, self_pause=False)
        self.warm, self.cold, self.spec = warm, cold, spec
        self.model = PrefixCache()

    def run(self, prompt, max_tokens, snapshot_at=None, expect=None):
        print(f"request n={len(prompt)} snapshot_at={snapshot_at} spec={self.spec}", flush=True)
        want = self.model.begin(prompt, snapshot_at)
        r = self.w.run(prompt, max_tokens, snapshot_at, spec=self.spec)
        c = self.cold.generate(prompt, max_tokens, self.spec)
        n = min(len(r["tokens"]), len(c["tokens"]))
        k = next((i for i in range(n) if r["tokens"][i] != c["tokens"][i]), n)
        if k < n:
            assert c["gaps"][k] < 1e-3, f"divergence at {k} with cold gap {c['gaps'][k]}"
        else:
            assert len(r["tokens"]) == len(c["tokens"])
        assert np.allclose(r["gaps"][:k], c["gaps"][:k], rtol=0, atol=1e-3)
        assert r["cached_tokens"] == want["cached"]
        if expect is not None:
            assert want["action"] == expect
        fed = self.warm.pos - len(prompt)
        assert fed in (len(r["tokens"]) - 1, len(r["tokens"]))
        self.model.decoded(r["tokens"][:fed])
        assert self.w.cache() == self.model.state()
        return r


@pytest.mark.parametrize("spec", [False, True], ids=["plain", "mtp"])
def test_conversation_reuses_the_cache(snl_mod, engines, spec):
    cfg, warm, cold = engines
    chk = Checked(snl_mod, warm, cold, spec)
    sys_prompt = _rand(24, cfg.vocab, 1)
    # turn 1: snapshot at the end of the shared prefix (the server's last <|im_start|>)
    p1 = sys_prompt + _rand(9, cfg.vocab, 2)
    r1 = chk.run(p1, 12, snapshot_at=len(sys_prompt), expect="reset")
    # turn 2 extends the whole first exchange: continues the live state
    p2 = p1 + r1["tokens"] + _rand(7, cfg.vocab, 3)
    r2 = chk.run(p2, 10, snapshot_at=len(p2) - 3, expect="live")
    assert r2["cached_tokens"] >= len(p1) + len(r1["tokens"]) - 1
    # a new question on the same system prompt: restores the first snapshot
    p3 = sys_prompt + _rand(11, cfg.vocab, 4)
    r3 = chk.run(p3, 10, expect="restore")
    assert r3["cached_tokens"] == len(sys_prompt)
    # back to the second turn's branch: its snapshot was dropped when turn 3 rewrote the
    # attention entries past the system prompt, so only the system prompt is reused
    p4 = p2[:len(p2) - 3] + _rand(5, cfg.vocab, 5)
    r4 = chk.run(p4, 8, expect="restore")
    assert r4["cached_tokens"] == len(sys_prompt)
    # an unrelated prompt starts over and drops every snapshot it overwrites
    chk.run(_rand(30, cfg.vocab, 6), 8, expect="reset")
    chk.run(p3, 8, expect="reset")
    chk.w.close()


def test_lru_over_nested_snapshots(snl_mod, engines):
    cfg, warm, cold = engines
    chk = Checked(snl_mod, warm, cold, True)
    seq = []
    for turn in range(6):
        seq = seq + _rand(6, cfg.vocab, 10 + turn)
        r = chk.run(seq, 4, snapshot_at=len(seq) - 2)
        seq = seq + r["tokens"]
    # branch from an early snapshot still held
    live, lens, used = chk.w.cache()
    held = sorted(k for k in lens if k > 0)
    assert len(held) == 4
    chk.run(seq[:held[0]] + _rand(5, cfg.vocab, 99), 6, expect="restore")
    chk.w.close()


def test_error_resets_the_worker(snl_mod, engines):
    cfg, warm, cold = engines
    chk = Checked(snl_mod, warm, cold, True)
    p = _rand(20, cfg.vocab, 21)
    chk.run(p, 6, snapshot_at=10)
    from snl.engine import SNL_ETOKEN, SnlError

    bad = p[:10] + [cfg.vocab]
    assert chk.model.begin(bad)["action"] == "restore"  # fails while feeding the bad token
    with pytest.raises(SnlError) as ei:
        chk.w.run(bad, 4)
    assert ei.value.code == SNL_ETOKEN
    chk.model.error()
    assert chk.w.cache() == (0, [-1] * 4, [0] * 4)
    with pytest.raises(SnlError):
        chk.w.run([], 4)
    with pytest.raises(SnlError):
        chk.w.run([1] * warm.ctx, 4)
    assert warm.pos == 0
    chk.run(p, 6, expect="reset")
    chk.w.close()


def test_worker_forgets_after_another_caller(snl_mod, engines):
    cfg, warm, cold = engines
    chk = Checked(snl_mod, warm, cold, True)
    p = _rand(18, cfg.vocab, 31)
    r = chk.run(p, 5, snapshot_at=9)
    warm.forward([1, 2, 3], None, 1)  # someone else moves the engine
    chk.model.error()  # the worker can no longer trust what it held
    chk.run(p + r["tokens"] + [7], 5, expect="reset")
    chk.w.close()


def test_worker_mtp_on_off_identical(snl_mod, engines):
    cfg, warm, cold = engines
    outs = []
    for spec in (False, True):
        w = snl_mod.Worker(warm, self_pause=False)
        p = _rand(16, cfg.vocab, 41)
        toks = []
        for k in range(3):
            r = w.run(p, 10, snapshot_at=len(p) - 1, spec=spec)
            toks.append(r["tokens"])
            p = p + r["tokens"] + _rand(3, cfg.vocab, 42 + k)
        outs.append(toks)
        w.close()
    assert outs[0] == outs[1]
