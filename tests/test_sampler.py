"""The sampler's host logic (src/sampler.rs) on the CPU: the restatement in oracle/sampler.py and
the library's host functions (snl_chacha_block, snl_rng_*, snl_draw, snl_finish_distribution),
against fixed vectors and hand-worked cases."""
import ctypes

import numpy as np
import pytest

import sampler as S


@pytest.fixture(scope="module")
def L():
    import snl

    return snl.lib()


def _u32p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))


def _f32p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


RFC7539_IN = [0x61707865, 0x3320646E, 0x79622D32, 0x6B206574] + \
    list(np.arange(32, dtype=np.uint8).view("<u4")) + [1, 0x09000000, 0x4A000000, 0]
# RFC 7539 section 2.3.2: the ChaCha20 block for that state
RFC7539_OUT = [0xE4E7F110, 0x15593BD1, 0x1FDD0F50, 0xC47120A3, 0xC7F4D1C7, 0x0368C033, 0x9AAA2204, 0x4E6CD4C3,
               0x466482D2, 0x09AA9F07, 0x05D7C214, 0xA2028BD9, 0xD19C12B5, 0xB94E16DE, 0xE883D0CB, 0x4E3C50A2]
ZERO_KEY_OUT = [0xADE0B876, 0x903DF1A0, 0xE56A5D40, 0x28BD8653]  # ChaCha20, zero key, nonce and counter


def test_chacha_block_vectors(L):
    assert S.chacha_block([int(x) for x in RFC7539_IN], 20) == RFC7539_OUT
    z = S.StdRng.CONST + [0] * 12
    assert S.chacha_block(z, 20)[:4] == ZERO_KEY_OUT
    inp = np.array(RFC7539_IN, np.uint32)
    out = np.zeros(16, np.uint32)
    L.snl_chacha_block(_u32p(inp), 20, _u32p(out))
    assert out.tolist() == RFC7539_OUT
    # 12 rounds: the library and the restatement agree
    L.snl_chacha_block(_u32p(inp), 12, _u32p(out))
    assert out.tolist() == S.chacha_block([int(x) for x in RFC7539_IN], 12)


@pytest.mark.parametrize("seed", [0, 1, 42, (1 << 63) + 5])
def test_rng_stream_matches_restatement(L, seed):
    import snl

    r, o = snl.Rng(seed), S.StdRng(seed)
    assert [r.u32() for _ in range(40)] == [o.u32() for _ in range(40)]  # crosses block boundaries
    fs = [r.f32() for _ in range(100)]
    assert fs == [o.f32() for _ in range(100)]
    assert all(0.0 <= f < 1.0 for f in fs)
    assert all(float(f * 16777216.0).is_integer() for f in fs)


def test_pcg32_known_answers():
    """The PCG32 step and output function of the seed expansion against the PCG reference
    implementation's demo program (pcg-c-basic): pcg32_srandom_r(42, 54), then six outputs of
    pcg32_random_r (which outputs the old state, then advances)."""
    inc = (54 << 1) | 1
    s = S.lcg(0, inc)
    s = S.lcg((s + 42) & ((1 << 64) - 1), inc)
    out = []
    for _ in range(6):
        out.append(S.xsh_rr(s))
        s = S.lcg(s, inc)
    assert out == [0xA15C02B7, 0x7B47F409, 0xBA1D3330, 0x83D2F293, 0xBFA4784B, 0xCBED606E]


def test_pcg32_seed_expansion_wiring():
    # rand_core's seed_from_u64 advances first and outputs the new state: from state 0 the first
    # state is the increment itself
    st, w = S.pcg32(0)
    assert st == S.SEED_INC
    assert w == S.xsh_rr(S.SEED_INC)
    st2, w2 = S.pcg32(st)
    assert st2 == S.lcg(S.SEED_INC) and w2 == S.xsh_rr(st2)


def test_draw_hand_cases(L):
    toks = np.array([7, 3, 9], np.uint32)
    probs = np.array([0.5, 0.3, 0.2], np.float32)
    cases = [(0.0, -1, 7), (0.49, -1, 7), (0.6, -1, 3), (0.81, -1, 9), (0.999, -1, 9),
             (0.0, 7, 3), (0.59, 7, 3), (0.61, 7, 9), (0.3, 3, 7), (0.9, 3, 9)]
    for u, ex, want in cases:
        assert S.draw(toks, probs, None if ex < 0 else ex, u) == want, (u, ex)
        assert L.snl_draw(_u32p(toks), _f32p(probs), 3, ex, u) == want, (u, ex)


def test_finish_distribution_cases(L):
    vals = np.array([2.0, 1.0, 0.0, -1.0], np.float32)
    e = np.exp(np.array([0.0, -1.0, -2.0, -3.0]))
    full = e / e.sum()
    for t, mp, tp, keep in [(1.0, 0.0, 1.0, 4), (1.0, 0.0, 0.9, 3), (1.0, 0.2, 1.0, 2), (1.0, 0.5, 1.0, 1),
                            (1.0, 0.0, 0.6, 1), (0.5, 0.0, 1.0, 4)]:
        got = S.finish(vals, t, mp, tp)
        assert len(got) == keep, (t, mp, tp)
        ref = np.exp((vals.astype(np.float64) - 2.0) / t)[:keep]
        assert np.allclose(got, ref / ref.sum(), rtol=1e-6)
        out = np.zeros(4, np.float32)
        n = L.snl_finish_distribution(_f32p(vals), 4, t, mp, tp, _f32p(out))
        assert n == keep
        assert np.allclose(out[:n], got, rtol=1e-6)
    assert np.allclose(S.finish(vals, 1.0, 0.0, 1.0), full, rtol=1e-6)


def test_penalties_and_topk_order():
    lg = np.array([1.0, 3.0, 3.0, -2.0, 0.5], np.float32)
    out = S.penalise(lg, {1: 2, 3: 1}, 1.5, 0.1, 0.25)
    assert out[1] == np.float32(np.float32(3.0 / 1.5) - np.float32(0.1 + 0.25 * 2))
    assert out[3] == np.float32(np.float32(-2.0 * 1.5) - np.float32(0.1 + 0.25))
    assert out[0] == 1.0 and out[2] == 3.0
    assert S.top_k(np.array([1.0, 3.0, 3.0, 2.0], np.float32), 3).tolist() == [1, 2, 3]  # ties: lower index first


def test_verify_output_is_distributed_as_p():
    """Integrate verify over a grid of uniforms: P(out = t) must equal p_t, draft or not."""
    toks = np.array([5, 1, 8, 2], np.uint32)
    probs = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    grid = (np.arange(400) + 0.5) / 400

    class Seq:
        def __init__(self, a, b):
            self.v = [a, b]

        def f32(self):
            return self.v.pop(0)

    for draft in (5, 8, 2, 99):
        hist = {}
        for ua in grid:
            for ud in grid:
                _, t = S.verify(False, toks, probs, draft, Seq(ua, ud))
                hist[t] = hist.get(t, 0) + 1
        got = np.array([hist.get(int(t), 0) for t in toks], np.float64) / len(grid) ** 2
        assert np.allclose(got, probs, atol=4e-3), (draft, got)
