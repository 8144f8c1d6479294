"""Pins the CPU oracle (oracle/snl_oracle.c) before the GPU results are compared with it.

The reference ships no golden vectors or tests for this path, so each oracle
function is pinned here by what the mathematics fixes: fp64 restatements of
the textbook operation, closed forms, invariants, special cases that reduce to
a library routine (numpy float16 rounding, transformers' Qwen3.5 gated
delta-rule / causal conv / gated RMSNorm / rotate-half RoPE), and brute force
on small inputs.  Each check is chosen so that a plausible mistake (a dropped
term, a wrong sign or index, a transposed operand, (1+w) vs w) fails it.
"""
import math

import numpy as np
import pytest


def rng(seed=0):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- generator
def test_randn_moments_and_determinism(oracle):
    key = oracle.stream_key(7, 123)
    v = np.array([oracle.randn(key, i) for i in range(20000)])
    assert abs(v.mean()) < 0.03 and abs(v.std() - 1.0) < 0.03
    assert np.abs(v).max() <= math.sqrt(12.0) + 1e-6  # Irwin-Hall(4) support is +-sqrt(12)
    assert oracle.randn(key, 5) == oracle.randn(key, 5)
    assert oracle.stream_key(7, 123) != oracle.stream_key(7, 124)
    u = np.array([oracle.randu(key, i) for i in range(20000)])
    assert u.min() >= 0.0 and u.max() < 1.0 and abs(u.mean() - 0.5) < 0.01


# ---------------------------------------------------------------- f16 packing
def test_f16_rne_matches_numpy(oracle):
    r = rng(1)
    vals = np.concatenate([
        r.standard_normal(4000).astype(np.float32) * 10,
        r.standard_normal(1000).astype(np.float32) * 1e-6,  # f16 subnormals
        (r.standard_normal(500) * 1e5).astype(np.float32),  # overflow to inf
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 1.0 + 2.0 ** -11,
                  1.0 + 3 * 2.0 ** -11], np.float32),
    ])
    ours = np.array([oracle.f32_to_f16_bits(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)
    back = np.array([oracle.lib().orc_f16_to_f32(int(b)) for b in ref[:2000]], np.float32)
    assert np.array_equal(back, ref[:2000].view(np.float16).astype(np.float32))


# ---------------------------------------------------------------- quantisation (weights.rs:123-153)
def test_q8_quantize_properties(oracle):
    r = rng(2)
    w = (r.standard_normal((64, 256)) * 0.02).astype(np.float32)
    w[3, :32] = 0.0  # all-zero block
    q, s = oracle.quantize(w, 0)
    blocks = w.reshape(-1, 32)
    qb = q.reshape(-1, 32).astype(np.int32)
    sb = s.reshape(-1)
    amax = np.abs(blocks).max(1)
    assert np.array_equal(sb, (amax / np.float32(127.0)).astype(np.float32))
    nz = amax > 0
    # the max-magnitude element lands on +-127 exactly
    idx = np.abs(blocks).argmax(1)
    assert np.all(np.abs(qb[np.arange(len(qb)), idx][nz]) == 127)
    # dequantisation error at most half a step
    deq = qb * sb[:, None]
    assert np.all(np.abs(deq - blocks) <= sb[:, None] * 0.5000001 + 1e-12)
    assert np.all(qb[~nz] == 0) and np.all(sb[~nz] == 0)


def test_q8_round_half_away_from_zero(oracle):
    # d = 127/127 = 1 exactly: v*id = v, so +-2.5 must round to +-3 (Rust f32::round), not to even.
    blk = np.zeros(32, np.float32)
    blk[0], blk[1], blk[2], blk[3] = 127.0, 2.5, -2.5, 0.5
    q, s = oracle.quantize(blk.reshape(1, 32), 0)
    assert s[0, 0] == 1.0
    assert q[0, 1] == 3 and q[0, 2] == -3 and q[0, 3] == 1


def test_q4_layout_and_rule(oracle):
    # Largest-magnitude value -> nibble 0 (value -8); nibble i of LE word w holds element w*8+i.
    blk = np.arange(32, dtype=np.float32) - 8.0  # values -8..23, largest magnitude 23
    blk = -blk  # largest magnitude -23 at element 31
    q, s = oracle.quantize(blk.reshape(1, 32), 1)
    d = s[0, 0]
    assert d == np.float32(-23.0) / np.float32(-8.0)
    words = q.reshape(4, 4).astype(np.uint32)
    words = words[:, 0] | (words[:, 1] << 8) | (words[:, 2] << 16) | (words[:, 3] << 24)
    nib = np.array([(words[e // 8] >> (4 * (e % 8))) & 15 for e in range(32)])
    assert nib[31] == 0
    # trunc(v*id + 8.5) clamped to [0, 15]
    idf = np.float32(1.0) / d
    expect = np.clip(np.trunc(blk * idf + np.float32(8.5)), 0, 15)
    assert np.array_equal(nib, expect)
    deq = oracle.dequant(q, s, 1, 32)[0]
    assert np.array_equal(deq, ((nib.astype(np.int64) - 8).astype(np.float32) * d).astype(np.float32))


# ---------------------------------------------------------------- GEMV (matmul.wgsl)
@pytest.mark.parametrize("quant", [0, 1])
@pytest.mark.parametrize("m", [1, 2, 5, 12])
def test_gemv_vs_fp64(oracle, quant, m):
    r = rng(3 + quant)
    n, k = 96, 1024
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    q, s = oracle.quantize(w, quant)
    x = r.standard_normal((m, k)).astype(np.float32)
    y = oracle.gemv(quant, q, s, x, n, k)
    deq = oracle.dequant(q, s, quant, k).astype(np.float64)
    ref = x.astype(np.float64) @ deq.T
    scale = np.abs(x.astype(np.float64)) @ np.abs(deq).T
    assert np.all(np.abs(y - ref) <= 1e-6 * scale + 1e-9)


def test_gemv_one_hot_selects_column(oracle):
    r = rng(4)
    n, k = 40, 256
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    for quant in (0, 1):
        q, s = oracle.quantize(w, quant)
        deq = oracle.dequant(q, s, quant, k)
        for col in (0, 31, 32, 255):
            x = np.zeros((1, k), np.float32)
            x[0, col] = 1.0
            y = oracle.gemv(quant, q, s, x, n, k)
            assert np.array_equal(y[0], deq[:, col])


def test_gemv_m1_equals_rows_of_m2(oracle):
    # matvec1 and matvec2 use the same per-row order, so each row is bitwise the same.
    r = rng(5)
    n, k = 64, 4096
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    q, s = oracle.quantize(w, 0)
    x = r.standard_normal((2, k)).astype(np.float32)
    y2 = oracle.gemv(0, q, s, x, n, k)
    assert np.array_equal(oracle.gemv(0, q, s, x[:1], n, k)[0], y2[0])
    assert np.array_equal(oracle.gemv(0, q, s, x[1:], n, k)[0], y2[1])


# ---------------------------------------------------------------- layers.wgsl
def test_branch_norm_modes(oracle):
    r = rng(6)
    h, m = 512, 3
    x = r.standard_normal((m, 2, h)).astype(np.float32)
    w = (r.standard_normal(h) * 0.1).astype(np.float32)
    coef = r.random((m, 8)).astype(np.float32)
    for mode in (0, 1):
        out = oracle.branch_norm(x, coef, w, h, m, m, mode, eps=1e-6)
        x64 = x.astype(np.float64)
        v = x64[:, 0] if mode == 0 else coef[:, :1] * x64[:, 0] + coef[:, 1:2] * x64[:, 1]
        ref = v / np.sqrt((v * v).mean(1, keepdims=True) + 1e-6) * (1.0 + w)
        assert np.allclose(out, ref, rtol=2e-6, atol=1e-6)
    # last_row: one output row, taken from step row m-1; weight_one=0 gives a plain-w norm
    out = oracle.branch_norm(x, coef, w, h, 1, m, 0, last_row=1, one=0.0)
    v = x[m - 1, 0].astype(np.float64)
    assert np.allclose(out[0], v / np.sqrt((v * v).mean() + 1e-6) * w, rtol=2e-6, atol=1e-7)
    # x_stride = h reads packed rows
    packed = x[:, 0].copy()
    out = oracle.branch_norm(packed, None, w, h, m, m, 0, x_stride=h)
    assert np.array_equal(out, oracle.branch_norm(x, None, w, h, m, m, 0))


def test_branch_norm_matches_transformers_rmsnorm(oracle):
    torch = pytest.importorskip("torch")
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5RMSNorm

    r = rng(7)
    h = 256
    x = r.standard_normal((2, 2, h)).astype(np.float32)
    w = (r.standard_normal(h) * 0.1).astype(np.float32)
    norm = Qwen3_5RMSNorm(h, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(torch.from_numpy(w))
        ref = norm(torch.from_numpy(x[:, 0].copy())).numpy()
    out = oracle.branch_norm(x, None, w, h, 2, 2, 0)
    assert np.allclose(out, ref, rtol=1e-5, atol=1e-6)


def _sinkhorn64(lg, iters):
    a, b, c, e = (float(v) for v in lg[4:8])

    def lse(u, v):
        mx = max(u, v)
        return mx + math.log(math.exp(u - mx) + math.exp(v - mx))

    for _ in range(iters):
        r0, r1 = lse(a, b), lse(c, e)
        a, b, c, e = a - r0, b - r0, c - r1, e - r1
        c0, c1 = lse(a, c), lse(b, e)
        a, c, b, e = a - c0, c - c0, b - c1, e - c1
    return np.exp([a, b, c, e])


def test_mhc_router_and_sinkhorn(oracle):
    r = rng(8)
    h, m, iters = 256, 2, 20
    x = r.standard_normal((m, 2 * h)).astype(np.float32)
    w = np.concatenate([(r.standard_normal(8 * 2 * h) * 0.02), r.standard_normal(8)]).astype(np.float32)
    raw, coef = oracle.mhc(x, w, h, m, iters)
    W = w[:16 * h].reshape(8, 2 * h).astype(np.float64)
    x64 = x.astype(np.float64)
    assert np.allclose(raw[:, :8], x64 @ W.T, rtol=1e-5, atol=1e-5)
    assert np.allclose(raw[:, 8], (x64 * x64).sum(1), rtol=1e-5)
    for i in range(m):
        lg = raw[i, :8].astype(np.float64) / np.sqrt(raw[i, 8] / (2 * h) + 1e-6) + w[16 * h:16 * h + 8]
        sig = 1.0 / (1.0 + np.exp(-lg[:4]))
        assert np.allclose(coef[i, :4], [sig[0], sig[1], 2 * sig[2], 2 * sig[3]], rtol=1e-5)
        mix = _sinkhorn64(lg, iters)
        assert np.allclose(coef[i, 4:], mix, rtol=1e-4, atol=1e-6)
        # after the last column step each column of exp(mix) sums to 1; rows converge to 1
        M = coef[i, 4:].reshape(2, 2).astype(np.float64)
        assert np.allclose(M.sum(0), 1.0, atol=1e-5)
        assert np.allclose(M.sum(1), 1.0, atol=1e-3)


def test_merge_modes(oracle):
    r = rng(9)
    h, m = 256, 2
    x = r.standard_normal((m, 2, h)).astype(np.float32)
    br = r.standard_normal((m, h)).astype(np.float32)
    coef = r.random((m, 8)).astype(np.float32)
    x0 = oracle.merge(x, coef, br, h, m, 0)
    assert np.array_equal(x0[:, 0], x[:, 0] + br) and np.array_equal(x0[:, 1], x[:, 1])
    x3 = oracle.merge(x, coef, br, h, m, 3)
    assert np.array_equal(x3[:, 1], x[:, 0]) and np.array_equal(x3[:, 0], x[:, 0])
    c = coef.astype(np.float64)[:, :, None]
    n0 = c[:, 4] * x[:, 0] + c[:, 5] * x[:, 1] + c[:, 2] * br
    n1 = c[:, 6] * x[:, 0] + c[:, 7] * x[:, 1] + c[:, 3] * br
    x1 = oracle.merge(x, coef, br, h, m, 1)
    assert np.allclose(x1[:, 0], n0, rtol=1e-5, atol=1e-6) and np.allclose(x1[:, 1], n1, rtol=1e-5, atol=1e-6)
    x2 = oracle.merge(x, coef, br, h, m, 2)
    assert np.allclose(x2[:, 0], 0.5 * (n0 + n1), rtol=1e-5, atol=1e-6)


def test_swiglu(oracle):
    r = rng(10)
    inter, m = 768, 2
    p = r.standard_normal((m, 2 * inter)).astype(np.float32) * 3
    act = oracle.swiglu(p, inter, m)
    g, u = p[:, :inter].astype(np.float64), p[:, inter:].astype(np.float64)
    assert np.allclose(act, g / (1 + np.exp(-g)) * u, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- linear.wgsl
def _lin_inputs(r, nk, nv, m):
    conv_dim = 2 * nk * 128 + nv * 128
    stride = conv_dim + nv * 128 + 2 * nv
    proj = r.standard_normal((m, stride)).astype(np.float32)
    lw = np.concatenate([r.standard_normal(conv_dim * 4) * 0.25, r.random(nv) * math.log(16),
                         r.standard_normal(nv) * 0.5, 1 + 0.1 * r.standard_normal(128)]).astype(np.float32)
    return conv_dim, stride, proj, lw


def test_conv_matches_transformers_causal_conv(oracle):
    torch = pytest.importorskip("torch")
    from transformers.models.qwen3_5.modeling_qwen3_5 import causal_conv1d_update

    r = rng(11)
    nk, nv, m = 2, 4, 2
    conv_dim, stride, proj, lw = _lin_inputs(r, nk, nv, m)
    st0 = r.standard_normal((3, conv_dim)).astype(np.float32)
    out, st, ck = oracle.conv(proj, stride, st0, lw, conv_dim, m, ckpt=1)
    hs = torch.from_numpy(proj[:, :conv_dim].T.copy()).unsqueeze(0)  # [1, C, T]
    cs = torch.from_numpy(st0.T.copy()).unsqueeze(0)  # [1, C, 3] oldest first
    wt = torch.from_numpy(lw[:conv_dim * 4].reshape(conv_dim, 4).copy())
    ref = causal_conv1d_update(hs, cs, wt, None, "silu")[0].numpy().T
    assert np.allclose(out, ref, rtol=1e-5, atol=1e-6)
    assert np.allclose(st, cs[0].numpy().T)
    # checkpoint after token 1 == state after a single-token step
    _, st1, _ = oracle.conv(proj[:1], stride, st0, lw, conv_dim, 1, ckpt=0)
    assert np.array_equal(ck, st1)


def _delta_ref_transformers(proj, conv_out, state, lw, conv_dim, nk, nv, eps, m):
    import torch
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5RMSNormGated, torch_recurrent_gated_delta_rule

    kd = nk * 128
    q = torch.from_numpy(conv_out[:, :kd].reshape(1, m, nk, 128).copy()).double()
    k = torch.from_numpy(conv_out[:, kd:2 * kd].reshape(1, m, nk, 128).copy()).double()
    v = torch.from_numpy(conv_out[:, 2 * kd:2 * kd + nv * 128].reshape(1, m, nv, 128).copy()).double()
    rep = nv // nk
    q, k = q.repeat_interleave(rep, dim=2), k.repeat_interleave(rep, dim=2)
    z_off, b_off = conv_dim, conv_dim + nv * 128
    a_off = b_off + nv
    b = torch.from_numpy(proj[:, b_off:b_off + nv].copy()).double().unsqueeze(0)
    a = torch.from_numpy(proj[:, a_off:a_off + nv].copy()).double().unsqueeze(0)
    a_log = torch.from_numpy(lw[conv_dim * 4:conv_dim * 4 + nv].copy()).double()
    dt = torch.from_numpy(lw[conv_dim * 4 + nv:conv_dim * 4 + 2 * nv].copy()).double()
    g = -a_log.exp() * torch.nn.functional.softplus(a + dt)
    beta = b.sigmoid()
    st = torch.from_numpy(state.copy()).double().unsqueeze(0)
    o, fs = torch_recurrent_gated_delta_rule(q.float(), k.float(), v.float(), g.float(), beta.float(), st.float(),
                                             True, use_qk_l2norm_in_kernel=True)
    norm = Qwen3_5RMSNormGated(128, eps=eps)
    with torch.no_grad():
        norm.weight.copy_(torch.from_numpy(lw[conv_dim * 4 + 2 * nv:].copy()))
        z = torch.from_numpy(proj[:, z_off:z_off + nv * 128].reshape(1, m, nv, 128).copy())
        out = norm(o.float(), z.float())
    return out.reshape(m, nv * 128).numpy(), fs[0].numpy()


@pytest.mark.parametrize("m", [1, 2])
def test_delta_matches_transformers(oracle, m):
    pytest.importorskip("torch")
    r = rng(12 + m)
    nk, nv = 2, 4
    conv_dim, stride, proj, lw = _lin_inputs(r, nk, nv, m)
    conv_out = r.standard_normal((m, conv_dim)).astype(np.float32)
    state = (r.standard_normal((nv, 128, 128)) * 0.1).astype(np.float32)
    out, st, ck = oracle.delta(proj, stride, conv_out, state, lw, conv_dim, nk, nv, 1e-6, m, ckpt=1 if m == 2 else 0)
    ref_out, ref_st = _delta_ref_transformers(proj, conv_out, state, lw, conv_dim, nk, nv, 1e-6, m)
    assert np.allclose(st, ref_st, rtol=1e-4, atol=1e-5)
    assert np.allclose(out, ref_out, rtol=1e-3, atol=1e-4)
    if m == 2:
        _, st1, _ = oracle.delta(proj[:1], stride, conv_out[:1], state, lw, conv_dim, nk, nv, 1e-6, 1, 0)
        assert np.array_equal(ck, st1)
        _, st2, _ = oracle.delta(proj[1:], stride, conv_out[1:], st1, lw, conv_dim, nk, nv, 1e-6, 1, 0)
        assert np.array_equal(st, st2)


def test_delta_invariants(oracle):
    r = rng(14)
    nk, nv = 1, 2
    conv_dim, stride, proj, lw = _lin_inputs(r, nk, nv, 1)
    conv_out = r.standard_normal((1, conv_dim)).astype(np.float32)
    state = (r.standard_normal((nv, 128, 128)) * 0.1).astype(np.float32)
    b_off = conv_dim + nv * 128
    a_off = b_off + nv
    # beta = 0 (b -> -inf): pure decay of the state
    p = proj.copy()
    p[0, b_off:b_off + nv] = -1e4
    _, st, _ = oracle.delta(p, stride, conv_out, state, lw, conv_dim, nk, nv, 1e-6, 1, 0)
    araw = p[0, a_off:a_off + nv].astype(np.float64) + lw[conv_dim * 4 + nv:conv_dim * 4 + 2 * nv]
    decay = np.exp(-np.exp(lw[conv_dim * 4:conv_dim * 4 + nv].astype(np.float64)) * np.log1p(np.exp(araw)))
    assert np.allclose(st, state * decay[:, None, None], rtol=1e-5, atol=1e-7)
    # decay = 1 (A_log -> -inf), beta = 1: after the update S^T k = v exactly (delta rule fixed point)
    lw2 = lw.copy()
    lw2[conv_dim * 4:conv_dim * 4 + nv] = -1e4
    p[0, b_off:b_off + nv] = 1e4
    _, st, _ = oracle.delta(p, stride, conv_out, state, lw2, conv_dim, nk, nv, 1e-6, 1, 0)
    k = conv_out[0, 128:256].astype(np.float64)
    k = k / np.sqrt((k * k).sum() + 1e-6)
    for h in range(nv):
        v = conv_out[0, 256 + h * 128:256 + (h + 1) * 128]
        assert np.allclose(st[h].astype(np.float64).T @ k, v, rtol=1e-4, atol=1e-4)


# ---------------------------------------------------------------- attention.wgsl
def _attn_case(r, n_heads, n_kv, m, pos0, ctx):
    q_dim, kv_dim = n_heads * 256, n_kv * 256
    stride = 2 * q_dim + 2 * kv_dim
    kc = np.zeros((ctx, kv_dim), np.uint16)
    vc = np.zeros((ctx, kv_dim), np.uint16)
    kc[:pos0] = (r.standard_normal((pos0, kv_dim))).astype(np.float16).view(np.uint16)
    vc[:pos0] = (r.standard_normal((pos0, kv_dim))).astype(np.float16).view(np.uint16)
    proj = r.standard_normal((m, stride)).astype(np.float32)
    norms = (r.standard_normal(512) * 0.1).astype(np.float32)
    return stride, kc, vc, proj, norms


def _rope64(x, pos, rot, theta):
    half = rot // 2
    fi = np.arange(half)
    inv = theta ** (-(2.0 * fi) / rot)
    ang = pos * inv
    out = x.copy()
    x1, x2 = x[:half], x[half:rot]
    out[:half] = x1 * np.cos(ang) - x2 * np.sin(ang)
    out[half:rot] = x2 * np.cos(ang) + x1 * np.sin(ang)
    return out


def test_attn_prep_norm_rope_and_cache(oracle):
    r = rng(15)
    n_heads, n_kv, m, pos0 = 4, 1, 2, 5
    stride, kc, vc, proj, norms = _attn_case(r, n_heads, n_kv, m, pos0, 16)
    ap = oracle.attn_params(n_heads, n_kv, 64, stride)
    rpos = np.array([[pos0 + i] * 3 + [0] for i in range(m)], np.uint32)
    qbuf = oracle.attn_prep(ap, proj, kc, vc, norms, rpos, m, pos0)
    for i in range(m):
        pos = pos0 + i
        for hh in range(n_heads):
            v = proj[i, hh * 512:hh * 512 + 256].astype(np.float64)
            v = v / np.sqrt((v * v).mean() + 1e-6) * (1 + norms[:256])
            assert np.allclose(qbuf[i, hh * 256:(hh + 1) * 256], _rope64(v, pos, 64, 1e7), rtol=1e-4, atol=1e-5)
        k = proj[i, 2 * 1024:2 * 1024 + 256].astype(np.float64)
        k = _rope64(k / np.sqrt((k * k).mean() + 1e-6) * (1 + norms[256:]), pos, 64, 1e7)
        kk = kc[pos].view(np.float16).astype(np.float64)
        assert np.allclose(kk, k, rtol=2e-3, atol=2e-3)
        vv = proj[i, 2 * 1024 + 256:2 * 1024 + 512]
        assert np.array_equal(vc[pos], vv.astype(np.float16).view(np.uint16))


def test_rope_matches_transformers_rotate_half(oracle):
    torch = pytest.importorskip("torch")
    from transformers.models.qwen3_5.modeling_qwen3_5 import apply_rotary_pos_emb

    r = rng(16)
    x = r.standard_normal(256)
    pos, rot, theta = 37, 64, 1e7
    inv = 1.0 / (theta ** (torch.arange(0, rot, 2, dtype=torch.float64) / rot))
    freqs = pos * inv
    emb = torch.cat([freqs, freqs])
    t = torch.from_numpy(x).reshape(1, 1, 1, 256)
    qe, _ = apply_rotary_pos_emb(t, t, emb.cos().reshape(1, 1, rot), emb.sin().reshape(1, 1, rot))
    assert np.allclose(_rope64(x, pos, rot, theta), qe.reshape(-1).numpy(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("parts", [1, 3])
def test_attend_vs_brute_force(oracle, parts):
    r = rng(17 + parts)
    n_heads, n_kv, m, pos0 = 8, 2, 2, 37
    stride, kc, vc, proj, norms = _attn_case(r, n_heads, n_kv, m, pos0, 64)
    ap = oracle.attn_params(n_heads, n_kv, 64, stride)
    rpos = np.array([[pos0 + i] * 3 + [0] for i in range(m)], np.uint32)
    qbuf = oracle.attn_prep(ap, proj, kc, vc, norms, rpos, m, pos0)
    out = oracle.attend(ap, proj, qbuf, kc, vc, m, pos0, parts)
    K = kc.view(np.float16).astype(np.float64)
    V = vc.view(np.float16).astype(np.float64)
    for i in range(m):
        total = pos0 + i + 1
        for hh in range(n_heads):
            kh = hh // 4
            q = qbuf[i, hh * 256:(hh + 1) * 256].astype(np.float64)
            s = K[:total, kh * 256:(kh + 1) * 256] @ q / 16.0
            p = np.exp(s - s.max())
            o = (p / p.sum()) @ V[:total, kh * 256:(kh + 1) * 256]
            gate = proj[i, hh * 512 + 256:hh * 512 + 512].astype(np.float64)
            ref = o / (1 + np.exp(-gate))
            assert np.allclose(out[i, hh * 256:(hh + 1) * 256], ref, rtol=1e-4, atol=1e-5)


def test_attend_split_invariance(oracle):
    r = rng(20)
    n_heads, n_kv, m, pos0 = 4, 1, 1, 300
    stride, kc, vc, proj, norms = _attn_case(r, n_heads, n_kv, m, pos0, 320)
    ap = oracle.attn_params(n_heads, n_kv, 64, stride)
    rpos = np.array([[pos0] * 3 + [0]], np.uint32)
    qbuf = oracle.attn_prep(ap, proj, kc, vc, norms, rpos, m, pos0)
    a = oracle.attend(ap, proj, qbuf, kc, vc, m, pos0, 1)
    for parts in (2, 5, 64):
        b = oracle.attend(ap, proj, qbuf, kc, vc, m, pos0, parts)
        assert np.allclose(a, b, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- argmax (sampler.rs:169-177)
def test_argmax_first_index_on_ties(oracle):
    v = np.array([0.5, 2.0, -1.0, 2.0, 2.0], np.float32)
    assert oracle.argmax(v) == 1
    r = rng(21)
    for _ in range(20):
        v = r.integers(0, 5, 1000).astype(np.float32)
        assert oracle.argmax(v) == int(np.argmax(v))  # numpy also returns the first maximum


# ---- engine composition (src/engine.rs:383-570, :653-697): self-consistency invariants ----
def _tiny_engines(oracle, n=2):
    import snl.config as C

    cfg = C.tiny_config()
    return cfg, [oracle.Engine(cfg, seed=5, quant=0, ctx=64, max_m=2) for _ in range(n)]


def _state_sizes(cfg):
    plan = cfg.execution_plan()
    n_lin = sum(1 for l in plan if not cfg.full_attention[l])
    conv_dim = 2 * cfg.lin_k_heads * cfg.lin_k_dim + cfg.lin_v_heads * cfg.lin_v_dim
    return n_lin * cfg.lin_v_heads * cfg.lin_v_dim * cfg.lin_v_dim, n_lin * 3 * conv_dim


def test_engine_stepwise_equals_batched(oracle):
    """A 2-token pass gives each row the logits of two 1-token passes (positions, caches and the
    recurrent state carried exactly between rows)."""
    cfg, (a, b) = _tiny_engines(oracle)
    p = np.random.default_rng(7).integers(0, cfg.vocab, 8).tolist()
    a.forward(p[:6], logit_rows=0)
    b.forward(p[:6], logit_rows=0)
    two = a.forward(p[6:8], logit_rows=2)
    one0 = b.forward(p[6:7], logit_rows=1)[0]
    one1 = b.forward(p[7:8], logit_rows=1)[0]
    assert np.array_equal(two[0], one0) and np.array_equal(two[1], one1)
    a.close()
    b.close()


def test_engine_rollback_equals_never_run(oracle):
    cfg, (a, b) = _tiny_engines(oracle)
    n_state, n_conv = _state_sizes(cfg)
    p = np.random.default_rng(8).integers(0, cfg.vocab, 9).tolist()
    a.forward(p[:6], logit_rows=0)
    b.forward(p[:6], logit_rows=0)
    a.forward(p[6:8], logit_rows=2, ckpt=True)
    a.rollback()
    b.forward(p[6:7], logit_rows=1)
    assert a.pos == b.pos == 7 and a.hid_rows == b.hid_rows == 1
    for bid, n in ((3, n_state), (4, n_conv), (2, cfg.hidden)):
        assert np.array_equal(a.buf(bid, n), b.buf(bid, n)), bid
    assert np.array_equal(a.forward(p[8:9])[0], b.forward(p[8:9])[0])
    a.close()
    b.close()


def test_engine_snapshot_restore(oracle):
    cfg, (a, b) = _tiny_engines(oracle)
    p = np.random.default_rng(9).integers(0, cfg.vocab, 12).tolist()
    a.forward(p[:6], logit_rows=0)
    a.snapshot(0)
    a.forward(p[6:10], logit_rows=0)
    a.restore(0, 6)
    b.forward(p[:6], logit_rows=0)
    assert a.pos == b.pos == 6
    assert np.array_equal(a.forward(p[10:12], logit_rows=2), b.forward(p[10:12], logit_rows=2))
    a.close()
    b.close()
