"""Kernel-level parity of the HIP library (through the C ABI) against the CPU oracle.

Tolerances: the path is required to agree within 1e-2 relative (fp32 accumulation) on
logits and DeltaNet state; the kernels here are held to much tighter bounds (GEMV 1e-5 of
the sum of |terms|), since the oracle and the GPU only differ in summation order.
Integer/index work (greedy pick) is bit-exact.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_cuda():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch


@pytest.fixture(scope="module")
def K(torch_cuda):
    import snl

    snl.lib()
    return snl.kernels


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _gemv_case(oracle, quant, n, k, m, seed):
    r = np.random.default_rng(seed)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    q, s = oracle.quantize(w, quant)
    x = r.standard_normal((m, k)).astype(np.float32)
    return q, s, x


@pytest.mark.parametrize("quant", [0, 1])
@pytest.mark.parametrize("n,k", [(96, 1024), (4096, 4096), (12288, 4096), (4096, 12288), (1544, 256), (512, 768)])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_gemv_matches_oracle(torch_cuda, K, oracle, quant, n, k, m):
    torch = torch_cuda
    print(f"gemv quant={quant} n={n} k={k} m={m}", flush=True)
    q, s, x = _gemv_case(oracle, quant, n, k, m, seed=n + k + m + quant)
    ref = oracle.gemv(quant, q, s, x, n, k)
    dq, ds, dx = _dev(torch, q), _dev(torch, s), _dev(torch, x)
    y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    K.gemv(quant, dq, ds, dx, y, m, n, k, k, n)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    deq = oracle.dequant(q, s, quant, k).astype(np.float64)
    scale = np.abs(x.astype(np.float64)) @ np.abs(deq).T
    assert np.all(np.abs(got - ref) <= 1e-5 * scale + 1e-7), np.abs(got - ref).max()
    exact = x.astype(np.float64) @ deq.T
    assert np.all(np.abs(got - exact) <= 1e-5 * scale + 1e-7)


@pytest.mark.parametrize("quant", [0, 1])
@pytest.mark.parametrize("n,k,m", [(96, 1024, 3), (4096, 4096, 512), (1544, 256, 37), (12352, 4096, 130),
                                   (4096, 12288, 64), (24576, 4096, 17)])
def test_gemm_matches_oracle(torch_cuda, K, oracle, quant, n, k, m):
    """The prefill GEMM against the oracle's GEMV and float64 products of the dequantised weights."""
    torch = torch_cuda
    print(f"gemm quant={quant} n={n} k={k} m={m}", flush=True)
    q, s, x = _gemv_case(oracle, quant, n, k, m, seed=7 * n + k + m + quant)
    x[0] *= 1e3  # rows of very different magnitudes keep their own scale
    if m > 2:
        x[2] *= 1e-4
    dq, ds, dx = _dev(torch, q), _dev(torch, s), _dev(torch, x)
    y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    K.gemm(quant, dq, ds, dx, y, m, n, k, k, n)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    deq = oracle.dequant(q, s, quant, k).astype(np.float64)
    scale = np.abs(x.astype(np.float64)) @ np.abs(deq).T
    exact = x.astype(np.float64) @ deq.T
    assert np.all(np.abs(got - exact) <= 1e-5 * scale + 1e-30), np.abs(got - exact).max()
    if m <= 64:
        ref = oracle.gemv(quant, q, s, x, n, k)
        assert np.all(np.abs(got - ref) <= 1e-5 * scale + 1e-30)


@pytest.mark.parametrize("quant", [0, 1])
def test_gemm_rows_independent_of_m(torch_cuda, K, oracle, quant):
    """A token row's result does not depend on how many rows share the call or where it sits."""
    torch = torch_cuda
    n, k = 1040, 1024
    q, s, x = _gemv_case(oracle, quant, n, k, 100, seed=5)
    dq, ds, dx = _dev(torch, q), _dev(torch, s), _dev(torch, x)
    y = torch.zeros((100, n), dtype=torch.float32, device="cuda")
    K.gemm(quant, dq, ds, dx, y, 100, n, k, k, n)
    full = y.cpu().numpy()
    for lo, hi in ((0, 3), (37, 100), (64, 65)):
        ys = torch.zeros((hi - lo, n), dtype=torch.float32, device="cuda")
        K.gemm(quant, dq, ds, dx[lo:hi], ys, hi - lo, n, k, k, n)
        assert np.array_equal(ys.cpu().numpy(), full[lo:hi])


def test_gemm_time_runs(torch_cuda, K):
    """The isolated GEMM timing used for the long-context roofline returns a positive mean."""
    for quant in (0, 1):
        ms = K.gemm_time(quant, 2048, 1024, 512, reps=3)
        assert 0.0 < ms < 100.0


@pytest.mark.parametrize("quant", [0, 1])
def test_gemv_rows_independent_of_m(torch_cuda, K, oracle, quant):
    """Row r of an M-row call is bitwise the M=1 result: the verify pass reproduces plain decode."""
    torch = torch_cuda
    n, k = 4096, 4096
    q, s, x = _gemv_case(oracle, quant, n, k, 4, seed=11)
    dq, ds, dx = _dev(torch, q), _dev(torch, s), _dev(torch, x)
    outs = {}
    for m in (1, 2, 4):
        y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
        K.gemv(quant, dq, ds, dx, y, m, n, k, k, n)
        outs[m] = y.cpu().numpy()
    for r in range(4):
        y1 = torch.zeros((1, n), dtype=torch.float32, device="cuda")
        K.gemv(quant, dq, ds, dx[r:r + 1], y1, 1, n, k, k, n)
        one = y1.cpu().numpy()[0]
        for m in (2, 4):
            if r < m:
                assert np.array_equal(outs[m][r], one)


@pytest.mark.parametrize("quant", [0, 1], ids=["q8", "q4"])
def test_gemv_lm_head_size(torch_cuda, K, oracle, quant):
    """Full LM-head shape (N=248320, K=4096, M=2): fp64 check on sampled rows, one-hot column check."""
    torch = torch_cuda
    n, k = 248320, 4096
    print(f"lm head gemv quant={quant}", flush=True)
    r = np.random.default_rng(5 + quant)
    rb = k if quant == 0 else k // 2
    q = r.integers(0, 256, size=(n, rb), dtype=np.uint8)
    s = (r.random((n, k // 32), dtype=np.float32) * 2e-4).astype(np.float32)
    x = r.standard_normal((2, k)).astype(np.float32)
    dq, ds = _dev(torch, q), _dev(torch, s)
    y = torch.zeros((2, n), dtype=torch.float32, device="cuda")
    K.gemv(quant, dq, ds, _dev(torch, x), y, 2, n, k, k, n)
    got = y.cpu().numpy()
    rows = np.sort(r.choice(n, 64, replace=False))
    deq = oracle.dequant(q[rows], s[rows], quant, k).astype(np.float64)
    exact = x.astype(np.float64) @ deq.T
    scale = np.abs(x.astype(np.float64)) @ np.abs(deq).T
    assert np.all(np.abs(got[:, rows] - exact) <= 1e-5 * scale + 1e-7)
    # one-hot x selects dequantized column 77 exactly
    e = np.zeros((1, k), np.float32)
    e[0, 77] = 1.0
    y1 = torch.zeros((1, n), dtype=torch.float32, device="cuda")
    K.gemv(quant, dq, ds, _dev(torch, e), y1, 1, n, k, k, n)
    if quant == 0:
        qv = q[:, 77].view(np.int8).astype(np.float32)
    else:  # element 77 = high nibble of byte 38 (element 2j low, 2j + 1 high)
        qv = ((q[:, 38] >> 4) & 15).astype(np.float32) - 8.0
    col = qv * s[:, 2]
    assert np.array_equal(y1.cpu().numpy()[0], col)


def _lin_inputs(r, nk, nv, m):
    conv_dim = 2 * nk * 128 + nv * 128
    stride = conv_dim + nv * 128 + 2 * nv
    proj = r.standard_normal((m, stride)).astype(np.float32)
    lw = np.concatenate([r.standard_normal(conv_dim * 4) * 0.25, r.random(nv) * np.log(16),
                         r.standard_normal(nv) * 0.5, 1 + 0.1 * r.standard_normal(128)]).astype(np.float32)
    return conv_dim, stride, proj, lw


@pytest.mark.parametrize("nk,nv,m", [(16, 32, 2), (16, 32, 1), (2, 4, 2), (2, 4, 4)])
def test_deltanet_matches_oracle(torch_cuda, K, oracle, nk, nv, m):
    """Gated DeltaNet verify step (16 QK / 32 V heads x 128, T=2): output and state vs the oracle."""
    torch = torch_cuda
    print(f"deltanet nk={nk} nv={nv} m={m}", flush=True)
    r = np.random.default_rng(100 + nk + m)
    conv_dim, stride, proj, lw = _lin_inputs(r, nk, nv, m)
    conv0 = r.standard_normal((3, conv_dim)).astype(np.float32)
    st0 = (r.standard_normal((nv, 128, 128)) * 0.1).astype(np.float32)
    ckpt = 1 if m >= 2 else 0
    conv_out, conv_ref, conv_ck = oracle.conv(proj, stride, conv0, lw, conv_dim, m, ckpt)
    out_ref, st_ref, st_ck = oracle.delta(proj, stride, conv_out, st0, lw, conv_dim, nk, nv, 1e-6, m, ckpt)
    cs = np.zeros((3, 3, conv_dim), np.float32)
    cs[0] = conv0
    ss = np.zeros((3, nv, 128, 128), np.float32)
    ss[0] = st0
    d_cs, d_ss = _dev(torch, cs), _dev(torch, ss)
    out = torch.zeros((m, nv * 128), dtype=torch.float32, device="cuda")
    K.deltanet(_dev(torch, proj), stride, _dev(torch, lw), d_cs, d_ss, out, conv_dim, nk, nv, 1e-6, m, ckpt, 0, 2, 1)
    got_out, got_cs, got_ss = out.cpu().numpy(), d_cs.cpu().numpy(), d_ss.cpu().numpy()
    assert np.allclose(got_out, out_ref, rtol=1e-3, atol=1e-4)
    assert np.allclose(got_ss[2], st_ref, rtol=1e-4, atol=1e-5)
    assert np.allclose(got_cs[2], conv_ref, rtol=1e-6, atol=1e-6)
    assert np.array_equal(got_ss[0], st0)  # the input slot is never written
    if ckpt:
        assert np.allclose(got_ss[1], st_ck, rtol=1e-4, atol=1e-5)
        assert np.allclose(got_cs[1], conv_ck, rtol=1e-6, atol=1e-6)
    # relative error of the state within the 1e-2 bound
    rel = np.abs(got_ss[2] - st_ref).max() / np.abs(st_ref).max()
    assert rel < 1e-2


def test_deltanet_two_steps_equal_one_verify(torch_cuda, K):
    """T=2 in one launch is bitwise two T=1 launches (state handed over through memory)."""
    torch = torch_cuda
    r = np.random.default_rng(7)
    nk, nv = 16, 32
    conv_dim, stride, proj, lw = _lin_inputs(r, nk, nv, 2)
    cs = np.zeros((3, 3, conv_dim), np.float32)
    cs[0] = r.standard_normal((3, conv_dim))
    ss = np.zeros((3, nv, 128, 128), np.float32)
    ss[0] = r.standard_normal((nv, 128, 128)) * 0.1
    dp, dl = _dev(torch, proj), _dev(torch, lw)
    a_cs, a_ss = _dev(torch, cs), _dev(torch, ss)
    out2 = torch.zeros((2, nv * 128), dtype=torch.float32, device="cuda")
    K.deltanet(dp, stride, dl, a_cs, a_ss, out2, conv_dim, nk, nv, 1e-6, 2, 1, 0, 2, 1)
    b_cs, b_ss = _dev(torch, cs), _dev(torch, ss)
    o1 = torch.zeros((1, nv * 128), dtype=torch.float32, device="cuda")
    o2 = torch.zeros((1, nv * 128), dtype=torch.float32, device="cuda")
    K.deltanet(dp[0:1], stride, dl, b_cs, b_ss, o1, conv_dim, nk, nv, 1e-6, 1, 0, 0, 1, 1)
    K.deltanet(dp[1:2], stride, dl, b_cs, b_ss, o2, conv_dim, nk, nv, 1e-6, 1, 0, 1, 2, 2)
    assert np.array_equal(out2.cpu().numpy()[0], o1.cpu().numpy()[0])
    assert np.array_equal(out2.cpu().numpy()[1], o2.cpu().numpy()[0])
    assert np.array_equal(a_ss.cpu().numpy()[1], b_ss.cpu().numpy()[1])  # checkpoint == state after token 1
    assert np.array_equal(a_ss.cpu().numpy()[2], b_ss.cpu().numpy()[2])
    assert np.array_equal(a_cs.cpu().numpy()[2], b_cs.cpu().numpy()[2])


def _attn_case(r, n_heads, n_kv, m, pos0, ctx):
    q_dim, kv_dim = n_heads * 256, n_kv * 256
    stride = 2 * q_dim + 2 * kv_dim
    kc = np.zeros((ctx, kv_dim), np.uint16)
    vc = np.zeros((ctx, kv_dim), np.uint16)
    kc[:pos0] = r.standard_normal((pos0, kv_dim)).astype(np.float16).view(np.uint16)
    vc[:pos0] = r.standard_normal((pos0, kv_dim)).astype(np.float16).view(np.uint16)
    proj = r.standard_normal((m, stride)).astype(np.float32)
    norms = (r.standard_normal(512) * 0.1).astype(np.float32)
    return stride, kc, vc, proj, norms


@pytest.mark.parametrize("n_heads,n_kv", [(16, 4), (4, 1)])
@pytest.mark.parametrize("m,pos0", [(1, 0), (2, 0), (1, 127), (2, 127), (2, 300), (1, 1535), (2, 4000)])
def test_attention_matches_oracle(torch_cuda, K, oracle, n_heads, n_kv, m, pos0):
    _attention_vs_oracle(torch_cuda, K, oracle, n_heads, n_kv, m, pos0, 4096 + 16)


@pytest.mark.parametrize("m,pos0,ctx", [(1, 32760, 32784), (2, 32760, 32784), (1, 70000, 70016),
                                        (2, 70000, 70016)])
def test_attention_long_context_matches_oracle(torch_cuda, K, oracle, m, pos0, ctx):
    """The 9B head shape at the end of a 32K cache (512 key parts) and past 64K keys (more parts
    than the combine's threads, so each thread merges several)."""
    _attention_vs_oracle(torch_cuda, K, oracle, 16, 4, m, pos0, ctx)


def _attention_vs_oracle(torch_cuda, K, oracle, n_heads, n_kv, m, pos0, ctx):
    torch = torch_cuda
    print(f"attention heads={n_heads}/{n_kv} m={m} pos0={pos0} ctx={ctx}", flush=True)
    r = np.random.default_rng(pos0 + m + n_heads)
    stride, kc, vc, proj, norms = _attn_case(r, n_heads, n_kv, m, pos0, ctx)
    ap = oracle.attn_params(n_heads, n_kv, 64, stride)
    rpos = np.array([[pos0 + i] * 3 + [0] for i in range(m)], np.uint32)
    kc_ref, vc_ref = kc.copy(), vc.copy()
    q_ref = oracle.attn_prep(ap, proj, kc_ref, vc_ref, norms, rpos, m, pos0)
    parts = max(1, min(64, (pos0 + m + 255) // 256))
    out_ref = oracle.attend(ap, proj, q_ref, kc_ref, vc_ref, m, pos0, parts)
    dk, dv = _dev(torch, kc.view(np.int16)), _dev(torch, vc.view(np.int16))
    qbuf = torch.zeros((m, n_heads * 256), dtype=torch.float32, device="cuda")
    out = torch.zeros((m, n_heads * 256), dtype=torch.float32, device="cuda")
    partial = torch.zeros(m * n_heads * ((ctx + 63) // 64) * 258, dtype=torch.float32, device="cuda")
    K.attention(_dev(torch, proj), stride, qbuf, dk, dv, _dev(torch, norms), out, partial, n_heads, n_kv, 64, 1e7,
                1e-6, (11, 11, 10), ctx, m, pos0, rpos[:, :3])
    torch.cuda.synchronize()
    # The rotary cos / sin come with the step record, formed on the host with the same libm calls
    # as the oracle, so q / k differ only by the order of the norm's sum (measured 1e-7 relative
    # up to position 70000; one f16 key word may round the other way) and the output by the
    # order of the softmax sums (measured 8e-7).  Held to 1e-3 of the largest value.
    tol = 1e-3

    def rel(a, b):
        return float(np.abs(a - b).max() / np.abs(b).max())

    assert rel(qbuf.cpu().numpy(), q_ref) < tol
    kv_got = dk.cpu().numpy().view(np.uint16)[pos0:pos0 + m].view(np.float16).astype(np.float32)
    kv_ref = kc_ref[pos0:pos0 + m].view(np.float16).astype(np.float32)
    assert rel(kv_got, kv_ref) < tol
    assert np.array_equal(dv.cpu().numpy().view(np.uint16)[pos0:pos0 + m], vc_ref[pos0:pos0 + m])
    assert rel(out.cpu().numpy(), out_ref) < tol


def test_attention_rows_independent_of_m(torch_cuda, K):
    """Token 0 of an M=2 call equals the M=1 call bitwise (fixed 128-key parts)."""
    torch = torch_cuda
    r = np.random.default_rng(3)
    n_heads, n_kv, pos0, ctx = 16, 4, 383, 1024
    stride, kc, vc, proj, norms = _attn_case(r, n_heads, n_kv, 2, pos0, ctx)
    res = []
    for m in (1, 2):
        dk, dv = _dev(torch, kc.view(np.int16)), _dev(torch, vc.view(np.int16))
        qbuf = torch.zeros((m, n_heads * 256), dtype=torch.float32, device="cuda")
        out = torch.zeros((m, n_heads * 256), dtype=torch.float32, device="cuda")
        partial = torch.zeros(m * n_heads * ((ctx + 63) // 64) * 258, dtype=torch.float32, device="cuda")
        rpos = np.array([[pos0 + i] * 3 for i in range(m)], np.uint32)
        K.attention(_dev(torch, proj[:m]), stride, qbuf, dk, dv, _dev(torch, norms), out, partial, n_heads, n_kv, 64,
                    1e7, 1e-6, (11, 11, 10), ctx, m, pos0, rpos)
        res.append(out.cpu().numpy())
    assert np.array_equal(res[0][0], res[1][0])


def test_pick_first_index_and_gap(torch_cuda, K):
    torch = torch_cuda
    import snl

    r = np.random.default_rng(9)
    V = 248320
    lg = r.standard_normal((2, V)).astype(np.float32)
    lg[0, 1000] = lg[0, 200000] = 9.0  # tie: first index wins
    lg[1, 5] = 7.0
    lg[1, 6] = 6.5
    picks = torch.zeros((2, 4), dtype=torch.int32, device="cuda")
    K.pick_rows(_dev(torch, lg), V, 2, picks)
    p = picks.cpu().numpy()
    tok = p[:, 0].view(np.uint32)
    top = p[:, 1:3].view(np.float32)
    assert tok[0] == 1000 and top[0, 0] == 9.0 and top[0, 1] == 9.0
    assert tok[1] == 5 and top[1, 0] == np.float32(7.0) and top[1, 1] == np.float32(6.5)
    for _ in range(3):
        v = r.integers(0, 50, V).astype(np.float32)
        K.pick_rows(_dev(torch, v.reshape(1, V)), V, 1, picks)
        assert picks.cpu().numpy()[0, 0] == int(np.argmax(v))
