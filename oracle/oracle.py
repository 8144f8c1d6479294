"""ctypes wrapper of the CPU oracle (liboracle.so, built from snl_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's CPU baseline, never by the shipped library.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

f32p = ctypes.POINTER(ctypes.c_float)
u32p = ctypes.POINTER(ctypes.c_uint32)
u16p = ctypes.POINTER(ctypes.c_uint16)
i32p = ctypes.POINTER(ctypes.c_int32)
vp = ctypes.c_void_p

# tensor kinds of the seeded initialiser (snl_oracle_engine.inc)
K_EMBED, K_LM_HEAD, K_NORM = 1, 2, 3
K_IN_LN, K_POST_LN, K_QK_NORM, K_LIN, K_QKV, K_O_PROJ, K_IN_PROJ = 1, 2, 3, 4, 5, 6, 7
K_OUT_PROJ, K_GATE_UP, K_DOWN, K_MHC_ATTN, K_MHC_FFN = 8, 9, 10, 11, 12
K_FC_E, K_FC_H, K_NORM_E, K_NORM_H, K_MTP_NORM = 20, 21, 22, 23, 24
MTP_LAYER = 0xFFF


class AttnP(ctypes.Structure):
    _fields_ = [("n_heads", ctypes.c_int), ("n_kv", ctypes.c_int), ("rot_dim", ctypes.c_int),
                ("proj_stride", ctypes.c_int), ("rope_theta", ctypes.c_float), ("eps", ctypes.c_float),
                ("scale", ctypes.c_float), ("mrope", ctypes.c_uint32)]


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run `make -C oracle` (or __graft_entry__.build())")
        L = ctypes.CDLL(path)
        L.orc_threads.restype = ctypes.c_int
        L.orc_stream_key.restype = ctypes.c_uint64
        L.orc_stream_key.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.orc_randn.restype = ctypes.c_float
        L.orc_randn.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.orc_randu.restype = ctypes.c_float
        L.orc_randu.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_quantize_q8.argtypes = [f32p, ctypes.c_int64, vp, f32p]
        L.orc_quantize_q4.argtypes = [f32p, ctypes.c_int64, vp, f32p]
        L.orc_dequant_q8_row.argtypes = [vp, f32p, ctypes.c_int64, f32p]
        L.orc_dequant_q4_row.argtypes = [vp, f32p, ctypes.c_int64, f32p]
        L.orc_gen_matrix.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.c_int64, ctypes.c_float, ctypes.c_int,
                                     vp, f32p]
        L.orc_gemv.argtypes = [ctypes.c_int, vp, f32p, f32p, f32p] + [ctypes.c_int] * 5
        L.orc_branch_norm.argtypes = [f32p, f32p, f32p, f32p] + [ctypes.c_int] * 5 + [ctypes.c_float,
                                                                                      ctypes.c_float, ctypes.c_int]
        L.orc_mhc_dots.argtypes = [f32p, f32p, f32p, ctypes.c_int, ctypes.c_int]
        L.orc_mhc_finish.argtypes = [f32p, f32p, f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.orc_merge.argtypes = [f32p, f32p, f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.orc_swiglu.argtypes = [f32p, f32p, ctypes.c_int, ctypes.c_int]
        L.orc_conv.argtypes = [f32p, ctypes.c_int, f32p, f32p, f32p, f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.orc_delta.argtypes = [f32p, ctypes.c_int, f32p, f32p, f32p, f32p, f32p, ctypes.c_int, ctypes.c_int,
                                ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_int]
        L.orc_attn_prep.argtypes = [ctypes.POINTER(AttnP), f32p, f32p, u16p, u16p, f32p, u32p, ctypes.c_int,
                                    ctypes.c_int]
        L.orc_attend.argtypes = [ctypes.POINTER(AttnP), f32p, f32p, u16p, u16p, f32p, f32p, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_int]
        L.orc_combine.argtypes = [ctypes.POINTER(AttnP), f32p, f32p, f32p, ctypes.c_int, ctypes.c_int]
        L.orc_argmax.restype = ctypes.c_uint32
        L.orc_argmax.argtypes = [f32p, ctypes.c_int64]
        L.orc_validate.argtypes = [vp]
        L.orc_execution_plan.argtypes = [vp, i32p]
        L.orc_engine_create.argtypes = [vp, ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.POINTER(vp)]
        L.orc_engine_destroy.argtypes = [vp]
        L.orc_forward.argtypes = [vp, u32p, ctypes.c_int, u32p, ctypes.c_int, ctypes.c_int, f32p]
        L.orc_mtp.argtypes = [vp, ctypes.c_int, u32p, ctypes.c_int, u32p, ctypes.c_int, ctypes.c_int, u32p, f32p]
        for n in ("orc_reset", "orc_rollback"):
            getattr(L, n).argtypes = [vp]
        L.orc_snapshot.argtypes = [vp, ctypes.c_int]
        L.orc_restore.argtypes = [vp, ctypes.c_int, ctypes.c_int]
        L.orc_pos.argtypes = [vp]
        L.orc_hid_rows.argtypes = [vp]
        L.orc_n_plan.argtypes = [vp]
        L.orc_engine_buf.restype = vp
        L.orc_engine_buf.argtypes = [vp, ctypes.c_int]
        L.orc_engine_tensor.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.POINTER(vp), ctypes.POINTER(f32p),
                                        i32p, i32p]
        L.orc_generate.argtypes = [vp, u32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, u32p, i32p, i32p, i32p, f32p,
                                   f32p]
        _LIB = L
    return _LIB


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def threads() -> int:
    return int(lib().orc_threads())


# ---------------------------------------------------------------- generator / quant
def stream_key(seed: int, stream: int) -> int:
    return lib().orc_stream_key(seed, stream)


def randn(key: int, i: int) -> float:
    return lib().orc_randn(key, i)


def randu(key: int, i: int) -> float:
    return lib().orc_randu(key, i)


def quantize(w: np.ndarray, quant: int):
    """Row-major [N, K] float matrix -> (quant bytes, f32 scales) with the reference quantizers."""
    w = f32(w)
    n = w.size
    if quant == 0:
        q = np.empty(n, np.int8)
        s = np.empty(n // 32, np.float32)
        lib().orc_quantize_q8(_p(w, f32p), n, q.ctypes.data, _p(s, f32p))
        return q.reshape(w.shape), s.reshape(w.shape[:-1] + (w.shape[-1] // 32,))
    q = np.empty(n // 2, np.uint8)
    s = np.empty(n // 32, np.float32)
    lib().orc_quantize_q4(_p(w, f32p), n, q.ctypes.data, _p(s, f32p))
    return q.reshape(w.shape[:-1] + (w.shape[-1] // 2,)), s.reshape(w.shape[:-1] + (w.shape[-1] // 32,))


def dequant(q: np.ndarray, s: np.ndarray, quant: int, k: int) -> np.ndarray:
    """Dequantize each row with the oracle (f32)."""
    rows = s.shape[0]
    out = np.empty((rows, k), np.float32)
    qc = np.ascontiguousarray(q)
    sc = f32(s)
    rb = k if quant == 0 else k // 2
    for r in range(rows):
        qr = qc.reshape(rows, rb)[r]
        sr = sc.reshape(rows, k // 32)[r]
        o = out[r]
        if quant == 0:
            lib().orc_dequant_q8_row(qr.ctypes.data, _p(sr, f32p), k, _p(o, f32p))
        else:
            lib().orc_dequant_q4_row(qr.ctypes.data, _p(sr, f32p), k, _p(o, f32p))
    return out


def gen_matrix(seed: int, stream: int, rows: int, cols: int, quant: int, std: float = 0.02):
    key = stream_key(seed, stream)
    q = np.empty(rows * cols if quant == 0 else rows * cols // 2, np.uint8)
    s = np.empty(rows * cols // 32, np.float32)
    lib().orc_gen_matrix(key, rows, cols, std, quant, q.ctypes.data, _p(s, f32p))
    return q, s


# ---------------------------------------------------------------- kernels
def gemv(quant: int, wq: np.ndarray, ws: np.ndarray, x: np.ndarray, n: int, k: int) -> np.ndarray:
    """y[m, n] = sum_k x[m, k] W[n, k] in the reference's summation order (matvec for M<=8, tiled beyond)."""
    x = f32(x).reshape(-1, k)
    m = x.shape[0]
    y = np.zeros((m, n), np.float32)
    wq = np.ascontiguousarray(wq)
    ws = f32(ws)
    lib().orc_gemv(quant, wq.ctypes.data, _p(ws, f32p), _p(x, f32p), _p(y, f32p), m, n, k, k, n)
    return y


def branch_norm(x, coef, w, h, count, step_m, mode, last_row=0, eps=1e-6, one=1.0, x_stride=0):
    x = f32(x)
    coef = f32(coef) if coef is not None else np.zeros(8 * max(step_m, 1), np.float32)
    w = f32(w)
    out = np.zeros((count, h), np.float32)
    lib().orc_branch_norm(_p(x, f32p), _p(coef, f32p), _p(w, f32p), _p(out, f32p), h, count, step_m, mode, last_row,
                          eps, one, x_stride)
    return out


def mhc(x, w, h, m, iterations):
    x = f32(x)
    w = f32(w)
    raw = np.zeros((m, 9), np.float32)
    coef = np.zeros((m, 8), np.float32)
    lib().orc_mhc_dots(_p(x, f32p), _p(w, f32p), _p(raw, f32p), h, m)
    lib().orc_mhc_finish(_p(raw, f32p), _p(w, f32p), _p(coef, f32p), h, m, iterations)
    return raw, coef


def merge(x, coef, br, h, m, mode):
    x = f32(x).copy()
    coef = f32(coef)
    br = f32(br)
    lib().orc_merge(_p(x, f32p), _p(coef, f32p), _p(br, f32p), h, m, mode)
    return x


def swiglu(proj, inter, m):
    proj = f32(proj)
    act = np.zeros((m, inter), np.float32)
    lib().orc_swiglu(_p(proj, f32p), _p(act, f32p), inter, m)
    return act


def conv(proj, proj_stride, conv_state, lw, conv_dim, m, ckpt):
    proj = f32(proj)
    st = f32(conv_state).copy()
    lw = f32(lw)
    out = np.zeros((m, conv_dim), np.float32)
    ck = np.zeros_like(st)
    lib().orc_conv(_p(proj, f32p), proj_stride, _p(out, f32p), _p(st, f32p), _p(lw, f32p), _p(ck, f32p), conv_dim, m,
                   ckpt)
    return out, st, ck


def delta(proj, proj_stride, conv_out, state, lw, conv_dim, n_k, n_v, eps, m, ckpt):
    proj = f32(proj)
    conv_out = f32(conv_out)
    st = f32(state).copy()
    lw = f32(lw)
    out = np.zeros((m, n_v * 128), np.float32)
    ck = np.zeros_like(st)
    lib().orc_delta(_p(proj, f32p), proj_stride, _p(conv_out, f32p), _p(st, f32p), _p(lw, f32p), _p(out, f32p),
                    _p(ck, f32p), conv_dim, n_k, n_v, eps, m, ckpt)
    return out, st, ck


def attn_params(n_heads, n_kv, rot_dim, proj_stride, rope_theta=1e7, eps=1e-6, mrope_section=(11, 11, 10)):
    return AttnP(n_heads, n_kv, rot_dim, proj_stride, rope_theta, eps, 1.0 / 16.0,
                 ((3 * mrope_section[1]) << 16) | (3 * mrope_section[2]))


def attn_prep(ap: AttnP, proj, kcache, vcache, norms, rpos, m, pos0):
    proj = f32(proj)
    qbuf = np.zeros((m, ap.n_heads * 256), np.float32)
    norms = f32(norms)
    rpos = np.ascontiguousarray(rpos, dtype=np.uint32)
    lib().orc_attn_prep(ctypes.byref(ap), _p(proj, f32p), _p(qbuf, f32p), _p(kcache, u16p), _p(vcache, u16p),
                        _p(norms, f32p), _p(rpos, u32p), m, pos0)
    return qbuf


def attend(ap: AttnP, proj, qbuf, kcache, vcache, m, pos0, parts):
    proj = f32(proj)
    qbuf = f32(qbuf)
    out = np.zeros((m, ap.n_heads * 256), np.float32)
    partial = np.zeros(max(1, m * ap.n_heads * parts * 258), np.float32)
    lib().orc_attend(ctypes.byref(ap), _p(proj, f32p), _p(qbuf, f32p), _p(kcache, u16p), _p(vcache, u16p),
                     _p(out, f32p), _p(partial, f32p), m, pos0, parts)
    if parts > 1:
        lib().orc_combine(ctypes.byref(ap), _p(proj, f32p), _p(partial, f32p), _p(out, f32p), m, parts)
    return out


def argmax(v) -> int:
    v = f32(v)
    return int(lib().orc_argmax(_p(v, f32p), v.size))


def f32_to_f16_bits(v: float) -> int:
    return int(lib().orc_f32_to_f16(v))


# ---------------------------------------------------------------- engine
class Engine:
    """The oracle engine: a CPU restatement of `Engine` (src/engine.rs) over seeded random weights."""

    def __init__(self, cfg, seed: int = 1, quant: int = 0, ctx: int = 512, max_m: int = 512):
        self.cfg = cfg
        self._cs = cfg.to_struct()
        h = vp()
        rc = lib().orc_engine_create(ctypes.byref(self._cs), seed, quant, ctx, max_m, ctypes.byref(h))
        if rc != 0:
            raise RuntimeError(f"orc_engine_create failed ({rc})")
        self.h = h
        self.vocab = cfg.vocab

    def close(self):
        if self.h:
            lib().orc_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def pos(self) -> int:
        return lib().orc_pos(self.h)

    @property
    def hid_rows(self) -> int:
        return lib().orc_hid_rows(self.h)

    def forward(self, tokens: Sequence[int], pos: Optional[Sequence[Sequence[int]]] = None, logit_rows: int = 1,
                ckpt: bool = False) -> Optional[np.ndarray]:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        p = None if pos is None else np.ascontiguousarray(pos, dtype=np.uint32).reshape(-1, 3)
        rows = min(logit_rows, len(t))
        out = np.zeros((max(rows, 1), self.vocab), np.float32)
        rc = lib().orc_forward(self.h, _p(t, u32p), len(t), None if p is None else _p(p, u32p), logit_rows, int(ckpt),
                               _p(out, f32p))
        if rc != 0:
            raise RuntimeError(f"orc_forward failed ({rc})")
        return out[:rows] if logit_rows > 0 else None

    def mtp(self, r0: int, tokens, pos, slot0: int, draft: bool):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        p = np.ascontiguousarray(pos, dtype=np.uint32).reshape(-1, 3)
        d = ctypes.c_uint32(0)
        lg = np.zeros(self.vocab, np.float32)
        rc = lib().orc_mtp(self.h, r0, _p(t, u32p), len(t), _p(p, u32p), slot0, int(draft), ctypes.byref(d),
                           _p(lg, f32p))
        if rc != 0:
            raise RuntimeError(f"orc_mtp failed ({rc})")
        return (int(d.value), lg) if draft else None

    def rollback(self):
        lib().orc_rollback(self.h)

    def reset(self):
        lib().orc_reset(self.h)

    def snapshot(self, slot: int):
        lib().orc_snapshot(self.h, slot)

    def restore(self, slot: int, pos: int):
        lib().orc_restore(self.h, slot, pos)

    def buf(self, bid: int, n: int, dtype=np.float32) -> np.ndarray:
        ptr = lib().orc_engine_buf(self.h, bid)
        return np.ctypeslib.as_array(ctypes.cast(ptr, ctypes.POINTER(np.ctypeslib.as_ctypes_type(dtype))),
                                     shape=(n,)).copy()

    def tensor(self, layer: int, kind: int):
        q = vp()
        s = f32p()
        rows = ctypes.c_int32()
        cols = ctypes.c_int32()
        qt = lib().orc_engine_tensor(self.h, layer, kind, ctypes.byref(q), ctypes.byref(s), ctypes.byref(rows),
                                     ctypes.byref(cols))
        if qt < 0:
            raise KeyError((layer, kind))
        r, c = rows.value, cols.value
        if qt == 2:
            return qt, np.ctypeslib.as_array(ctypes.cast(q, f32p), shape=(c,)).copy(), None
        nq = r * c if qt == 0 else r * c // 2
        qa = np.ctypeslib.as_array(ctypes.cast(q, ctypes.POINTER(ctypes.c_uint8)), shape=(nq,)).copy()
        sa = np.ctypeslib.as_array(s, shape=(r * c // 32,)).copy()
        return qt, qa.reshape(r, -1), sa.reshape(r, -1)

    def set_vector(self, layer: int, kind: int, values) -> None:
        """Overwrite an f32 parameter vector of the engine in place (tests that need chosen values,
        such as a zero mHC router with given biases)."""
        q = vp()
        s = f32p()
        rows = ctypes.c_int32()
        cols = ctypes.c_int32()
        qt = lib().orc_engine_tensor(self.h, layer, kind, ctypes.byref(q), ctypes.byref(s), ctypes.byref(rows),
                                     ctypes.byref(cols))
        if qt != 2:
            raise KeyError((layer, kind))
        v = f32(values).reshape(-1)
        if v.size != cols.value:
            raise ValueError(f"expected {cols.value} values, got {v.size}")
        ctypes.memmove(q.value, v.ctypes.data, v.nbytes)

    def zero_rows(self, layer: int, kind: int, first: int) -> None:
        """Set the block scales of rows first.. of a quantised matrix to zero, so those rows dequantise
        to exactly 0 (a head whose argmax is confined to the first rows)."""
        q = vp()
        s = f32p()
        rows = ctypes.c_int32()
        cols = ctypes.c_int32()
        qt = lib().orc_engine_tensor(self.h, layer, kind, ctypes.byref(q), ctypes.byref(s), ctypes.byref(rows),
                                     ctypes.byref(cols))
        if qt not in (0, 1):
            raise KeyError((layer, kind))
        nb = cols.value // 32
        sa = np.ctypeslib.as_array(s, shape=(rows.value * nb,))
        sa[first * nb:] = 0.0

    def generate(self, prompt: Sequence[int], max_tokens: int, spec: bool):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max_tokens, np.uint32)
        gaps = np.zeros(max_tokens, np.float32)
        dgaps = np.zeros(max_tokens, np.float32)
        n_out = ctypes.c_int32()
        dr = ctypes.c_int32()
        ac = ctypes.c_int32()
        rc = lib().orc_generate(self.h, _p(p, u32p), len(p), max_tokens, int(spec), _p(out, u32p), ctypes.byref(n_out),
                                ctypes.byref(dr), ctypes.byref(ac), _p(gaps, f32p), _p(dgaps, f32p))
        if rc != 0:
            raise RuntimeError(f"orc_generate failed ({rc})")
        n = n_out.value
        return dict(tokens=out[:n].tolist(), gaps=gaps[:n], drafted=dr.value, accepted=ac.value,
                    draft_gaps=dgaps[:dr.value])
