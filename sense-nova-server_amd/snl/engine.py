"""ctypes binding of libsnl.so: the engine API (src/engine.rs) and the kernel-level entry points."""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

from .config import ModelConfig, SnlConfig

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "libsnl.so")
_LIB = None

SNL_OK, SNL_EARG, SNL_ECTX, SNL_ETOKEN, SNL_EDEVICE, SNL_ENOMEM, SNL_ESTATE = range(7)
_NAMES = {1: "EARG", 2: "ECTX", 3: "ETOKEN", 4: "EDEVICE", 5: "ENOMEM", 6: "ESTATE"}

# tensor kinds of the seeded initialiser
K_EMBED, K_LM_HEAD, K_NORM = 1, 2, 3
K_IN_LN, K_POST_LN, K_QK_NORM, K_LIN, K_QKV, K_O_PROJ, K_IN_PROJ = 1, 2, 3, 4, 5, 6, 7
K_OUT_PROJ, K_GATE_UP, K_DOWN, K_MHC_ATTN, K_MHC_FFN = 8, 9, 10, 11, 12
K_FC_E, K_FC_H, K_NORM_E, K_NORM_H, K_MTP_NORM = 20, 21, 22, 23, 24
MTP_LAYER = 0xFFF

vp = ctypes.c_void_p
u32p = ctypes.POINTER(ctypes.c_uint32)
f32p = ctypes.POINTER(ctypes.c_float)
i32p = ctypes.POINTER(ctypes.c_int32)


class Pick(ctypes.Structure):
    _fields_ = [("token", ctypes.c_uint32), ("top1", ctypes.c_float), ("top2", ctypes.c_float),
                ("_pad", ctypes.c_uint32)]


class GenStats(ctypes.Structure):
    _fields_ = [("generated", ctypes.c_int32), ("drafted", ctypes.c_int32), ("accepted", ctypes.c_int32),
                ("_pad", ctypes.c_int32), ("prefill_s", ctypes.c_double), ("decode_s", ctypes.c_double),
                ("draft_s", ctypes.c_double), ("verify_s", ctypes.c_double)]


class Finish(ctypes.Structure):
    _fields_ = [("reason", ctypes.c_int32), ("prompt_tokens", ctypes.c_int32),
                ("completion_tokens", ctypes.c_int32), ("cached_tokens", ctypes.c_int32),
                ("drafted", ctypes.c_int32), ("accepted", ctypes.c_int32), ("prefill_s", ctypes.c_double),
                ("decode_s", ctypes.c_double)]


SNAPSHOTS = 4


class Sampling(ctypes.Structure):
    """SamplingParams (src/sampler.rs:4-29); the reference's defaults."""
    _fields_ = [("temperature", ctypes.c_float), ("top_p", ctypes.c_float), ("min_p", ctypes.c_float),
                ("presence_penalty", ctypes.c_float), ("frequency_penalty", ctypes.c_float),
                ("repetition_penalty", ctypes.c_float), ("top_k", ctypes.c_int32), ("_pad", ctypes.c_int32)]

    def __init__(self, temperature=1.0, top_p=0.95, top_k=20, min_p=0.0, presence_penalty=0.0,
                 frequency_penalty=0.0, repetition_penalty=1.0):
        super().__init__(temperature, top_p, min_p, presence_penalty, frequency_penalty, repetition_penalty, top_k, 0)


class Rng(ctypes.Structure):
    """The reference's StdRng (ChaCha12, seed_from_u64) inside the library."""
    _fields_ = [("key", ctypes.c_uint32 * 8), ("counter", ctypes.c_uint64), ("buf", ctypes.c_uint32 * 16),
                ("idx", ctypes.c_int32), ("_pad", ctypes.c_int32)]

    def __init__(self, seed: int):
        super().__init__()
        lib().snl_rng_seed(ctypes.byref(self), ctypes.c_uint64(seed))

    def u32(self) -> int:
        return int(lib().snl_rng_u32(ctypes.byref(self)))

    def f32(self) -> float:
        return float(lib().snl_rng_f32(ctypes.byref(self)))


class OpTime(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 24), ("bytes", ctypes.c_double), ("ms", ctypes.c_double)]


class SnlError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{_NAMES.get(code, code)}: {msg}")
        self.code = code


def lib() -> ctypes.CDLL:
    """Load libsnl.so (built by sense-nova-server_amd/build.py); raises if it was not built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with sense-nova-server_amd/build.py")
        L = ctypes.CDLL(LIB_PATH)
        L.snl_engine_create.argtypes = [ctypes.POINTER(SnlConfig), ctypes.c_uint64, ctypes.c_int, ctypes.c_int,
                                        ctypes.POINTER(vp)]
        L.snl_engine_load.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(vp)]
        L.snl_engine_save.argtypes = [vp, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p]
        L.snl_engine_config.argtypes = [vp, ctypes.POINTER(SnlConfig)]
        L.snl_engine_destroy.argtypes = [vp]
        L.snl_last_error.restype = ctypes.c_char_p
        L.snl_last_error.argtypes = [vp]
        L.snl_create_error.restype = ctypes.c_char_p
        L.snl_forward.argtypes = [vp, u32p, ctypes.c_int, u32p, ctypes.c_int, ctypes.c_int, f32p,
                                  ctypes.POINTER(Pick)]
        L.snl_mtp.argtypes = [vp, ctypes.c_int, u32p, ctypes.c_int, u32p, ctypes.c_int, ctypes.c_int, u32p,
                              ctypes.POINTER(Pick), f32p]
        L.snl_rollback.argtypes = [vp]
        L.snl_snapshot.argtypes = [vp, ctypes.c_int]
        L.snl_restore.argtypes = [vp, ctypes.c_int, ctypes.c_int]
        L.snl_reset.argtypes = [vp]
        for n in ("snl_pos", "snl_ctx", "snl_hid_rows", "snl_has_mtp", "snl_prefill_chunk"):
            getattr(L, n).argtypes = [vp]
        L.snl_generate.argtypes = [vp, u32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, u32p, f32p,
                                   ctypes.POINTER(GenStats)]
        L.snl_forward_profiled.argtypes = [vp, u32p, ctypes.c_int, u32p, ctypes.c_int, ctypes.c_int,
                                           ctypes.POINTER(OpTime), ctypes.c_int, i32p]
        L.snl_time_op.argtypes = [vp, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                  ctypes.POINTER(ctypes.c_double), i32p]
        L.snl_decoder_create.argtypes = [vp, u32p, ctypes.c_int, ctypes.c_int, ctypes.POINTER(vp)]
        L.snl_decoder_step.argtypes = [vp, u32p, f32p, i32p]
        L.snl_decoder_steps.argtypes = [vp, ctypes.c_int, u32p, f32p, i32p]
        L.snl_decoder_stats.argtypes = [vp, ctypes.POINTER(GenStats)]
        L.snl_decoder_destroy.argtypes = [vp]
        L.snl_worker_create.argtypes = [vp, ctypes.c_int, ctypes.POINTER(vp)]
        L.snl_worker_destroy.argtypes = [vp]
        L.snl_worker_run.argtypes = [vp, u32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, u32p, f32p,
                                     ctypes.POINTER(Finish)]
        L.snl_worker_cache.argtypes = [vp, i32p, i32p, ctypes.POINTER(ctypes.c_uint64)]
        L.snl_worker_run_sampled.argtypes = [vp, u32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             ctypes.POINTER(Sampling), ctypes.c_uint64, ctypes.c_int, u32p,
                                             ctypes.POINTER(Finish)]
        L.snl_chacha_block.argtypes = [u32p, ctypes.c_int, u32p]
        L.snl_chacha_block.restype = None
        L.snl_rng_seed.argtypes = [ctypes.POINTER(Rng), ctypes.c_uint64]
        L.snl_rng_seed.restype = None
        L.snl_rng_u32.argtypes = [ctypes.POINTER(Rng)]
        L.snl_rng_u32.restype = ctypes.c_uint32
        L.snl_rng_f32.argtypes = [ctypes.POINTER(Rng)]
        L.snl_rng_f32.restype = ctypes.c_float
        L.snl_draw.argtypes = [u32p, f32p, ctypes.c_int, ctypes.c_int64, ctypes.c_float]
        L.snl_draw.restype = ctypes.c_uint32
        L.snl_finish_distribution.argtypes = [f32p, ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_float, f32p]
        L.snl_sampler_create.argtypes = [vp, ctypes.POINTER(Sampling), ctypes.c_uint64, ctypes.c_int,
                                         ctypes.POINTER(vp)]
        L.snl_sampler_destroy.argtypes = [vp]
        L.snl_sampler_destroy.restype = None
        L.snl_sampler_accept.argtypes = [vp, ctypes.c_uint32]
        L.snl_sampler_accept.restype = None
        L.snl_sampler_sample.argtypes = [vp, ctypes.c_int, u32p]
        L.snl_sampler_verify.argtypes = [vp, ctypes.c_int, ctypes.c_uint32, i32p, u32p]
        L.snl_sampler_distribution.argtypes = [vp, ctypes.c_int, u32p, f32p, ctypes.c_int, i32p]
        L.snl_tensor_info.argtypes = [vp, ctypes.c_int, ctypes.c_int, i32p, i32p]
        L.snl_tensor_read.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, f32p]
        L.snl_tensor_zero_rows.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.snl_buffer_read.argtypes = [vp, ctypes.c_int, vp, ctypes.c_size_t]
        L.snl_buffer_size.restype = ctypes.c_size_t
        L.snl_buffer_size.argtypes = [vp, ctypes.c_int]
        L.snl_gemv.argtypes = [ctypes.c_int, vp, vp, vp, vp] + [ctypes.c_int] * 5 + [vp]
        L.snl_gemm.argtypes = [ctypes.c_int, vp, vp, vp, vp] + [ctypes.c_int] * 5 + [vp]
        L.snl_gemm_time.argtypes = [ctypes.c_int] * 5 + [ctypes.POINTER(ctypes.c_double)]
        L.snl_gemv_time.argtypes = [ctypes.c_int] * 5 + [ctypes.POINTER(ctypes.c_double)] * 2 + [i32p]
        L.snl_deltanet.argtypes = [vp, ctypes.c_int, vp, vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_float] + [ctypes.c_int] * 5 + [vp]
        L.snl_attention.argtypes = [vp, ctypes.c_int, vp, vp, vp, vp, vp, vp, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_float, ctypes.c_float, i32p, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, u32p, vp]
        L.snl_pick_rows.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, vp]
        L.snl_pick_rows_noalloc.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, vp]
        _LIB = L
    return _LIB


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint32)


def _ptr(a: np.ndarray, t):
    return a.ctypes.data_as(t)


class Engine:
    """Engine API of the reference (src/engine.rs) on one MI355X.  Weights are drawn on the device
    from `seed` (quant 0 = Q8_0, 1 = Q4_0), or read from the reference's `.snl` files with
    Engine.load."""

    def __init__(self, cfg: ModelConfig, seed: int = 1, quant: int = 0, ctx: int = 512):
        cfg.validate()
        self.cfg = cfg
        self._cs = cfg.to_struct()
        h = vp()
        rc = lib().snl_engine_create(ctypes.byref(self._cs), seed, quant, ctx, ctypes.byref(h))
        if rc != SNL_OK:
            raise SnlError(rc, lib().snl_create_error().decode())
        self.h = h
        self.vocab = cfg.vocab

    @classmethod
    def load(cls, path: str, mtp_path: str | None = None, ctx: int = 512) -> "Engine":
        """Engine::load (src/engine.rs:230) from a text-model `.snl` file and an optional MTP file."""
        h = vp()
        rc = lib().snl_engine_load(os.fsencode(path), os.fsencode(mtp_path) if mtp_path else None, ctx,
                                   ctypes.byref(h))
        if rc != SNL_OK:
            raise SnlError(rc, lib().snl_create_error().decode())
        self = cls.__new__(cls)
        self.h = h
        cs = SnlConfig()
        lib().snl_engine_config(h, ctypes.byref(cs))
        self._cs = cs
        self.cfg = ModelConfig.from_struct(cs)
        self.vocab = self.cfg.vocab
        return self

    def save(self, path: str, mtp_path: str | None = None, model_name: str = "") -> None:
        """Write the weights as the converter does (src/convert.rs:316-427)."""
        self._check(lib().snl_engine_save(self.h, os.fsencode(path), os.fsencode(mtp_path) if mtp_path else None,
                                          model_name.encode()))

    def close(self):
        if getattr(self, "h", None):
            lib().snl_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int):
        if rc != SNL_OK:
            raise SnlError(rc, lib().snl_last_error(self.h).decode())

    @property
    def pos(self) -> int:
        return lib().snl_pos(self.h)

    @property
    def ctx(self) -> int:
        return lib().snl_ctx(self.h)

    @property
    def hid_rows(self) -> int:
        return lib().snl_hid_rows(self.h)

    @property
    def prefill_chunk(self) -> int:
        return lib().snl_prefill_chunk(self.h)

    def has_mtp(self) -> bool:
        return bool(lib().snl_has_mtp(self.h))

    def forward(self, tokens: Sequence[int], pos: Optional[Sequence[Sequence[int]]] = None, logit_rows: int = 1,
                ckpt: bool = False, want_logits: bool = True):
        """Engine::forward_mm for text; returns (logits [rows, V] or None, picks list)."""
        t = _u32(tokens)
        p = None if pos is None else _u32(pos).reshape(-1, 3)
        rows = min(logit_rows, len(t))
        lg = np.zeros((max(rows, 1), self.vocab), np.float32) if (want_logits and rows > 0) else None
        picks = (Pick * 2)()
        rc = lib().snl_forward(self.h, _ptr(t, u32p), len(t), None if p is None else _ptr(p, u32p), logit_rows,
                               int(ckpt), None if lg is None else _ptr(lg, f32p), picks)
        self._check(rc)
        return (lg[:rows] if lg is not None else None), [picks[i] for i in range(rows)]

    def forward_profiled(self, tokens: Sequence[int], pos=None, logit_rows: int = 1, ckpt: bool = False):
        """One pass launched op by op with device timestamps: list of (name, bytes, ms)."""
        t = _u32(tokens)
        p = None if pos is None else _u32(pos).reshape(-1, 3)
        recs = (OpTime * 4096)()
        n = ctypes.c_int32()
        rc = lib().snl_forward_profiled(self.h, _ptr(t, u32p), len(t), None if p is None else _ptr(p, u32p),
                                        logit_rows, int(ckpt), recs, 4096, ctypes.byref(n))
        self._check(rc)
        return [(recs[i].name.decode(), recs[i].bytes, recs[i].ms) for i in range(n.value)]

    def time_op(self, name: str, reps: int = 4):
        """Launch only the `name` ops of a verify pass, `reps` passes back to back:
        (ms per launch, algorithmic bytes per launch, launches per pass)."""
        ms, b, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_int32()
        rc = lib().snl_time_op(self.h, name.encode(), reps, ctypes.byref(ms), ctypes.byref(b), ctypes.byref(n))
        self._check(rc)
        return ms.value, b.value, n.value

    def decoder(self, prompt: Sequence[int], spec: bool) -> "Decoder":
        return Decoder(self, prompt, spec)

    def mtp(self, r0: int, tokens, pos, slot0: int, draft: bool, want_logits: bool = False):
        t = _u32(tokens)
        p = _u32(pos).reshape(-1, 3)
        d = ctypes.c_uint32(0)
        pk = Pick()
        lg = np.zeros(self.vocab, np.float32) if want_logits else None
        rc = lib().snl_mtp(self.h, r0, _ptr(t, u32p), len(t), _ptr(p, u32p), slot0, int(draft), ctypes.byref(d),
                           ctypes.byref(pk), None if lg is None else _ptr(lg, f32p))
        self._check(rc)
        return (int(d.value), pk, lg) if draft else None

    def rollback(self):
        self._check(lib().snl_rollback(self.h))

    def snapshot(self, slot: int):
        self._check(lib().snl_snapshot(self.h, slot))

    def restore(self, slot: int, pos: int):
        self._check(lib().snl_restore(self.h, slot, pos))

    def reset(self):
        self._check(lib().snl_reset(self.h))

    def generate(self, prompt: Sequence[int], max_tokens: int, spec: bool):
        """Greedy decode (src/worker.rs:123-255) inside the library."""
        p = _u32(prompt)
        out = np.zeros(max_tokens, np.uint32)
        gaps = np.zeros(max_tokens, np.float32)
        st = GenStats()
        rc = lib().snl_generate(self.h, _ptr(p, u32p), len(p), max_tokens, int(spec), _ptr(out, u32p),
                                _ptr(gaps, f32p), ctypes.byref(st))
        self._check(rc)
        n = st.generated
        return dict(tokens=out[:n].tolist(), gaps=gaps[:n], drafted=st.drafted, accepted=st.accepted,
                    prefill_s=st.prefill_s, decode_s=st.decode_s, draft_s=st.draft_s, verify_s=st.verify_s)

    def tensor(self, layer: int, kind: int):
        rows = ctypes.c_int32()
        cols = ctypes.c_int32()
        qt = lib().snl_tensor_info(self.h, layer, kind, ctypes.byref(rows), ctypes.byref(cols))
        if qt < 0:
            raise KeyError((layer, kind))
        r, c = rows.value, cols.value
        if qt == 2:
            v = np.zeros(c, np.float32)
            self._check(lib().snl_tensor_read(self.h, layer, kind, v.ctypes.data, None))
            return qt, v, None
        q = np.zeros(r * c if qt == 0 else r * c // 2, np.uint8)
        s = np.zeros(r * c // 32, np.float32)
        self._check(lib().snl_tensor_read(self.h, layer, kind, q.ctypes.data, _ptr(s, f32p)))
        return qt, q.reshape(r, -1), s.reshape(r, -1)

    def zero_rows(self, layer: int, kind: int, first: int) -> None:
        """Zero the block scales of rows first.. of a quantised matrix (those rows dequantise to 0):
        a head whose argmax is confined to its first rows, as the oracle's zero_rows."""
        self._check(lib().snl_tensor_zero_rows(self.h, layer, kind, first))

    def buffer(self, bid: int) -> np.ndarray:
        n = lib().snl_buffer_size(self.h, bid)
        out = np.zeros(n // 4, np.float32)
        self._check(lib().snl_buffer_read(self.h, bid, out.ctypes.data, n))
        return out


class Decoder:
    """The greedy MTP loop of src/worker.rs:182-255 one speculative step at a time."""

    def __init__(self, engine: Engine, prompt: Sequence[int], spec: bool):
        self.engine = engine
        p = _u32(prompt)
        h = vp()
        engine._check(lib().snl_decoder_create(engine.h, _ptr(p, u32p), len(p), int(spec), ctypes.byref(h)))
        self.h = h
        self._out = np.zeros(2, np.uint32)
        self._gaps = np.zeros(2, np.float32)

    def step(self):
        """Emit the pending token and run one draft + verify; returns the emitted tokens (1 or 2)."""
        n = ctypes.c_int32()
        self.engine._check(lib().snl_decoder_step(self.h, _ptr(self._out, u32p), _ptr(self._gaps, f32p),
                                                  ctypes.byref(n)))
        return self._out[:n.value].tolist()

    def steps(self, k: int):
        """k steps in one native call (each queued on the device before the previous one is read);
        returns the emitted tokens."""
        out = np.zeros(2 * max(k, 1), np.uint32)
        n = ctypes.c_int32()
        self.engine._check(lib().snl_decoder_steps(self.h, int(k), _ptr(out, u32p), None, ctypes.byref(n)))
        return out[:n.value].tolist()

    def stats(self) -> dict:
        st = GenStats()
        lib().snl_decoder_stats(self.h, ctypes.byref(st))
        return {f: getattr(st, f) for f, _ in GenStats._fields_ if f != "_pad"}

    def close(self):
        if getattr(self, "h", None):
            lib().snl_decoder_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Worker:
    """The generation worker with its prefix cache (src/worker.rs:57-272) over one engine."""

    def __init__(self, engine: Engine, self_pause: bool = True):
        self.engine = engine
        h = vp()
        engine._check(lib().snl_worker_create(engine.h, int(self_pause), ctypes.byref(h)))
        self.h = h

    def run(self, prompt: Sequence[int], max_tokens: int, snapshot_at: Optional[int] = None, spec: bool = True):
        """One request (Worker::run, greedy); returns the tokens, their top-2 margins and the Finish fields."""
        p = _u32(prompt)
        cap = max(1, max_tokens)
        out = np.zeros(cap, np.uint32)
        gaps = np.zeros(cap, np.float32)
        fin = Finish()
        rc = lib().snl_worker_run(self.h, _ptr(p, u32p), len(p), -1 if snapshot_at is None else snapshot_at,
                                  max_tokens, int(spec), _ptr(out, u32p), _ptr(gaps, f32p), ctypes.byref(fin))
        self.engine._check(rc)
        n = fin.completion_tokens
        res = {f: getattr(fin, f) for f, _ in Finish._fields_}
        res["reason"] = "stop" if fin.reason == 1 else "length"
        res.update(tokens=out[:n].tolist(), gaps=gaps[:n])
        return res

    def run_sampled(self, prompt: Sequence[int], max_tokens: int, params: "Sampling", seed: Optional[int] = None,
                    snapshot_at: Optional[int] = None, spec: bool = True):
        """One request with SamplingParams (Worker::run with a Sampler); returns tokens and Finish fields."""
        p = _u32(prompt)
        out = np.zeros(max(1, max_tokens), np.uint32)
        fin = Finish()
        rc = lib().snl_worker_run_sampled(self.h, _ptr(p, u32p), len(p), -1 if snapshot_at is None else snapshot_at,
                                          max_tokens, int(spec), ctypes.byref(params),
                                          ctypes.c_uint64(seed or 0), int(seed is not None), _ptr(out, u32p),
                                          ctypes.byref(fin))
        self.engine._check(rc)
        res = {f: getattr(fin, f) for f, _ in Finish._fields_}
        res["reason"] = "stop" if fin.reason == 1 else "length"
        res["tokens"] = out[:fin.completion_tokens].tolist()
        return res

    def cache(self):
        """(live length, per-slot key counts with -1 for empty, per-slot last use)."""
        live = ctypes.c_int32()
        lens = (ctypes.c_int32 * SNAPSHOTS)()
        used = (ctypes.c_uint64 * SNAPSHOTS)()
        self.engine._check(lib().snl_worker_cache(self.h, ctypes.byref(live), lens, used))
        return live.value, list(lens), list(used)

    def close(self):
        if getattr(self, "h", None):
            lib().snl_worker_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Sampler:
    """Sampler (src/sampler.rs:32-96) over the engine's logits rows of its last forward."""

    def __init__(self, engine: "Engine", params: "Sampling", seed: Optional[int] = None):
        self.engine = engine
        h = vp()
        engine._check(lib().snl_sampler_create(engine.h, ctypes.byref(params), ctypes.c_uint64(seed or 0),
                                               int(seed is not None), ctypes.byref(h)))
        self.h = h

    def accept(self, token: int):
        lib().snl_sampler_accept(self.h, token)

    def sample(self, row: int = 0) -> int:
        t = ctypes.c_uint32()
        self.engine._check(lib().snl_sampler_sample(self.h, row, ctypes.byref(t)))
        return int(t.value)

    def verify(self, row: int, draft: int):
        ok = ctypes.c_int32()
        t = ctypes.c_uint32()
        self.engine._check(lib().snl_sampler_verify(self.h, row, draft, ctypes.byref(ok), ctypes.byref(t)))
        return bool(ok.value), int(t.value)

    def distribution(self, row: int = 0, cap: int = 1 << 18):
        toks = np.zeros(cap, np.uint32)
        probs = np.zeros(cap, np.float32)
        n = ctypes.c_int32()
        self.engine._check(lib().snl_sampler_distribution(self.h, row, _ptr(toks, u32p), _ptr(probs, f32p), cap,
                                                          ctypes.byref(n)))
        return toks[:n.value], probs[:n.value]

    def close(self):
        if getattr(self, "h", None):
            lib().snl_sampler_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class kernels:
    """Kernel-level entry points over torch device tensors (tests and microbenchmarks)."""

    @staticmethod
    def _stream():
        import torch

        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    @staticmethod
    def gemv(quant: int, wq, ws, x, y, M: int, N: int, K: int, x_stride: int, y_stride: int):
        rc = lib().snl_gemv(quant, wq.data_ptr(), ws.data_ptr(), x.data_ptr(), y.data_ptr(), M, N, K, x_stride,
                            y_stride, kernels._stream())
        if rc != SNL_OK:
            raise SnlError(rc, "snl_gemv")

    @staticmethod
    def gemm(quant: int, wq, ws, x, y, M: int, N: int, K: int, x_stride: int, y_stride: int):
        """The prefill GEMM (M up to 512 rows) over reference-layout weights."""
        rc = lib().snl_gemm(quant, wq.data_ptr(), ws.data_ptr(), x.data_ptr(), y.data_ptr(), M, N, K, x_stride,
                            y_stride, kernels._stream())
        if rc != SNL_OK:
            raise SnlError(rc, "snl_gemm")

    @staticmethod
    def gemv_time(quant: int, N: int, K: int, M: int, reps: int = 40):
        """(ms per launch, algorithmic bytes per launch, distinct weight copies) of the decode GEMV
        alone, weights rotated over at least 1 GB."""
        ms = ctypes.c_double()
        b = ctypes.c_double()
        c = ctypes.c_int32()
        rc = lib().snl_gemv_time(quant, N, K, M, reps, ctypes.byref(ms), ctypes.byref(b), ctypes.byref(c))
        if rc != SNL_OK:
            raise SnlError(rc, "snl_gemv_time")
        return ms.value, b.value, c.value

    @staticmethod
    def gemm_time(quant: int, N: int, K: int, M: int, reps: int = 20) -> float:
        """Mean ms per launch of the prefill GEMM alone (seeded weights, random rows)."""
        ms = ctypes.c_double()
        rc = lib().snl_gemm_time(quant, N, K, M, reps, ctypes.byref(ms))
        if rc != SNL_OK:
            raise SnlError(rc, "snl_gemm_time")
        return ms.value

    @staticmethod
    def deltanet(proj, proj_stride, lw, conv_state, state, out, conv_dim, n_k, n_v, eps, M, ckpt, s_in, s_out,
                 s_ck):
        rc = lib().snl_deltanet(proj.data_ptr(), proj_stride, lw.data_ptr(), conv_state.data_ptr(), state.data_ptr(),
                                out.data_ptr(), conv_dim, n_k, n_v, eps, M, ckpt, s_in, s_out, s_ck,
                                kernels._stream())
        if rc != SNL_OK:
            raise SnlError(rc, "snl_deltanet")

    @staticmethod
    def attention(proj, proj_stride, qbuf, kcache, vcache, norms, out, partial, n_heads, n_kv, rot_dim, rope_theta,
                  eps, mrope_section, ctx, M, pos0, rpos):
        ms = np.ascontiguousarray(mrope_section, dtype=np.int32)
        rp = _u32(rpos).reshape(-1, 3)
        rc = lib().snl_attention(proj.data_ptr(), proj_stride, qbuf.data_ptr(), kcache.data_ptr(), vcache.data_ptr(),
                                 norms.data_ptr(), out.data_ptr(), partial.data_ptr(), n_heads, n_kv, rot_dim,
                                 rope_theta, eps, _ptr(ms, i32p), ctx, M, pos0, _ptr(rp, u32p), kernels._stream())
        if rc != SNL_OK:
            raise SnlError(rc, "snl_attention")

    @staticmethod
    def pick_rows(logits, V: int, rows: int, picks):
        rc = lib().snl_pick_rows(logits.data_ptr(), V, rows, picks.data_ptr(), kernels._stream())
        if rc != SNL_OK:
            raise SnlError(rc, "snl_pick_rows")

    @staticmethod
    def pick_rows_noalloc(logits, V: int, rows: int, picks):
        """snl_pick_rows_noalloc: enqueued on torch's current stream, no device allocation."""
        rc = lib().snl_pick_rows_noalloc(logits.data_ptr(), V, rows, picks.data_ptr(), kernels._stream())
        if rc != SNL_OK:
            raise SnlError(rc, "snl_pick_rows_noalloc")
