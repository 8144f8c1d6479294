"""Model hyper-parameters and the two synthetic model shapes.

Mirrors `ModelConfig` of the reference (src/config.rs:6-37), its `validate`
(src/config.rs:195-240), `execution_plan` (src/config.rs:243-250) and derived
dims (src/config.rs:256-278).  The C layout of `snl_config` lives in
include/snl.h; `to_struct` fills it.
"""
from __future__ import annotations

import ctypes
import dataclasses
from typing import List, Tuple

MAX_LAYERS = 64


class SnlConfig(ctypes.Structure):
    """ctypes mirror of `snl_config` (include/snl.h)."""

    _fields_ = [
        ("hidden", ctypes.c_int32),
        ("intermediate", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("n_layers", ctypes.c_int32),
        ("n_heads", ctypes.c_int32),
        ("n_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("rot_dim", ctypes.c_int32),
        ("rope_theta", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("mrope_section", ctypes.c_int32 * 3),
        ("lin_k_heads", ctypes.c_int32),
        ("lin_v_heads", ctypes.c_int32),
        ("lin_k_dim", ctypes.c_int32),
        ("lin_v_dim", ctypes.c_int32),
        ("conv_kernel", ctypes.c_int32),
        ("loop_start", ctypes.c_int32),
        ("loop_end", ctypes.c_int32),
        ("loop_count", ctypes.c_int32),
        ("mhc_start", ctypes.c_int32),
        ("mhc_end", ctypes.c_int32),
        ("mhc_streams", ctypes.c_int32),
        ("mhc_iterations", ctypes.c_int32),
        ("has_mtp", ctypes.c_int32),
        ("n_eos", ctypes.c_int32),
        ("eos", ctypes.c_uint32 * 4),
        ("full_attention", ctypes.c_uint8 * MAX_LAYERS),
    ]


@dataclasses.dataclass
class ModelConfig:
    hidden: int
    intermediate: int
    vocab: int
    n_layers: int
    full_attention: List[bool]
    n_heads: int
    n_kv_heads: int
    head_dim: int
    rot_dim: int
    rope_theta: float = 1e7
    mrope_section: Tuple[int, int, int] = (11, 11, 10)
    lin_k_heads: int = 16
    lin_v_heads: int = 32
    lin_k_dim: int = 128
    lin_v_dim: int = 128
    conv_kernel: int = 4
    eps: float = 1e-6
    loop_start: int = 0
    loop_end: int = 1
    loop_count: int = 1
    mhc: Tuple[int, int, int, int] | None = None  # (start, end, streams, iterations)
    has_mtp: bool = True
    eos: Tuple[int, ...] = ()

    # derived dims, src/config.rs:256-278
    @property
    def q_dim(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim

    @property
    def lin_key_dim(self) -> int:
        return self.lin_k_heads * self.lin_k_dim

    @property
    def lin_value_dim(self) -> int:
        return self.lin_v_heads * self.lin_v_dim

    @property
    def conv_dim(self) -> int:
        return 2 * self.lin_key_dim + self.lin_value_dim

    @property
    def lin_proj_rows(self) -> int:
        return self.conv_dim + self.lin_value_dim + 2 * self.lin_v_heads

    @property
    def attn_proj_rows(self) -> int:
        return 2 * self.q_dim + 2 * self.kv_dim

    def is_mhc(self, layer: int) -> bool:
        return self.mhc is not None and self.mhc[0] <= layer < self.mhc[1]

    def execution_plan(self) -> List[int]:
        """src/config.rs:243-250: prefix, looped block `loop_count` times, suffix."""
        plan = list(range(self.loop_start))
        for _ in range(self.loop_count):
            plan.extend(range(self.loop_start, self.loop_end))
        plan.extend(range(self.loop_end, self.n_layers))
        return plan

    def validate(self) -> None:
        """src/config.rs:195-240; raises ValueError like the reference's bail!."""
        checks = [
            (self.head_dim == 256, "head_dim must be 256"),
            (self.lin_k_dim == 128 and self.lin_v_dim == 128, "linear head dims must be 128"),
            (self.conv_kernel == 4, "linear conv kernel must be 4"),
            (self.hidden % 256 == 0, "hidden size must be a multiple of 256"),
            (len(self.full_attention) == self.n_layers, "layer_types length mismatch"),
            (self.n_heads == 4 * self.n_kv_heads, "attention must have 4 query heads per KV head"),
            (self.lin_v_heads % self.lin_k_heads == 0, "linear value heads must be a multiple of key heads"),
            (self.rot_dim % 2 == 0 and self.rot_dim <= self.head_dim, "invalid rotary dim"),
            (sum(self.mrope_section) == self.rot_dim // 2, "M-RoPE sections must cover the rotary dims"),
            (self.loop_start < self.loop_end <= self.n_layers and self.loop_count >= 1, "invalid loop range"),
            (self.n_layers <= MAX_LAYERS, "too many layers"),
        ]
        for ok, msg in checks:
            if not ok:
                raise ValueError(f"unsupported model configuration: {msg}")
        if self.mhc is not None:
            start, end, streams, _ = self.mhc
            if streams != 2:
                raise ValueError("unsupported model configuration: only 2 mHC streams are supported")

            def inside(a: int, b: int) -> bool:
                return a <= start and end <= b

            if not (inside(0, self.loop_start) or inside(self.loop_start, self.loop_end)
                    or inside(self.loop_end, self.n_layers)):
                raise ValueError("mHC range crosses a loop boundary")

    @staticmethod
    def from_struct(s: SnlConfig) -> "ModelConfig":
        """The inverse of to_struct (used for models loaded from a weight file)."""
        mhc = None
        if s.mhc_streams > 0:
            mhc = (s.mhc_start, s.mhc_end, s.mhc_streams, s.mhc_iterations)
        return ModelConfig(
            hidden=s.hidden, intermediate=s.intermediate, vocab=s.vocab, n_layers=s.n_layers,
            full_attention=[bool(s.full_attention[i]) for i in range(s.n_layers)],
            n_heads=s.n_heads, n_kv_heads=s.n_kv_heads, head_dim=s.head_dim, rot_dim=s.rot_dim,
            rope_theta=float(s.rope_theta), mrope_section=tuple(int(s.mrope_section[i]) for i in range(3)),
            lin_k_heads=s.lin_k_heads, lin_v_heads=s.lin_v_heads, lin_k_dim=s.lin_k_dim, lin_v_dim=s.lin_v_dim,
            conv_kernel=s.conv_kernel, eps=float(s.eps), loop_start=s.loop_start, loop_end=s.loop_end,
            loop_count=s.loop_count, mhc=mhc, has_mtp=bool(s.has_mtp),
            eos=tuple(int(s.eos[i]) for i in range(s.n_eos)))

    def to_struct(self) -> SnlConfig:
        s = SnlConfig()
        for f in ("hidden", "intermediate", "vocab", "n_layers", "n_heads", "n_kv_heads", "head_dim", "rot_dim",
                  "lin_k_heads", "lin_v_heads", "lin_k_dim", "lin_v_dim", "conv_kernel", "loop_start", "loop_end",
                  "loop_count"):
            setattr(s, f, int(getattr(self, f)))
        s.rope_theta = float(self.rope_theta)
        s.eps = float(self.eps)
        for i in range(3):
            s.mrope_section[i] = int(self.mrope_section[i])
        if self.mhc is not None:
            s.mhc_start, s.mhc_end, s.mhc_streams, s.mhc_iterations = (int(v) for v in self.mhc)
        s.has_mtp = int(bool(self.has_mtp))
        if len(self.eos) > 4:
            raise ValueError("at most 4 EOS ids")
        s.n_eos = len(self.eos)
        for i, t in enumerate(self.eos):
            s.eos[i] = int(t)
        for i, f in enumerate(self.full_attention):
            s.full_attention[i] = int(bool(f))
        return s


def tiny_config() -> ModelConfig:
    """Tiny SenseNova-Loop-style plumbing model: hidden 256, FFN 768, vocab 4096, 8 layers with
    full attention at i % 4 == 3, layers 2-5 looped twice, 2-stream mHC over the loop, 1 MTP layer."""
    return ModelConfig(
        hidden=256, intermediate=768, vocab=4096, n_layers=8,
        full_attention=[i % 4 == 3 for i in range(8)],
        n_heads=4, n_kv_heads=1, head_dim=256, rot_dim=64,
        lin_k_heads=2, lin_v_heads=4,
        loop_start=2, loop_end=6, loop_count=2,
        mhc=(2, 6, 2, 20), has_mtp=True,
    )


def nine_b_config() -> ModelConfig:
    """SenseNova-Loop-9B shape: hidden 4096, FFN 12288, vocab 248320, 32 layers (3 DeltaNet : 1 gated
    attention), layers 4-27 run twice, 16 q / 4 kv heads x 256 with 25% RoPE, DeltaNet 16 k / 32 v
    heads x 128, 2-stream mHC over the looped block, 1-layer MTP head."""
    return ModelConfig(
        hidden=4096, intermediate=12288, vocab=248320, n_layers=32,
        full_attention=[i % 4 == 3 for i in range(32)],
        n_heads=16, n_kv_heads=4, head_dim=256, rot_dim=64,
        lin_k_heads=16, lin_v_heads=32,
        loop_start=4, loop_end=28, loop_count=2,
        mhc=(4, 28, 2, 20), has_mtp=True,
    )
