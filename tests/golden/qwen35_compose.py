"""The reference's decoder composition, restated over transformers' Qwen3.5 modules.

Test infrastructure.  Builds `Qwen3_5Attention`, `Qwen3_5GatedDeltaNet`, `Qwen3_5MLP` and
`Qwen3_5RMSNorm` modules (transformers 5.15.0, installed locally) from the oracle's
dequantised weights.  The weights are mapped back through the converter's fused layouts
(src/convert.rs:203-311): in_proj = in_proj_qkv | in_proj_z | in_proj_b | in_proj_a;
qkv = q_proj | k_proj | v_proj; gate_up = gate_proj | up_proj; lin = conv1d | A_log | dt_bias |
norm; qk_norm = q_norm | k_norm; mtp.fc_e / mtp.fc_h = the column halves of mtp.fc.

The modules are composed in the order of src/engine.rs:383-493 (execution plan, branch norms,
merges, final norm, LM head) and :495-570 (MTP head).  transformers has no module for the mHC
router and merge, so those two are restated here from src/shaders/layers.wgsl:75-162, or
replaced by closed-form coefficients when a test fixes the router (`coef_override`).

A whole token sequence runs in one call from empty caches, so the composition shares no state,
chunking or buffer logic with the oracle it checks.
"""
from __future__ import annotations

import numpy as np
import torch
from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
from transformers.models.qwen3_5.modeling_qwen3_5 import (Qwen3_5Attention, Qwen3_5GatedDeltaNet, Qwen3_5MLP,
                                                          Qwen3_5RMSNorm, Qwen3_5TextRotaryEmbedding)

K_EMBED, K_LM_HEAD, K_NORM = 1, 2, 3
K_IN_LN, K_POST_LN, K_QK_NORM, K_LIN, K_QKV, K_O_PROJ, K_IN_PROJ = 1, 2, 3, 4, 5, 6, 7
K_OUT_PROJ, K_GATE_UP, K_DOWN, K_MHC_ATTN, K_MHC_FFN = 8, 9, 10, 11, 12
K_FC_E, K_FC_H, K_NORM_E, K_NORM_H, K_MTP_NORM = 20, 21, 22, 23, 24
MTP_LAYER = 0xFFF

DT = torch.float64


def hf_config(cfg) -> Qwen3_5TextConfig:
    c = Qwen3_5TextConfig(
        vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.intermediate,
        num_hidden_layers=cfg.n_layers, num_attention_heads=cfg.n_heads, num_key_value_heads=cfg.n_kv_heads,
        head_dim=cfg.head_dim, linear_num_key_heads=cfg.lin_k_heads, linear_num_value_heads=cfg.lin_v_heads,
        linear_key_head_dim=cfg.lin_k_dim, linear_value_head_dim=cfg.lin_v_dim,
        linear_conv_kernel_dim=cfg.conv_kernel, rms_norm_eps=cfg.eps,
        layer_types=["full_attention" if f else "linear_attention" for f in cfg.full_attention],
        rope_parameters={"rope_type": "default", "rope_theta": float(cfg.rope_theta),
                         "partial_rotary_factor": cfg.rot_dim / cfg.head_dim,
                         "mrope_section": list(cfg.mrope_section)},
    )
    c._attn_implementation = "eager"
    return c


def _set(param, value):
    with torch.no_grad():
        param.copy_(torch.as_tensor(np.asarray(value), dtype=param.dtype).reshape(param.shape))


def causal_mask(t: int) -> torch.Tensor:
    m = torch.full((t, t), float("-inf"), dtype=DT).triu(1)
    return m[None, None]


def router_coef(x0: torch.Tensor, x1: torch.Tensor, w: np.ndarray, h: int, iterations: int) -> torch.Tensor:
    """mhc_dots + mhc_finish (src/shaders/layers.wgsl:75-126) in float64: [T, 8] coefficients
    pre0, pre1, post0, post1, mix00, mix01, mix10, mix11."""
    d = 2 * h
    wt = torch.as_tensor(w, dtype=DT)
    W, b = wt[: 8 * d].reshape(8, d), wt[8 * d: 8 * d + 8]
    xx = torch.cat([x0, x1], dim=-1)
    rinv = 1.0 / torch.sqrt((xx * xx).sum(-1) / d + 1e-6)
    lg = (xx @ W.T) * rinv[:, None] + b
    a, bb, c, e = lg[:, 4], lg[:, 5], lg[:, 6], lg[:, 7]
    for _ in range(iterations):
        r0 = torch.logaddexp(a, bb)
        r1 = torch.logaddexp(c, e)
        a, bb, c, e = a - r0, bb - r0, c - r1, e - r1
        c0 = torch.logaddexp(a, c)
        c1 = torch.logaddexp(bb, e)
        a, c, bb, e = a - c0, c - c0, bb - c1, e - c1
    return torch.stack([torch.sigmoid(lg[:, 0]), torch.sigmoid(lg[:, 1]), 2 * torch.sigmoid(lg[:, 2]),
                        2 * torch.sigmoid(lg[:, 3]), a.exp(), bb.exp(), c.exp(), e.exp()], dim=-1)


def merge(x0, x1, br, coef, mode):
    """src/shaders/layers.wgsl:128-162, modes 0-2."""
    if mode == 0:
        return x0 + br, x1
    n0 = coef[:, 4:5] * x0 + coef[:, 5:6] * x1 + coef[:, 2:3] * br
    n1 = coef[:, 6:7] * x0 + coef[:, 7:8] * x1 + coef[:, 3:4] * br
    if mode == 2:
        return 0.5 * (n0 + n1), x1
    return n0, n1


class F16Cache:
    """Stands in for a key/value cache: the reference stores the normed, rotated keys and the
    values as f16 (pack2x16float, src/shaders/attention.wgsl:59-127) and attends over those."""

    def update(self, k, v, layer_idx):
        return k.to(torch.float16).to(k.dtype), v.to(torch.float16).to(v.dtype)


class Composed:
    """Main model and MTP head of the oracle engine `o` (weights read back from it)."""

    def __init__(self, o, cfg, dequant, coef_override=None):
        self.cfg = cfg
        self.coef_override = coef_override or {}
        hc = hf_config(cfg)
        self.hc = hc
        h, inter = cfg.hidden, cfg.intermediate

        def mat(layer, kind):
            qt, q, s = o.tensor(layer, kind)
            return torch.as_tensor(dequant(q, s, qt, s.shape[1] * 32), dtype=DT)

        def vec(layer, kind):
            return o.tensor(layer, kind)[1]

        def rms(w):
            n = Qwen3_5RMSNorm(w.size, eps=cfg.eps).to(DT)
            _set(n.weight, w)
            return n

        self.embed = mat(-1, K_EMBED)
        self.lm_head = mat(-1, K_LM_HEAD)
        self.final_norm = rms(vec(-1, K_NORM))
        self.rot = Qwen3_5TextRotaryEmbedding(hc)
        self.layers = []
        q_dim, kv_dim = cfg.q_dim, cfg.kv_dim
        for l in range(cfg.n_layers):
            L = {"in_ln": rms(vec(l, K_IN_LN)), "post_ln": rms(vec(l, K_POST_LN))}
            if cfg.full_attention[l]:
                L["mixer"] = self._attention(hc, l, mat(l, K_QKV), mat(l, K_O_PROJ), vec(l, K_QK_NORM))
            else:
                dn = Qwen3_5GatedDeltaNet(hc, l).to(DT)
                ip = mat(l, K_IN_PROJ)
                cd, vd, nv = cfg.conv_dim, cfg.lin_value_dim, cfg.lin_v_heads
                _set(dn.in_proj_qkv.weight, ip[:cd])
                _set(dn.in_proj_z.weight, ip[cd:cd + vd])
                _set(dn.in_proj_b.weight, ip[cd + vd:cd + vd + nv])
                _set(dn.in_proj_a.weight, ip[cd + vd + nv:cd + vd + 2 * nv])
                lw = vec(l, K_LIN)
                _set(dn.conv1d.weight, lw[:4 * cd])
                _set(dn.A_log, lw[4 * cd:4 * cd + nv])
                _set(dn.dt_bias, lw[4 * cd + nv:4 * cd + 2 * nv])
                _set(dn.norm.weight, lw[4 * cd + 2 * nv:4 * cd + 2 * nv + cfg.lin_v_dim])
                _set(dn.out_proj.weight, mat(l, K_OUT_PROJ))
                L["mixer"] = dn
            L["mlp"] = self._mlp(hc, mat(l, K_GATE_UP), mat(l, K_DOWN), inter)
            if cfg.is_mhc(l):
                L["mhc_attn"] = vec(l, K_MHC_ATTN)
                L["mhc_ffn"] = vec(l, K_MHC_FFN)
            self.layers.append(L)
        if cfg.has_mtp:
            M = MTP_LAYER
            self.fc = torch.cat([mat(M, K_FC_E), mat(M, K_FC_H)], dim=1)  # mtp.fc [H, 2H]
            self.norm_e, self.norm_h, self.m_norm = rms(vec(M, K_NORM_E)), rms(vec(M, K_NORM_H)), rms(vec(M, K_MTP_NORM))
            self.m_in_ln, self.m_post_ln = rms(vec(M, K_IN_LN)), rms(vec(M, K_POST_LN))
            self.m_att = self._attention(hc, 0, mat(M, K_QKV), mat(M, K_O_PROJ), vec(M, K_QK_NORM))
            self.m_mlp = self._mlp(hc, mat(M, K_GATE_UP), mat(M, K_DOWN), inter)
        _ = (h, q_dim, kv_dim)

    def _attention(self, hc, l, qkv, o_proj, qk_norm):
        q_dim, kv_dim = self.cfg.q_dim, self.cfg.kv_dim
        a = Qwen3_5Attention(hc, l).to(DT)
        _set(a.q_proj.weight, qkv[:2 * q_dim])
        _set(a.k_proj.weight, qkv[2 * q_dim:2 * q_dim + kv_dim])
        _set(a.v_proj.weight, qkv[2 * q_dim + kv_dim:])
        _set(a.o_proj.weight, o_proj)
        hd = self.cfg.head_dim
        _set(a.q_norm.weight, qk_norm[:hd])
        _set(a.k_norm.weight, qk_norm[hd:2 * hd])
        return a

    def _mlp(self, hc, gate_up, down, inter):
        m = Qwen3_5MLP(hc, inter).to(DT)
        _set(m.gate_proj.weight, gate_up[:inter])
        _set(m.up_proj.weight, gate_up[inter:])
        _set(m.down_proj.weight, down)
        return m

    def _rope(self, positions):
        p = torch.as_tensor(positions, dtype=torch.long)
        x = torch.zeros(1, len(p), self.cfg.hidden, dtype=DT)
        return self.rot(x, p[None, None, :].expand(3, 1, len(p)))

    def _mix(self, module, xn, rope, mask):
        if isinstance(module, Qwen3_5Attention):
            out, _ = module(hidden_states=xn[None], position_embeddings=rope, attention_mask=mask,
                            past_key_values=F16Cache())
            return out[0]
        return module(hidden_states=xn[None])[0]

    def _site(self, x0, x1, li, which, t):
        key = (li, which)
        if key in self.coef_override:
            return torch.as_tensor(self.coef_override[key], dtype=DT)[None].expand(t, 8)
        return router_coef(x0, x1, self.layers[li]["mhc_" + which], self.cfg.hidden, self.cfg.mhc[3])

    @torch.no_grad()
    def forward(self, tokens):
        """Logits [T, V] and final-normed hidden rows [T, H] of the token sequence from position 0."""
        cfg = self.cfg
        t = len(tokens)
        x0 = self.embed[torch.as_tensor(tokens, dtype=torch.long)].clone()
        x1 = torch.zeros_like(x0)
        rope = self._rope(range(t))
        mask = causal_mask(t)
        mhc_start = cfg.mhc[0] if cfg.mhc else None
        mhc_end = cfg.mhc[1] if cfg.mhc else None
        for li in cfg.execution_plan():
            L = self.layers[li]
            mhc = cfg.is_mhc(li)
            if mhc and li == mhc_start:
                x1 = x0.clone()  # merge mode 3
            coef = None
            if mhc:
                coef = self._site(x0, x1, li, "attn", t)
                inp = coef[:, 0:1] * x0 + coef[:, 1:2] * x1
            else:
                inp = x0
            br = self._mix(L["mixer"], L["in_ln"](inp), rope, mask)
            x0, x1 = merge(x0, x1, br, coef, 1 if mhc else 0)
            if mhc:
                coef = self._site(x0, x1, li, "ffn", t)
                inp = coef[:, 0:1] * x0 + coef[:, 1:2] * x1
            else:
                inp = x0
            br = L["mlp"](L["post_ln"](inp)[None])[0]
            mode = 0 if not mhc else (2 if li + 1 == mhc_end else 1)
            x0, x1 = merge(x0, x1, br, coef, mode)
        hid = self.final_norm(x0)
        return hid @ self.lm_head.T, hid

    @torch.no_grad()
    def mtp(self, hid_rows, tokens, positions):
        """MTP head over the pairs (hid_rows[i], tokens[i]) at cache slots 0.. and rotary positions
        `positions` (src/engine.rs:549-570, :713-774); the draft logits of the last pair."""
        e = self.norm_e(self.embed[torch.as_tensor(tokens, dtype=torch.long)])
        x = torch.cat([e, self.norm_h(hid_rows)], dim=-1) @ self.fc.T
        rope = self._rope(positions)
        x = x + self._mix(self.m_att, self.m_in_ln(x), rope, causal_mask(len(tokens)))
        x = x + self.m_mlp(self.m_post_ln(x)[None])[0]
        return self.m_norm(x[-1]) @ self.lm_head.T
