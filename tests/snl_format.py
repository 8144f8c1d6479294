"""Test helper: the reference's `.snl` weight file in Python (src/weights.rs:1-121 reader,
src/convert.rs:316-427 writer), used to check the engine's C++ reader and writer.

Layout: b"SNLQ", u32 version 1, u64 header length, the JSON header {model_name, quant, config,
tensors: {name: {dtype, shape, offset, scales_offset}}}, then every region 256-byte aligned, data
from align(16 + len(header with unshifted offsets) + 4096)."""
from __future__ import annotations

import json
import struct

import numpy as np

MAGIC = b"SNLQ"
VERSION = 1
ALIGN = 256


def align(x: int) -> int:
    return (x + ALIGN - 1) // ALIGN * ALIGN


def sizes(dtype: str, rows: int, cols: int):
    """DType::sizes (src/weights.rs:47-55): (quant bytes, scale bytes)."""
    n = rows * cols
    if dtype == "f32":
        return n * 4, 0
    if dtype == "q8_0":
        return n, n // 32 * 4
    if dtype == "q4_0":
        return n // 2, n // 32 * 4
    raise ValueError(dtype)


def rows_cols(shape):
    return (1, shape[0]) if len(shape) == 1 else (shape[0], shape[-1])


def config_dict(cfg, max_position: int) -> dict:
    """ModelConfig (src/config.rs:6-37) as the reference serialises it, fields in order."""
    return {
        "hidden": cfg.hidden, "intermediate": cfg.intermediate, "vocab": cfg.vocab, "n_layers": cfg.n_layers,
        "full_attention": [bool(f) for f in cfg.full_attention], "n_heads": cfg.n_heads,
        "n_kv_heads": cfg.n_kv_heads, "head_dim": cfg.head_dim, "rot_dim": cfg.rot_dim,
        "rope_theta": float(cfg.rope_theta), "mrope_section": list(cfg.mrope_section),
        "lin_k_heads": cfg.lin_k_heads, "lin_v_heads": cfg.lin_v_heads, "lin_k_dim": cfg.lin_k_dim,
        "lin_v_dim": cfg.lin_v_dim, "conv_kernel": cfg.conv_kernel, "eps": float(cfg.eps),
        "loop_start": cfg.loop_start, "loop_end": cfg.loop_end, "loop_count": cfg.loop_count,
        "mhc": None if cfg.mhc is None else dict(zip(("start", "end", "streams", "iterations"), cfg.mhc)),
        "eos": list(cfg.eos), "max_position": max_position, "vision": None,
    }


def write(path: str, model_name: str, quant: str, config: dict, tensors):
    """tensors: [(name, dtype, shape, quants bytes-like, scales float32 array or None)] in file order."""
    table, cursor = {}, 0
    for name, dtype, shape, _, _ in tensors:
        qb, sb = sizes(dtype, *rows_cols(shape))
        off = cursor
        cursor = align(cursor + qb)
        soff = cursor
        cursor = align(cursor + sb)
        table[name] = {"dtype": dtype, "shape": list(shape), "offset": off, "scales_offset": soff}
    header = {"model_name": model_name, "quant": quant, "config": config,
              "tensors": dict(sorted(table.items()))}
    probe = json.dumps(header, separators=(",", ":")).encode()
    start = align(16 + len(probe) + 4096)
    for t in table.values():
        t["offset"] += start
        t["scales_offset"] += start
    hdr = json.dumps(header, separators=(",", ":")).encode()
    assert 16 + len(hdr) <= start
    buf = bytearray(start + cursor)
    buf[0:16] = MAGIC + struct.pack("<IQ", VERSION, len(hdr))
    buf[16:16 + len(hdr)] = hdr
    for name, dtype, shape, q, s in tensors:
        t = table[name]
        qb = bytes(q)
        buf[t["offset"]:t["offset"] + len(qb)] = qb
        if s is not None:
            sb = np.asarray(s, np.float32).tobytes()
            buf[t["scales_offset"]:t["scales_offset"] + len(sb)] = sb
    with open(path, "wb") as f:
        f.write(buf)


def read(path: str):
    """(header dict, {name: (dtype, shape, quants uint8 array, scales float32 array or None)}, raw bytes)."""
    data = open(path, "rb").read()
    assert data[:4] == MAGIC, "magic"
    version, n = struct.unpack("<IQ", data[4:16])
    assert version == VERSION
    header = json.loads(data[16:16 + n])
    out = {}
    for name, t in header["tensors"].items():
        qb, sb = sizes(t["dtype"], *rows_cols(t["shape"]))
        q = np.frombuffer(data, np.uint8, qb, t["offset"])
        s = np.frombuffer(data, np.float32, sb // 4, t["scales_offset"]) if sb else None
        out[name] = (t["dtype"], t["shape"], q, s)
    return header, out, data


def tensor_kinds(cfg, mtp: bool, mtp_layer: int = 0xFFF):
    """(layer, kind, name) of each tensor of the main or MTP file in the converter's order
    (src/convert.rs:203-311); layer -1 for the globals, `mtp_layer` for the MTP head."""
    if mtp:
        ks = [(20, "fc_e"), (21, "fc_h"), (22, "norm_e"), (23, "norm_h"), (24, "norm"), (1, "in_ln"), (2, "post_ln"),
              (3, "qk_norm"), (5, "qkv"), (6, "o_proj"), (9, "gate_up"), (10, "down")]
        return [(mtp_layer, k, "mtp." + n) for k, n in ks]
    out = [(-1, 1, "embed"), (-1, 2, "lm_head"), (-1, 3, "norm")]
    for i in range(cfg.n_layers):
        out += [(i, 1, f"l{i}.in_ln"), (i, 2, f"l{i}.post_ln")]
        out += [(i, 3, f"l{i}.qk_norm")] if cfg.full_attention[i] else [(i, 4, f"l{i}.lin")]
        if cfg.is_mhc(i):
            out += [(i, 11, f"l{i}.mhc_attn"), (i, 12, f"l{i}.mhc_ffn")]
    for i in range(cfg.n_layers):
        if cfg.full_attention[i]:
            out += [(i, 5, f"l{i}.qkv"), (i, 6, f"l{i}.o_proj")]
        else:
            out += [(i, 7, f"l{i}.in_proj"), (i, 8, f"l{i}.out_proj")]
        out += [(i, 9, f"l{i}.gate_up"), (i, 10, f"l{i}.down")]
    return out


def write_engine_files(o, cfg, quant: int, main_path: str, mtp_path: str, max_position: int = 4096) -> None:
    """Write the weights of an oracle engine `o` as the converter's two files."""
    for is_mtp, path in ((False, main_path), (True, mtp_path)):
        tensors = []
        for layer, kind, name in tensor_kinds(cfg, is_mtp):
            ot, oq, os_ = o.tensor(layer, kind)
            if ot == 2:
                tensors.append((name, "f32", (oq.size,), oq.astype(np.float32).tobytes(), None))
            else:
                cols = oq.shape[1] * (1 if ot == 0 else 2)
                tensors.append((name, "q8_0" if ot == 0 else "q4_0", (oq.shape[0], cols), oq.tobytes(),
                                os_.reshape(-1)))
        write(path, "oracle", "q8_0" if is_mtp or quant == 0 else "q4_0", config_dict(cfg, max_position), tensors)
