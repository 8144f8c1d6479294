"""The reference's `.snl` weight file (src/weights.rs:1-121, src/convert.rs:316-427) on the CPU:
the Python restatement used by the GPU tests round-trips and follows the converter's layout rules,
and the engine's C++ reader rejects malformed files (header checks run before any device work)."""
import ctypes
import json
import os
import struct

import numpy as np
import pytest

import snl_format as F

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "sense-nova-server_amd", "libsnl.so")


def _tiny_file(path, cfg, max_position=1024, drop=None, quant="q8_0"):
    rng = np.random.default_rng(0)
    tensors = []
    for name, dtype, shape in [("embed", "q8_0", (cfg.vocab, cfg.hidden)), ("norm", "f32", (cfg.hidden,)),
                               ("l0.down", quant, (cfg.hidden, cfg.intermediate))]:
        if name == drop:
            continue
        r, c = F.rows_cols(shape)
        qb, sb = F.sizes(dtype, r, c)
        q = rng.integers(0, 256, qb, dtype=np.uint8)
        s = rng.standard_normal(sb // 4).astype(np.float32) if sb else None
        tensors.append((name, dtype, shape, q, s))
    F.write(path, "tiny", quant, F.config_dict(cfg, max_position), tensors)
    return tensors


def test_python_format_roundtrip(tmp_path):
    import snl

    cfg = snl.tiny_config()
    p = str(tmp_path / "m.snl")
    written = _tiny_file(p, cfg)
    header, got, data = F.read(p)
    assert data[:4] == b"SNLQ" and struct.unpack("<I", data[4:8])[0] == 1
    assert list(header["tensors"]) == sorted(header["tensors"])  # a BTreeMap in the reference
    assert header["config"]["hidden"] == cfg.hidden and header["config"]["max_position"] == 1024
    offs = []
    for name, dtype, shape, q, s in written:
        d, sh, gq, gs = got[name]
        assert d == dtype and sh == list(shape)
        assert np.array_equal(gq, q)
        assert (gs is None and s is None) or np.array_equal(gs, s)
        t = header["tensors"][name]
        assert t["offset"] % 256 == 0 and t["scales_offset"] % 256 == 0
        offs.append(t["offset"])
    assert offs == sorted(offs)  # regions in the order given
    n = struct.unpack("<Q", data[8:16])[0]
    assert min(offs) >= 16 + n and min(offs) % 256 == 0
    assert len(data) % 256 == 0


def _load(path, mtp=None):
    L = ctypes.CDLL(LIB)
    L.snl_engine_load.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)]
    L.snl_create_error.restype = ctypes.c_char_p
    h = ctypes.c_void_p()
    rc = L.snl_engine_load(path.encode(), mtp.encode() if mtp else None, 64, ctypes.byref(h))
    return rc, L.snl_create_error().decode()


@pytest.mark.parametrize("case", ["magic", "version", "truncated", "json", "no_config", "tensor_past_end",
                                  "bad_dtype", "config_field", "unsupported"])
def test_reader_rejects_malformed_files(tmp_path, case):
    import snl

    if not os.path.exists(LIB):
        pytest.skip("libsnl.so not built")
    cfg = snl.tiny_config()
    p = str(tmp_path / "m.snl")
    _tiny_file(p, cfg)
    data = bytearray(open(p, "rb").read())
    n = struct.unpack("<Q", data[8:16])[0]
    header = json.loads(data[16:16 + n])

    def put_header(h):
        b = json.dumps(h, separators=(",", ":")).encode()
        assert len(b) <= n + 4000
        data[8:16] = struct.pack("<Q", len(b))
        data[16:16 + len(b)] = b

    if case == "magic":
        data[0:4] = b"GGUF"
    elif case == "version":
        data[4:8] = struct.pack("<I", 2)
    elif case == "truncated":
        data[8:16] = struct.pack("<Q", len(data))
    elif case == "json":
        data[16] = ord("[")
    elif case == "no_config":
        del header["config"]
        put_header(header)
    elif case == "tensor_past_end":
        header["tensors"]["norm"]["offset"] = len(data)
        put_header(header)
    elif case == "bad_dtype":
        header["tensors"]["norm"]["dtype"] = "bf16"
        put_header(header)
    elif case == "config_field":
        del header["config"]["n_heads"]
        put_header(header)
    elif case == "unsupported":
        header["config"]["head_dim"] = 128
        put_header(header)
    open(p, "wb").write(data)
    rc, msg = _load(p)
    assert rc == 1, (rc, msg)  # SNL_EARG
    expect = {"magic": "not a SenseNova Loop weight file", "version": "version", "truncated": "past the end",
              "json": "malformed", "no_config": "header lacks", "tensor_past_end": "past the end",
              "bad_dtype": "unknown dtype", "config_field": "n_heads", "unsupported": "unsupported model"}[case]
    assert expect in msg, msg


def test_reader_reports_a_missing_file(tmp_path):
    if not os.path.exists(LIB):
        pytest.skip("libsnl.so not built")
    rc, msg = _load(str(tmp_path / "nope.snl"))
    assert rc == 1 and "opening" in msg
