"""The `.snl` reader (csrc/snl_file.cpp: its JSON header parser, tensor table and config) on the
CPU, under the address and undefined-behaviour sanitizers: tests/snl_file_fuzz.cpp is built with
g++ and run over seeded mutations of a small valid file (bytes flipped, files cut short, header
lengths, JSON text edits, fields replaced by hostile values, deep nesting).  No input may trip a
sanitizer or leave an accepted tensor outside the file, and four inputs that earlier builds
accepted are rejected."""
import json
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

import snl_format as F

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "sense-nova-server_amd", "csrc")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("g++ not available")
    out = str(tmp_path_factory.mktemp("fuzz") / "snl_file_fuzz")
    cmd = [gxx, "-std=c++17", "-O1", "-g", *SAN, "-I", CSRC, os.path.join(REPO, "tests", "snl_file_fuzz.cpp"),
           os.path.join(CSRC, "snl_file.cpp"), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return out


def _run(driver, paths):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    res = {}
    for i0 in range(0, len(paths), 200):
        chunk = paths[i0:i0 + 200]
        r = subprocess.run([driver, *chunk], capture_output=True, text=True, env=env, timeout=300)
        assert "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
        assert r.returncode in (0, 1), (r.returncode, r.stderr[-4000:])
        for line in r.stdout.splitlines():
            k, rest = line.split(" ", 1)
            res[chunk[int(k) - 1]] = rest
    assert len(res) == len(paths)
    return res


def _base(tmp_path):
    """A small valid file: a tiny model's config and three small tensors, one of each dtype."""
    import snl

    rng = np.random.default_rng(0)
    tensors = []
    for name, dtype, shape in [("embed", "q8_0", (4, 64)), ("norm", "f32", (64,)), ("l0.down", "q4_0", (8, 64))]:
        r, c = F.rows_cols(shape)
        qb, sb = F.sizes(dtype, r, c)
        q = rng.integers(0, 256, qb, dtype=np.uint8)
        s = rng.standard_normal(sb // 4).astype(np.float32) if sb else None
        tensors.append((name, dtype, shape, q, s))
    p = str(tmp_path / "base.snl")
    F.write(p, "tiny", "q8_0", F.config_dict(snl.tiny_config(), 1024), tensors)
    data = bytearray(open(p, "rb").read())
    n = struct.unpack("<Q", data[8:16])[0]
    return data, json.loads(bytes(data[16:16 + n]))


def _with_header(data, text: bytes):
    d = bytearray(data)
    d[8:16] = struct.pack("<Q", len(text))
    d[16:16 + len(text)] = text
    return d


HOSTILE = [0, 1, 31, 33, 1 << 30, (1 << 30) + 1, 1 << 31, 1 << 32, (1 << 62), (1 << 64) - 1, (1 << 64) - 256,
           -1, -(1 << 63), 1.5, 1e300, "x", None, True, [], {}, [1, 2, 3], [[1]], [1 << 31, 1 << 31]]


def _mutate(rng, data, header):
    n = struct.unpack("<Q", data[8:16])[0]
    kind = int(rng.integers(0, 6))
    if kind == 0:  # bytes flipped in the preamble and header
        d = bytearray(data)
        for _ in range(int(rng.integers(1, 9))):
            d[int(rng.integers(0, 16 + n))] = int(rng.integers(0, 256))
        return d
    if kind == 1:  # cut short
        return bytearray(data[:int(rng.integers(0, len(data)))])
    if kind == 2:  # header length
        d = bytearray(data)
        lens = [0, 1, n - 1, n + 1, len(data), (1 << 64) - 1, int(rng.integers(0, 1 << 62))]
        d[8:16] = struct.pack("<Q", lens[int(rng.integers(0, len(lens)))])
        return d
    if kind == 3:  # JSON text edits
        t = bytearray(data[16:16 + n])
        alphabet = b'{}[]":,\\u0123456789abcdefgxyzEe+-. \x00\n'
        for _ in range(int(rng.integers(1, 6))):
            op, at = int(rng.integers(0, 3)), int(rng.integers(0, len(t) + 1))
            c = alphabet[int(rng.integers(0, len(alphabet)))]
            if op == 0 and at < len(t):
                del t[at]
            elif op == 1:
                t.insert(at, c)
            elif at < len(t):
                t[at] = c
        return _with_header(data, bytes(t))
    h = json.loads(json.dumps(header))
    if kind == 4:  # one field of a tensor entry or of the config replaced by a hostile value
        if rng.integers(0, 2):
            ent = h["tensors"][str(rng.choice(sorted(h["tensors"])))]
            ent[str(rng.choice(["dtype", "shape", "offset", "scales_offset"]))] = HOSTILE[int(rng.integers(0, len(HOSTILE)))]
        else:
            h["config"][str(rng.choice(sorted(h["config"])))] = HOSTILE[int(rng.integers(0, len(HOSTILE)))]
        return _with_header(data, json.dumps(h).encode())
    # deep nesting, long strings and escapes where a value is expected
    depth = int(rng.integers(1, 200))
    v = "[" * depth + "1" + "]" * depth if rng.integers(0, 2) else '"' + "\\u00e9\\\\\\n" * int(rng.integers(1, 500)) + '"'
    text = json.dumps(h).replace('"quant": "q8_0"', '"quant": ' + v)
    return _with_header(data, text.encode())


def test_reader_survives_mutated_files(tmp_path, driver):
    data, header = _base(tmp_path)
    rng = np.random.default_rng(20261202)
    paths = [str(tmp_path / "base.snl")]
    for i in range(1500):
        p = str(tmp_path / f"m{i}.snl")
        open(p, "wb").write(bytes(_mutate(rng, data, header)))
        paths.append(p)
    res = _run(driver, paths)
    assert res[paths[0]] == "ok", res[paths[0]]
    bad = [p for p, v in res.items() if v.startswith("bounds")]
    assert not bad, [(p, res[p]) for p in bad[:5]]
    rejected = sum(v.startswith("rejected") for v in res.values())
    assert 300 < rejected < len(paths)  # the mutations reach past the first checks


def test_reader_rejects_inputs_earlier_builds_accepted(tmp_path, driver):
    data, header = _base(tmp_path)
    n = struct.unpack("<Q", data[8:16])[0]
    text = bytes(data[16:16 + n])
    off = header["tensors"]["norm"]["offset"]
    cases = {}
    # a NUL byte inside a number was read as part of it (strchr finds the terminator)
    cases["nul"] = text.replace(b'"offset":%d' % off, b'"offset":%d\x00' % off, 1)
    # a \u escape with a non-hex digit that did not push the value past 0xFFFF
    cases["uhex"] = text.replace(b'"model_name":"tiny"', b'"model_name":"ti\\u00g0ny"', 1)
    # an f32 tensor of 2^31 x 2^31 elements: rows * cols * 4 wrapped to 0 bytes
    h = json.loads(text)
    h["tensors"]["norm"]["shape"] = [1 << 31, 1 << 31]
    cases["wrap"] = json.dumps(h).encode()
    # a float field that does not fit a float
    h = json.loads(text)
    h["config"]["rope_theta"] = 1e300
    cases["inf"] = json.dumps(h).encode()
    assert all(v != text for v in cases.values())
    paths = []
    for k, t in cases.items():
        p = str(tmp_path / f"{k}.snl")
        open(p, "wb").write(bytes(_with_header(data, t)))
        paths.append(p)
    res = _run(driver, paths)
    for k, p in zip(cases, paths):
        assert res[p].startswith("rejected"), (k, res[p])
