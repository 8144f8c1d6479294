"""Writes the small golden fixtures of the decode-step tests (run from the repository root).

    python tests/golden/make_golden.py

The reference ships no test vectors for this path, so the fixtures come from three sources,
each stated in the fixture:

* quant_kat.npz: hand-chosen Q8_0 / Q4_0 blocks whose quantised bytes follow from the
  rules of src/weights.rs:123-153 by inspection (half-away-from-zero ties, clamps, the Q4
  sign convention), written out literally below, not computed by the oracle.
* gemv_small.npz: random Q8_0 / Q4_0 matrices and token rows with the product computed in
  float64 from the dequantised weights (numpy), independent of the oracle's summation.
* tiny_stream_q8.npz / tiny_stream_q4.npz: the tiny random-init model (seed 3) decoding a
  32-token prompt greedily for 24 tokens with MTP on and off, and the prompt's last-row logits,
  produced by the C oracle; they pin the oracle against regressions and give the GPU engine a
  fixed target (token ids exact except at oracle near-ties, logits within 1e-3 relative).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, os.path.join(REPO, "sense-nova-server_amd"))


def quant_kat():
    # Q8_0 block 0: amax 127 -> d = 1, id = 1: x.5 rounds away from zero, 127.4 clamps to 127
    b0 = np.zeros(32, np.float32)
    b0[:8] = [2.5, -2.5, 0.5, -0.5, 126.5, -126.5, 127.0, 1.49]
    q0 = np.zeros(32, np.int8)
    q0[:8] = [3, -3, 1, -1, 127, -127, 127, 1]
    # Q8_0 block 1: all zero -> d = 0, id = 0, every quant 0
    b1 = np.zeros(32, np.float32)
    q1 = np.zeros(32, np.int8)
    # Q8_0 block 2: amax 254 -> d = 2, id = 0.5: 5 -> 2.5 -> 3, -254 -> -127, 1 -> 0.5 -> 1
    b2 = np.zeros(32, np.float32)
    b2[:4] = [5.0, -254.0, 1.0, -1.0]
    q2 = np.zeros(32, np.int8)
    q2[:4] = [3, -127, 1, -1]
    q8_x = np.stack([b0, b1, b2])
    q8_q = np.stack([q0, q1, q2])
    q8_s = np.array([1.0, 0.0, 2.0], np.float32)

    # Q4_0: d = (signed value of largest magnitude) / -8, id = 1/d, nibble = clamp(trunc(v*id + 8.5), 0, 15)
    # block 0: max-magnitude value -8 -> d = 1: v = -8 -> 0, 7 -> 15, 0 -> 8, -0.5 -> trunc(8.0) = 8,
    #          0.49 -> trunc(8.99) = 8, 0.5 -> 9, -1.5 -> trunc(7.0) = 7
    c0 = np.zeros(32, np.float32)
    c0[:7] = [-8.0, 7.0, 0.0, -0.5, 0.49, 0.5, -1.5]
    n0 = np.full(32, 8, np.uint8)
    n0[:7] = [0, 15, 8, 8, 8, 9, 7]
    # block 1: max-magnitude value +8 -> d = -1: v = 8 -> trunc(0.5) = 0, -7 -> 15, 1 -> 7
    c1 = np.zeros(32, np.float32)
    c1[:3] = [8.0, -7.0, 1.0]
    n1 = np.full(32, 8, np.uint8)
    n1[:3] = [0, 15, 7]
    q4_x = np.stack([c0, c1])
    q4_n = np.stack([n0, n1])
    q4_s = np.array([1.0, -1.0], np.float32)
    # pack: element 8w + i is nibble i of little-endian word w
    q4_bytes = np.zeros((2, 16), np.uint8)
    for r in range(2):
        for e in range(32):
            w, i = divmod(e, 8)
            byte = 4 * w + i // 2
            q4_bytes[r, byte] |= q4_n[r, e] << (4 * (i % 2))
    np.savez(os.path.join(HERE, "quant_kat.npz"), q8_x=q8_x, q8_q=q8_q, q8_s=q8_s, q4_x=q4_x,
             q4_bytes=q4_bytes, q4_s=q4_s)


def gemv_small():
    import oracle as O

    rng = np.random.default_rng(2024)
    out = {}
    for quant in (0, 1):
        for (n, k) in ((64, 256), (48, 512)):
            w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
            q, s = O.quantize(w, quant)
            x = rng.standard_normal((2, k)).astype(np.float32)
            deq = O.dequant(q, s, quant, k).astype(np.float64)
            tag = f"q{quant}_{n}x{k}"
            out[tag + "_q"] = q
            out[tag + "_s"] = s
            out[tag + "_x"] = x
            out[tag + "_y64"] = x.astype(np.float64) @ deq.T
            out[tag + "_abs"] = np.abs(x.astype(np.float64)) @ np.abs(deq).T
    np.savez(os.path.join(HERE, "gemv_small.npz"), **out)


def tiny_streams():
    import oracle as O
    import snl.config as C

    cfg = C.tiny_config()
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, 32).astype(np.uint32)
    for quant in (0, 1):
        # 2-row passes, as the GPU engine prefills
        runs = []
        for what in ("logits", True, False):
            e = O.Engine(cfg, seed=3, quant=quant, ctx=256, max_m=2)
            runs.append(e.forward(prompt.tolist(), logit_rows=1)[0] if what == "logits"
                        else e.generate(prompt.tolist(), 24, what))
            e.close()
        lg, on, off = runs
        np.savez(os.path.join(HERE, f"tiny_stream_q{'8' if quant == 0 else '4'}.npz"), prompt=prompt,
                 logits=lg.astype(np.float32), seed=np.int64(3),
                 tokens_spec=np.array(on["tokens"], np.uint32), gaps_spec=on["gaps"].astype(np.float32),
                 drafted=np.int64(on["drafted"]), accepted=np.int64(on["accepted"]),
                 tokens_plain=np.array(off["tokens"], np.uint32), gaps_plain=off["gaps"].astype(np.float32))


if __name__ == "__main__":
    quant_kat()
    gemv_small()
    tiny_streams()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
