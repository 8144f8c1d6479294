"""`.snl` weight files on the GPU engine (snl_engine_save / snl_engine_load, restating
src/convert.rs:316-427 and src/engine.rs:230-644) on the tiny model:

* the files the engine writes follow the converter's layout and hold exactly the weights the
  oracle draws (bit-exact), tensor by tensor;
* loading them back gives bitwise the same logits, drafts and decode stream;
* a file written independently in Python from the oracle's weights loads into an engine that
  matches the seeded one bitwise;
* a file that lacks a tensor is rejected with the reference's message."""
import numpy as np
import pytest

import snl_format as F

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def snl_mod():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import snl

    snl.lib()
    return snl


def _kinds(snl, cfg, mtp):
    """(layer, kind, name) of each tensor in the converter's order (src/convert.rs:203-311)."""
    return F.tensor_kinds(cfg, mtp, snl.engine.MTP_LAYER)


def _prompt(n, vocab, seed=1):
    return np.random.default_rng(seed).integers(0, vocab, n).tolist()


@pytest.fixture(scope="module", params=[0, 1], ids=["q8", "q4"])
def saved(request, snl_mod, oracle, tmp_path_factory):
    cfg = snl_mod.tiny_config()
    quant = request.param
    print(f"snl files quant={quant}", flush=True)
    g = snl_mod.Engine(cfg, seed=5, quant=quant, ctx=256)
    o = oracle.Engine(cfg, seed=5, quant=quant, ctx=256, max_m=g.prefill_chunk)
    d = tmp_path_factory.mktemp(f"snl{quant}")
    main, mtp = str(d / "model.snl"), str(d / "mtp.snl")
    g.save(main, mtp, model_name="tiny")
    yield cfg, quant, g, o, main, mtp
    g.close()
    o.close()


def test_saved_files_follow_the_converter_layout(snl_mod, saved):
    cfg, quant, g, o, main, mtp = saved
    for path, is_mtp in ((main, False), (mtp, True)):
        header, tensors, data = F.read(path)
        assert header["model_name"] == "tiny"
        assert header["quant"] == ("q8_0" if is_mtp or quant == 0 else "q4_0")
        assert header["config"] == F.config_dict(cfg, 262144)
        kinds = _kinds(snl_mod, cfg, is_mtp)
        assert sorted(tensors) == sorted(n for _, _, n in kinds)
        offs = [header["tensors"][n]["offset"] for _, _, n in kinds]
        assert offs == sorted(offs) and all(x % 256 == 0 for x in offs)
        for layer, kind, name in kinds:
            dtype, shape, q, s = tensors[name]
            ot, oq, os_ = o.tensor(layer, kind)
            if ot == 2:
                assert dtype == "f32" and shape == [oq.size], name
                assert np.array_equal(q.view(np.uint32), oq.view(np.uint32)), name
            else:
                assert dtype == ("q8_0" if ot == 0 else "q4_0"), name
                assert shape == [oq.shape[0], oq.shape[1] * (1 if ot == 0 else 2)], name
                assert np.array_equal(q, oq.reshape(-1)), name
                assert np.array_equal(s.view(np.uint32), os_.reshape(-1).view(np.uint32)), name


def test_loaded_engine_is_bitwise_the_saved_one(snl_mod, saved):
    cfg, quant, g, o, main, mtp = saved
    e = snl_mod.Engine.load(main, mtp, ctx=256)
    try:
        assert e.cfg.hidden == cfg.hidden and e.cfg.mhc == cfg.mhc and e.cfg.has_mtp
        for layer, kind, name in _kinds(snl_mod, cfg, False) + _kinds(snl_mod, cfg, True):
            a, b = g.tensor(layer, kind), e.tensor(layer, kind)
            assert a[0] == b[0], name
            assert np.array_equal(a[1].view(np.uint8), b[1].view(np.uint8)), name
            assert (a[2] is None) == (b[2] is None) and (a[2] is None or np.array_equal(a[2], b[2])), name
        prompt = _prompt(11, cfg.vocab, seed=9)
        pos = [[i] * 3 for i in range(len(prompt))]
        g.reset()
        e.reset()
        lg_g, _ = g.forward(prompt, pos, logit_rows=1)
        lg_e, _ = e.forward(prompt, pos, logit_rows=1)
        assert np.array_equal(lg_g.view(np.uint32), lg_e.view(np.uint32))
        g.reset()
        e.reset()
        sg = g.generate(prompt, 12, spec=True)
        se = e.generate(prompt, 12, spec=True)
        assert sg["tokens"] == se["tokens"] and sg["accepted"] == se["accepted"]
    finally:
        e.close()


def test_file_written_from_the_oracle_loads(snl_mod, saved, tmp_path):
    cfg, quant, g, o, main, mtp = saved
    paths = [str(tmp_path / "model.snl"), str(tmp_path / "mtp.snl")]
    F.write_engine_files(o, cfg, quant, paths[0], paths[1])
    e = snl_mod.Engine.load(paths[0], paths[1], ctx=256)
    try:
        prompt = _prompt(7, cfg.vocab, seed=2)
        pos = [[i] * 3 for i in range(len(prompt))]
        g.reset()
        e.reset()
        lg_g, _ = g.forward(prompt, pos, logit_rows=1)
        lg_e, _ = e.forward(prompt, pos, logit_rows=1)
        assert np.array_equal(lg_g.view(np.uint32), lg_e.view(np.uint32))
    finally:
        e.close()


def test_missing_tensor_is_rejected(snl_mod, saved, tmp_path):
    cfg, quant, g, o, main, mtp = saved
    header, tensors, _ = F.read(main)
    kinds = _kinds(snl_mod, cfg, False)
    drop = "l1.lin"
    items = []
    for _, _, name in kinds:
        if name == drop:
            continue
        dtype, shape, q, s = tensors[name]
        items.append((name, dtype, tuple(shape), q.tobytes(), s))
    p = str(tmp_path / "broken.snl")
    F.write(p, "broken", header["quant"], header["config"], items)
    with pytest.raises(snl_mod.SnlError) as ei:
        snl_mod.Engine.load(p, None, ctx=256)
    assert "missing tensor `l1.lin`" in str(ei.value)
