"""Checkpoint loading (rs_mlx_weights_load, native/mlx_bridge.cpp:108-118) into
the engine and the device session.

A seeded synthetic engine's tensors are split into the MLX-named checkpoint
tensors (tests/ckpt.py) and written as safetensors files; loaded back, the
engine must assemble exactly the same fused tensors (bit-exact on every row
that comes from a named tensor, zero on padding rows) and, with the same tiled
weights, the device session must produce bit-identical logits for the target
and the MTP head. The shifted-norm rule (mlx_bridge.cpp:115, qwen_model.inc:
21-31, qwen_mtp.inc:30) is checked with norms stored as offsets from 1, which
restore exactly (w - 1 is exact in f32 for w in [0.5, 2]).
"""
import numpy as np
import pytest

import ckpt

pytestmark = pytest.mark.gpu

SEED = 29


@pytest.fixture(scope="module")
def world(bridge, tmp_path_factory):
    from hip_bridge.engine import Engine, tiny_config

    cfg = tiny_config(layers=2, interval=2, chunk=8, context=96)
    print("case: checkpoint tiny config (DeltaNet + attention) synthetic engine", flush=True)
    ref = Engine(cfg, 1, 96, 8, 8, seed=SEED, mtp=True)
    d = tmp_path_factory.mktemp("ckpt")
    files = {
        "target": d / "model.safetensors",
        "mtp": d / "mtp.safetensors",
        "shifted": d / "shifted.safetensors",
        "shifted_mtp_key": d / "shifted_mtp_key.safetensors",
    }
    ckpt.write_safetensors(files["target"], ckpt.split_target(cfg, ref.export), {"format": "mlx"})
    ckpt.write_safetensors(files["mtp"], ckpt.split_mtp(cfg, ref.export))
    ckpt.write_safetensors(files["shifted"], ckpt.split_target(cfg, ref.export, shift=True, raw_conv=True))
    ckpt.write_safetensors(files["shifted_mtp_key"], ckpt.split_target(cfg, ref.export, shift=True,
                                                                     with_mtp_key=True))
    yield cfg, ref, files
    ref.close()


def stores(files, *names):
    from hip_bridge.session import WeightStore

    out = []
    for n in names:
        s = WeightStore()
        s.load(files[n])
        out.append(s)
    return out


def assert_same_tensors(cfg, got, want, mtp=True, what=""):
    for tid in ckpt.all_tensor_ids(cfg, mtp):
        a, b = got.export(tid), want.export(tid)
        rows = ckpt.filled_rows(cfg, tid)
        if isinstance(a, tuple):
            for part, x, y in zip("wsb", a, b):
                n = x.shape[0] if rows is None else rows
                assert np.array_equal(x[:n], y[:n]), f"{what} tensor {tid} part {part}"
                assert not x[n:].any(), f"{what} tensor {tid} part {part}: padding rows not zero"
        else:
            assert np.array_equal(a, b), f"{what} vector {tid}"


def test_checkpoint_assembles_engine_tensors(world):
    from hip_bridge.engine import Engine

    cfg, ref, files = world
    target, side = stores(files, "target", "mtp")
    print("case: checkpoint engine from named tensors", flush=True)
    e = Engine(cfg, 1, 96, 8, 8, store=target, mtp_store=side)
    try:
        assert_same_tensors(cfg, e, ref, what="checkpoint")
    finally:
        e.close()


@pytest.mark.parametrize("name", ["shifted", "shifted_mtp_key"])
def test_shifted_norms_restore(world, name):
    from hip_bridge.engine import Engine

    cfg, ref, files = world
    (target,) = stores(files, name)
    print(f"case: shifted checkpoint ({name})", flush=True)
    e = Engine(cfg, 1, 96, 8, 8, store=target)
    try:
        assert_same_tensors(cfg, e, ref, mtp=False, what=name)
    finally:
        e.close()


def test_unshifted_offsets_are_not_restored(world, tmp_path):
    """Norms stored as offsets in a checkpoint with neither trigger stay offsets."""
    from hip_bridge.engine import Engine

    cfg, ref, files = world
    t = ckpt.split_target(cfg, ref.export, shift=True)
    ckpt.write_safetensors(tmp_path / "plain.safetensors", t)
    files = dict(files, plain=tmp_path / "plain.safetensors")
    (target,) = stores(files, "plain")
    e = Engine(cfg, 1, 96, 8, 8, store=target)
    try:
        got, want = e.export(ckpt.FINAL_NORM), ref.export(ckpt.FINAL_NORM)
        assert np.array_equal(got, (want - np.float32(1)).astype(np.float32))
    finally:
        e.close()


def test_checkpoint_session_matches_synthetic(world):
    from hip_bridge.session import DeviceSession, WeightStore

    cfg, _, files = world
    target, side = stores(files, "target", "mtp")
    syn, syn_side = WeightStore(SEED, 0), WeightStore(SEED, 1)
    print("case: device sessions over checkpoint and synthetic stores", flush=True)
    a, b = DeviceSession(target, cfg, slots=8), DeviceSession(syn, cfg, slots=8)
    try:
        a.mtp_attach(side)
        b.mtp_attach(syn_side)
        toks = np.random.default_rng(5).integers(0, cfg.vocab, 11).astype(np.uint32)
        ra, la = a.block(None, 0, toks[:8])
        rb, lb = b.block(None, 0, toks[:8])
        assert np.array_equal(la, lb), "prefill logits"
        sa, la2, _ = a.step(ra, 8, toks[8:11])
        sb, lb2, _ = b.step(rb, 8, toks[8:11])
        assert np.array_equal(la2, lb2), "step logits"
        ha, _ = a.hidden_block(None, 0, toks[:6])
        hb, _ = b.hidden_block(None, 0, toks[:6])
        da, ma = a.mtp_step(None, ha, 0, 0, toks[1:7])
        db, mb = b.mtp_step(None, hb, 0, 0, toks[1:7])
        assert np.array_equal(ma, mb), "MTP logits"
        for s, ids in ((a, (da,)), (b, (db,))):
            for i in ids:
                s.mtp_release(i)
        for s, ids in ((a, (ra, sa, ha)), (b, (rb, sb, hb))):
            for i in ids:
                s.release(i)
    finally:
        a.close()
        b.close()


def test_loader_rejections(world, tmp_path):
    from hip_bridge import HipBridgeError
    from hip_bridge.engine import Engine
    from hip_bridge.session import DeviceSession, WeightStore

    cfg, ref, files = world
    # a name already held (mlx_bridge.cpp:114): the second load stores nothing
    (target,) = stores(files, "target")
    with pytest.raises(HipBridgeError, match="duplicate native parameter"):
        target.load(files["target"])
    # a missing tensor names itself at engine creation
    t = ckpt.split_target(cfg, ref.export)
    del t[ckpt.MODEL + ".layers.1.self_attn.k_proj.scales"]
    ckpt.write_safetensors(tmp_path / "missing.safetensors", t)
    s = WeightStore()
    s.load(tmp_path / "missing.safetensors")
    with pytest.raises(HipBridgeError, match="missing tensor .*k_proj.scales"):
        Engine(cfg, 1, 96, 8, 8, store=s)
    # a tensor of the wrong shape
    t = ckpt.split_target(cfg, ref.export)
    name = ckpt.MODEL + ".layers.0.linear_attn.out_proj.weight"
    t[name] = ("U32", t[name][1][:-16])
    ckpt.write_safetensors(tmp_path / "shape.safetensors", t)
    s = WeightStore()
    s.load(tmp_path / "shape.safetensors")
    with pytest.raises(HipBridgeError, match="out_proj.weight is"):
        DeviceSession(s, cfg, slots=2)
    # a target store is not an MTP sidecar, and 8-bit modules are not run
    (target,) = stores(files, "target")
    sess = DeviceSession(target, cfg, slots=2)
    try:
        (other,) = stores(files, "target")
        with pytest.raises(HipBridgeError, match="not an MTP sidecar store"):
            sess.mtp_attach(other)
    finally:
        sess.close()
    # an override whose module tensors are not at the declared bits
    (q8,) = stores(files, "target")
    q8.quant(ckpt.MODEL + ".layers.0.mlp.gate", 64, 8)
    with pytest.raises(HipBridgeError, match="mlp.gate.weight is .*8-bit group 64 needs"):
        DeviceSession(q8, cfg, slots=2)
