"""Per-module quantization overrides (rs_qwen_quant, native/qwen_model.inc:16
and 273-276) and the MTP sidecar's dense BF16 fc (native/qwen_model.inc:34,
src/serving/native_mtp.rs:121-123) through checkpoint stores.

A seeded synthetic engine's tensors are split into MLX-named checkpoint
tensors (tests/ckpt.py); a set of modules spread over every kind of matrix
slot (embedding, DeltaNet in-projection, router and shared-expert gate,
attention out-projection, routed and shared expert matrices, lm_head, the MTP
layer's router) is replaced by fresh random modules at other (group, bits),
and the sidecar's fc by a dense BF16 matrix. The engine built from those stores
runs such slots from the checkpoint tensors in place; every layer is checked
teacher-forced against the oracle model with the same per-module quantization
(layer_check.py: mixer, then MoE, near-tie routing judged against the swapped
experts), then the final norm and lm_head, and the MTP head over the dense fc.
A device session over the same stores must give the engine's logits bit for
bit, and a synthetic store refuses overrides.
"""
import numpy as np
import pytest

import ckpt
import oracle
from layer_check import Row, check_layer, check_layers
from numerics import assert_bf16_close
from oracle import bf16_round, from_bf16_bits, to_bf16_bits
from oracle.model import LM_HEAD, MTP_FC, MTP_NORM, HybridModel, layer_tensor

SEED = 37
TIE = 2e-3
M = ckpt.MODEL

# module -> (group, bits), all different from the default 64/4
OVERRIDES = {
    M + ".embed_tokens": (32, 8),
    M + ".layers.0.linear_attn.in_proj_z": (128, 6),
    M + ".layers.0.mlp.gate": (64, 8),
    M + ".layers.0.mlp.shared_expert_gate": (64, 8),
    M + ".layers.1.self_attn.o_proj": (32, 3),
    M + ".layers.1.mlp.switch_mlp.gate_proj": (64, 5),
    M + ".layers.1.mlp.switch_mlp.down_proj": (32, 2),
    M + ".layers.1.mlp.shared_expert.up_proj": (128, 8),
    "language_model.lm_head": (64, 6),
}
MTP_OVERRIDES = {ckpt.MTP + ".layers.0.mlp.gate": (32, 8)}


def pack_codes(codes, bits):
    """Codes [..., K] (< 2^bits) as the MLX bit stream: code k at bit k * bits of
    its row, LSB first, in little-endian u32 words."""
    *lead, K = codes.shape
    b = ((codes[..., None].astype(np.uint64) >> np.arange(bits, dtype=np.uint64)) & 1).astype(np.uint8)
    b = b.reshape(*lead, K * bits)
    return np.packbits(b, axis=-1, bitorder="little").view(np.uint32).reshape(*lead, K * bits // 32)


def random_module(rng, shape, K, group, bits, std=0.02):
    """(codes u32, scales bf16 bits, biases bf16 bits) of a random affine module
    of rows `shape` x K whose weights spread like the synthetic ones."""
    codes = rng.integers(0, 1 << bits, (*shape, K)).astype(np.uint32)
    G = K // group
    s = rng.uniform(0.5, 1.5, (*shape, G)) * std * np.sqrt(12.0) / (1 << bits)
    b = -s * (1 << (bits - 1)) * rng.uniform(0.9, 1.1, (*shape, G))
    return pack_codes(codes, bits), to_bf16_bits(s.astype(np.float32)), to_bf16_bits(b.astype(np.float32))


def test_packing_matches_the_oracle_dequantization():
    """pack_codes against oracle.dequant (orc_dequant): every bits x group."""
    rng = np.random.default_rng(3)
    for bits in (2, 3, 4, 5, 6, 8):
        for group in (32, 64, 128):
            K = 256
            codes = rng.integers(0, 1 << bits, (5, K)).astype(np.uint32)
            s = rng.uniform(0.1, 1, (5, K // group)).astype(np.float32)
            b = rng.uniform(-1, 1, (5, K // group)).astype(np.float32)
            got = oracle.dequant(pack_codes(codes, bits), s, b, K, group, bits)
            want = np.repeat(s, group, 1).astype(np.float64) * codes + np.repeat(b, group, 1)
            assert np.allclose(got, want, rtol=0, atol=1e-6), (bits, group)


class QG:
    """One checkpoint module at its own (group, bits)."""

    def __init__(self, w, s, b, group, bits):
        self.w, self.s, self.b, self.group, self.bits = w, from_bf16_bits(s), from_bf16_bits(b), group, bits

    def __call__(self, x):
        return oracle.qmm(np.asarray(x, np.float32), self.w, self.s, self.b, self.group, self.bits)


class Parts:
    """A fused engine matrix as its modules, each into its own output columns."""

    def __init__(self, parts, N):
        self.parts, self.N = parts, N
        self.w = np.empty((N, 0))  # rows as the oracle's head reads them

    def __call__(self, x):
        y = np.zeros((len(x), self.N))
        for col, q in self.parts:
            y[:, col:col + q.w.shape[0]] = q(x)
        return y


class Dense:
    """A dense BF16 matrix [N][K]: y = x . W^T in FP64."""

    def __init__(self, wbits):
        self.W = from_bf16_bits(wbits).astype(np.float64)
        self.w = self.W

    def __call__(self, x):
        return np.asarray(x, np.float64) @ self.W.T


class NamedModel(HybridModel):
    """The oracle model over named checkpoint tensors with per-module
    quantization: overridden slots become Parts, expert matrices at other
    (group, bits) go through gather_qmm per module."""

    def __init__(self, cfg, engine_export, named, quant):
        super().__init__(cfg.dims(), engine_export)
        self.named, self.quant, self.gen_experts = named, quant, {}
        d = self.d
        H, E, I, V = d["hidden"], d["experts"], d["intermediate"], d["vocab"]

        def mod(name):
            g, b = quant.get(name, (64, 4))
            return QG(named[name + ".weight"][1], named[name + ".scales"][1], named[name + ".biases"][1], g, b)

        def slot(tid, mods, N):
            if any(n in quant for n, _ in mods):
                self.cache[tid] = Parts([(col, mod(n)) for n, col in mods], N)

        self.mod = mod
        if M + ".embed_tokens" in quant:
            self.gen_embed = mod(M + ".embed_tokens")
        slot(LM_HEAD, [("language_model.lm_head", 0)], V)
        for layer in range(d["layers"] + 1):
            p = f"{M}.layers.{layer}" if layer < d["layers"] else ckpt.MTP + ".layers.0"
            if p + ".mlp.gate.weight" not in named:
                continue
            attn = ckpt.is_attention(cfg, layer)
            if attn:
                q, kv = d["q_heads"] * 2 * d["head_dim"], d["kv_heads"] * d["head_dim"]
                slot(layer_tensor(layer, 2), [(p + ".self_attn.q_proj", 0), (p + ".self_attn.k_proj", q),
                                              (p + ".self_attn.v_proj", q + kv)], self.attn_rows)
                slot(layer_tensor(layer, 3), [(p + ".self_attn.o_proj", 0)], H)
            else:
                C, Z, Hv = self.C, d["value_heads"] * d["value_dim"], d["value_heads"]
                slot(layer_tensor(layer, 2), [(p + ".linear_attn.in_proj_qkv", 0), (p + ".linear_attn.in_proj_z", C),
                                              (p + ".linear_attn.in_proj_a", C + Z),
                                              (p + ".linear_attn.in_proj_b", C + Z + Hv)], C + Z + 2 * Hv)
                slot(layer_tensor(layer, 3), [(p + ".linear_attn.out_proj", 0)], H)
            slot(layer_tensor(layer, 10), [(p + ".mlp.gate", 0), (p + ".mlp.shared_expert_gate", E)], E + 1)
            ex = [p + ".mlp.switch_mlp." + n for n in ("gate_proj", "up_proj", "down_proj")] + \
                [p + ".mlp.shared_expert." + n for n in ("gate_proj", "up_proj", "down_proj")]
            if any(n in quant for n in ex):
                self.gen_experts[layer] = [mod(n) for n in ex]

    def embed(self, tokens):
        if not hasattr(self, "gen_embed"):
            return super().embed(tokens)
        q, t = self.gen_embed, np.asarray(tokens, np.int64)
        return oracle.dequant(q.w[t], q.s[t], q.b[t], self.d["hidden"], q.group, q.bits).astype(np.float32)

    def _experts(self, h, layer, idx, wts, shared_logit):
        if layer not in self.gen_experts:
            return super()._experts(h, layer, idx, wts, shared_logit)
        gate, up, down, sgate, sup, sdown = self.gen_experts[layer]
        d = self.d
        E, I, H = d["experts"], d["intermediate"], d["hidden"]
        n, top = idx.shape

        def routed(q, x, rows, sel):
            return oracle.gather_qmm(x, q.w.reshape(E, rows, -1), q.s.reshape(E, rows, -1), q.b.reshape(E, rows, -1),
                                     sel, q.group, q.bits)

        g, u = routed(gate, h, I, idx), routed(up, h, I, idx)
        act = bf16_round((oracle.silu(g.astype(np.float32)) * u).astype(np.float32)).reshape(n * top, I)
        dn = routed(down, act, H, np.ascontiguousarray(idx.reshape(-1, 1), np.int32)).reshape(n, top, H)
        dn = bf16_round(dn.astype(np.float32)).astype(np.float64)
        sa = bf16_round((oracle.silu(sgate(h).astype(np.float32)) * sup(h)).astype(np.float32))
        sd = bf16_round(sdown(sa).astype(np.float32)).astype(np.float64)
        out = np.einsum("bj,bjh->bh", np.asarray(wts, np.float64), dn)
        return out + 1.0 / (1.0 + np.exp(-np.asarray(shared_logit, np.float64)))[:, None] * sd


@pytest.fixture(scope="module")
def world(bridge, tmp_path_factory):
    from hip_bridge.engine import Engine, tiny_config
    from hip_bridge.session import WeightStore

    cfg = tiny_config(layers=2, interval=2, chunk=8, context=96)
    print("case: override checkpoints (tiny config, DeltaNet + attention + MTP)", flush=True)
    ref = Engine(cfg, 1, 96, 8, 8, seed=SEED, mtp=True)
    rng = np.random.default_rng(SEED)
    target = ckpt.split_target(cfg, ref.export)
    side = ckpt.split_mtp(cfg, ref.export)
    for named, table in ((target, OVERRIDES), (side, MTP_OVERRIDES)):
        for name, (group, bits) in table.items():
            w0 = named[name + ".weight"][1]
            shape, K = w0.shape[:-1], w0.shape[-1] * 8
            w, s, b = random_module(rng, shape, K, group, bits)
            named[name + ".weight"], named[name + ".scales"], named[name + ".biases"] = \
                ("U32", w), ("BF16", s), ("BF16", b)
    H = cfg.hidden
    fc = to_bf16_bits((rng.standard_normal((H, 2 * H)) * 0.02).astype(np.float32))
    for k in (".weight", ".scales", ".biases"):
        side.pop(ckpt.MTP + ".fc" + k)
    side[ckpt.MTP + ".fc.weight"] = ("BF16", fc)
    d = tmp_path_factory.mktemp("overrides")
    ckpt.write_safetensors(d / "model.safetensors", target, {"format": "mlx"})
    ckpt.write_safetensors(d / "mtp.safetensors", side)

    def stores():
        t, m = WeightStore(), WeightStore()
        t.load(d / "model.safetensors")
        m.load(d / "mtp.safetensors")
        for name, (group, bits) in OVERRIDES.items():
            t.quant(name, group, bits)
        for name, (group, bits) in MTP_OVERRIDES.items():
            m.quant(name, group, bits)
        return t, m

    model = NamedModel(cfg, ref.export, {**target, **side}, {**OVERRIDES, **MTP_OVERRIDES})
    model.cache[MTP_FC] = Dense(fc)
    model.tie_window = TIE
    yield cfg, ref, stores, model
    ref.close()


@pytest.mark.gpu
def test_override_engine_matches_oracle_layer_by_layer(world):
    from hip_bridge.engine import Engine

    cfg, _, stores, model = world
    t, m = stores()
    L, H, V = cfg.layers, cfg.hidden, cfg.vocab
    e = Engine(cfg, 4, 96, 8, 32, store=t, mtp_store=m)
    try:
        e.trace(True)
        rng = np.random.default_rng(8)
        seqs = [rng.integers(0, V, n).astype(np.uint32) for n in (7, 1, 8, 5)]
        lens = [len(s) for s in seqs]
        T = sum(lens)
        cu = np.cumsum([0] + lens)
        print("case: override engine prefill rows 7,1,8,5", flush=True)
        e.forward(lens, [0] * 4, [0, 1, 2, 3], np.concatenate(seqs), logit_rows=list(range(T)))
        logits, hidden = e.read("logits", T), e.read("hidden", T)
        trace, mid = e.read("trace", T), e.read("mid_trace", T)
        ties = 0
        for r, s in enumerate(seqs):
            row = Row(L, H)
            row.extend(trace[:, cu[r]:cu[r + 1]], mid[:, cu[r]:cu[r + 1]])
            ties += check_layers(model, row, len(s), s, f"row {r}")
            hn, want = model.head(row.x[L])
            assert_bf16_close(hidden[cu[r]:cu[r + 1]], hn, f"hidden row {r}")
            assert_bf16_close(logits[cu[r]:cu[r + 1]], want, f"logits row {r}")
        print(f"near-tie tokens judged against the swapped routing: {ties}", flush=True)

        # MTP head over (hidden q, token q + 1) through the dense BF16 fc
        nxt = [np.append(s[1:], np.uint32(np.argmax(logits[cu[r + 1] - 1]))) for r, s in enumerate(seqs)]
        print("case: override engine MTP head (dense fc)", flush=True)
        e.mtp_forward(lens, [0] * 4, [0, 1, 2, 3], np.concatenate(nxt), list(range(T)), logit_rows=list(range(T)))
        got, got_h, trace = e.read("logits", T), e.read("mtp_hidden", T), e.read("trace", T)
        mid = e.read("mid_trace", T)
        for r in range(len(seqs)):
            sl = slice(cu[r], cu[r + 1])
            assert_bf16_close(trace[0, sl], model.mtp_input(nxt[r], hidden[sl]), f"MTP dense fc row {r}")
            check_layer(model, L, trace[0, sl], mid[L, sl], trace[1, sl], lens[r], f"MTP row {r}")
            mh, want = model.head(trace[1, sl], norm=MTP_NORM)
            assert_bf16_close(got_h[sl], mh, f"MTP hidden row {r}")
            assert_bf16_close(got[sl], want, f"MTP logits row {r}")
    finally:
        e.close()


@pytest.mark.gpu
def test_override_session_equals_engine(world):
    """A device session over the same stores (overrides applied with
    rs_qwen_quant) gives the named engine's logits bit for bit."""
    from hip_bridge.engine import Engine
    from hip_bridge.session import DeviceSession

    cfg, _, stores, _ = world
    t, m = stores()
    toks = np.random.default_rng(11).integers(0, cfg.vocab, 8).astype(np.uint32)
    e = Engine(cfg, 1, 96, 8, 8, store=t, mtp_store=m)
    try:
        e.forward([8], [0], [0], toks, logit_rows=list(range(8)))
        want = e.read("logits", 8)
    finally:
        e.close()
    t2, m2 = stores()
    sess = DeviceSession(t2, cfg, slots=8)
    try:
        sess.mtp_attach(m2)
        sid, got = sess.block(None, 0, toks)
        assert np.array_equal(got.reshape(-1, cfg.vocab)[-1], want[-1]), "session logits"
        sess.release(sid)
    finally:
        sess.close()


@pytest.mark.gpu
def test_synthetic_store_refuses_overrides(bridge):
    from hip_bridge import HipBridgeError
    from hip_bridge.engine import tiny_config
    from hip_bridge.session import DeviceSession, WeightStore

    cfg = tiny_config(layers=2, interval=2, chunk=8, context=96)
    s = WeightStore(SEED, 0)
    s.quant(M + ".layers.0.mlp.gate", 64, 8)
    with pytest.raises(HipBridgeError, match="synthetic store"):
        DeviceSession(s, cfg, slots=8)
