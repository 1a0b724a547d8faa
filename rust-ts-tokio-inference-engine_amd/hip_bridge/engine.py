"""Host mirror of the decode engine and the speculative decode loop.

The engine owns the hybrid decoder's device-resident weights (seeded
synthetic 4-bit), the per-sequence KV pages and recurrent state, and runs the
packed ragged forward (qwen_forward_core, native/qwen_model.inc:277-373; the
batched packer native/qwen_batch.inc:2-50). The decode loop mirrors
mtp_prepare/mtp_commit (src/serving/native_mtp_decode.rs:124-295) with the
acceptance plan on the device.
"""
import ctypes as C

import numpy as np

from . import ERR_CAP, HipBridgeError, _err, call, load

# rs_qwen_config field order (native/mlx_bridge.h:50-53; src/serving/native_qwen.rs:62-98)
CONFIG_INTS = ["hidden", "layers", "vocab", "q_heads", "kv_heads", "head_dim", "key_heads", "value_heads", "key_dim",
               "value_dim", "conv", "interval", "experts", "top", "intermediate", "shared", "group", "bits",
               "context", "chunk", "rope_dims", "activation_precision", "layer_group", "fused_recurrent",
               "execution_timing", "compiled_decode", "operator_profile", "fused_attention", "validation_mode",
               "validation_interval", "expert_kernel"]


class QwenConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in CONFIG_INTS] + [("epsilon", C.c_float), ("theta", C.c_float)]

    def dims(self):
        return {n: getattr(self, n) for n in CONFIG_INTS + ["epsilon", "theta"]}


def hybrid_config(**overrides) -> QwenConfig:
    """48-layer hybrid decoder: 3 Gated-DeltaNet layers then 1 gated GQA layer,
    hidden 2048, vocab 151936, 512 experts top-10 of width 512 plus a shared
    expert, 16/2 x 256 attention heads (64 rotary dims, theta 1e7), 16 key and
    32 value heads of 128 for DeltaNet, conv width 4, 4-bit group 64."""
    d = dict(hidden=2048, layers=48, vocab=151936, q_heads=16, kv_heads=2, head_dim=256, key_heads=16,
             value_heads=32, key_dim=128, value_dim=128, conv=4, interval=4, experts=512, top=10, intermediate=512,
             shared=512, group=64, bits=4, context=8448, chunk=64, rope_dims=64, activation_precision=0,
             layer_group=1, validation_interval=1, epsilon=1e-6, theta=1e7)
    d.update(overrides)
    c = QwenConfig()
    for k, v in d.items():
        setattr(c, k, v)
    return c


def tiny_config(**overrides) -> QwenConfig:
    """A small geometry of the same family for parity tests: 4 layers (3
    DeltaNet + 1 attention), hidden 256, vocab 512, 8/1 attention heads, 2/4
    DeltaNet heads, 8 experts top-2."""
    d = dict(hidden=256, layers=4, vocab=512, q_heads=8, kv_heads=1, head_dim=256, key_heads=2, value_heads=4,
             key_dim=128, value_dim=128, conv=4, interval=4, experts=8, top=2, intermediate=128, shared=128,
             context=512)
    d.update(overrides)
    return hybrid_config(**d)


# tensor ids (engine weight generation and export)
EMBED, FINAL_NORM, LM_HEAD, MTP_PRE_E, MTP_PRE_H, MTP_FC, MTP_NORM = range(7)
IN_NORM, POST_NORM, IN_PROJ, OUT_PROJ, CONV_W, A_LOG, DT_BIAS, G_NORM, Q_NORM, K_NORM, ROUTER, GATE_UP, DOWN = \
    range(13)


def layer_tensor(layer, slot):
    return 16 + 16 * layer + slot


def _i32(a):
    return None if a is None else np.ascontiguousarray(a, np.int32)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class Engine:
    def __init__(self, config: QwenConfig, max_rows, max_context, max_row_tokens, max_step_tokens, seed=20261201,
                 mtp=True, store=None, mtp_store=None):
        """Seeded synthetic weights, or with `store` (a loaded WeightStore, plus
        `mtp_store` for the MTP sidecar) the checkpoint's tensors."""
        err = _err()
        self.config = config
        if store is not None:
            name = "hb_engine_create_named"
            self.handle = load().hb_engine_create_named(C.byref(config), max_rows, max_context, max_row_tokens,
                                                        max_step_tokens, store.handle,
                                                        None if mtp_store is None else mtp_store.handle, err,
                                                        ERR_CAP)
        else:
            name = "hb_engine_create"
            self.handle = load().hb_engine_create(C.byref(config), max_rows, max_context, max_row_tokens,
                                                  max_step_tokens, seed, int(mtp), err, ERR_CAP)
        if not self.handle:
            raise HipBridgeError(f"{name}: {err.value.decode(errors='replace')}")
        self.max_rows, self.max_context = max_rows, max_context
        self.max_row_tokens, self.max_step_tokens = max_row_tokens, max_step_tokens
        info = np.zeros(4, np.uint64)
        call("hb_engine_info", self.handle, info.ctypes.data_as(C.c_void_p), 4)
        self.weight_bytes, self.state_bytes, self.max_pages, self.stream = (int(v) for v in info)

    def fused_heads(self):
        """Vocabulary-head passes so far that fused the selection (wrote no logits)."""
        info = np.zeros(5, np.uint64)
        call("hb_engine_info", self.handle, info.ctypes.data_as(C.c_void_p), 5)
        return int(info[4])

    def close(self):
        if getattr(self, "handle", None):
            load().hb_engine_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor_shape(self, tid):
        n, k, q = C.c_int32(), C.c_int32(), C.c_int32()
        call("hb_engine_tensor_shape", self.handle, tid, C.byref(n), C.byref(k), C.byref(q))
        return n.value, k.value, bool(q.value)

    def export(self, tid):
        """Tensor `tid` in checkpoint layout: (w u32 [N][K/8], s, b as bf16 bits) or an f32 vector."""
        from . import DeviceBuffer

        n, k, q4 = self.tensor_shape(tid)
        if q4:
            w = DeviceBuffer(n * k // 2)
            s = DeviceBuffer(n * (k // 64) * 2)
            b = DeviceBuffer(n * (k // 64) * 2)
            call("hb_engine_export", self.handle, tid, w, s, b)
            return (w.download(np.uint32, (n, k // 8)), s.download(np.uint16, (n, k // 64)),
                    b.download(np.uint16, (n, k // 64)))
        w = DeviceBuffer(n * 4)
        call("hb_engine_export", self.handle, tid, w, None, None)
        return w.download(np.float32, (n,))

    def forward(self, row_tokens, positions, seq, tokens, speculative=False, logit_rows=None, src_slot=None,
                dst_slot=None, hist_off=None, log_count=None):
        rt, pos, sq = _i32(row_tokens), _i32(positions), _i32(seq)
        tok = np.ascontiguousarray(tokens, np.uint32)
        lr = _i32(logit_rows if logit_rows is not None else [])
        src, dst, ho, lc = _i32(src_slot), _i32(dst_slot), _i32(hist_off), _i32(log_count)
        call("hb_engine_forward", self.handle, len(rt), _ptr(rt), _ptr(pos), _ptr(sq), _ptr(src), _ptr(dst),
             _ptr(ho), _ptr(lc), _ptr(tok), int(speculative), _ptr(lr) if len(lr) else None, len(lr))

    def mtp_forward(self, row_tokens, positions, seq, tokens, hidden_idx, hidden_source=0, logit_rows=None):
        rt, pos, sq = _i32(row_tokens), _i32(positions), _i32(seq)
        tok = np.ascontiguousarray(tokens, np.uint32)
        hi = _i32(hidden_idx)
        lr = _i32(logit_rows if logit_rows is not None else [])
        call("hb_engine_mtp_forward", self.handle, len(rt), _ptr(rt), _ptr(pos), _ptr(sq), _ptr(tok),
             hidden_source, _ptr(hi), _ptr(lr) if len(lr) else None, len(lr))

    def read(self, which, count, offset=0):
        """which: 'hidden' / 'mtp_hidden' ([count][H] f32), 'logits' ([count][V] f32),
        'winners' (u32), 'margins' (f32), 'status' (i32); 'trace' ([L+1][count][H]: the
        residual stream of the last forward, needs trace(True)); 'mid_trace' ([L+1][count][H]:
        each layer's residual after its mixer, slot L the MTP layer)."""
        if which in ("trace", "mid_trace"):
            c = self.config
            out = np.empty((c.layers + 1, count, c.hidden), np.float32)
            for i in range(c.layers + 1):
                call("hb_engine_read", self.handle, 6 if which == "trace" else 7,
                     i * self.max_step_tokens * c.hidden * 4, out[i].ctypes.data_as(C.c_void_p), out[i].nbytes)
            return out
        c = self.config
        kind = {"hidden": (0, np.float32, (count, c.hidden)), "mtp_hidden": (1, np.float32, (count, c.hidden)),
                "logits": (2, np.float32, (count, c.vocab)), "winners": (3, np.uint32, (count,)),
                "margins": (4, np.float32, (count,)), "status": (5, np.int32, (count,))}[which]
        out = np.empty(kind[2], kind[1])
        call("hb_engine_read", self.handle, kind[0], offset, out.ctypes.data_as(C.c_void_p), out.nbytes)
        return out

    def profile(self, stride=1):
        """Probe every `stride`-th launch of the grouped MoE GEMMs, attention and the
        DeltaNet recurrence (0: off; enabling resets the probes)."""
        call("hb_engine_profile", self.handle, int(stride))

    def profile_read(self, kind):
        """kind 0 grouped gate/up, 1 grouped down, 2 paged attention + combine, 3 DeltaNet
        recurrence: dict(launches, ms, tokens, active, bytes), summed over sampled launches."""
        out = np.zeros(5, np.float64)
        call("hb_engine_profile_read", self.handle, kind, out.ctypes.data_as(C.c_void_p), 5)
        return dict(launches=int(out[0]), ms=float(out[1]), tokens=float(out[2]), active=float(out[3]),
                    bytes=float(out[4]))

    def trace(self, enable=True):
        call("hb_engine_trace", self.handle, int(enable))

    def synthetic_context(self, positions, seed=7):
        pos = _i32(positions)
        call("hb_engine_synthetic_context", self.handle, len(pos), _ptr(pos), seed)


class DecodeLoop:
    def __init__(self, engine: Engine, width=4, gate_margin=1.25, eos=()):
        err = _err()
        self.engine = engine
        e = np.ascontiguousarray(eos, np.uint32)
        self.handle = load().hb_decode_create(engine.handle, width, gate_margin, _ptr(e) if len(e) else None, len(e),
                                              err, ERR_CAP)
        if not self.handle:
            raise HipBridgeError(f"hb_decode_create: {err.value.decode(errors='replace')}")

    def close(self):
        if getattr(self, "handle", None):
            load().hb_decode_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def admit(self, seq, position, pending, budget, hist_off=0):
        call("hb_decode_admit", self.handle, seq, position, pending, budget, hist_off)

    def set_drafts(self, seq, tokens):
        t = np.ascontiguousarray(tokens, np.uint32)
        call("hb_decode_set_drafts", self.handle, seq, _ptr(t) if len(t) else None, len(t))

    def step(self):
        n = C.c_int32()
        call("hb_decode_step", self.handle, C.byref(n))
        return n.value

    def stats(self):
        s = np.zeros(9, np.uint64)
        call("hb_decode_stats", self.handle, s.ctypes.data_as(C.c_void_p), 9)
        keys = ["steps", "emitted", "target_tokens", "proposed", "accepted", "mtp_calls", "mtp_tokens", "finished",
                "live"]
        return {k: int(v) for k, v in zip(keys, s)}

    def output(self, seq):
        n, pos = C.c_int32(), C.c_int32()
        call("hb_decode_output", self.handle, seq, None, 0, C.byref(n), C.byref(pos))
        out = np.zeros(n.value, np.uint32)
        call("hb_decode_output", self.handle, seq, out.ctypes.data_as(C.c_void_p), n.value, C.byref(n),
             C.byref(pos))
        return out, pos.value
