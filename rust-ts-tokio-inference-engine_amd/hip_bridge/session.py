"""Host mirror of the device-session ABI (native/mlx_bridge.h:50-133): weight
stores, immutable StateId versions, the target steps, the batched and ragged
packers and the MTP operator. It plays the role of the Rust `Session`
wrapper (src/serving/native_device.rs:130-345): every call passes a 1024-byte
error buffer and raises on a nonzero status; ids are released exactly once.
"""
import ctypes as C

import numpy as np

from . import ERR_CAP, HipBridgeError, _err, load
from .engine import QwenConfig

STATS_LEN = 17 + 19 * 3  # native/qwen_device.inc:62


class StateId(C.Structure):
    """40-byte value descriptor of a published state version (native/state_table.h:11-13)."""
    _fields_ = [(n, C.c_uint64) for n in ("owner", "slot", "generation", "position", "bytes")]

    def key(self):
        return (self.owner, self.slot, self.generation, self.position, self.bytes)

    def copy(self):
        return StateId(*self.key())

    def __repr__(self):
        return "StateId(owner={}, slot={}, generation={}, position={}, bytes={})".format(*self.key())


class Layer(C.Structure):
    _fields_ = [("index", C.c_uint32), ("mixer", C.c_uint32)]


def layer_program(config: QwenConfig):
    """The mixer program: attention iff (i + 1) % interval == 0 (src/serving/model_ir.rs:170)."""
    arr = (Layer * config.layers)()
    for i in range(config.layers):
        arr[i].index = i
        arr[i].mixer = int((i + 1) % config.interval == 0)
    return arr


def state_count(c: QwenConfig) -> int:
    """qwen_state_count (native/qwen_model.inc:268-271), fixed capacity."""
    full = c.layers // c.interval
    linear = c.layers - full
    conv = (c.conv - 1) * (2 * c.key_heads * c.key_dim + c.value_heads * c.value_dim)
    rec = c.value_heads * c.value_dim * c.key_dim
    return linear * (conv + rec) + full * 2 * c.kv_heads * c.context * c.head_dim


def _check(rc, name, err):
    if rc != 0:
        raise HipBridgeError(f"{name}: {err.value.decode(errors='replace')}")


def _call(name, *args):
    err = _err()
    _check(getattr(load(), name)(*args, err, ERR_CAP), name, err)


def _u32(a):
    return np.ascontiguousarray(a, np.uint32)


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def safetensors_check(path):
    """Host-only header validation (hb_safetensors_check): the tensor count."""
    n = C.c_size_t()
    _call("hb_safetensors_check", str(path).encode(), C.byref(n))
    return n.value


class WeightStore:
    """rs_mlx_weights_create store; `seed` marks it as the seeded random-init
    model (part 0) or its MTP sidecar (part 1)."""

    def __init__(self, seed=None, part=0):
        err = _err()
        self.handle = load().rs_mlx_weights_create(err, ERR_CAP)
        if not self.handle:
            raise HipBridgeError(f"rs_mlx_weights_create: {err.value.decode(errors='replace')}")
        if seed is not None:
            _call("hb_weights_synthetic", self.handle, C.c_uint64(seed), part)

    def load(self, path):
        """rs_mlx_weights_load: every tensor of a safetensors file, as device arrays."""
        _call("rs_mlx_weights_load", self.handle, str(path).encode())

    def quant(self, module: str, group: int, bits: int):
        _call("rs_qwen_quant", self.handle, module.encode(), group, bits)

    def forward(self, config, tokens, offset=0, old_state=None, trace=False):
        """Stateless rs_qwen_forward: (new_state, logits [V], trace or None)."""
        tokens = _u32(tokens)
        n = state_count(config)
        new = np.empty(n, np.float32)
        logits = np.empty(config.vocab, np.float32)
        old = None if old_state is None else np.ascontiguousarray(old_state, np.float32)
        tr = np.empty(config.layers * 5 * len(tokens) * config.hidden, np.float32) if trace else None
        prog = layer_program(config)
        _call("rs_qwen_forward", self.handle, 1, C.byref(config), prog, config.layers, _p(tokens), len(tokens), offset,
              _p(old), 0 if old is None else old.size, _p(new), n, _p(logits), logits.size, 0, None, 0, _p(tr),
              0 if tr is None else tr.size)
        return new, logits, tr

    def close(self):
        if getattr(self, "handle", None):
            load().rs_mlx_weights_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceSession:
    """rs_qwen_device_create over a synthetic store (gpu = 1)."""

    def __init__(self, store: WeightStore, config: QwenConfig, slots=8, budget=1 << 50):
        err = _err()
        self.config = config
        self.vocab, self.hidden = config.vocab, config.hidden
        self.handle = load().rs_qwen_device_create(store.handle, 1, C.byref(config), layer_program(config),
                                                   config.layers, slots, C.c_uint64(budget), err, ERR_CAP)
        if not self.handle:
            raise HipBridgeError(f"rs_qwen_device_create: {err.value.decode(errors='replace')}")

    def close(self):
        if getattr(self, "handle", None):
            load().rs_qwen_device_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---------------------------------------------------------------- target steps
    def _step(self, name, prev, position, tokens, rows, trace=False):
        tokens = _u32(tokens)
        out = StateId()
        logits = np.empty((rows, self.vocab), np.float32)
        args = [self.handle, None if prev is None else C.byref(prev), position, _p(tokens), len(tokens), C.byref(out),
                _p(logits), logits.size]
        tr = None
        if name == "rs_qwen_device_step":
            tr = np.empty(self.config.layers * 5 * len(tokens) * self.hidden, np.float32) if trace else None
            args += [_p(tr), 0 if tr is None else tr.size]
        _call(name, *args)
        return out, logits, tr

    def step(self, prev, position, tokens, trace=False):
        """(id, logits [V] of the last token, trace [L][5][n][H] or None)."""
        sid, lg, tr = self._step("rs_qwen_device_step", prev, position, tokens, 1, trace)
        if tr is not None:
            tr = tr.reshape(self.config.layers, 5, len(tokens), self.hidden)
        return sid, lg[0], tr

    def block(self, prev, position, tokens):
        sid, lg, _ = self._step("rs_qwen_device_block", prev, position, tokens, len(tokens))
        return sid, lg

    def hidden_step(self, prev, position, tokens):
        sid, lg, _ = self._step("rs_qwen_device_hidden_step", prev, position, tokens, 1)
        return sid, lg[0]

    def hidden_block(self, prev, position, tokens):
        sid, lg, _ = self._step("rs_qwen_device_hidden_block", prev, position, tokens, len(tokens))
        return sid, lg

    def step_sampled(self, prev, position, tokens):
        tokens = _u32(tokens)
        out, tok = StateId(), C.c_uint32()
        _call("rs_qwen_device_step_sampled", self.handle, None if prev is None else C.byref(prev), position,
              _p(tokens), len(tokens), C.byref(out), C.byref(tok))
        return out, tok.value

    def decode_batch(self, parents, tokens):
        B = len(parents)
        par = (StateId * B)(*[p.copy() for p in parents])
        outs = (StateId * B)()
        tokens = _u32(tokens)
        logits = np.empty((B, self.vocab), np.float32)
        _call("rs_qwen_device_decode_batch", self.handle, par, _p(tokens), B, outs, _p(logits), logits.size)
        return list(outs), logits

    def ragged(self, parents, seqs, per_token=False, hidden=False, logits=False):
        """parents: StateId or None (a fresh row at position 0) per row; seqs:
        token lists. Returns (ids, winners, margins, logits or None)."""
        B = len(seqs)
        par = (StateId * B)(*[(p.copy() if p is not None else StateId()) for p in parents])
        outs = (StateId * B)()
        rt = _u32([len(s) for s in seqs])
        toks = _u32(np.concatenate([np.asarray(s, np.uint32) for s in seqs]))
        n = len(toks) if per_token else B
        win = np.empty(n, np.uint32)
        mar = np.empty(n, np.float32)
        lg = np.empty((n, self.vocab), np.float32) if logits else None
        flags = (1 if per_token else 0) | (2 if hidden else 0)
        _call("rs_qwen_device_ragged_step", self.handle, par, _p(rt), B, _p(toks), len(toks), flags, outs, _p(win),
              _p(mar), _p(lg), 0 if lg is None else lg.size)
        return list(outs), win, mar, lg

    # ---------------------------------------------------------------- versions
    def release(self, sid):
        _call("rs_qwen_device_release", self.handle, C.byref(sid))

    def snapshot(self, sid):
        out = np.empty(state_count(self.config), np.float32)
        _call("rs_qwen_device_snapshot", self.handle, C.byref(sid), _p(out), out.size)
        return out

    def hidden_snapshot(self, sid, rows):
        out = np.empty((rows, self.hidden), np.float32)
        _call("rs_qwen_device_hidden_snapshot", self.handle, C.byref(sid), _p(out), out.size)
        return out

    def stats(self):
        out = np.zeros(STATS_LEN, np.uint64)
        _call("rs_qwen_device_stats", self.handle, _p(out), out.size)
        return out

    def info(self):
        """Bridge diagnostics (hb_session_info): vocabulary-head passes that
        fused the greedy selection."""
        out = np.zeros(1, np.uint64)
        _call("hb_session_info", self.handle, _p(out), out.size)
        return {"fused_heads": int(out[0])}

    def drain(self):
        n = C.c_uint64()
        _call("rs_qwen_device_drain", self.handle, C.byref(n))
        return n.value

    # ---------------------------------------------------------------- MTP operator
    def mtp_attach(self, store: WeightStore):
        _call("rs_qwen_device_mtp_attach", self.handle, store.handle)

    def mtp_step(self, prev, source, draft_source, row, tokens):
        tokens = _u32(tokens)
        out = StateId()
        logits = np.empty(self.vocab, np.float32)
        _call("rs_qwen_device_mtp_step", self.handle, None if prev is None else C.byref(prev), C.byref(source),
              draft_source, row, _p(tokens), len(tokens), C.byref(out), _p(logits), logits.size, 0)
        return out, logits

    def mtp_release(self, sid):
        _call("rs_qwen_device_mtp_release", self.handle, C.byref(sid))

    def mtp_snapshot(self, sid):
        out = np.empty(sid.bytes // 4, np.float32)
        _call("rs_qwen_device_mtp_snapshot", self.handle, C.byref(sid), _p(out), out.size)
        return out
