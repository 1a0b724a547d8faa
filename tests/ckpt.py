"""Checkpoint files for the loader tests: a safetensors writer and the split of
an engine's fused tensors back into the MLX-named tensors the reference's model
code reads (native/qwen_model.inc:34-206 for the target, native/qwen_mtp.inc:
37-45 for the MTP sidecar).

The fused layouts undone here:
- attention in-projection rows: q_proj (q and gate per head), k_proj, v_proj;
- DeltaNet in-projection rows: in_proj_qkv, in_proj_z, in_proj_a, in_proj_b;
- router rows: mlp.gate (experts), then mlp.shared_expert_gate;
- expert gate/up rows: per expert (the shared expert last) 16-row tiles of 8
  gate_proj rows then the matching 8 up_proj rows;
- expert down rows: every expert's down_proj, then the shared expert's;
- conv taps [C][W] as MLX's [C, W, 1] (or the raw [C, 1, W]).
Rows past the named tensors (padding to the kernels' tile) are dropped.
"""
import json
import struct

import numpy as np

EMBED, FINAL_NORM, LM_HEAD, MTP_PRE_E, MTP_PRE_H, MTP_FC, MTP_NORM = range(7)
IN_NORM, POST_NORM, IN_PROJ, OUT_PROJ, CONV_W, A_LOG, DT_BIAS, G_NORM, Q_NORM, K_NORM, ROUTER, GATE_UP, DOWN = \
    range(13)
MODEL, MTP = "language_model.model", "language_model.mtp"


def layer_tensor(layer, slot):
    return 16 + 16 * layer + slot


def write_safetensors(path, tensors, metadata=None):
    """tensors: name -> (dtype string, numpy array of that item size)."""
    header, blobs, off = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, (dt, a) in tensors.items():
        b = np.ascontiguousarray(a).tobytes()
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        f.write(b"".join(blobs))


def is_attention(cfg, layer):
    return layer == cfg.layers or (layer + 1) % cfg.interval == 0


def _q4(out, name, w, s, b, shape=None):
    if shape is not None:
        w = w.reshape(*shape, w.shape[-1])
        s = s.reshape(*shape, s.shape[-1])
        b = b.reshape(*shape, b.shape[-1])
    out[name + ".weight"] = ("U32", w)
    out[name + ".scales"] = ("BF16", s)
    out[name + ".biases"] = ("BF16", b)


def _split_rows(out, prefix, t, parts):
    w, s, b = t
    at = 0
    for name, rows in parts:
        _q4(out, f"{prefix}.{name}", w[at:at + rows], s[at:at + rows], b[at:at + rows])
        at += rows
    return at


def split_layer(cfg, export, layer, prefix, shift=False, raw_conv=False):
    """The named tensors of one decoder layer (layer == cfg.layers: the MTP layer)."""
    out = {}
    H, E, I = cfg.hidden, cfg.experts, cfg.intermediate
    attn = is_attention(cfg, layer)
    t = lambda slot: export(layer_tensor(layer, slot))
    off = (lambda v: (v - np.float32(1)).astype(np.float32)) if shift else (lambda v: v)
    out[prefix + ".input_layernorm.weight"] = ("F32", off(t(IN_NORM)))
    out[prefix + ".post_attention_layernorm.weight"] = ("F32", off(t(POST_NORM)))
    if attn:
        D, Hq, Hkv = cfg.head_dim, cfg.q_heads, cfg.kv_heads
        _split_rows(out, prefix + ".self_attn", t(IN_PROJ),
                    [("q_proj", Hq * 2 * D), ("k_proj", Hkv * D), ("v_proj", Hkv * D)])
        _q4(out, prefix + ".self_attn.o_proj", *t(OUT_PROJ))
        out[prefix + ".self_attn.q_norm.weight"] = ("F32", off(t(Q_NORM)))
        out[prefix + ".self_attn.k_norm.weight"] = ("F32", off(t(K_NORM)))
    else:
        Hk, Hv, Dk, Dv, W = cfg.key_heads, cfg.value_heads, cfg.key_dim, cfg.value_dim, cfg.conv
        C = 2 * Hk * Dk + Hv * Dv
        _split_rows(out, prefix + ".linear_attn", t(IN_PROJ),
                    [("in_proj_qkv", C), ("in_proj_z", Hv * Dv), ("in_proj_a", Hv), ("in_proj_b", Hv)])
        _q4(out, prefix + ".linear_attn.out_proj", *t(OUT_PROJ))
        conv = t(CONV_W).reshape(C, W)
        out[prefix + ".linear_attn.conv1d.weight"] = ("F32", conv[:, None, :] if raw_conv else conv[:, :, None])
        out[prefix + ".linear_attn.A_log"] = ("F32", t(A_LOG))
        out[prefix + ".linear_attn.dt_bias"] = ("F32", t(DT_BIAS))
        out[prefix + ".linear_attn.norm.weight"] = ("F32", t(G_NORM))  # never shifted
    _split_rows(out, prefix + ".mlp", t(ROUTER), [("gate", E), ("shared_expert_gate", 1)])
    w, s, b = t(GATE_UP)
    tiles = lambda a: a[:(E + 1) * 2 * I].reshape(E + 1, I // 8, 2, 8, a.shape[-1])
    gw, gs, gb = (tiles(a)[:, :, 0].reshape(E + 1, I, a.shape[-1]) for a in (w, s, b))
    uw, us, ub = (tiles(a)[:, :, 1].reshape(E + 1, I, a.shape[-1]) for a in (w, s, b))
    _q4(out, prefix + ".mlp.switch_mlp.gate_proj", gw[:E], gs[:E], gb[:E])
    _q4(out, prefix + ".mlp.switch_mlp.up_proj", uw[:E], us[:E], ub[:E])
    _q4(out, prefix + ".mlp.shared_expert.gate_proj", gw[E], gs[E], gb[E])
    _q4(out, prefix + ".mlp.shared_expert.up_proj", uw[E], us[E], ub[E])
    w, s, b = t(DOWN)
    _q4(out, prefix + ".mlp.switch_mlp.down_proj", w[:E * H], s[:E * H], b[:E * H], shape=(E, H))
    _q4(out, prefix + ".mlp.shared_expert.down_proj", w[E * H:], s[E * H:], b[E * H:])
    return out


def split_target(cfg, export, shift=False, raw_conv=False, with_mtp_key=False):
    """The target model's named tensors; `shift` stores norms as offsets from 1
    (a checkpoint the loader must mark shifted: raw conv layout or an mtp. key)."""
    V = cfg.vocab
    out = {}
    w, s, b = export(EMBED)
    _q4(out, MODEL + ".embed_tokens", w[:V], s[:V], b[:V])
    w, s, b = export(LM_HEAD)
    _q4(out, "language_model.lm_head", w[:V], s[:V], b[:V])
    norm = export(FINAL_NORM)
    out[MODEL + ".norm.weight"] = ("F32", (norm - np.float32(1)).astype(np.float32) if shift else norm)
    for layer in range(cfg.layers):
        out.update(split_layer(cfg, export, layer, f"{MODEL}.layers.{layer}", shift, raw_conv))
    if with_mtp_key:
        out["mtp.unused_marker"] = ("F32", np.zeros(4, np.float32))
    return out


def split_mtp(cfg, export):
    """The MTP sidecar's named tensors (never shifted)."""
    out = {
        MTP + ".pre_fc_norm_embedding.weight": ("F32", export(MTP_PRE_E)),
        MTP + ".pre_fc_norm_hidden.weight": ("F32", export(MTP_PRE_H)),
        MTP + ".norm.weight": ("F32", export(MTP_NORM)),
    }
    _q4(out, MTP + ".fc", *export(MTP_FC))
    out.update(split_layer(cfg, export, cfg.layers, MTP + ".layers.0"))
    return out


def all_tensor_ids(cfg, mtp=True):
    ids = [EMBED, FINAL_NORM, LM_HEAD] + ([MTP_PRE_E, MTP_PRE_H, MTP_FC, MTP_NORM] if mtp else [])
    for layer in range(cfg.layers + (1 if mtp else 0)):
        slots = [IN_NORM, POST_NORM, IN_PROJ, OUT_PROJ, ROUTER, GATE_UP, DOWN]
        slots += [Q_NORM, K_NORM] if is_attention(cfg, layer) else [CONV_W, A_LOG, DT_BIAS, G_NORM]
        ids += [layer_tensor(layer, s) for s in slots]
    return ids


def filled_rows(cfg, tid):
    """Rows of fused tensor `tid` that come from named tensors (the rest is padding)."""
    if tid in (EMBED, LM_HEAD):
        return cfg.vocab
    if tid < 16:
        return None
    layer, slot = (tid - 16) // 16, (tid - 16) % 16
    if slot == IN_PROJ:
        if is_attention(cfg, layer):
            return cfg.q_heads * 2 * cfg.head_dim + 2 * cfg.kv_heads * cfg.head_dim
        return 2 * cfg.key_heads * cfg.key_dim + 2 * cfg.value_heads * cfg.value_dim + 2 * cfg.value_heads
    if slot == ROUTER:
        return cfg.experts + 1
    return None
