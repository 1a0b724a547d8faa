"""Write tests/golden/ref_vectors.npz: seeded inputs and the outputs of the
reference's own FP64 scalar oracles (native/projection_reference.h,
native/operator_reference.h, native/attention_reference.h), compiled in place
from /root/reference by `make -C oracle ref` into oracle/_ref/libref.so.

Run in the build container (where /root/reference exists):
    python tests/golden/make_ref_vectors.py
The fixture is data only (inputs and expected outputs); no reference source is
stored in this repository.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

SEED = 20261201


def main():
    oracle.build(reference=True)
    R = oracle.ref()
    if R is None:
        raise SystemExit("oracle/_ref/libref.so is not built (reference tree absent?)")
    rng = np.random.default_rng(SEED)
    out = {}

    # projection: 8 rows x 256 outputs x 2048, 4-bit g64, plus odd widths
    for tag, (rows, outputs, width, group, bits) in {
        "p4": (8, 256, 2048, 64, 4),
        "p3": (3, 64, 512, 128, 3),
        "p5": (2, 32, 256, 32, 5),
    }.items():
        x = rng.standard_normal((rows, width)).astype(np.float32)
        words = width * bits // 32
        packed = rng.integers(0, 2**32, (outputs, words), dtype=np.uint64).astype(np.uint32)
        scales = oracle.bf16_round(rng.uniform(0.001, 0.01, (outputs, width // group)))
        biases = oracle.bf16_round(rng.uniform(-0.08, 0, (outputs, width // group)))
        y = np.zeros(rows * outputs)
        assert R.ref_projection(x.reshape(-1), rows, packed.reshape(-1), scales.reshape(-1), biases.reshape(-1),
                                outputs, width, group, bits, y) == 0
        out.update({f"{tag}_x": x, f"{tag}_packed": packed, f"{tag}_scales": scales, f"{tag}_biases": biases,
                    f"{tag}_y": y.reshape(rows, outputs), f"{tag}_geom": np.array([group, bits])})
        emb = np.zeros(min(outputs, 8) * width)
        r8 = min(outputs, 8)
        assert R.ref_embedding(packed[:r8].reshape(-1), scales[:r8].reshape(-1), biases[:r8].reshape(-1), r8, width,
                               group, bits, emb) == 0
        out[f"{tag}_embed"] = emb.reshape(r8, width)

    # RMS with and without weight
    x = rng.standard_normal((8, 2048)).astype(np.float32) * 3
    w = rng.standard_normal(2048).astype(np.float32)
    y = np.zeros(x.size)
    assert R.ref_rms(x.reshape(-1), x.size, w.ctypes.data, 2048, 1e-6, y) == 0
    out.update(rms_x=x, rms_w=w, rms_y=y.reshape(x.shape))
    x2 = rng.standard_normal((16, 256)).astype(np.float32)
    y2 = np.zeros(x2.size)
    assert R.ref_rms(x2.reshape(-1), x2.size, None, 256, 1e-6, y2) == 0
    out.update(rms0_x=x2, rms0_y=y2.reshape(x2.shape))

    # SiLU
    x = (rng.standard_normal(4096) * 6).astype(np.float32)
    y = np.zeros(x.size)
    assert R.ref_silu(x, x.size, y) == 0
    out.update(silu_x=x, silu_y=y)

    # RoPE: reference layout [heads][tokens][dim], 64 of 256 dims, theta 1e7, offset 100
    heads, tokens, dim = 16, 4, 256
    x = rng.standard_normal((heads, tokens, dim)).astype(np.float32)
    y = np.zeros(x.size)
    assert R.ref_rope(x.reshape(-1), heads, tokens, dim, 64, 100, 1e7, y) == 0
    out.update(rope_x=x, rope_y=y.reshape(x.shape), rope_geom=np.array([64, 100]))

    # Gated DeltaNet mixer core at the model head size (128), 2 value heads per key head, 3 tokens, conv width 4
    t, hk, hv, dk, dv, kernel = 3, 4, 8, 128, 128, 4
    channels = 2 * hk * dk + hv * dv
    qkv = rng.standard_normal((t, channels)).astype(np.float32)
    hist = rng.standard_normal((kernel - 1, channels)).astype(np.float32)
    conv = (rng.standard_normal((channels, kernel)) * 0.5).astype(np.float32)
    a = rng.standard_normal((t, hv)).astype(np.float32)
    b = rng.standard_normal((t, hv)).astype(np.float32)
    alog = np.log(rng.uniform(0.01, 1, hv)).astype(np.float32)
    dt = (rng.standard_normal(hv) * 0.1).astype(np.float32)
    init = (rng.standard_normal((hv, dv, dk)) * 0.01).astype(np.float32)
    act = np.zeros(t * channels)
    hist_out = np.zeros((kernel - 1) * channels)
    o = np.zeros(t * hv * dv)
    st = np.zeros(hv * dv * dk)
    assert R.ref_delta(qkv.reshape(-1), hist.reshape(-1), conv.reshape(-1), a.reshape(-1), b.reshape(-1), alog, dt,
                       init.reshape(-1), t, hk, hv, dk, dv, kernel, act, hist_out, o, st) == 0
    out.update(gdn_qkv=qkv, gdn_hist=hist, gdn_conv=conv, gdn_a=a, gdn_b=b, gdn_alog=alog, gdn_dt=dt, gdn_init=init,
               gdn_act=act.reshape(t, channels), gdn_hist_out=hist_out.reshape(kernel - 1, channels),
               gdn_out=o.reshape(t, hv, dv), gdn_state=st.reshape(hv, dv, dk))

    # Routing: 8 rows x 256 experts, top 8 (reference oracle bounds); selection
    # from the C oracle, weights and membership validated by the reference.
    logits = rng.standard_normal((8, 256)).astype(np.float32)
    idx, _ = oracle.route_topk(logits, 8)
    w = np.zeros(8 * 8)
    assert R.ref_routing(logits.reshape(-1), idx.reshape(-1), 8, 256, 8, w) == 0
    out.update(route_logits=logits, route_idx=idx, route_w=w.reshape(8, 8))

    # Attention: 16 heads, 2 kv heads, 4 new tokens after 37 cached, dim 256
    heads, kvh, tokens, offset, dim = 16, 2, 4, 37, 256
    n = offset + tokens
    q = rng.standard_normal((heads, tokens, dim)).astype(np.float32)
    k = rng.standard_normal((kvh, n, dim)).astype(np.float32)
    v = rng.standard_normal((kvh, n, dim)).astype(np.float32)
    y = np.zeros(q.size)
    assert R.ref_attention(q.reshape(-1), k.reshape(-1), v.reshape(-1), heads, kvh, tokens, offset, dim, y) == 0
    out.update(att_q=q, att_k=k, att_v=v, att_y=y.reshape(q.shape), att_geom=np.array([offset]))

    path = os.path.join(HERE, "ref_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
