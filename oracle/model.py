"""CPU restatement of the hybrid decoder's forward (whole-step composition).

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the device
engine; the product library never loads it.

Composition, scales and epsilon placement follow qwen_forward_core
(native/qwen_model.inc:277-373): the layer loop (:321-352) with the mixer
program "attention iff (i+1) % interval == 0" (src/serving/model_ir.rs:170),
Qwen::attention (:101-153), Qwen::recurrent (:154-206), Qwen::moe (:75-100),
final norm + lm_head (:353-366), and the MTP head (native/qwen_mtp.inc:32-46).
Every operator is the oracle's own FP64 restatement (oracle.c). Activations
are rounded to bf16 exactly where the device path stores them in bf16
(matmul inputs, the KV cache, the mixer outputs), so a deviation measures
arithmetic, not storage format.

Weights come in the checkpoint layout, addressed by the engine's tensor ids:
tensors(id) -> (packed u32 [N][K/8], scales bits, biases bits) or an f32 vector.
The fused projections concatenate the reference's separate matrices by rows:
  attention in-projection = q_proj (q | gate per head) ; k_proj ; v_proj
  DeltaNet in-projection  = in_proj_qkv ; in_proj_z ; in_proj_a ; in_proj_b (; zero pad to 16)
  router                  = router ; shared_expert_gate (; pad)
  expert gate/up          = per expert, per 16-row tile: 8 gate rows then the 8 matching up rows
  expert down             = per expert [H][I]
Expert index E is the shared expert.
"""
from __future__ import annotations

import numpy as np

from . import bf16_round, from_bf16_bits, gdn, paged_attention, qmm, qmm4_f32, rms, rope, route_topk, silu

EMBED, FINAL_NORM, LM_HEAD, MTP_PRE_E, MTP_PRE_H, MTP_FC, MTP_NORM = range(7)
IN_NORM, POST_NORM, IN_PROJ, OUT_PROJ, CONV_W, A_LOG, DT_BIAS, G_NORM, Q_NORM, K_NORM, ROUTER, GATE_UP, DOWN = \
    range(13)


def layer_tensor(layer, slot):
    return 16 + 16 * layer + slot


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))


class Q4:
    """A 4-bit g64 matrix in checkpoint layout with bf16 scales/biases widened to f32.
    fp32: products in the oracle's FP32 form (the CPU baseline's timing path)."""

    def __init__(self, t, fp32=False):
        w, s, b = t
        self.w, self.s, self.b = w, from_bf16_bits(s), from_bf16_bits(b)
        self.fp32 = fp32

    def rows(self, idx):
        return Q4.__new__(Q4)._set(self.w[idx], self.s[idx], self.b[idx], self.fp32)

    def _set(self, w, s, b, fp32=False):
        self.w, self.s, self.b, self.fp32 = w, s, b, fp32
        return self

    def __call__(self, x):
        """x [M][K] (float) -> FP64 [M][N] = x . W^T (mx::quantized_matmul, qwen_model.inc:34)."""
        if self.fp32:
            return qmm4_f32(np.asarray(x, np.float32), self.w, self.s, self.b).astype(np.float64)
        return qmm(np.asarray(x, np.float32), self.w, self.s, self.b)


class HybridModel:
    def __init__(self, dims: dict, tensors, fp32=False):
        """fp32: every 4-bit product in the oracle's FP32 form (the CPU
        baseline's timing path); FP64 otherwise (the parity checker)."""
        self.d = dims
        self.t = tensors
        self.fp32 = fp32
        self.cache = {}
        d = dims
        self.attn_rows = d["q_heads"] * 2 * d["head_dim"] + 2 * d["kv_heads"] * d["head_dim"]
        self.C = 2 * d["key_heads"] * d["key_dim"] + d["value_heads"] * d["value_dim"]
        self.min_route_gap = np.inf
        # router-logit gap below which a top-k boundary counts as a near-tie
        # (0: no alternatives are recorded)
        self.tie_window = 0.0
        self.moe_alternatives = {}
        self.layer_alternatives = {}

    def w(self, tid):
        if tid not in self.cache:
            t = self.t(tid)
            self.cache[tid] = Q4(t, self.fp32) if isinstance(t, tuple) else np.asarray(t, np.float32)
        return self.cache[tid]

    # ------------------------------------------------------------ operators
    def embed(self, tokens):
        """Dequantised embedding rows (qwen_model.inc:306-309)."""
        e = self.w(EMBED)
        H = self.d["hidden"]
        tokens = np.asarray(tokens, np.int64)
        codes = np.stack([(e.w[tokens] >> np.uint32(4 * j)) & np.uint32(15) for j in range(8)], -1)
        codes = codes.reshape(len(tokens), H).astype(np.float64)
        g = np.arange(H) // 64
        return (e.s[tokens][:, g].astype(np.float64) * codes + e.b[tokens][:, g]).astype(np.float32)

    def norm(self, x, tid):
        """bf16(rms(x, w)) with eps (Qwen::norm, qwen_model.inc:19-32)."""
        return bf16_round(rms(x, self.w(tid), self.d["epsilon"]).astype(np.float32))

    def attention(self, h, layer, positions, last=None):
        """Gated GQA over the whole sequence 0..len-1 (Qwen::attention, qwen_model.inc:101-153).
        h bf16 [n][H]; positions = 0..n-1 (the full causal prefix is recomputed).
        With `last`, only the last `last` tokens' outputs are formed: the keys and
        values still come from every token, q, gate and the output projection only
        from those rows (each projected row is independent of the others)."""
        d = self.d
        hq, hkv, D = d["q_heads"], d["kv_heads"], d["head_dim"]
        n = h.shape[0]
        m = n if last is None else int(last)
        inp = self.w(layer_tensor(layer, IN_PROJ))
        nq = hq * 2 * D
        qg = bf16_round(inp.rows(np.arange(nq))(h[n - m:]).astype(np.float32)).reshape(m, hq, 2 * D)
        kv = bf16_round(inp.rows(np.arange(nq, nq + 2 * hkv * D))(h).astype(np.float32))
        k = kv[:, :hkv * D].reshape(n, hkv, D)
        v = kv[:, hkv * D:].reshape(n, hkv, D)
        eps = d["epsilon"]
        q = rope(rms(qg[:, :, :D], self.w(layer_tensor(layer, Q_NORM)), eps).astype(np.float32), positions[n - m:],
                 d["rope_dims"], d["theta"])
        k = rope(rms(k, self.w(layer_tensor(layer, K_NORM)), eps).astype(np.float32), positions, d["rope_dims"],
                 d["theta"])
        q, k = bf16_round(q.astype(np.float32)), bf16_round(k.astype(np.float32))
        page = 16
        pages = (n + page - 1) // page
        kc = np.zeros((pages * page, hkv, D), np.float32)
        vc = np.zeros((pages * page, hkv, D), np.float32)
        kc[:n], vc[:n] = k, v
        kc = kc.reshape(pages, page, hkv, D).transpose(0, 2, 1, 3)
        vc = vc.reshape(pages, page, hkv, D).transpose(0, 2, 1, 3)
        bt = np.arange(pages, dtype=np.int32)[None, :]
        out = paged_attention(q, kc, vc, bt, np.array([0, m], np.int32), np.array([n], np.int32),
                              1.0 / np.sqrt(D), gate=qg[:, :, D:].copy())
        out = bf16_round(out.astype(np.float32)).reshape(m, hq * D)
        return self.w(layer_tensor(layer, OUT_PROJ))(out)

    def recurrent(self, h, layer, last=None):
        """Gated DeltaNet over the whole sequence from a zero state and zero
        conv history (Qwen::recurrent, qwen_model.inc:154-206); with `last`,
        the output of the last `last` tokens only."""
        d = self.d
        hk, hv, dk, dv, conv = d["key_heads"], d["value_heads"], d["key_dim"], d["value_dim"], d["conv"]
        C = self.C
        n = h.shape[0]
        proj = bf16_round(self.w(layer_tensor(layer, IN_PROJ))(h).astype(np.float32))
        qkv = proj[:, :C]
        z = proj[:, C:C + hv * dv]
        a = proj[:, C + hv * dv:C + hv * dv + hv]
        b = proj[:, C + hv * dv + hv:C + hv * dv + 2 * hv]
        conv_w = self.w(layer_tensor(layer, CONV_W)).reshape(C, conv)
        _, _, o, _ = gdn(qkv, np.zeros((conv - 1, C), np.float32), conv_w, a, b, self.w(layer_tensor(layer, A_LOG)),
                         self.w(layer_tensor(layer, DT_BIAS)), np.zeros((hv, dv, dk), np.float32), hk, hv, dk, dv)
        y = rms(o.astype(np.float32), self.w(layer_tensor(layer, G_NORM)), 1e-6) * silu(z.reshape(n, hv, dv))
        y = bf16_round(y.astype(np.float32)).reshape(n, hv * dv)
        m = n if last is None else int(last)
        return self.w(layer_tensor(layer, OUT_PROJ))(y[n - m:])

    def moe(self, h, layer):
        """Routed experts plus the sigmoid-gated shared expert (Qwen::moe, qwen_model.inc:75-100),
        one gather_qmm per matrix over all tokens (the shared expert is expert E).

        Near-ties: a token whose top-th and (top+1)-th router logits lie within
        `self.tie_window` has a second legitimate outcome (any rounding of the
        logits may pick either expert). Its MoE output with those two experts
        swapped is kept in `self.moe_alternatives[token]`."""
        d = self.d
        E, top = d["experts"], d["top"]
        logits = self.w(layer_tensor(layer, ROUTER))(h).astype(np.float32)
        rl = np.ascontiguousarray(logits[:, :E])
        idx, wts = route_topk(rl, top)
        self.moe_alternatives = {}
        if top < E:
            srt = np.sort(rl, axis=1)[:, ::-1]
            gaps = srt[:, top - 1] - srt[:, top]
            self.min_route_gap = min(self.min_route_gap, float(np.min(gaps)))
            near = np.nonzero(gaps < self.tie_window)[0]
            if len(near):
                alt_idx, alt_w = self._swap_boundary(rl[near], top)
                alt = self._experts(h[near], layer, alt_idx, alt_w, logits[near, E])
                self.moe_alternatives = {int(t): alt[i] for i, t in enumerate(near)}
        return self._experts(h, layer, idx, wts, logits[:, E])

    @staticmethod
    def _swap_boundary(logits, top):
        """Top-k sets with the top-th expert replaced by the (top+1)-th, and
        their renormalised softmax weights (same rule as route_topk)."""
        order = np.argsort(-logits.astype(np.float64), axis=1, kind="stable")
        idx = np.concatenate([order[:, :top - 1], order[:, top:top + 1]], axis=1).astype(np.int32)
        sel = np.take_along_axis(logits.astype(np.float64), idx, axis=1)
        w = np.exp(sel - sel.max(axis=1, keepdims=True))
        return idx, w / w.sum(axis=1, keepdims=True)

    def _experts(self, h, layer, idx, wts, shared_logit):
        """sum_j w_j * expert_{idx_j}(h) + sigmoid(shared_logit) * expert_E(h) with
        SwiGLU experts: act = bf16(silu(gate) * up), out = bf16(down(act))."""
        from . import gather_qmm

        d = self.d
        E, I, H = d["experts"], d["intermediate"], d["hidden"]
        n, top = idx.shape
        full = np.concatenate([idx, np.full((n, 1), E, np.int32)], axis=1)
        gu, dn = self.w(layer_tensor(layer, GATE_UP)), self.w(layer_tensor(layer, DOWN))
        y = gather_qmm(h, gu.w.reshape(E + 1, 2 * I, -1), gu.s.reshape(E + 1, 2 * I, -1),
                       gu.b.reshape(E + 1, 2 * I, -1), full)
        tile = y.reshape(n, top + 1, -1, 16)
        g, u = tile[..., :8].reshape(n, top + 1, I), tile[..., 8:].reshape(n, top + 1, I)
        act = bf16_round((silu(g.astype(np.float32)) * u).astype(np.float32)).reshape(n * (top + 1), I)
        down = gather_qmm(act, dn.w.reshape(E + 1, H, -1), dn.s.reshape(E + 1, H, -1), dn.b.reshape(E + 1, H, -1),
                          np.ascontiguousarray(full.reshape(-1, 1), np.int32))
        down = bf16_round(down.reshape(n, top + 1, H).astype(np.float32)).astype(np.float64)
        out = np.einsum("bj,bjh->bh", np.asarray(wts, np.float64), down[:, :top])
        return out + _sigmoid(shared_logit)[:, None] * down[:, top]

    def moe_per_token(self, h, layer):
        """The same MoE as `moe`, written as a per-token, per-expert loop over
        row slices of the fused matrices (the independent form the gathered
        one is checked against)."""
        d = self.d
        E, top, I = d["experts"], d["top"], d["intermediate"]
        n = h.shape[0]
        logits = self.w(layer_tensor(layer, ROUTER))(h).astype(np.float32)
        idx, wts = route_topk(np.ascontiguousarray(logits[:, :E]), top)
        gu, dn = self.w(layer_tensor(layer, GATE_UP)), self.w(layer_tensor(layer, DOWN))
        tile = np.arange(2 * I).reshape(-1, 16)
        g_rows, u_rows = tile[:, :8].reshape(-1), tile[:, 8:].reshape(-1)
        out = np.zeros((n, d["hidden"]), np.float64)

        def expert(x, e):
            base = e * 2 * I
            g = gu.rows(base + g_rows)(x)
            u = gu.rows(base + u_rows)(x)
            act = bf16_round((silu(g.astype(np.float32)) * u).astype(np.float32))
            return bf16_round(dn.rows(np.arange(e * d["hidden"], (e + 1) * d["hidden"]))(act).astype(np.float32))

        for t in range(n):
            x = h[t:t + 1]
            for j in range(top):
                out[t] += wts[t, j] * expert(x, int(idx[t, j]))[0]
            out[t] += _sigmoid(logits[t, E]) * expert(x, E)[0]
        return out

    # ------------------------------------------------------------ programs
    def layer_mixer(self, layer, x, last=None):
        """The residual after the mixer, x + mixer(rms(x, input_layernorm)), over a
        whole sequence (positions 0..n-1) from the f32 residual x [n][H]
        (qwen_model.inc:328-331); with `last`, the rows of the last `last`
        tokens only (every token still feeds their keys and recurrence)."""
        d = self.d
        x = np.asarray(x, np.float32).astype(np.float64)
        n = x.shape[0]
        m = n if last is None else int(last)
        pos = np.arange(n, dtype=np.int32)
        h = self.norm(x.astype(np.float32), layer_tensor(layer, IN_NORM))
        if layer == d["layers"] or (layer + 1) % d["interval"] == 0:
            y = x[n - m:] + self.attention(h, layer, pos, last=m)
        else:
            y = x[n - m:] + self.recurrent(h, layer, last=m)
        return y.astype(np.float32)

    def layer_moe(self, layer, x):
        """x + moe(rms(x, post_attention_layernorm)) for residual rows x [n][H]
        after the mixer (qwen_model.inc:332-335); per token, so any subset of a
        sequence's rows may be passed. Near-tie alternatives of the whole
        output land in `self.layer_alternatives` (token -> row)."""
        x = np.asarray(x, np.float32).astype(np.float64)
        h = self.norm(x.astype(np.float32), layer_tensor(layer, POST_NORM))
        out = (x + self.moe(h, layer)).astype(np.float32)
        self.layer_alternatives = {t: (x[t] + alt).astype(np.float32) for t, alt in self.moe_alternatives.items()}
        return out

    def layer(self, layer, x):
        """One decoder layer over a whole sequence (positions 0..n-1) from the
        f32 residual x [n][H] (qwen_model.inc:328-335):
        x += mixer(rms(x, input_layernorm)); x += moe(rms(x, post_attention_layernorm))."""
        return self.layer_moe(layer, self.layer_mixer(layer, x))

    def head(self, x, norm=FINAL_NORM):
        """(post-norm hidden f32 [n][H], lm_head logits FP64 [n][V]) (qwen_model.inc:353-366);
        rows of the lm_head beyond the vocabulary are padding."""
        hn = rms(np.asarray(x, np.float32), self.w(norm), self.d["epsilon"]).astype(np.float32)
        lm = self.w(LM_HEAD)
        lm = lm.rows(np.arange(self.d["vocab"])) if lm.w.shape[0] > self.d["vocab"] else lm
        return hn, lm(bf16_round(hn))

    def forward(self, tokens):
        """One sequence from position 0: (post-final-norm hidden f32 [n][H], logits FP64 [n][V])."""
        x = self.embed(tokens)
        for layer in range(self.d["layers"]):
            x = self.layer(layer, x)
        return self.head(x)

    def mtp_input(self, next_tokens, hidden):
        """fc([rms(embed(t_{q+1}), pre_fc_norm_embedding) | rms(h_q, pre_fc_norm_hidden)])
        (qwen_mtp.inc:37-39): f32 [n][H]."""
        e = self.norm(self.embed(next_tokens), MTP_PRE_E)
        hh = self.norm(np.asarray(hidden, np.float32), MTP_PRE_H)
        return self.w(MTP_FC)(np.concatenate([e, hh], axis=1)).astype(np.float32)

    def mtp(self, next_tokens, hidden):
        """MTP head over pairs (target hidden row q, token q+1) for q = 0..n-1
        (qwen_mtp.inc:32-46): (MTP hidden f32 [n][H], logits FP64 [n][V])."""
        x = self.layer(self.d["layers"], self.mtp_input(next_tokens, hidden))
        return self.head(x, MTP_NORM)


class DecodeStepCPU:
    """One greedy decode step (one new token per row) of rows that already hold
    a context, restated with the oracle's primitives: per attention layer a
    paged KV cache of the context, per DeltaNet layer the recurrent state and
    the conv history. Same composition as HybridModel.layer for T = 1; the
    routed experts go through one gather_qmm per matrix (shared expert as
    expert E). Timing baseline for the device decode step."""

    def __init__(self, model: HybridModel, layers, contexts, seed=0, zero=False):
        d = model.d
        self.m, self.layers = model, list(layers)
        self.ctx = np.asarray(contexts, np.int32)
        rng = np.random.default_rng(seed)
        fill = (lambda shape: np.zeros(shape, np.float32)) if zero else (
            lambda shape: rng.standard_normal(shape, dtype=np.float32))
        B = len(self.ctx)
        hkv, D = d["kv_heads"], d["head_dim"]
        hv, dv, dk, conv = d["value_heads"], d["value_dim"], d["key_dim"], d["conv"]
        page = 16
        self.pages = [(int(c) + 1 + page - 1) // page for c in self.ctx]
        self.bt = np.zeros((B, max(self.pages)), np.int32)
        cur = 0
        for r, n in enumerate(self.pages):
            self.bt[r, :n] = np.arange(cur, cur + n)
            self.bt[r, n:] = cur + n - 1
            cur += n
        self.cache = {}
        for layer in self.layers:
            if (layer + 1) % d["interval"] == 0:
                shape = (cur, hkv, page, D)
                self.cache[layer] = (bf16_round(fill(shape)), bf16_round(fill(shape)))
            else:
                self.cache[layer] = (fill((B, hv, dv, dk)) * 0.01, bf16_round(fill((B, conv - 1, model.C))))

    def layer(self, layer, x):
        m, d = self.m, self.m.d
        x = np.asarray(x, np.float32).astype(np.float64)
        B = x.shape[0]
        h = m.norm(x.astype(np.float32), layer_tensor(layer, IN_NORM))
        if (layer + 1) % d["interval"] == 0:
            hq, hkv, D = d["q_heads"], d["kv_heads"], d["head_dim"]
            proj = bf16_round(m.w(layer_tensor(layer, IN_PROJ))(h).astype(np.float32))
            qg = proj[:, :hq * 2 * D].reshape(B, hq, 2 * D)
            k = proj[:, hq * 2 * D:hq * 2 * D + hkv * D].reshape(B, hkv, D)
            v = proj[:, hq * 2 * D + hkv * D:].reshape(B, hkv, D)
            q = rope(rms(qg[:, :, :D], m.w(layer_tensor(layer, Q_NORM)), d["epsilon"]).astype(np.float32), self.ctx,
                     d["rope_dims"], d["theta"])
            k = rope(rms(k, m.w(layer_tensor(layer, K_NORM)), d["epsilon"]).astype(np.float32), self.ctx,
                     d["rope_dims"], d["theta"])
            kc, vc = self.cache[layer]
            for r in range(B):
                pg, off = self.bt[r, self.ctx[r] // 16], self.ctx[r] % 16
                kc[pg, :, off] = bf16_round(k[r].astype(np.float32))
                vc[pg, :, off] = v[r]
            out = paged_attention(bf16_round(q.astype(np.float32)), kc, vc, self.bt,
                                  np.arange(B + 1, dtype=np.int32), self.ctx + 1, 1.0 / np.sqrt(D),
                                  gate=qg[:, :, D:].copy())
            y = bf16_round(out.astype(np.float32)).reshape(B, hq * D)
        else:
            hk, hv, dk, dv = d["key_heads"], d["value_heads"], d["key_dim"], d["value_dim"]
            C = m.C
            proj = bf16_round(m.w(layer_tensor(layer, IN_PROJ))(h).astype(np.float32))
            state, hist = self.cache[layer]
            conv_w = m.w(layer_tensor(layer, CONV_W)).reshape(C, d["conv"])
            o = np.zeros((B, hv, dv))
            for r in range(B):
                a0 = C + hv * dv
                _, hist_r, o_r, st = gdn(proj[r:r + 1, :C], hist[r], conv_w, proj[r:r + 1, a0:a0 + hv],
                                         proj[r:r + 1, a0 + hv:a0 + 2 * hv], m.w(layer_tensor(layer, A_LOG)),
                                         m.w(layer_tensor(layer, DT_BIAS)), state[r], hk, hv, dk, dv)
                hist[r], state[r], o[r] = hist_r, st, o_r[0]
            z = proj[:, C:C + hv * dv].reshape(B, hv, dv)
            y = rms(o.astype(np.float32), m.w(layer_tensor(layer, G_NORM)), 1e-6) * silu(z)
            y = bf16_round(y.astype(np.float32)).reshape(B, hv * dv)
        x = (x + m.w(layer_tensor(layer, OUT_PROJ))(y)).astype(np.float32).astype(np.float64)
        h = m.norm(x.astype(np.float32), layer_tensor(layer, POST_NORM))
        return (x + self.moe(h, layer)).astype(np.float32)

    def moe(self, h, layer):
        from . import gather_qmm as gq64, gather_qmm4_f32

        m, d = self.m, self.m.d
        gather_qmm = (lambda *a: gather_qmm4_f32(*a).astype(np.float64)) if m.fp32 else gq64
        E, top, I, H = d["experts"], d["top"], d["intermediate"], d["hidden"]
        B = h.shape[0]
        logits = m.w(layer_tensor(layer, ROUTER))(h).astype(np.float32)
        idx, wts = route_topk(np.ascontiguousarray(logits[:, :E]), top)
        idx = np.concatenate([idx, np.full((B, 1), E, np.int32)], axis=1)
        gu, dn = m.w(layer_tensor(layer, GATE_UP)), m.w(layer_tensor(layer, DOWN))
        gu_w = gu.w.reshape(E + 1, 2 * I, -1)
        y = gather_qmm(h, gu_w, gu.s.reshape(E + 1, 2 * I, -1), gu.b.reshape(E + 1, 2 * I, -1), idx)
        tile = y.reshape(B, top + 1, -1, 16)
        g, u = tile[..., :8].reshape(B, top + 1, I), tile[..., 8:].reshape(B, top + 1, I)
        act = bf16_round((silu(g.astype(np.float32)) * u).astype(np.float32)).reshape(B * (top + 1), I)
        down = gather_qmm(act, dn.w.reshape(E + 1, H, -1), dn.s.reshape(E + 1, H, -1), dn.b.reshape(E + 1, H, -1),
                          np.ascontiguousarray(idx.reshape(-1, 1), np.int32))
        down = bf16_round(down.reshape(B, top + 1, H).astype(np.float32))
        out = np.einsum("bj,bjh->bh", wts, down[:, :top].astype(np.float64))
        return out + _sigmoid(logits[:, E])[:, None] * down[:, top]
