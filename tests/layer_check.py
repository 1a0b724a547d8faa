"""Teacher-forced layer checks of the decode engine against the oracle model.

Each layer is judged in two halves, each from the engine's own residual
stream: the mixer (x -> x + mixer(norm(x)), attention or DeltaNet, over the
whole sequence) against the residual the engine kept after its mixer, then the
MoE from that residual to the layer output. Top-k routing has near-ties: the
oracle records, for every token whose k-th and (k+1)-th router logits lie
within its tie window, the MoE output with those two experts swapped, and the
device must match one of the two outcomes (any rounding of the router logits
may legitimately pick either expert).
"""
import numpy as np

from numerics import assert_bf16_close, assert_close


class Row:
    """One sequence's residual stream as the engine computed it: x [L+1][n][H]
    (layer inputs, then the output) and mid [L+1][n][H] (after each mixer)."""

    def __init__(self, L, H):
        self.x = np.zeros((L + 1, 0, H), np.float32)
        self.mid = np.zeros((L + 1, 0, H), np.float32)

    def extend(self, trace_rows, mid_rows):
        self.x = np.concatenate([self.x, trace_rows], axis=1)
        self.mid = np.concatenate([self.mid, mid_rows], axis=1)

    def copy(self):
        r = Row(0, 0)
        r.x, r.mid = self.x.copy(), self.mid.copy()
        return r


def judged_against(got, want, alts, first):
    """`want` with every near-tie token (index >= first in the sequence)
    replaced by its alternative when the device is closer to that one."""
    want = np.array(want, copy=True)
    swapped = 0
    for t, alt in alts.items():
        i = t - first
        if 0 <= i < len(want) and np.max(np.abs(got[i] - alt)) < np.max(np.abs(got[i] - want[i])):
            want[i] = alt
            swapped += 1
    return want, swapped


def check_layer(model, layer, x_in, mid, out, new, what):
    """Mixer over the whole sequence from x_in (outputs formed for the last
    `new` tokens), then the MoE of those tokens from the engine's mid residual;
    returns the near-tie tokens judged against the swapped routing."""
    want_mid = model.layer_mixer(layer, x_in, last=new)
    assert_bf16_close(mid[-new:], want_mid[-new:], f"{what} layer {layer} mixer")
    want = model.layer_moe(layer, mid[-new:])
    want, swapped = judged_against(out[-new:], want, model.layer_alternatives, 0)
    assert_bf16_close(out[-new:], want, f"{what} layer {layer} MoE")
    return swapped


def check_layers(model, row, new, tokens, what):
    """Embedding of the last `new` tokens, then every layer; returns the number
    of near-tie tokens judged against the swapped routing."""
    L = model.d["layers"]
    assert_close(row.x[0, -new:], model.embed(tokens[-new:]), 1e-6, f"{what} embedding")
    return sum(check_layer(model, layer, row.x[layer], row.mid[layer], row.x[layer + 1], new, what)
               for layer in range(L))
