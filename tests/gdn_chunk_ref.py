"""The chunked form of the gated delta rule, in FP64, as the device's chunked
prefill kernel computes it (the test infrastructure's statement of it).

Token-serial rule per (row, value head), state S [dv][dk] (native/
qwen_model.inc:191-200): S <- g_t S; d = (v_t - S k_t) beta_t; S <- S + d k_t^T;
o_t = S q_t.

Over a chunk of C tokens with log-decay prefix L_t = sum_{j <= t} log g_j,
Gamma_t = exp(L_t), and U the chunk's corrected values:
  (I + A) U = diag(beta) (V - diag(Gamma) K S0^T),
      A[t][i] = beta_t exp(L_t - L_i) k_t . k_i   (i < t, else 0)
  O = diag(Gamma) Q S0^T + P U,  P[t][i] = exp(L_t - L_i) q_t . k_i  (i <= t)
  S_C = Gamma_C S0 + U^T diag(exp(L_C - L)) K
The triangular system is solved in 16-token blocks: each block first takes
the earlier blocks' contributions, then a forward substitution within the block.
"""
import numpy as np


def serial(q, k, v, g, beta, S):
    """Token by token: (outputs [T][dv], final state [dv][dk])."""
    S = np.array(S, np.float64)
    out = np.zeros((len(q), S.shape[0]))
    for t in range(len(q)):
        S *= g[t]
        d = (v[t] - S @ k[t]) * beta[t]
        S += np.outer(d, k[t])
        out[t] = S @ q[t]
    return out, S


def chunk(q, k, v, g, beta, S, block=16):
    """One chunk in the closed form above (T <= 64 tokens)."""
    q, k, v, S = (np.asarray(a, np.float64) for a in (q, k, v, S))
    g, beta = np.asarray(g, np.float64), np.asarray(beta, np.float64)
    T = len(q)
    L = np.cumsum(np.log(g))
    gam = np.exp(L)
    ratio = np.exp(L[:, None] - L[None, :])
    A = np.tril(beta[:, None] * ratio * (k @ k.T), -1)
    R = beta[:, None] * (v - gam[:, None] * (k @ S.T))
    U = np.zeros_like(R)
    for b0 in range(0, T, block):
        b1 = min(b0 + block, T)
        r = R[b0:b1] - A[b0:b1, :b0] @ U[:b0]
        for t in range(b1 - b0):  # forward substitution within the block
            U[b0 + t] = r[t] - A[b0 + t, b0:b0 + t] @ U[b0:b0 + t]
    P = np.tril(ratio * (q @ k.T))
    O = gam[:, None] * (q @ S.T) + P @ U
    S_new = gam[-1] * S + (U * np.exp(L[-1] - L)[:, None]).T @ k
    return O, S_new


def chunked(q, k, v, g, beta, S, C=64):
    """A sequence in chunks of C tokens."""
    outs = []
    for c0 in range(0, len(q), C):
        sl = slice(c0, c0 + C)
        o, S = chunk(q[sl], k[sl], v[sl], g[sl], beta[sl], S)
        outs.append(o)
    return np.concatenate(outs), S
