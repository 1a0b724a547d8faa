// Gated DeltaNet mixer core (Qwen::recurrent, native/qwen_model.inc:154-206;
// scalar oracle native/operator_reference.h:20-44) for ragged packed rows.
#pragma once
#include "hb_common.h"

namespace hb {

struct GdnGeom {
  int key_heads, value_heads, key_dim, value_dim;  // 16, 32, 128, 128
  int conv;                                        // conv width (4)
  int max_tokens;                                  // window capacity per row beyond the history
};

// Per row r the conv window holds (conv-1) history rows followed by the row's
// new input rows: window [rows][conv-1+max_tokens][channels] bf16. The
// committed history of a row starts at window row hist_off[r] (the number of
// new rows the previous step committed; 0 for a fresh row with a zero window).
// The kernel reads that history, rewrites the window as [history | new rows]
// and emits, per packed token: q_hat, k_hat f32 [T][key_heads][key_dim],
// v f32 [T][value_heads][value_dim], decay and beta f32 [T][value_heads]:
//   act = silu(sum_tau stream[j+tau] * w[c][tau]),
//   q_hat = q / (sqrt(mean q^2 + 1e-6) * key_dim), k_hat = k / (sqrt(mean k^2 + 1e-6) * sqrt(key_dim)),
//   beta = sigmoid(b), decay = exp(-exp(A_log) * softplus(a + dt_bias)).
// Per-row storage slots: row r reads its parent's window/state/log at slot
// src[r] and writes its own at slot dst[r] (equal slots update in place; null
// arrays mean slot r). Distinct slots leave the parent version untouched at no
// extra traffic, since every step reads and writes the state once anyway.
struct GdnSlots {
  const int32_t* src;
  const int32_t* dst;
};
void gdn_prep(const bf16_t* qkv, int ld_qkv, const bf16_t* a, const bf16_t* b, int ld_ab, const float* conv_w,
              const float* a_log, const float* dt_bias, bf16_t* window, const int32_t* hist_off,
              const GdnSlots& slots, const int32_t* cu_seqlens, int rows, const GdnGeom& g, float* q_hat,
              float* k_hat, float* v, float* decay, float* beta, hipStream_t stream);

// The fp32 state of a (slot, value head) is stored key-major: element
// S[value i][key c] at [slot][value_heads][key c][value i].
// Recurrence per (row, value head) with the state in registers:
//   S <- decay*S; m = S k; delta = (v - m)*beta; S += delta k^T; o = S q.
// Pending log: before its own tokens a row replays log_count[r] logged
// updates S <- g*S + delta k^T (the accepted part of its previous speculative
// step). speculative != 0: the state written back is the state after the
// pending log (the committed state) and this step's updates are logged to
// log_out (capacity log_cap tokens per row); speculative == 0: the state after
// all tokens is written back and nothing is logged.
// Outputs: o f32 [T][value_heads][value_dim] when o_out != null, and the gated
// norm y = rms(o, norm_w, 1e-6) * silu(z) as bf16 [T][value_heads*value_dim]
// when y_out != null (z bf16 at z + i*ld_z).
struct GdnLog {
  float* k;      // [rows][cap][value_heads][key_dim]
  float* delta;  // [rows][cap][value_heads][value_dim]
  float* g;      // [rows][cap][value_heads]
};
void gdn_recurrence(const float* q_hat, const float* k_hat, const float* v, const float* decay, const float* beta,
                    const int32_t* cu_seqlens, int rows, const GdnGeom& g, float* state, const GdnSlots& slots,
                    const GdnLog& log_in, const int32_t* log_count, const GdnLog& log_out, int log_cap,
                    int speculative, float* o_out, const bf16_t* z, int ld_z, const float* norm_w, bf16_t* y_out,
                    hipStream_t stream);

// gdn_prep then gdn_recurrence in one launch for conv width 4 and 128-wide
// heads (the decode step): the same arguments as the two, without the
// intermediate q_hat / k_hat / v / decay / beta arrays, and bit-identical
// results (outputs, state, logs, conv window). False, with nothing launched,
// for another geometry.
bool gdn_decode(const bf16_t* qkv, int ld_qkv, const bf16_t* a, const bf16_t* b, int ld_ab, const float* conv_w,
                const float* a_log, const float* dt_bias, bf16_t* window, const int32_t* hist_off,
                const int32_t* cu_seqlens, int rows, const GdnGeom& g, float* state, const GdnSlots& slots,
                const GdnLog& log_in, const int32_t* log_count, const GdnLog& log_out, int log_cap, int speculative,
                float* o_out, const bf16_t* z, int ld_z, const float* norm_w, bf16_t* y_out, hipStream_t stream);

// Chunked form of the same recurrence for prefill steps (no pending log, not
// speculative): per row, chunks of 64 tokens run as matrix products (the
// corrected values of a chunk solve a unit lower-triangular system) instead
// of 64 dependent token updates. Same inputs and outputs as gdn_recurrence
// with speculative == 0; results agree with it to FP32 rounding, not bitwise.
// One 256-thread workgroup per (value head, row) with gdn_chunked_lds_bytes()
// of LDS.
void gdn_chunked(const float* q_hat, const float* k_hat, const float* v, const float* decay, const float* beta,
                 const int32_t* cu_seqlens, int rows, const GdnGeom& g, float* state, const GdnSlots& slots,
                 float* o_out, const bf16_t* z, int ld_z, const float* norm_w, bf16_t* y_out, hipStream_t stream);
size_t gdn_chunked_lds_bytes();

}  // namespace hb
