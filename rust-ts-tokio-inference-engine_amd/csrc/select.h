// Greedy selection and MTP acceptance on the device.
#pragma once
#include "hb_common.h"

namespace hb {

// Per row of logits f32 [rows][ld] (vocab columns): winner under f32 total
// order with the lowest index on ties, margin = top1 - top2 (f32; +inf when the
// row has one element), status = 1 if the row holds a non-finite value.
// Reference: winner_with_margin, src/serving/native_speculative.rs:45-73;
// device_total_argmax, native/selection.h:5-13.
// workspace (optional, argmax_workspace_bytes): rows longer than one chunk
// are scanned by several workgroups and merged in column order.
size_t argmax_workspace_bytes(int rows, int vocab);
// Size of the static device scratch that stands in for the workspace when the
// caller cannot allocate (hb_argmax_margin_noalloc): 65,536 (row, chunk)
// summaries.
constexpr size_t kSelectScratchBytes = size_t(1) << 20;
// Device address of that scratch on the current device (resolved once per
// device with hipGetSymbolAddress; allocates nothing). Every call on one GPU
// shares it.
void* select_scratch();
void argmax_margin(const float* logits, int ld, int rows, int vocab, uint32_t* winner, float* margin,
                   int32_t* status, hipStream_t stream, void* workspace = nullptr);

// MTP acceptance per row (src/serving/native_speculative.rs:74-128):
//   draft[r][0..n_draft[r]) proposed tokens, target[r][i] = winner after input i
//   (target[r][0] is the winner of the row's initial logits, target[r][i] for
//   i >= 1 the winner of verify row i-1), eos list, remaining[r] budget.
// emitted[r][0..n_emitted[r]) (capacity max_draft+1), accepted[r], terminal[r];
// status[r] = 1 for a malformed row (n_draft > 8, > remaining, remaining == 0,
// or tokens outside the vocabulary).
void mtp_plan(const uint32_t* draft, const int32_t* n_draft, int max_draft, const uint32_t* target,
              const uint32_t* eos, int n_eos, const int32_t* remaining, int rows, int vocab, uint32_t* emitted,
              int32_t* n_emitted, int32_t* accepted, int32_t* terminal, int32_t* status, hipStream_t stream);

}  // namespace hb
