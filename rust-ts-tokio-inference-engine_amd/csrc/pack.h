// Device-built ragged packing tables (see pack.hip).
#pragma once
#include "hb_common.h"

namespace hb {

// All pointers are device pointers. status[0] is set to 1 when a row has a
// negative count/position or runs past its block table (tables are then not
// expanded), else 0.
void pack_tables(const int32_t* row_tokens, const int32_t* positions, const int32_t* block_table, int max_pages,
                 int rows, int page, int32_t* cu_seqlens, int32_t* token_row, int32_t* token_pos, int32_t* kv_slot,
                 int32_t* context, int32_t* status, hipStream_t stream);

// Page copies across KV pools for copy-on-write page sharing and snapshots.
// pools: device array of pool base pointers (bf16), each holding pages of
// page_elems elements; pairs: device i32 [n][2] (source page, destination page).
// Pool p of pools[0..n_pools) copies page pairs[i][0] to page pairs[i][1] of the
// same pool, or, when `gather` is set, to gather + (p * n + i) * page_elems.
// page_elems must be a multiple of 8.
void copy_pages(bf16_t* const* pools, int n_pools, const int32_t* pairs, int n, int page_elems, bf16_t* gather,
                hipStream_t stream);

}  // namespace hb
