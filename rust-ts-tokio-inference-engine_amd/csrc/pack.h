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

}  // namespace hb
