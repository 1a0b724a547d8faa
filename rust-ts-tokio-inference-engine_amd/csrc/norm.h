// Embedding gather and RMSNorm (native/qwen_model.inc:19-32, :306-309).
#pragma once
#include "hb_common.h"

namespace hb {

// out f32 [T][H] = s * q + b of the 4-bit g64 embedding rows tokens[t]
// (checkpoint layout: w u32 [V][H/8], s/b bf16 [V][H/64]).
void embed_gather(const uint32_t* tokens, int T, const uint32_t* w, const bf16_t* s, const bf16_t* b, int H,
                  float* out, hipStream_t stream);

// out bf16 [T][ld_out] = x * rsqrt(mean(x^2) + eps) * w for x f32 [T][ld_x] (first H columns);
// out_f32 (optional) receives the same values unrounded, row stride H; gsum
// (optional, H % 64 == 0) the sums of each 64-column group of the bf16 out
// row, f32 [T][H / 64], in the order the 4-bit projections use (q4_device.h).
void rmsnorm(const float* x, int ld_x, const float* w, int T, int H, float eps, bf16_t* out, int ld_out,
             hipStream_t stream, float* out_f32 = nullptr, float* gsum = nullptr);

// dst[i][:] = src[idx[i]][:] for n rows of `width` 32-bit words.
void gather_rows_f32(const float* src, int ld_src, const int32_t* idx, int n, int width, float* dst, int ld_dst,
                     hipStream_t stream);
void gather_rows_i32(const int32_t* src, int ld_src, const int32_t* idx, int n, int width, int32_t* dst, int ld_dst,
                     hipStream_t stream);

}  // namespace hb
