// Seeded synthetic tensors on the device (see synth.hip).
#pragma once
#include "hb_common.h"

namespace hb {

// W [N][K] ~ N(0, std) quantised to affine 4-bit group 64 in the checkpoint
// layout: w u32 [N][K/8], s and b bf16 [N][K/64].
void random_q4(uint64_t seed, int N, int K, float std_dev, uint32_t* w, bf16_t* s, bf16_t* b, hipStream_t stream);
// out[i] = mean + std * N(0,1) (dtype 0 f32, 4 bf16)
void random_normal(uint64_t seed, size_t n, float std_dev, float mean, int dtype, void* out, hipStream_t stream);
// out[i] ~ U[lo, hi)
void random_uniform(uint64_t seed, size_t n, float lo, float hi, int dtype, void* out, hipStream_t stream);
// out[i] ~ U{0 .. bound-1}
void random_ints(uint64_t seed, size_t n, uint32_t bound, uint32_t* out, hipStream_t stream);

}  // namespace hb
