// Checkpoint-layout projections for modules outside the tiled 4-bit g64 form:
// per-module affine quantization overrides (rs_qwen_quant, native/qwen_model.inc:
// 16 and 273-276: any bits in {2,3,4,5,6,8}, group in {32,64,128}) and the MTP
// sidecar's dense BF16 fc (native/qwen_model.inc:34, src/serving/native_mtp.rs:
// 121-123). The tensors stay where the checkpoint loader put them (MLX layout:
// codes as an LSB-first bit stream per row, bf16 scales and biases [rows][K /
// group]); these kernels read them in place with FP32 accumulation.
#pragma once
#include "hb_common.h"

namespace hb {

// One quantized module: rows x K (lead experts of rows each when lead > 0),
// placed at output column `col` of the engine tensor it stands in for.
struct QMod {
  const uint32_t* w = nullptr;
  const bf16_t* s = nullptr;
  const bf16_t* b = nullptr;
  int rows = 0, K = 0, group = 64, bits = 4, lead = 0, col = 0;
  __host__ __device__ size_t words_per_row() const { return size_t(K) * bits / 32; }
};

// act[j][n] = bf16(silu(g) * u) for the sorted routed rows j < P (token
// order[j] / top, expert idx[order[j]]) and the shared expert's rows P + t,
// g and u the rows' projections through gate/up (experts) or sgate/sup
// (shared); x bf16 [T][ldx].
void moe_generic_gate_up(const bf16_t* x, int ldx, const int32_t* order, const int32_t* idx, int top, int P, int T,
                         const QMod& gate, const QMod& up, const QMod& sgate, const QMod& sup, bf16_t* act,
                         hipStream_t stream);
// dout[j][n] = bf16(act[j] . down[expert(j)][n]) over the same rows.
void moe_generic_down(const bf16_t* act, const int32_t* order, const int32_t* idx, int top, int P, int T,
                      const QMod& down, const QMod& sdown, bf16_t* dout, hipStream_t stream);
// x[t][c] = s * q + b of embedding row tokens[t] (f32 [T][K]).
void embed_generic(const uint32_t* tokens, int T, const QMod& emb, float* x, hipStream_t stream);
// y (ldy) = x (bf16 [M][K]) . W^T with W bf16 [N][K], FP32 accumulation; out
// 0 bf16, 1 f32, 2 f32 +=.
void dense_bf16(const bf16_t* x, int M, int K, const bf16_t* W, int N, void* y, int out_mode, int ldy,
                hipStream_t stream);

}  // namespace hb
