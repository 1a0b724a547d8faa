// The continuous-batching decode engine: device-resident weights of the hybrid
// decoder, per-sequence state pools, and the packed forward over ragged rows.
// Reference: qwen_forward_core (native/qwen_model.inc:277-373), the batched
// packer (native/qwen_batch.inc:2-50) and the MTP head (native/qwen_mtp.inc:8-56).
#pragma once
#include <array>
#include <cstdint>
#include <string>
#include <vector>

#include "../../include/hip_bridge.h"
#include "attention.h"
#include "deltanet.h"
#include "generic.h"
#include "graph.h"
#include "hb_common.h"
#include "moe.h"

namespace hb {

// The one activation profile this bridge computes: BF16 matrix operands and
// stored activations (norm outputs, projections, the KV cache), an FP32
// residual stream, FP32 accumulation and FP32 recurrent state. The reference's
// rs_qwen_config.activation_precision calls this profile 0; its profile 1
// (FP32 activations, native/qwen_model.inc:308-309) is refused at creation.
constexpr const char* kFp32ProfileRefused =
    "activation precision 1 (FP32) is not built into this bridge: it computes BF16 activations with an FP32 "
    "residual stream and FP32 accumulation (activation precision 0)";

struct Geom {
  int H, L, V, Hq, Hkv, D, Hk, Hv, Dk, Dv, conv, interval, E, top, I, rotary;
  float eps, theta;
  bool attn(int l) const { return (l + 1) % interval == 0; }
  int conv_channels() const { return 2 * Hk * Dk + Hv * Dv; }
  // Fused projections are padded to whole 256-row groups (the streaming GEMM's
  // workgroup tile); padding rows produce outputs nobody reads.
  static int round256(int n) { return (n + 255) / 256 * 256; }
  int dn_in_rows() const { return round256(conv_channels() + Hv * Dv + 2 * Hv); }  // qkv | z | a | b
  int attn_in_rows() const { return round256(Hq * 2 * D + 2 * Hkv * D); }        // (q|gate) per head | k | v
  int router_rows() const { return round256(E + 1); }                            // experts | shared gate
  int vocab_rows() const { return round256(V); }                                 // lm_head rows
  int z_col() const { return conv_channels(); }
  int a_col() const { return conv_channels() + Hv * Dv; }
  int b_col() const { return a_col() + Hv; }
};

Geom geom_from(const rs_qwen_config& c);

// Checkpoint tensors by name (rs_mlx_weights_load), as the engine's source
// of weights instead of the seeded synthetic ones; shift: the store's norm
// weights are offsets from 1 (native/mlx_bridge.cpp:115, qwen_model.inc:25);
// quant: per-module (group, bits) overrides of the model's default
// (rs_qwen_quant, native/qwen_model.inc:16).
struct NamedWeights {
  std::map<std::string, std::shared_ptr<Tensor>> arrays;
  std::map<std::string, std::pair<int, int>> quant;
  bool shift = false;
};

struct Q4T {  // 4-bit g64 matrix in the tiled layout
  uint32_t* w = nullptr;
  bf16_t* sb = nullptr;
  int N = 0, K = 0;
  size_t bytes() const { return size_t(N) * K / 2 + size_t(N) * (K / 64) * 4; }
};

// A matrix slot held as checkpoint-layout modules instead of a tiled Q4T: any
// of its modules has a (group, bits) other than 64/4. The modules stay in the
// weight store; each fills the output columns [col, col + rows) of the slot.
struct GSlot {
  std::vector<QMod> mods;
  bool on() const { return !mods.empty(); }
};

struct LayerW {
  bool attn = false;
  float *in_norm = nullptr, *post_norm = nullptr;
  Q4T in_proj, out_proj;
  float *conv_w = nullptr, *a_log = nullptr, *dt_bias = nullptr, *gnorm = nullptr;  // DeltaNet
  float *q_norm = nullptr, *k_norm = nullptr;                                       // attention
  Q4T router, gate_up, down;                                                        // MoE (+ shared expert at E)
  GSlot g_in, g_out, g_router, g_gate_up, g_down;  // checkpoint-layout forms (override models)
};

// Tensor ids: the synthetic weights of tensor `id` are generated from seed*1000003+id.
enum TensorSlot : int {
  kTInNorm = 0, kTPostNorm, kTInProj, kTOutProj, kTConvW, kTALog, kTDtBias, kTGNorm, kTQNorm, kTKNorm,
  kTRouter, kTGateUp, kTDown, kTLayerStride = 16
};
int tensor_id(int layer, int slot);      // layer == L means the MTP layer
int tensor_id_global(int which);         // 0 embedding, 1 final norm, 2 lm_head, 3 mtp pre_e, 4 mtp pre_h, 5 mtp fc, 6 mtp norm

struct Weights {
  uint32_t* emb_w = nullptr;  // checkpoint layout [V][H/8]
  bf16_t *emb_s = nullptr, *emb_b = nullptr;
  GSlot g_emb;                // the embedding at another (group, bits)
  std::vector<LayerW> layers;
  float* final_norm = nullptr;
  Q4T lm_head;
  GSlot g_head;
  bool has_mtp = false;
  float *mtp_pre_e = nullptr, *mtp_pre_h = nullptr, *mtp_norm = nullptr;
  Q4T mtp_fc;
  GSlot g_mtp_fc;
  const bf16_t* mtp_fc_dense = nullptr;  // the sidecar's dense BF16 fc [H][2H] (in the store)
  LayerW mtp_layer;
};

struct ProbeStats {
  int launches;
  double ms, tokens, active, bytes;  // summed over launches (bytes: algorithmic HBM bytes)
};

// Operator stages of the diagnostic profile, in the order of the reference's
// OperatorStage (native/operator_timing.h:5-9); the stats export them at
// [17 + 3 i] (calls, host ns, wait ns).
enum class OpStage : int {
  Embedding, InputNorm, RecurrentProjection, RecurrentPrepare, RecurrentUpdate, RecurrentOutput,
  AttentionProjection, AttentionReduction, AttentionOutput, ResidualNorm, MoeRouting, MoeUpGate,
  MoeDown, MoeMixture, MoeShared, MoeMerge, LayerOutput, FinalProjection, StateValidation, Count
};
constexpr int kOpStages = int(OpStage::Count);
struct OpMetrics {
  uint64_t calls = 0, host_ns = 0, wait_ns = 0;
};

// One packed step as the host describes it.
struct StepRows {
  int rows = 0;
  std::vector<int32_t> row_tokens, positions, seq, src_slot, dst_slot, hist_off, log_count;
  std::vector<uint32_t> tokens;
  int total() const;
};

class Engine {
 public:
  // named: checkpoint tensors for the target model (nullptr: seeded synthetic
  // weights); named_mtp: the MTP sidecar's, when mtp is set.
  Engine(const rs_qwen_config& cfg, int max_rows, int max_context, int max_row_tokens, int max_step_tokens,
         uint64_t seed, bool mtp, std::shared_ptr<const NamedWeights> named = nullptr,
         std::shared_ptr<const NamedWeights> named_mtp = nullptr);
  ~Engine();
  Engine(const Engine&) = delete;
  Engine& operator=(const Engine&) = delete;

  const Geom& geom() const { return g_; }
  hipStream_t stream() const { return stream_; }
  size_t weight_bytes() const { return weight_bytes_; }
  size_t state_bytes() const { return state_bytes_; }

  // Regenerates tensor `id` in the checkpoint layout into caller buffers
  // (device). For q4 tensors w/s/b; for f32 vectors only w (as float*).
  void export_tensor(int id, void* w, void* s, void* b);
  // shape of tensor id: N rows, K cols (K = 0 for f32 vectors: N elements); is_q4
  void tensor_shape(int id, int& N, int& K, bool& q4) const;

  // Packed target forward: uploads the step tables, runs the layer program and
  // the final norm (rows at position 0 start from a cleared recurrent state);
  // optional lm_head + selection over `logit_rows` packed token indices (host
  // list). Results stay in the engine's buffers:
  //   hidden_f32() [T][H], logits() [n][V], winners()/margins() [n].
  void forward(const StepRows& s, bool speculative, const std::vector<int32_t>& logit_rows);
  // MTP head forward over packed (token, hidden) pairs at the given positions,
  // with per-row tables like forward(); hidden rows come from `hidden_src`
  // (device f32, ld H) gathered by `hidden_idx` (host list, one per token).
  // Produces logits/winners/margins for `logit_rows` and the head's f32 hidden.
  void mtp_forward(const StepRows& s, const float* hidden_src, const std::vector<int32_t>& hidden_idx,
                   const std::vector<int32_t>& logit_rows);

  // Synthetic context for decode benchmarks: rows 0..n-1 hold positions[r]
  // tokens of seeded random KV / recurrent state / conv history.
  void synthetic_context(int n, const int32_t* positions, uint64_t seed);

  // Residual-stream trace for layer-by-layer checks: when on, forward() keeps
  // x after the embedding and after every layer ([L+1][max_step_tokens][H]
  // f32, slot i = input of layer i), mtp_forward() x after the fc (slot 0)
  // and after its layer (slot 1). The mid trace keeps x after each layer's
  // mixer, before its MoE ([L+1][max_step_tokens][H] f32, slot l for target
  // layer l, slot L for the MTP layer).
  void set_trace(bool on);
  float* trace() const { return trace_; }
  float* mid_trace() const { return mid_trace_; }
  // Live kernel probes: with stride k > 0, HIP events bracket every k-th
  // launch of each probed kernel: kind 0 the grouped MoE gate/up GEMM with
  // SwiGLU, 1 the grouped down GEMM, 2 paged attention with its split
  // combine, 3 the DeltaNet recurrence. A census records the routed experts
  // each sampled gate/up launch touched, and kinds 2 and 3 sum the
  // algorithmic bytes of their sampled launches (from the step's row
  // contexts and token count). Sampling keeps the event records (each stalls
  // the stream for a few microseconds) from perturbing the step being
  // measured. set_profile resets every kind; 0 turns the probes off.
  void set_profile(int stride);
  ProbeStats profile_read(int kind);
  // Operator profile: when on, every stage of a forward is a cut. The host
  // clock is read when the stage's first launch is enqueued (op_begin) and
  // after its last (host ns), then the stream is synchronised (wait ns), as
  // the reference's OperatorInterval does around its eval. Stages fused into
  // a neighbour's kernel are counted where the kernel runs: the input norm of
  // layers after the first and the final norm in the MoE combine (MoeMerge,
  // which also holds the mixture, the shared-expert merge and the residual
  // add), the DeltaNet prep in the fused decode step (RecurrentUpdate), the
  // output gate in the attention combine (AttentionReduction). Off: no clock
  // is read and nothing is synchronised.
  void set_operator_profile(bool on) { op_profile_ = on; }
  bool operator_profile() const { return op_profile_; }
  const std::array<OpMetrics, kOpStages>& operator_metrics() const { return ops_; }
  void op_begin();
  void op_cut(OpStage stage);

  // --- state versions (device sessions) ---
  // Builds the MTP head's weights and KV pool on an engine created without them.
  void enable_mtp(std::shared_ptr<const NamedWeights> named_mtp = nullptr);
  // Number of target attention layers; their KV pools come first, the MTP pool last.
  int attn_layers() const { return n_attn_; }
  int page_count() const { return pages_; }
  // Overwrites block-table row `row` (a sequence slot) with a host page list
  // (at most max_pages entries; the rest of the row keeps stale entries that no
  // context reaches). Synchronous.
  void write_block_row(int row, const std::vector<int32_t>& pages);
  // Copies whole pages, (source, destination) pairs, in every target KV pool
  // (mtp = false) or in the MTP pool. Enqueued on the engine's stream.
  void copy_kv_pages(bool mtp, const std::vector<int32_t>& pairs);
  // Synchronous reads in the reference's state layouts (f32):
  //   DeltaNet layer dn (0-based among DeltaNet layers), recurrent slot `slot`:
  //   conv history [conv-1][C] starting at window row hist_off, state [Hv][Dv][Dk];
  void read_recurrent(int dn, int slot, int hist_off, float* conv, float* state);
  //   KV pool `pool`: K and V [Hkv][context][D] of the first `position`
  //   tokens held in `pages`, zero beyond.
  void read_kv(int pool, const std::vector<int32_t>& pages, int position, int context, float* k, float* v);
  // The inverse imports (synchronous): the window rows [0, conv-1) of `slot`
  // become the conv history (so hist_off = 0), the state is transposed to the
  // device layout, and K/V positions [0, position) are written to `pages`.
  void write_recurrent(int dn, int slot, const float* conv, const float* state);
  void write_kv(int pool, const std::vector<int32_t>& pages, int position, int context, const float* k, const float* v);
  // Per-layer stage trace of a target forward (device f32 [L][5][T][H], T the
  // step's packed tokens): input norm, mixer output, residual, MoE output,
  // layer output. Null turns it off.
  void set_stage_trace(float* buffer) { stage_trace_ = buffer; }

  float* hidden_f32() const { return hn_f32_; }
  float* mtp_hidden_f32() const { return mtp_h_f32_; }
  float* logits() const { return logits_; }  // [n][vocab_rows()], first V columns are the logits
  // False when the last vocabulary-head pass fused the selection and wrote
  // no logits (logits() then holds an earlier pass's values).
  bool logits_valid() const { return logits_valid_; }
  // Vocabulary-head passes that took the fused selection (no logits written).
  uint64_t fused_heads() const { return fused_heads_; }
  uint32_t* winners() const { return winners_; }
  // Off: the vocabulary head may leave logits() unwritten and give only the
  // selection (winners, margins, status), fused into its GEMM when the shape
  // allows. On (the default): logits() is always written.
  void set_logits_export(bool on) { logits_export_ = on; }
  float* margins() const { return margins_; }
  int32_t* sel_status() const { return sel_status_; }
  // winners(), margins() and sel_status() are consecutive regions of
  // max_step_tokens() entries each, starting at winners().
  int max_rows() const { return max_rows_; }
  int max_context() const { return max_context_; }
  int max_row_tokens() const { return max_row_tokens_; }
  int max_step_tokens() const { return max_step_tokens_; }
  bool has_mtp() const { return w_.has_mtp; }
  int max_pages() const { return max_pages_; }
  // Device block table [max_rows][max_pages] (row = sequence slot).
  int32_t* block_table() const { return block_table_; }

 private:
  void alloc_weights();
  void gen_q4(Q4T& m, int id, int N, int K, float std_dev);
  // The tiled form of matrix `id`, or its checkpoint-layout modules (gs) when
  // a named source quantizes any of them other than 4-bit g64.
  void gen_slot(Q4T& m, GSlot& gs, int id, int N, int K);
  float* gen_vec(int id, int n, int kind);  // kind 0 norm (1 + 0.02 N), 1 conv N(0,0.3), 2 U[0,1], 3 zeros
  void upload_tables(const StepRows& s);
  // Rows at position 0 start from a zero recurrent state and conv history.
  void clear_fresh_rows(const StepRows& s);
  void trace_point(int i, int T);
  // A sampled probe times the launches between probe_begin and probe_end
  // through the kernels' own dispatch timestamps: the first timed launch
  // takes the start event, the last (the same one unless probe_last marks
  // another) the stop event. A sample whose events no launch took is dropped.
  void probe_begin(int kind, bool sampled, bool one_launch = true);
  void probe_last(int kind, bool sampled);
  void probe_end(int kind, int tokens, bool sampled, double bytes = 0);
  bool probe_sample(int kind);  // every profile stride-th launch of a kind
  // normed_in: h_ already holds the layer's input norm (fused into the previous
  // layer's MoE combine); next: the norm to fuse into this layer's combine
  void layer_forward(const LayerW& w, int attn_index, int dn_index, int T, int B, int max_t, bool speculative,
                     bool mtp_pool, bool normed_in, const CombineNorm* next);
  // next: the following norm fused into the combine (null: none)
  // cut_norm: the post-attention norm is its own operator stage (target
  // layers; the MTP layer's norms are not cut, as in the reference)
  void moe_block(const LayerW& w, int T, const CombineNorm* next, bool cut_norm);
  void lm_head_select(const bf16_t* h, const std::vector<int32_t>& rows);
  // Projection through a matrix slot: the tiled form, or its checkpoint-layout
  // modules, each into its own output columns.
  // gsum: the group sums of x written with it (see qmm), or null
  void project(const Q4T& m, const GSlot& g, const bf16_t* x, int M, void* y, int out_mode, int ldy,
               const float* gsum = nullptr);
  void embed(int T);  // x_ = the embedding rows of the step's tokens
  // Checkpoint modules of matrix tensor `id` (named sources): name, experts
  // (0: dense), rows per expert, K, first output column.
  struct ModSpec {
    std::string name;
    int lead, rows, K, col;
  };
  std::vector<ModSpec> slot_modules(int id) const;
  const NamedWeights& source_of(int id) const;
  std::pair<int, int> quant_of(const NamedWeights& src, const std::string& module) const;
  // The checkpoint-layout form of tensor `id` when a named source gives any of
  // its modules a (group, bits) other than 64/4; empty otherwise.
  GSlot generic_slot(int id) const;
  void head_select(int n);  // lm_head + selection over the n rows of sel_h_
  void* dalloc(size_t bytes, size_t* counter);

  Geom g_;
  int qgroup_ = 64, qbits_ = 4;  // the model's default quantization (rs_qwen_config group, bits)
  hipStream_t stream_ = nullptr;
  uint64_t seed_;
  std::shared_ptr<const NamedWeights> named_, named_mtp_;  // checkpoint sources (kept for export_tensor)
  void export_named(int id, void* w, void* s, void* b);
  int max_rows_, max_context_, max_row_tokens_, max_step_tokens_, max_pages_, pages_;
  bool mtp_;
  size_t weight_bytes_ = 0, state_bytes_ = 0, work_bytes_ = 0;
  std::vector<void*> allocations_;
  Weights w_;
  // scratch for regenerating checkpoint-layout tensors before tiling
  uint32_t* gen_w_ = nullptr;
  bf16_t *gen_s_ = nullptr, *gen_b_ = nullptr;
  size_t gen_cap_ = 0;
  // pools
  std::vector<float*> dn_state_;
  std::vector<bf16_t*> dn_window_;
  std::vector<float*> dn_log_k_, dn_log_d_, dn_log_g_;
  std::vector<bf16_t*> kc_, vc_;  // per attention layer, then the MTP layer
  int n_attn_ = 0;
  bf16_t** d_pools_ = nullptr;    // device [2 * (n_attn + 1)]: K0, V0, K1, V1, ..., K_mtp, V_mtp
  int32_t* d_pairs_ = nullptr;    // device [2 * max_rows] page pairs
  int pairs_cap_ = 0;
  void alloc_kv_pool();
  void sync_pool_table();
  LayerW make_layer(int l, bool attn);
  void build_mtp_weights();
  int32_t* block_table_ = nullptr;
  // step tables
  int32_t* d_tab_ = nullptr;     // step table block (see the constructor)
  int32_t* sel_block_ = nullptr;  // [winners | margins | status], max_step_tokens each
  int32_t *d_row_tokens_, *d_positions_, *d_seq_, *d_src_, *d_dst_, *d_hist_, *d_logc_, *d_cu_, *d_tok_row_,
      *d_tok_pos_, *d_slot_, *d_ctx_, *d_status_, *d_bt_rows_, *d_sel_idx_;
  uint32_t* d_tokens_;
  // Pinned staging ring: every upload takes the next slot, and a slot is
  // reused only after the copies that read it have executed (one event per
  // slot), so table uploads never drain the stream.
  static constexpr int kStageSlots = 8;
  int32_t* h_pinned_ = nullptr;  // kStageSlots slots of h_pinned_cap_ int32
  size_t h_pinned_cap_ = 0;
  hipEvent_t stage_ev_[kStageSlots] = {};
  bool stage_used_[kStageSlots] = {};
  int stage_next_ = 0, stage_cur_ = 0;
  int32_t* stage_begin();
  void stage_end();
  void upload_index(const std::vector<int32_t>& idx);  // into d_sel_idx_
  // work
  float *x_, *hn_f32_, *mtp_h_f32_, *mtp_in_f32_, *rlog_, *moe_w_, *logits_, *margins_, *attn_wo_, *attn_wml_;
  float *gq_, *gk_, *gv_, *gg_, *gb_;
  float* hgs_ = nullptr;  // per-64-column group sums of h_ from the norm that wrote it (null: hidden % 64 != 0)
  bf16_t *h_, *proj_, *q_, *aout_, *y_, *act_, *dout_, *hn_, *sel_h_;
  int32_t *moe_idx_, *moe_counts_, *moe_offsets_, *moe_order_, *moe_inverse_, *moe_items_, *sel_status_;
  uint32_t* winners_;
  void* sel_ws_ = nullptr;
  void* sel_part_ = nullptr;  // fused selection partials
  size_t sel_part_bytes_ = 0;
  bool logits_export_ = true;
  bool logits_valid_ = false;
  uint64_t fused_heads_ = 0;
  int attn_split_ = 256;
  int32_t* attn_plan_ = nullptr;  // the step's attention piece list
  AttnWork attn_work_{};
  float* trace_ = nullptr;
  bool tracing_ = false;
  float* mid_trace_ = nullptr;
  float* stage_trace_ = nullptr;
  int trace_layer_ = 0;
  static constexpr int kProbeCap = 8192;
  struct Probe {
    std::vector<hipEvent_t> ev;
    int n = 0;
    double tokens = 0, bytes = 0;
    uint64_t calls = 0;  // launches seen, sampled or not
  };
  // 0 grouped gate/up, 1 grouped down, 2 paged attention + combine, 3 DeltaNet recurrence
  static constexpr int kProbes = 4;
  Probe probe_[kProbes];
  // the current step as uploaded: rows, packed tokens, sum of row contexts
  int step_rows_ = 0, step_tokens_ = 0;
  bool step_logs_ = false;  // some row of the step replays a pending speculative log
  // Non-speculative steps whose longest row has at least this many tokens
  // (prefill chunks) run the DeltaNet recurrence in 64-token chunks on MFMA.
  static constexpr int kChunkedRowTokens = 64;
  double step_ctx_sum_ = 0;
  int32_t* census_ = nullptr;
  int profile_stride_ = 0;
  bool op_profile_ = false;
  uint64_t op_start_ = 0;
  std::array<OpMetrics, kOpStages> ops_{};
};

}  // namespace hb
