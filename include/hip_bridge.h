/*
 * hip_bridge: MI355X (gfx950) drop-in for the C ABI of the reference's
 * native/mlx_bridge.h, plus additive device-pointer entry points (hb_*).
 *
 * Conventions (same as native/mlx_bridge.cpp:19-31):
 *   - int-returning calls return 0 on success and -1 on failure; constructors
 *     return NULL on failure;
 *   - the message is copied into the caller's `error` buffer of `capacity`
 *     bytes, truncated and NUL-terminated; no C++ exception crosses the ABI;
 *   - failed calls leave caller outputs untouched;
 *   - handles are owned by the caller and freed only by the matching destroy.
 * Threading: handles are confined to one host thread (native/mlx_bridge.h:7).
 */
#ifndef HIP_BRIDGE_H
#define HIP_BRIDGE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ===================================================================== */
/* Graph API. Replaces native/mlx_bridge.h:8-16 (rs_mlx_create .. version),  */
/* :23 (cleanup), :30-34 (weights, parameter), :41-43 (kernel), :64          */
/* (weight_bytes). Nodes are device tensors; ops execute eagerly on the      */
/* graph's HIP stream; finish synchronises and copies one node to the host.  */
/* dtype codes: 0 f32, 1 i32, 2 u32, 3 f16, 4 bf16 (native/mlx_bridge.cpp:127). */
/* ===================================================================== */
void* rs_mlx_create(int gpu, char* error, size_t capacity);              /* mlx_bridge.h:8  */
void rs_mlx_destroy(void* graph);                                          /* mlx_bridge.h:9  */
int rs_mlx_input(void* graph, int dtype, const void* data, const int32_t* shape, size_t rank, char* error,
                 size_t capacity);                                         /* mlx_bridge.h:10 */
/* op 0 add, 1 multiply, 2 matmul, 3 affine 4-bit qmm, 4 rms_norm,
 * 100+bits affine qmm with `group` (native/mlx_bridge.cpp:56-79). */
int rs_mlx_op(void* graph, int op, const uint32_t* inputs, size_t count, int group, float epsilon, char* error,
              size_t capacity);                                            /* mlx_bridge.h:12 */
int rs_mlx_finish(void* graph, uint32_t output, void* data, size_t elements, char* error,
                  size_t capacity);                                        /* mlx_bridge.h:14 */
const char* rs_mlx_version(void);                                          /* mlx_bridge.h:16 */
void rs_mlx_cleanup(void);                                                 /* mlx_bridge.h:23 */
void* rs_mlx_weights_create(char* error, size_t capacity);                 /* mlx_bridge.h:30 */
void rs_mlx_weights_destroy(void* store);                                  /* mlx_bridge.h:31 */
int rs_mlx_weights_load(void* store, const char* file, char* error, size_t capacity); /* mlx_bridge.h:32 */
/* Host-only check of a safetensors header (the validation rs_mlx_weights_load
 * applies before touching the device); *tensors = tensor count. No reference
 * counterpart (the manifest checks of src/serving/weights.rs:236-301). */
int hb_safetensors_check(const char* file, size_t* tensors, char* error, size_t capacity);
int rs_mlx_parameter(void* graph, void* store, const char* name, const int32_t* shape, size_t rank, int dtype,
                     char* error, size_t capacity);                        /* mlx_bridge.h:33 */
/* op 1 rope, 2 sdpa, 3 gated delta, 4 route top-k, 5 gather qmm, 6 expert mix,
 * 7 silu, 8 flat concat (native/mlx_bridge.cpp:132-174). */
int rs_mlx_kernel(void* graph, int op, const uint32_t* inputs, size_t count, const int32_t* ints, size_t ni,
                  const float* floats, size_t nf, char* error, size_t capacity); /* mlx_bridge.h:41 */
int rs_mlx_weight_bytes(void* store, const char* name, const int32_t* shape, size_t rank, int dtype, size_t offset,
                        uint8_t* output, size_t count, char* error, size_t capacity); /* mlx_bridge.h:64 */

/* ===================================================================== */
/* Model configuration and session API. Replaces native/mlx_bridge.h:50-57, */
/* :71-133. Struct layouts are fixed by the Rust #[repr(C)] mirrors         */
/* (src/serving/native_qwen.rs:62-98, src/serving/model_ir.rs:135-140).     */
/* ===================================================================== */
typedef struct {
  int32_t hidden, layers, vocab, q_heads, kv_heads, head_dim, key_heads, value_heads, key_dim, value_dim, conv,
      interval, experts, top, intermediate, shared, group, bits, context, chunk, rope_dims, activation_precision,
      layer_group, fused_recurrent, execution_timing, compiled_decode, operator_profile, fused_attention,
      validation_mode, validation_interval, expert_kernel;
  float epsilon, theta;
} rs_qwen_config; /* mlx_bridge.h:50-53 (132 bytes) */
typedef struct {
  uint32_t index, mixer;
} rs_qwen_layer; /* mlx_bridge.h:54 */
#ifndef RS_QWEN_STATE_ID_DEFINED
#define RS_QWEN_STATE_ID_DEFINED
typedef struct StateId {
  uint64_t owner, slot, generation, position, bytes;
} StateId; /* native/state_table.h:11 (40 bytes) */
#endif

/* Model entry points (native/mlx_bridge.h:55-57). rs_qwen_quant records a
 * per-module quantisation override in the store (bits 2/3/4/5/6/8, group
 * 32/64/128): checkpoint stores apply it, synthetic stores (4-bit group 64 by
 * construction) refuse it at session creation. rs_qwen_forward is the stateless full-state forward
 * (qwen_forward_core, native/qwen_model.inc:277-373): old_state/new_state in the
 * reference layout of qwen_state_count (:268-271); logits of the last token.
 * gpu must be 1; projection diagnostics are refused. */
int rs_qwen_quant(void* store, const char* module, int group, int bits, char* error, size_t capacity);
int rs_qwen_forward(void* store, int gpu, const rs_qwen_config* config, const rs_qwen_layer* layers,
                    size_t layer_count, const uint32_t* tokens, size_t count, size_t offset, const float* old_state,
                    size_t old_count, float* new_state, size_t new_count, float* logits, size_t logits_count,
                    int projection_checks, const uint32_t* projection_outputs, size_t projection_output_count,
                    float* trace, size_t trace_count, char* error, size_t capacity);

/* Device sessions (native/mlx_bridge.h:71-96; native/qwen_device.inc:5-75).
 * Published StateId versions are immutable; each is released exactly once.
 * Activation profile: config->activation_precision must be 0 (BF16 matrix
 * operands and stored activations, FP32 residual stream, accumulation and
 * recurrent state). Profile 1 (FP32 activations) is refused at creation with a
 * message, here and in rs_qwen_forward, instead of being run in BF16; the
 * reference's FP32-only guards (qwen_batch.inc:5, qwen_mtp.inc:4) therefore
 * admit profile 0 for decode_batch and the MTP operator.
 * A session takes a store marked with hb_weights_synthetic(part 0), or a
 * checkpoint store loaded by rs_mlx_weights_load, and any
 * geometry the kernels support (the reference accepts only its 40-layer
 * checkpoint, qwen_device.inc:27-28). config->chunk bounds the tokens per row
 * and step (<= 64; step/block/hidden calls take at most 8 as in the reference). */
void* rs_qwen_device_create(void* weights, int gpu, const rs_qwen_config* config, const rs_qwen_layer* layers,
                            size_t count, size_t slots, uint64_t bytes, char* error, size_t capacity); /* :76 */
int rs_qwen_device_decode_batch(void* session, const StateId* parents, const uint32_t* tokens, size_t batch,
                                StateId* outputs, float* logits, size_t logits_count, char* error,
                                size_t capacity); /* :77; batch <= slots (the reference stops at 3) */
int rs_qwen_device_step(void* session, const StateId* previous, size_t position, const uint32_t* tokens, size_t count,
                        StateId* output, float* logits, size_t logits_count, float* trace, size_t trace_count,
                        char* error, size_t capacity); /* :78; trace [layers][5][count][hidden] */
int rs_qwen_device_step_sampled(void* session, const StateId* previous, size_t position, const uint32_t* tokens,
                                size_t count, StateId* output, uint32_t* token, char* error, size_t capacity); /* :79 */
int rs_qwen_device_block(void* session, const StateId* previous, size_t position, const uint32_t* tokens,
                         size_t count, StateId* output, float* logits, size_t logits_count, char* error,
                         size_t capacity); /* :81, position-major logits */
int rs_qwen_device_release(void* session, const StateId* id, char* error, size_t capacity);          /* :82 */
int rs_qwen_device_snapshot(void* session, const StateId* id, float* output, size_t count, char* error,
                            size_t capacity);                                                          /* :83 */
int rs_qwen_device_stats(void* session, uint64_t* output, size_t count, char* error, size_t capacity); /* :84, 74 */
int rs_qwen_device_drain(void* session, uint64_t* invalidated, char* error, size_t capacity);         /* :85 */
void rs_qwen_device_destroy(void* session);                                                            /* :86 */
int rs_qwen_device_hidden_step(void* session, const StateId* previous, size_t position, const uint32_t* tokens,
                               size_t count, StateId* output, float* logits, size_t logits_count, char* error,
                               size_t capacity); /* :94 */
int rs_qwen_device_hidden_block(void* session, const StateId* previous, size_t position, const uint32_t* tokens,
                                size_t count, StateId* output, float* logits, size_t logits_count, char* error,
                                size_t capacity); /* :95 */
int rs_qwen_device_hidden_snapshot(void* session, const StateId* id, float* output, size_t count, char* error,
                                   size_t capacity); /* :96 */
/* MTP operator (native/mlx_bridge.h:103-112; native/qwen_mtp.inc:2-63): attach
 * takes a store marked hb_weights_synthetic(part 1) before any admission. */
int rs_qwen_device_mtp_attach(void* session, void* weights, char* error, size_t capacity); /* :103 */
int rs_qwen_device_mtp_step(void* session, const StateId* previous, const StateId* source, int draft_source,
                            size_t row, const uint32_t* tokens, size_t count, StateId* output, float* logits,
                            size_t logits_count, int diagnostics, char* error, size_t capacity); /* :104 */
int rs_qwen_device_mtp_release(void* session, const StateId* id, char* error, size_t capacity); /* :105 */
int rs_qwen_device_mtp_snapshot(void* session, const StateId* id, float* output, size_t count, char* error,
                                size_t capacity); /* :112 */
/* DSpark drafter (native/mlx_bridge.h:120-133): exported stubs that always fail. */
int rs_qwen_device_dspark_step(void* session, const StateId* parent, size_t position, const uint32_t* tokens,
                               size_t count, StateId* output, float* logits, size_t logits_count, int mode,
                               char* error, size_t capacity);
void* rs_qwen_dspark_create(void* session, const char* path, int mode, size_t slots, uint64_t bytes, char* error,
                            size_t capacity);
void rs_qwen_dspark_destroy(void* drafter);
int rs_qwen_dspark_ingest(void* drafter, const StateId* target, const StateId* previous, StateId* output,
                          char* error, size_t capacity);
int rs_qwen_dspark_propose(void* drafter, const StateId* state, uint32_t token, size_t count, uint32_t* tokens,
                           float* scores, size_t capacity_tokens, char* error, size_t capacity);
int rs_qwen_dspark_release(void* drafter, const StateId* id, char* error, size_t capacity);
int rs_qwen_dspark_stats(void* drafter, uint64_t* output, size_t count, char* error, size_t capacity);
int rs_qwen_device_dspark_snapshot(void* session, const StateId* id, float* output, size_t count, char* error,
                                   size_t capacity);

/* Additive session entry points (no counterpart in native/mlx_bridge.h).
 * hb_weights_synthetic marks an rs_mlx_weights_create store as the seeded
 * random-init model (part 0) or its MTP sidecar (part 1); sessions generate
 * the weights on the device from the seed.
 * rs_qwen_device_ragged_step is the ragged generalisation of decode_batch:
 * rows with their own parents (owner 0 = a fresh row at position 0), positions
 * and token counts (1..chunk) in one packed forward. flags: 1 = per-token
 * winners/margins/logits (else the last token of each row), 2 = keep hidden
 * rows for the MTP head. winners/margins get the device greedy selection
 * (IEEE total order, lowest index on ties, margin = top1 - top2); logits are
 * optional (NULL with logits_count 0). */
int hb_weights_synthetic(void* store, uint64_t seed, int part, char* error, size_t capacity);
int rs_qwen_device_ragged_step(void* session, const StateId* parents, const uint32_t* row_tokens, size_t rows,
                               const uint32_t* tokens, size_t total_tokens, int flags, StateId* outputs,
                               uint32_t* winners, float* margins, float* logits, size_t logits_count, char* error,
                               size_t capacity);

/* ===================================================================== */
/* Additive device-pointer API (no counterpart in the reference: these take */
/* HBM-resident operands, which the reference's host-buffer graph API      */
/* cannot express). Pointers are device addresses; `stream` is a           */
/* hipStream_t or NULL for the null stream. bf16 tensors are uint16 bits.  */
/* ===================================================================== */
int hb_device_count(void);
const char* hb_device_name(int device);
void* hb_malloc(size_t bytes, char* error, size_t capacity);
int hb_free(void* ptr);
int hb_memcpy_h2d(void* dst, const void* src, size_t bytes, char* error, size_t capacity);
int hb_memcpy_d2h(void* dst, const void* src, size_t bytes, char* error, size_t capacity);
int hb_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream, char* error, size_t capacity);
int hb_memset(void* ptr, int value, size_t bytes, void* stream, char* error, size_t capacity);
int hb_synchronize(void* stream, char* error, size_t capacity);
void* hb_stream_create(char* error, size_t capacity);
void hb_stream_destroy(void* stream);
void* hb_event_create(char* error, size_t capacity);
void hb_event_destroy(void* event);
int hb_event_record(void* event, void* stream, char* error, size_t capacity);
/* Milliseconds between two recorded events (synchronises on `end`). */
int hb_event_elapsed(void* start, void* end, float* ms, char* error, size_t capacity);

/* Memory-rate probes (no reference counterpart; the benchmark runs them beside
 * the kernels it measures). hb_stream_read reads `bytes` (a multiple of 16)
 * grid-stride with `blocks` workgroups of 256 threads, 16-byte loads
 * (streaming when `nontemporal`), and XOR-folds them into `sink` of
 * hb_stream_read_sink_bytes(blocks) bytes; hb_stream_copy copies with
 * streaming loads and stores. */
size_t hb_stream_read_sink_bytes(int blocks);
int hb_stream_read(const void* src, size_t bytes, void* sink, int blocks, int nontemporal, void* stream,
                   char* error, size_t capacity);
int hb_stream_copy(void* dst, const void* src, size_t bytes, int blocks, void* stream, char* error,
                   size_t capacity);
/* The same probes over contiguous chunks: workgroup b reads (copies) bytes
 * [b chunk_bytes, (b + 1) chunk_bytes), 64 KiB in flight per workgroup, as a
 * kernel owning a block of state per workgroup reads it (chunk_bytes a
 * multiple of 64 KiB, bytes a multiple of chunk_bytes, at most 65536 chunks;
 * the sink takes hb_stream_read_sink_bytes(bytes / chunk_bytes) bytes). */
int hb_stream_read_chunked(const void* src, size_t bytes, size_t chunk_bytes, void* sink, int nontemporal,
                           void* stream, char* error, size_t capacity);
int hb_stream_copy_chunked(void* dst, const void* src, size_t bytes, size_t chunk_bytes, void* stream, char* error,
                           size_t capacity);

/* HIP graph capture of work issued on `stream` (plumbing for launch-bound
 * loops: capture once, replay many times). */
int hb_graph_begin(void* stream, char* error, size_t capacity);
void* hb_graph_end(void* stream, char* error, size_t capacity); /* returns an executable graph */
int hb_graph_launch(void* graph_exec, void* stream, char* error, size_t capacity);
void hb_graph_destroy(void* graph_exec);

/* Repack checkpoint-format 4-bit group-64 weights (u32 [N][K/8], bf16 scales and
 * biases [N][K/64]) into the tiled device layout of the MFMA path: w_tiled has
 * N*K/8 words, sb_tiled 2*N*K/64 bf16 (scale and bias interleaved per tile).
 * Needs N % 16 == 0 and K % 128 == 0. */
int hb_q4_tile(const uint32_t* w, const void* scales, const void* biases, uint32_t* w_tiled, void* sb_tiled, int N,
               int K, void* stream, char* error, size_t capacity);

/* Affine quantised matmul, y[M][N] = x[M][K] . (s*q+b)[N][K]^T.
 * Replaces mx::quantized_matmul at native/qwen_model.inc:34 / mlx_bridge.cpp:72,75.
 * x bf16 [M][K]; y bf16 (y_f32=0) or f32 [M][ldy].
 * layout 0: w u32 [N][K*bits/32] checkpoint stream, scales/biases bf16 [N][K/group];
 * layout 1: 4-bit g64 tiled (hb_q4_tile): w = w_tiled, scales = sb_tiled, biases unused. */
int hb_qmm(const void* x, const uint32_t* w, const void* scales, const void* biases, void* y, int M, int N, int K,
           int group, int bits, int layout, int y_f32, int ldy, void* stream, char* error, size_t capacity);

/* Ragged packing tables for one continuous-batching step (device pointers).
 * Generalises the equal-position concat packer rs_qwen_device_decode_batch
 * (native/qwen_batch.inc:2-50) to rows with different token counts/positions:
 *   cu_seqlens[rows+1] (exclusive prefix sum of row_tokens), token_row[T],
 *   token_pos[T] = positions[r] + j, kv_slot[T] = block_table[r][pos/page]*page + pos%page,
 *   context[rows] = positions[r] + row_tokens[r].
 * status[0] = 1 when a row is malformed or overruns its block table (tables not expanded). */
int hb_pack_tables(const int32_t* row_tokens, const int32_t* positions, const int32_t* block_table, int max_pages,
                   int rows, int page, int32_t* cu_seqlens, int32_t* token_row, int32_t* token_pos, int32_t* kv_slot,
                   int32_t* context, int32_t* status, void* stream, char* error, size_t capacity);

/* Attention input stage (Qwen::attention, native/qwen_model.inc:103-113): per-head
 * RMSNorm of q and k with q_norm/k_norm, partial non-traditional RoPE
 * (native/operator_reference.h:15-18), then k and v appended at kv_slot of the
 * paged cache (K [pages][kv_heads][16][head_dim], V [pages][kv_heads][head_dim][16]).
 * qg bf16 [T][q_heads][2*head_dim] (q then gate), k at kv + i*ld_kv, v at kv + i*ld_kv + kv_off. */
int hb_attn_prep(const void* qg, int ld_qg, const void* kv, int ld_kv, int kv_off, const float* q_norm,
                 const float* k_norm, const int32_t* token_pos, const int32_t* kv_slot, int tokens, int q_heads,
                 int kv_heads, int head_dim, int rotary, float theta, float eps, void* qout, void* kcache,
                 void* vcache, void* stream, char* error, size_t capacity);

/* f32 elements of the split-K workspace work_o: the partial outputs plus the
 * int32 piece list (work_ml needs 2/head_dim of it). */
size_t hb_attn_workspace_floats(int rows, int kv_heads, int head_dim, int max_tokens, int group, int max_context,
                                int split_len);

/* Causal ragged GQA over the paged cache plus sigmoid output gate
 * (native/qwen_model.inc:116-152; FP64 oracle native/attention_reference.h:8-21).
 * q bf16 [T][q_heads][head_dim]; token t of row r sits at context[r]-T_r+t.
 * out bf16 [T][q_heads][head_dim] = softmax(q k^T * scale) v * sigmoid(gate).
 * split_len (keys per split-K piece): a multiple of 32, at most 256. */
int hb_paged_attention(const void* q, const void* kcache, const void* vcache, const int32_t* block_table,
                       int max_pages, const int32_t* cu_seqlens, const int32_t* context, const int32_t* token_row,
                       const void* qg, int ld_qg, int rows, int tokens, int max_tokens, int max_context, int q_heads,
                       int kv_heads, int head_dim, float scale, int split_len, float* work_o, float* work_ml,
                       void* out, void* stream, char* error, size_t capacity);

/* Gated DeltaNet input stage (Qwen::recurrent, native/qwen_model.inc:157-186;
 * native/operator_reference.h:25-34): causal depthwise conv (width `conv`) over
 * the row's committed history and new inputs, SiLU, q/k normalisation
 * (q / (rms*key_dim), k / (rms*sqrt(key_dim)), eps 1e-6), beta = sigmoid(b),
 * decay = exp(-exp(A_log) * softplus(a + dt_bias)).
 * window bf16 [rows][conv-1+max_tokens][channels]: history starts at row
 * hist_off[r]; rewritten as [history | new rows]. Row r reads window slot
 * src_slot[r] and writes slot dst_slot[r] (null: slot r). Outputs f32: q_hat, k_hat
 * [T][key_heads][key_dim], v [T][value_heads][value_dim], decay, beta [T][value_heads]. */
int hb_gdn_prep(const void* qkv, int ld_qkv, const void* a, const void* b, int ld_ab, const float* conv_w,
                const float* a_log, const float* dt_bias, void* window, const int32_t* hist_off,
                const int32_t* src_slot, const int32_t* dst_slot, const int32_t* cu_seqlens, int rows, int key_heads,
                int value_heads, int key_dim, int value_dim, int conv, int max_tokens, float* q_hat, float* k_hat,
                float* v, float* decay, float* beta, void* stream, char* error, size_t capacity);

/* Gated delta recurrence with fp32 state [slots][value_heads][key_dim][value_dim] (key-major)
 * (native/qwen_model.inc:191-200, mlx_bridge.cpp:143-156). A row first replays
 * log_count[r] logged updates (S <- g*S + delta k^T) from its previous
 * speculative step. speculative=1: the state written back is that committed
 * state and this step's per-token (k, delta, g) are logged (log_cap tokens per
 * row); speculative=0: the state after all tokens is written back.
 * Logs: log_k, log_delta f32 [slots][log_cap][value_heads][128], log_g [slots][log_cap][value_heads].
 * State and log of row r are read at slot src_slot[r] and written at dst_slot[r] (null: slot r).
 * o_out (optional) f32 [T][value_heads][value_dim]; y_out (optional) bf16
 * [T][value_heads*value_dim] = rms(o, norm_w, 1e-6) * silu(z) (qwen_model.inc:203-204). */
int hb_gdn_recurrence(const float* q_hat, const float* k_hat, const float* v, const float* decay, const float* beta,
                      const int32_t* cu_seqlens, int rows, int key_heads, int value_heads, int key_dim,
                      int value_dim, float* state, const int32_t* src_slot, const int32_t* dst_slot, float* log_k,
                      float* log_delta, float* log_g, const int32_t* log_count, int log_cap, int speculative,
                      float* o_out, const void* z, int ld_z, const float* norm_w, void* y_out, void* stream,
                      char* error, size_t capacity);

/* hb_gdn_prep followed by hb_gdn_recurrence in one launch (the decode step;
 * no reference counterpart beyond those two): the same arguments without the
 * intermediate q_hat / k_hat / v / decay / beta arrays, bit-identical outputs,
 * state, logs and conv window. Needs conv width 4, 128-wide heads and two value
 * heads per key head; fails with a message otherwise. */
int hb_gdn_decode(const void* qkv, int ld_qkv, const void* a, const void* b, int ld_ab, const float* conv_w,
                  const float* a_log, const float* dt_bias, void* window, const int32_t* hist_off,
                  const int32_t* src_slot, const int32_t* dst_slot, const int32_t* cu_seqlens, int rows, int key_heads,
                  int value_heads, int key_dim, int value_dim, int conv, int max_tokens, float* state, float* log_k,
                  float* log_delta, float* log_g, const int32_t* log_count, int log_cap, int speculative,
                  float* o_out, const void* z, int ld_z, const float* norm_w, void* y_out, void* stream, char* error,
                  size_t capacity);

/* Chunked form of hb_gdn_recurrence for prefill steps (speculative = 0, no
 * pending log): per row, chunks of 64 tokens run as matrix products on MFMA
 * (the chunk's corrected values solve a unit lower-triangular system) instead
 * of 64 dependent token updates. Same recurrence as native/qwen_model.inc:
 * 189-200 (the prefill half of mlx_bridge.cpp:143-156's gated-delta op), same
 * arguments and layouts as hb_gdn_recurrence without the log; results agree
 * with the token-serial kernel to FP32 rounding, not bitwise. */
int hb_gdn_chunked(const float* q_hat, const float* k_hat, const float* v, const float* decay, const float* beta,
                   const int32_t* cu_seqlens, int rows, int key_heads, int value_heads, int key_dim, int value_dim,
                   float* state, const int32_t* src_slot, const int32_t* dst_slot, float* o_out, const void* z,
                   int ld_z, const float* norm_w, void* y_out, void* stream, char* error, size_t capacity);

/* Seeded synthetic data on the device (random-init weights and inputs; the
 * reference quantises nothing at run time). Counter-based generator: element i
 * of (seed) is reproducible independently of launch shape.
 * hb_random_q4: W [N][K] ~ N(0, std) quantised affine 4-bit g64 (scale =
 * (max-min)/15, bias = min, both bf16) into w u32 [N][K/8], s/b bf16 [N][K/64].
 * dtype: 0 f32, 4 bf16. */
int hb_random_q4(uint64_t seed, int N, int K, float std_dev, uint32_t* w, void* scales, void* biases, void* stream,
                 char* error, size_t capacity);
int hb_random_normal(uint64_t seed, size_t n, float std_dev, float mean, int dtype, void* out, void* stream,
                     char* error, size_t capacity);
int hb_random_uniform(uint64_t seed, size_t n, float lo, float hi, int dtype, void* out, void* stream, char* error,
                      size_t capacity);
int hb_random_ints(uint64_t seed, size_t n, uint32_t bound, uint32_t* out, void* stream, char* error,
                   size_t capacity);

/* MoE router (native/qwen_model.inc:77-81; mlx_bridge.cpp:157-163 kernel op 4):
 * per token the top-k of logits[t][0..experts) under IEEE total order (lower
 * expert index first on ties; MLX argpartition leaves that order open), weights
 * = softmax renormalised over the selection; then the stable counting sort of
 * the (token, slot) pairs by expert: order[offsets[e]+i] = i-th pair of expert e,
 * inverse[p] = position of pair p, counts[e], offsets[experts+1]. tokens*top <= 4096. */
int hb_moe_route(const float* logits, int ld_logits, int tokens, int experts, int top, int32_t* idx, float* weights,
                 int32_t* counts, int32_t* offsets, int32_t* order, int32_t* inverse, int32_t* items, void* stream,
                 char* error, size_t capacity);
/* Capacity (int32 elements) of the work list hb_moe_route writes to `items`:
 * items[0] = count, then slot << 16 | tile per 16-row tile, the shared
 * expert's token tiles (slot 0) first, then each routed expert e's pair tiles
 * (slot e + 1). */
size_t hb_moe_items_capacity(int tokens, int experts, int top);

/* Grouped affine 4-bit GEMM over the routed experts plus the shared expert
 * (gather_qmm at native/qwen_model.inc:36-41,89; shared expert :97). Weights are
 * [experts+1] tiled matrices of n_rows x K (hb_q4_tile), index `experts` being the
 * shared expert. swiglu=1: x bf16 [tokens][K], rows of each 16-row tile are 8 gate
 * then the 8 matching up rows, y bf16 [P+tokens][n_rows/2] = silu(gate)*up;
 * swiglu=0: x bf16 [P+tokens][K] in sorted pair order, y bf16 [P+tokens][n_rows].
 * Routed rows are in sorted pair order (P = tokens*top), shared rows at P+token. */
int hb_moe_grouped_qmm(const void* x, int K, const uint32_t* w_tiled, const void* sb_tiled, int n_rows,
                       const int32_t* counts, const int32_t* offsets, const int32_t* order, const int32_t* items,
                       int experts, int top, int tokens, int swiglu, void* y, void* stream, char* error,
                       size_t capacity);

/* residual[t] += sum_j weights[t][j]*down[inverse[t*top+j]] + sigmoid(logits[t][sg_col])*down[P+t]
 * (mixture and shared-expert merge, native/qwen_model.inc:95-98; mlx_bridge.cpp:167). */
int hb_moe_combine(const void* down, const float* weights, const int32_t* inverse, const float* logits, int ld_logits,
                   int sg_col, int top, int tokens, int hidden, float* residual, void* stream, char* error,
                   size_t capacity);

/* Greedy selection per row of logits f32 [rows][ld] over `vocab` columns:
 * winner under f32 total order (lowest index on ties), margin = top1 - top2
 * (+inf for one column), status 1 for a row with a non-finite value.
 * Replaces the host scans winner_with_margin (src/serving/native_speculative.rs:45-73)
 * and device_total_argmax (native/selection.h:5-13). */
int hb_argmax_margin(const float* logits, int ld, int rows, int vocab, uint32_t* winner, float* margin,
                     int32_t* status, void* workspace, void* stream, char* error, size_t capacity);
/* Optional workspace of hb_argmax_margin (device, bytes): with it, long rows
 * are scanned by several workgroups and merged in column order. */
size_t hb_argmax_workspace_bytes(int rows, int vocab);
/* No counterpart in the reference. hb_argmax_margin with its multi-workgroup
 * scan, for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): the
 * per-(row, 8192-column chunk) partial summaries live in a static device array
 * of hb_argmax_noalloc_limit_bytes() = 1 MiB per GPU instead of a workspace.
 * Fails when rows * ceil(vocab / 8192) * 16 exceeds it. Allocates nothing;
 * every entry read is written by the same call. Calls that overlap on one GPU
 * (concurrent streams or threads) race on the array. */
int hb_argmax_margin_noalloc(const float* logits, int ld, int rows, int vocab, uint32_t* winner, float* margin,
                             int32_t* status, void* stream, char* error, size_t capacity);
size_t hb_argmax_noalloc_limit_bytes(void);
/* The same selection fused into the vocabulary head: over the logits
 * x (bf16 [rows][K]) . W^T of a tiled 4-bit W ([n][K], n % 256 == 0), columns
 * [0, vocab), without writing them; the lm_head epilogue fusion the reference
 * plans for device_total_argmax (docs/NATIVE_TUNING_PLAN.md:898). *fused = 0
 * (nothing launched, outputs untouched) for shapes the fused kernel does not
 * cover: 16 < rows <= 256, K = 2048, enough work to fill the GPU.
 * workspace: hb_qmm_select_workspace_bytes(rows, n) device bytes. */
int hb_qmm_select(const void* x, int rows, int K, const uint32_t* w_tiled, const void* sb_tiled, int n, int vocab,
                  void* workspace, size_t workspace_bytes, uint32_t* winner, float* margin, int32_t* status,
                  int* fused, void* stream, char* error, size_t capacity);
size_t hb_qmm_select_workspace_bytes(int rows, int n);
/* MTP acceptance per row (plan(), src/serving/native_speculative.rs:74-128):
 * draft [rows][max_draft] with n_draft[r] used, target [rows][max_draft+1]
 * (target[r][0] = winner of the initial logits, target[r][i] = winner of verify
 * row i-1), eos [n_eos], remaining [rows] -> emitted [rows][max_draft+1],
 * n_emitted, accepted, terminal; status 1 marks a malformed row. */
int hb_mtp_plan(const uint32_t* draft, const int32_t* n_draft, int max_draft, const uint32_t* target,
                const uint32_t* eos, int n_eos, const int32_t* remaining, int rows, int vocab, uint32_t* emitted,
                int32_t* n_emitted, int32_t* accepted, int32_t* terminal, int32_t* status, void* stream,
                char* error, size_t capacity);
/* Embedding rows: out f32 [count][hidden] = s*q + b of the 4-bit g64 rows
 * tokens[i] (checkpoint layout; native/qwen_model.inc:306-309). */
int hb_embed_gather(const uint32_t* tokens, int count, const uint32_t* w, const void* scales, const void* biases,
                    int hidden, float* out, void* stream, char* error, size_t capacity);
/* RMSNorm of f32 rows into bf16 (and optionally f32): x*rsqrt(mean x^2 + eps)*w
 * (Qwen::norm, native/qwen_model.inc:19-32). */
int hb_rmsnorm(const float* x, int ld_x, const float* weight, int rows, int hidden, float epsilon, void* out,
               int ld_out, float* out_f32, void* stream, char* error, size_t capacity);
/* The same RMSNorm writing also the per-64-column group sums of each bf16
 * output row, gsum f32 [rows][hidden / 64] (hidden % 64 == 0), in the fixed
 * order the 4-bit projections use, and hb_qmm (tiled layout) reading them
 * instead of recomputing them: the decoder's input norm feeds its
 * in-projection this way (no reference counterpart: an internal fusion of
 * Qwen::norm and the quantized matmul, native/qwen_model.inc:19-34). Outputs
 * are bit-identical to hb_rmsnorm and hb_qmm. */
int hb_rmsnorm_gs(const float* x, int ld_x, const float* weight, int rows, int hidden, float epsilon, void* out,
                  int ld_out, float* gsum, void* stream, char* error, size_t capacity);
int hb_qmm_gs(const void* x, const uint32_t* w_tiled, const void* sb_tiled, void* y, int M, int N, int K,
              int out_mode, int ld_y, const float* gsum, void* stream, char* error, size_t capacity);

/* ===================================================================== */
/* Decode engine: the hybrid decoder's device-resident weights (seeded     */
/* synthetic 4-bit), per-sequence state pools and the packed ragged        */
/* forward (qwen_forward_core, native/qwen_model.inc:277-373; batched      */
/* packer native/qwen_batch.inc:2-50; MTP head native/qwen_mtp.inc:8-56).  */
/* Geometry-generic over rs_qwen_config; hidden and intermediate multiples  */
/* of 128, head_dim 256, key/value dims 128.                              */
/* ===================================================================== */
void* hb_engine_create(const rs_qwen_config* config, int max_rows, int max_context, int max_row_tokens,
                       int max_step_tokens, uint64_t seed, int mtp, char* error, size_t capacity);
/* The same engine over checkpoint tensors held by rs_mlx_weights_load stores
 * (the target's, and the MTP sidecar's or NULL): each engine tensor is
 * assembled from the named MLX tensors (qwen_model.inc:34-206, qwen_mtp.inc:
 * 37-45) and tiled. No reference counterpart: the engine-level entry that the
 * loader's parity tests use. */
void* hb_engine_create_named(const rs_qwen_config* config, int max_rows, int max_context, int max_row_tokens,
                             int max_step_tokens, void* weights, void* mtp_weights, char* error, size_t capacity);
void hb_engine_destroy(void* engine);
/* out[0..count) of: weight bytes, state bytes, pages per sequence, hipStream_t,
 * vocabulary-head passes that fused the selection (count >= 4). */
int hb_engine_info(void* engine, uint64_t* out, size_t count, char* error, size_t capacity);
/* out[0] = vocabulary-head passes of a rs_qwen_device_create session that fused
 * the greedy selection (count >= 1). No reference counterpart: a diagnostic
 * beside rs_qwen_device_stats, whose 74-entry layout is the reference's. */
int hb_session_info(void* session, uint64_t* out, size_t count, char* error, size_t capacity);
/* Tensor ids: 0 embedding, 1 final norm, 2 lm_head, 3/4 MTP pre-fc norms
 * (embedding, hidden), 5 MTP fc, 6 MTP norm; 16 + 16*layer + slot for layer
 * tensors (layer == layers is the MTP layer), slots 0 input norm, 1 post norm,
 * 2 in-projection, 3 out-projection, 4 conv weight [C][conv], 5 A_log,
 * 6 dt_bias, 7 gated-norm weight, 8 q norm, 9 k norm, 10 router, 11 expert
 * gate/up [(E+1)*2I][H], 12 expert down [(E+1)*H][I]. */
int hb_engine_tensor_shape(void* engine, int id, int32_t* rows, int32_t* cols, int32_t* q4, char* error,
                           size_t capacity);
/* Regenerates tensor `id` in checkpoint layout into device buffers (4-bit:
 * w u32 [rows][cols/8], scales and biases bf16 [rows][cols/64]; else f32 w). */
int hb_engine_export(void* engine, int id, void* w, void* scales, void* biases, char* error, size_t capacity);
/* One packed target forward. Per row: row_tokens, positions (tokens already in
 * the state), seq (sequence slot: KV pages), src/dst recurrent slots (null =
 * seq), hist_off / log_count (rows committed by the previous speculative step;
 * null = 0). speculative != 0 logs this step's recurrent updates instead of
 * committing them. Logits, winners and margins for the packed token indices
 * logit_rows (read back with hb_engine_read). */
int hb_engine_forward(void* engine, int rows, const int32_t* row_tokens, const int32_t* positions, const int32_t* seq,
                      const int32_t* src_slot, const int32_t* dst_slot, const int32_t* hist_off,
                      const int32_t* log_count, const uint32_t* tokens, int speculative, const int32_t* logit_rows,
                      int n_logit_rows, char* error, size_t capacity);
/* MTP head over packed (token, hidden row) pairs; hidden rows are taken from
 * the last target forward (hidden_source 0) or the last MTP forward (1). */
int hb_engine_mtp_forward(void* engine, int rows, const int32_t* row_tokens, const int32_t* positions,
                          const int32_t* seq, const uint32_t* tokens, int hidden_source, const int32_t* hidden_idx,
                          const int32_t* logit_rows, int n_logit_rows, char* error, size_t capacity);
/* which: 0 hidden f32 [T][H], 1 MTP hidden f32 [T][H], 2 logits f32 [n][V]
 * (fails when the last head pass fused the selection and wrote none),
 * 3 winners u32 [n], 4 margins f32 [n], 5 selection status i32 [n],
 * 6 residual trace f32 [layers+1][max_step_tokens][H] (layer inputs, then the
 * output), 7 mid trace f32 [layers+1][max_step_tokens][H] (each layer's
 * residual after its mixer, before its MoE; slot `layers` = the MTP layer). */
int hb_engine_read(void* engine, int which, size_t offset, void* out, size_t bytes, char* error, size_t capacity);
/* Residual-stream trace (the reference's per-layer trace of rs_qwen_forward,
 * native/mlx_bridge.h:56): when enabled, forward keeps x after the embedding
 * and after each layer, the MTP forward x after its fc and after its layer. */
int hb_engine_trace(void* engine, int enable, char* error, size_t capacity);
/* Live kernel probes: with stride k > 0, HIP events on the engine's stream
 * around every k-th launch of each kind: 0 grouped MoE gate/up + SwiGLU,
 * 1 grouped down, 2 paged attention + split combine, 3 DeltaNet recurrence;
 * a census of the routed experts each sampled gate/up launch touched (0 turns
 * the probes off; enabling resets them). read: out[0..count) of launches,
 * summed ms, summed tokens, summed experts touched (kinds 0-1), summed
 * algorithmic HBM bytes (kinds 2-3; count >= 5). */
int hb_engine_profile(void* engine, int stride, char* error, size_t capacity);
int hb_engine_profile_read(void* engine, int kind, double* out, size_t count, char* error, size_t capacity);
/* Seeded synthetic context (KV, recurrent state, conv history) standing in
 * for prompts of positions[r] tokens in sequence slots 0..rows-1. */
int hb_engine_synthetic_context(void* engine, int rows, const int32_t* positions, uint64_t seed, char* error,
                                size_t capacity);

/* Continuous-batching greedy decode with MTP speculation over an engine
 * (mtp_prepare / mtp_commit, src/serving/native_mtp_decode.rs:124-295):
 * width = block width (drafts + 1), gate_margin = draft margin gate (1.25). */
void* hb_decode_create(void* engine, int width, float gate_margin, const uint32_t* eos, int n_eos, char* error,
                       size_t capacity);
void hb_decode_destroy(void* loop);
/* hist_off = row count of the last forward that wrote the sequence's conv
 * window (its last prefill chunk; 0 after hb_engine_synthetic_context). */
int hb_decode_admit(void* loop, int seq, int position, uint32_t pending, int budget, int hist_off, char* error,
                    size_t capacity);
int hb_decode_set_drafts(void* loop, int seq, const uint32_t* tokens, int count, char* error, size_t capacity);
int hb_decode_step(void* loop, int32_t* emitted, char* error, size_t capacity);
/* stats[0..9): steps, emitted, target tokens, proposed, accepted, MTP calls,
 * MTP tokens, finished rows, live rows */
int hb_decode_stats(void* loop, uint64_t* stats, size_t count, char* error, size_t capacity);
int hb_decode_output(void* loop, int seq, uint32_t* tokens, size_t capacity_tokens, int32_t* count,
                     int32_t* position, char* error, size_t capacity);

#ifdef __cplusplus
}
#endif
#endif
