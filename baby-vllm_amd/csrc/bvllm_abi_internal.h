// Argument blocks passed from the C-ABI entry points to the kernel launchers.
// All strides are in elements. Tensors are bf16 unless noted.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bvllm {

struct RopeArgs {
  void* q;        int64_t q_st, q_sh;      // [T, H, D], last-dim stride 1
  void* k;        int64_t k_st, k_sh;      // [T, Hkv, D]
  const void* v;  int64_t v_st, v_sh;      // [T, Hkv, D]
  const void* cos; int64_t cs_st;          // [T, D]
  const void* sin; int64_t sn_st;          // [T, D]
  void* k_cache;  int64_t kc_slot, kc_head;  // flat [NB·BS, Hkv, D] view of kv_cache[0]
  void* v_cache;  int64_t vc_slot, vc_head;  // flat view of kv_cache[1]
  const int64_t* slot_mapping;             // [T]
  int64_t num_slots;                       // NB·BS; slots outside [0, num_slots) are not written
  int32_t num_tokens, num_heads, num_kv_heads, head_dim;
  int32_t has_cache;
  int32_t vec_ok;                          // every row start and stride is 16-byte aligned
};

struct DecodeArgs {
  const void* q;  int64_t q_sb, q_sh;      // [B, H, D]
  const void* k_cache; const void* v_cache;  // [NB, BS, Hkv, D] each
  int64_t c_sb, c_st, c_sh;                // page, token, head strides (shared by K and V)
  int32_t num_pages;                       // NB; table entries are clamped into [0, NB)
  const int32_t* block_tables; int64_t bt_stride; int32_t max_blocks;
  const int32_t* seq_lens;                 // [B]
  float scale_log2;                        // softmax scale · log2(e)
  void* out;      int64_t o_sb, o_sh;      // [B, H, D], written when num_splits == 1
  float* part_out;                         // [B, H, parts, D] fp32 partial outputs
  float* part_lse;                         // [B, H, parts] fp32 (log2 units)
  int32_t num_splits, blocks_per_split;
  int32_t batch, num_heads, num_kv_heads, head_dim;
  int32_t waves;                           // waves per single-pass work-group (4; 0 = default)
  // Set by the launcher for split launches (decode_plan):
  int32_t splits_per_item;                 // consecutive splits one streaming wave computes
  int32_t num_partials;                    // partial states per (row, head) the launch writes
  int32_t ws_partials;                     // partial states per (row, head) the workspace holds
  int32_t item_order;                      // 0: KV head fastest in the wave numbering; 1: split unit fastest
  // Prefill view (both null for a decode batch): row b is sequence b of a
  // varlen prefill batch. Only sequences with exactly one query token are
  // computed; their q / out row is query_start_loc[b] and they attend keys
  // 0 .. min(seq_lens[b], context_lens[b] + 1) - 1.
  const int32_t* query_start_loc;
  const int32_t* context_lens;
};

struct PrefillArgs {
  const void* q;  int64_t q_st, q_sh;      // [T, H, D]
  const void* k_cache; const void* v_cache;
  int64_t c_sb, c_st, c_sh;
  int32_t num_pages;
  const int32_t* block_tables; int64_t bt_stride; int32_t max_blocks;
  const int32_t* query_start_loc;          // [S+1]
  const int32_t* seq_lens;                 // [S]
  const int32_t* context_lens;             // [S]
  float scale_log2;
  void* out;      int64_t o_st, o_sh;      // [T, H, D]
  int32_t num_seqs, num_tokens, max_query_len;
  int32_t num_heads, num_kv_heads, head_dim;
  // Sequences with exactly one query token: -1 = unknown, 0 = none. When not 0
  // those sequences run on the decode kernel and the prefill kernel skips them.
  int32_t single_query_seqs;
};

struct ArgmaxArgs {
  const void* logits; int64_t row_stride;  // [rows, vocab], unit column stride
  int32_t rows, vocab;
  int32_t fp32;                            // 1: fp32 logits, 0: bf16
  int32_t vec_ok;                          // 16-byte loads cover whole rows exactly
  void* workspace;                         // argmax_workspace_bytes(rows, vocab)
  int64_t* out;                            // [rows]
};

struct NormArgs {
  const void* input; int64_t in_stride;    // [rows, n] bf16
  void* residual;    int64_t res_stride;   // [rows, n] bf16 or null; receives input + residual
  const void* weight;                      // [n], bf16 or fp32
  int32_t weight_fp32;
  void* out;         int64_t out_stride;   // [rows, n] bf16
  int32_t rows, n;
  float eps;
  int32_t vec_ok;                          // 16-byte aligned rows, n % 8 == 0
};

struct SiluArgs {
  const void* gate_up;                     // [rows, 2d] bf16, contiguous
  void* out;                               // [rows, d] bf16, contiguous
  int64_t rows;
  int32_t d;
  int32_t vec_ok;                          // 16-byte aligned, d % 8 == 0
};

hipError_t rope_kv_append(const RopeArgs& a, hipStream_t stream);
int64_t argmax_workspace_bytes(int32_t rows, int32_t vocab);
hipError_t greedy_argmax(const ArgmaxArgs& a, hipStream_t stream);
hipError_t fused_add_rms_norm(const NormArgs& a, hipStream_t stream);
hipError_t silu_mul(const SiluArgs& a, hipStream_t stream);
hipError_t paged_decode(const DecodeArgs& a, hipStream_t stream);

// How a decode launch with the caller's split plan runs (paged_decode.hip).
struct DecodePlan {
  bool single_pass;        // one split: single-pass work-groups, no workspace
  int32_t group;           // consecutive splits folded into one partial (level 2 of the merge)
  int32_t splits_per_item; // splits per streaming wave: 1, or `group` when the wave folds them
  int32_t partials;        // partial states per (row, head) in the workspace
  bool fold_in_reduce;     // the reduce folds the per-split partials into groups
  bool pair;               // one split or group per work-group of two waves (two states each)
  bool quad;               // (with pair) one split of at most 32 pages per work-group of four waves
};
DecodePlan decode_plan(int32_t batch, int32_t num_kv_heads, int32_t num_splits, int32_t blocks_per_split);
// Column groups of a decode launch: its KV heads, each cut into ceil(G / 16)
// groups of at most 16 query heads (one MFMA tile of columns) when G > 16.
inline int64_t decode_col_groups(const DecodeArgs& a) {
  const int G = a.num_heads / a.num_kv_heads;
  return (int64_t)a.num_kv_heads * ((G + 15) / 16);
}
// Partial states per (row, head) the decode workspace holds: the most any
// plan of these splits writes, independent of the tuning knobs.
int32_t decode_partials(int32_t batch, int32_t num_kv_heads, int32_t num_splits, int32_t blocks_per_split);

// Process-wide tuning switches (bvllm_set_tuning). Knob values: 0 = default.
enum TuneKnob {
  kTuneDecodeSplitMode = 0,         // 1: one wave per split, 2: one wave per group of splits, 3: two
                                    // waves per group, 4: two waves per split also for splits of at most
                                    // 32 pages (same bits); by default single splits run on four waves
                                    // (at most 32 pages) or two, groups on two waves when at most one
                                    // group per CU
  kTunePrefillBlocksPerWg = 1,      // n > 0: prefill column blocks per work-group when the table allows it
  kTuneDecodeOrder = 2,             // 1: split units fastest in the streaming wave numbering (same bits)
  kTuneDecodeSinglePassStream = 3,  // 1: single-pass launches on streaming waves too (same bits)
  kTuneDecodeCached = 4,            // 1: streaming page loads without the nontemporal hint (same bits)
  kTuneAppendChunks = 5,            // 1: aligned appends on the per-chunk kernel (same bits, NaN payloads aside)
  kTunePrefillShortGrid = 6,        // 1: short prefill grids on the single key walk instead of the key split
  kTuneKnobs = 7,
};
int tuning(int knob);
int set_tuning(int knob, int value);
hipError_t paged_prefill(const PrefillArgs& a, hipStream_t stream);
// Compute units of the current device (cached per device).
int device_cus();

}  // namespace bvllm
