// C-ABI entry points: argument validation and packing, then the launchers.
#include "../../include/babyvllm_amd.h"
#include "bvllm_abi_internal.h"
#include "bvllm_device.h"

#include <algorithm>

using namespace bvllm;

namespace {

constexpr int kBad = (int)hipErrorInvalidValue;

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

bool valid_heads(int32_t h, int32_t hkv) { return h > 0 && hkv > 0 && h % hkv == 0; }

}  // namespace

extern "C" int bvllm_abi_version(void) { return BVLLM_ABI_VERSION; }

extern "C" const char* bvllm_error_string(int code) {
  if (code == kBad) return "invalid argument (rejected by babyvllm_amd)";
  if (code == BVLLM_ERROR_SCRATCH_LIMIT)
    return "decode split scratch exceeds BVLLM_NOALLOC_SCRATCH_BYTES (use bvllm_paged_decode with a workspace)";
  return hipGetErrorString((hipError_t)code);
}

extern "C" int bvllm_rope_kv_append(void* q, int64_t q_stride_t, int64_t q_stride_h,
                                    void* k, int64_t k_stride_t, int64_t k_stride_h,
                                    const void* v, int64_t v_stride_t, int64_t v_stride_h,
                                    const void* cos, int64_t cos_stride_t,
                                    const void* sin, int64_t sin_stride_t,
                                    void* k_cache, void* v_cache,
                                    int64_t cache_stride_slot, int64_t cache_stride_head,
                                    int64_t num_slots, const int64_t* slot_mapping,
                                    int32_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
                                    int32_t head_dim, void* stream) {
  if (num_tokens < 0 || !valid_heads(num_heads, num_kv_heads)) return kBad;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return kBad;
  if (num_tokens == 0) return 0;
  if (!q || !k || !cos || !sin) return kBad;
  const bool has_cache = k_cache != nullptr;
  if (has_cache && (!v_cache || !v || !slot_mapping || num_slots <= 0)) return kBad;

  RopeArgs a{};
  a.q = q; a.q_st = q_stride_t; a.q_sh = q_stride_h;
  a.k = k; a.k_st = k_stride_t; a.k_sh = k_stride_h;
  a.v = v; a.v_st = v_stride_t; a.v_sh = v_stride_h;
  a.cos = cos; a.cs_st = cos_stride_t;
  a.sin = sin; a.sn_st = sin_stride_t;
  a.k_cache = k_cache; a.kc_slot = cache_stride_slot; a.kc_head = cache_stride_head;
  a.v_cache = v_cache; a.vc_slot = cache_stride_slot; a.vc_head = cache_stride_head;
  a.slot_mapping = slot_mapping;
  a.num_slots = num_slots;
  a.num_tokens = num_tokens; a.num_heads = num_heads; a.num_kv_heads = num_kv_heads;
  a.head_dim = head_dim;
  a.has_cache = has_cache ? 1 : 0;

  bool vec = aligned16(q) && aligned16(k) && aligned16(cos) && aligned16(sin) &&
             q_stride_t % 8 == 0 && q_stride_h % 8 == 0 && k_stride_t % 8 == 0 && k_stride_h % 8 == 0 &&
             cos_stride_t % 8 == 0 && sin_stride_t % 8 == 0;
  if (has_cache)
    vec = vec && aligned16(v) && aligned16(k_cache) && aligned16(v_cache) && v_stride_t % 8 == 0 &&
          v_stride_h % 8 == 0 && cache_stride_slot % 8 == 0 && cache_stride_head % 8 == 0;
  a.vec_ok = vec ? 1 : 0;
  return (int)rope_kv_append(a, (hipStream_t)stream);
}

extern "C" int64_t bvllm_decode_workspace_bytes(int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                                int32_t head_dim, int32_t num_splits,
                                                int32_t blocks_per_split) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_splits < 1 || blocks_per_split < 1) return 0;
  const int64_t parts = decode_partials(batch, num_kv_heads, num_splits, blocks_per_split);
  if (parts <= 0) return 0;
  const int64_t rows = (int64_t)batch * num_heads * parts;
  return rows * head_dim * (int64_t)sizeof(float) + rows * (int64_t)sizeof(float);
}

static bool cache_ok(const void* kc, const void* vc, int64_t sb, int64_t st, int64_t sh, int32_t nb) {
  // The page stride is a 32-bit factor of the kernels' page-offset products.
  return kc && vc && nb > 0 && aligned16(kc) && aligned16(vc) && sb % 8 == 0 && st % 8 == 0 &&
         sh % 8 == 0 && sb > 0 && st > 0 && sh > 0 && sb <= 0x7fffffff;
}

extern "C" int bvllm_paged_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                  const void* k_cache, const void* v_cache,
                                  int64_t cache_stride_block, int64_t cache_stride_tok,
                                  int64_t cache_stride_head, int32_t num_blocks,
                                  const int32_t* block_tables, int64_t bt_stride, int32_t max_blocks,
                                  const int32_t* seq_lens, float scale,
                                  void* out, int64_t out_stride_b, int64_t out_stride_h,
                                  void* workspace, int32_t num_splits, int32_t blocks_per_split,
                                  int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                  int32_t head_dim, int32_t block_size, int32_t waves, void* stream) {
  if (batch < 0 || !valid_heads(num_heads, num_kv_heads)) return kBad;
  if (head_dim != 64 && head_dim != 128) return kBad;
  if (block_size != 16) return kBad;
  if (batch == 0) return 0;
  if (!q || !out || !block_tables || !seq_lens) return kBad;
  if (!cache_ok(k_cache, v_cache, cache_stride_block, cache_stride_tok, cache_stride_head, num_blocks))
    return kBad;
  if (!aligned16(q) || !aligned16(out) || q_stride_b % 8 || q_stride_h % 8 || out_stride_b % 8 ||
      out_stride_h % 8)
    return kBad;
  if (max_blocks < 1 || bt_stride < max_blocks) return kBad;
  if (num_splits < 1 || blocks_per_split < 1) return kBad;
  // Offsets inside one page are 32-bit.
  if ((int64_t)16 * cache_stride_tok > 0x7fffffff) return kBad;
  const int64_t ws_bytes = bvllm_decode_workspace_bytes(batch, num_heads, num_kv_heads, head_dim, num_splits,
                                                        blocks_per_split);
  if (ws_bytes > 0 && (!workspace || !aligned16(workspace))) return kBad;
  if (waves != 0 && waves != 4) return kBad;

  DecodeArgs a{};
  a.q = q; a.q_sb = q_stride_b; a.q_sh = q_stride_h;
  a.k_cache = k_cache; a.v_cache = v_cache;
  a.c_sb = cache_stride_block; a.c_st = cache_stride_tok; a.c_sh = cache_stride_head;
  a.num_pages = num_blocks;
  a.block_tables = block_tables; a.bt_stride = bt_stride; a.max_blocks = max_blocks;
  a.seq_lens = seq_lens;
  a.scale_log2 = scale * kLog2e;
  a.out = out; a.o_sb = out_stride_b; a.o_sh = out_stride_h;
  if (ws_bytes > 0) {
    a.ws_partials = decode_partials(batch, num_kv_heads, num_splits, blocks_per_split);
    const int64_t rows = (int64_t)batch * num_heads * a.ws_partials;
    a.part_out = reinterpret_cast<float*>(workspace);
    a.part_lse = a.part_out + rows * head_dim;
  }
  a.num_splits = num_splits; a.blocks_per_split = blocks_per_split;
  a.batch = batch; a.num_heads = num_heads; a.num_kv_heads = num_kv_heads; a.head_dim = head_dim;
  a.waves = waves;
  return (int)paged_decode(a, (hipStream_t)stream);
}

extern "C" int bvllm_paged_prefill(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                   const void* k_cache, const void* v_cache,
                                   int64_t cache_stride_block, int64_t cache_stride_tok,
                                   int64_t cache_stride_head, int32_t num_blocks,
                                   const int32_t* block_tables, int64_t bt_stride, int32_t max_blocks,
                                   const int32_t* query_start_loc, const int32_t* seq_lens,
                                   const int32_t* context_lens, float scale,
                                   void* out, int64_t out_stride_t, int64_t out_stride_h,
                                   int32_t num_seqs, int32_t num_tokens, int32_t max_query_len,
                                   int32_t single_query_seqs,
                                   int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                   int32_t block_size, void* stream) {
  if (num_seqs < 0 || num_tokens < 0 || max_query_len < 0) return kBad;
  if (single_query_seqs < -1 || single_query_seqs > num_seqs) return kBad;
  if (!valid_heads(num_heads, num_kv_heads)) return kBad;
  if (head_dim != 64 && head_dim != 128) return kBad;
  if (block_size != 16) return kBad;
  if (num_tokens == 0 || num_seqs == 0 || max_query_len == 0) return 0;
  if (!q || !out || !block_tables || !query_start_loc || !seq_lens || !context_lens) return kBad;
  if (!cache_ok(k_cache, v_cache, cache_stride_block, cache_stride_tok, cache_stride_head, num_blocks))
    return kBad;
  if (!aligned16(q) || !aligned16(out) || q_stride_t % 8 || q_stride_h % 8 || out_stride_t % 8 ||
      out_stride_h % 8)
    return kBad;
  if (max_blocks < 1 || bt_stride < max_blocks) return kBad;
  // Offsets inside one page are 32-bit (decode kernel).
  if ((int64_t)16 * cache_stride_tok > 0x7fffffff) return kBad;

  PrefillArgs a{};
  a.q = q; a.q_st = q_stride_t; a.q_sh = q_stride_h;
  a.k_cache = k_cache; a.v_cache = v_cache;
  a.c_sb = cache_stride_block; a.c_st = cache_stride_tok; a.c_sh = cache_stride_head;
  a.num_pages = num_blocks;
  a.block_tables = block_tables; a.bt_stride = bt_stride; a.max_blocks = max_blocks;
  a.query_start_loc = query_start_loc; a.seq_lens = seq_lens; a.context_lens = context_lens;
  a.scale_log2 = scale * kLog2e;
  a.out = out; a.o_st = out_stride_t; a.o_sh = out_stride_h;
  a.num_seqs = num_seqs; a.num_tokens = num_tokens; a.max_query_len = max_query_len;
  a.num_heads = num_heads; a.num_kv_heads = num_kv_heads; a.head_dim = head_dim;
  a.single_query_seqs = single_query_seqs;
  return (int)paged_prefill(a, (hipStream_t)stream);
}

extern "C" int bvllm_set_tuning(int32_t knob, int32_t value) { return set_tuning(knob, value); }

extern "C" int64_t bvllm_argmax_workspace_bytes(int32_t rows, int32_t vocab) {
  if (rows <= 0 || vocab <= 0) return 0;
  return argmax_workspace_bytes(rows, vocab);
}

extern "C" int bvllm_greedy_argmax(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab,
                                   int32_t logits_fp32, void* workspace, int64_t* out, void* stream) {
  if (rows < 0 || vocab < 1 || (logits_fp32 != 0 && logits_fp32 != 1)) return kBad;
  if (rows == 0) return 0;
  if (!logits || !out || !workspace || row_stride < vocab) return kBad;
  if (((uintptr_t)workspace & 3u) != 0) return kBad;
  ArgmaxArgs a{};
  a.logits = logits; a.row_stride = row_stride;
  a.rows = rows; a.vocab = vocab;
  a.fp32 = logits_fp32;
  const int64_t esize = logits_fp32 ? 4 : 2;
  a.vec_ok = aligned16(logits) && (row_stride * esize) % 16 == 0 && ((int64_t)vocab * esize) % 16 == 0;
  a.workspace = workspace;
  a.out = out;
  return (int)greedy_argmax(a, (hipStream_t)stream);
}

extern "C" int bvllm_fused_add_rms_norm(const void* input, int64_t input_stride, void* residual,
                                        int64_t residual_stride, const void* weight, int32_t weight_fp32,
                                        void* out, int64_t out_stride, int32_t rows, int32_t hidden, float eps,
                                        void* stream) {
  if (rows < 0 || hidden < 1 || (weight_fp32 != 0 && weight_fp32 != 1)) return kBad;
  if (rows == 0) return 0;
  if (!input || !weight || !out || input_stride < hidden || out_stride < hidden) return kBad;
  if (residual && residual_stride < hidden) return kBad;
  NormArgs a{};
  a.input = input; a.in_stride = input_stride;
  a.residual = residual; a.res_stride = residual_stride;
  a.weight = weight; a.weight_fp32 = weight_fp32;
  a.out = out; a.out_stride = out_stride;
  a.rows = rows; a.n = hidden; a.eps = eps;
  a.vec_ok = hidden % 8 == 0 && aligned16(input) && aligned16(out) && aligned16(weight) &&
             input_stride % 8 == 0 && out_stride % 8 == 0 &&
             (!residual || (aligned16(residual) && residual_stride % 8 == 0));
  return (int)fused_add_rms_norm(a, (hipStream_t)stream);
}

extern "C" int bvllm_silu_mul(const void* gate_up, int64_t rows, int32_t d, void* out, void* stream) {
  if (rows < 0 || d < 1) return kBad;
  if (rows == 0) return 0;
  if (!gate_up || !out) return kBad;
  SiluArgs a{};
  a.gate_up = gate_up; a.out = out; a.rows = rows; a.d = d;
  a.vec_ok = d % 8 == 0 && aligned16(gate_up) && aligned16(out);
  return (int)silu_mul(a, (hipStream_t)stream);
}
