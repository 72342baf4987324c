/*
 * babyvllm_amd — C ABI of the MI355X (gfx950) paged-KV hot path.
 *
 * Three operations, each a drop-in for one Python entry point of the
 * reference's babyvllm/kernels package:
 *
 *   bvllm_rope_kv_append  <- fused_rope_and_cache      (babyvllm/kernels/rope.py:101-153)
 *   bvllm_paged_decode    <- paged_decode_attention    (babyvllm/kernels/paged_attn.py:259-346)
 *   bvllm_paged_prefill   <- paged_prefill_attention   (babyvllm/kernels/paged_prefill.py:104-146)
 *
 * Conventions shared by every entry point:
 *   - Tensors are device pointers to bf16 (uint16 bit patterns) unless noted;
 *     strides are in ELEMENTS; the last (head_dim) stride is always 1.
 *   - The KV cache of one layer is the reference's [2, num_blocks, block_size,
 *     num_kv_heads, head_dim] tensor (babyvllm/worker/model_runner.py:224-239);
 *     k_cache = &cache[0], v_cache = &cache[1], and the page / token / head
 *     strides are those of cache[0] (cache[1] must have the same).
 *   - block_size must be 16; head_dim must be 64 or 128 (RoPE also takes 256);
 *     num_heads must be a multiple of num_kv_heads (any ratio; the attention
 *     kernels compute a group of more than 16 query heads per KV head as
 *     ceil(ratio / 16) column groups of at most 16 heads, each reading the KV
 *     head's pages).
 *   - `stream` is a hipStream_t (NULL = the legacy default stream). Every call is
 *     asynchronous, does no host<->device copy and no host synchronisation, and
 *     allocates nothing, so it may be captured in a hipGraph.
 *   - Returns 0 on success, otherwise a hipError_t value
 *     (hipErrorInvalidValue = 1 for rejected arguments); bvllm_error_string
 *     turns it into text.
 *   - Table entries outside [0, num_blocks) are clamped into the pool and
 *     slots outside [0, num_blocks*block_size) are not written (the reference
 *     would access memory outside the cache in both cases).
 */
#ifndef BABYVLLM_AMD_H
#define BABYVLLM_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version of this header; bumped on any signature change. */
#define BVLLM_ABI_VERSION 6

#if defined(__GNUC__)
#define BVLLM_API __attribute__((visibility("default")))
#else
#define BVLLM_API
#endif

BVLLM_API int bvllm_abi_version(void);

/* Text for a return code of this library. */
BVLLM_API const char* bvllm_error_string(int code);

/*
 * Fused RoPE + KV-store append. Replaces fused_rope_and_cache
 * (babyvllm/kernels/rope.py:101-153, kernel rope.py:5-98).
 *
 * Rotates q [T, H, D] and k [T, Hkv, D] in place with rotate-half RoPE:
 *   x[:D/2] <- x[:D/2]·cos[:D/2] − x[D/2:]·sin[:D/2]
 *   x[D/2:] <- x[D/2:]·cos[D/2:] + x[:D/2]·sin[D/2:]
 * each product and the sum rounded to bf16 (torch's eager bf16 ops).
 * If k_cache is non-NULL, writes the rotated k and the raw v [T, Hkv, D] into
 * the cache row of slot_mapping[t] (int64 [T]); slot = page·16 + offset.
 * cos/sin are [T, D] bf16 rows (one per token).
 */
BVLLM_API int bvllm_rope_kv_append(void* q, int64_t q_stride_t, int64_t q_stride_h,
                         void* k, int64_t k_stride_t, int64_t k_stride_h,
                         const void* v, int64_t v_stride_t, int64_t v_stride_h,
                         const void* cos, int64_t cos_stride_t,
                         const void* sin, int64_t sin_stride_t,
                         void* k_cache, void* v_cache,
                         int64_t cache_stride_slot, int64_t cache_stride_head,
                         int64_t num_slots, const int64_t* slot_mapping,
                         int32_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
                         int32_t head_dim, void* stream);

/*
 * Bytes of device scratch bvllm_paged_decode needs for one launch (0 = none):
 * fp32 partial outputs [B, H, P, D] and log-sum-exps [B, H, P], the
 * reference's part_out / part_lse (babyvllm/kernels/paged_attn.py:317-318),
 * where P is the number of splits, or, for plans of more than 32 splits whose
 * pages per split are a multiple of 4, the number of groups of 4 consecutive
 * splits (those launches fold each group before writing it). The size and
 * layout depend only on these arguments, never on bvllm_set_tuning: knob 0
 * may make a launch write fewer partials than P, never more.
 */
BVLLM_API int64_t bvllm_decode_workspace_bytes(int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                               int32_t head_dim, int32_t num_splits,
                                               int32_t blocks_per_split);

/*
 * Paged decode attention, one query token per sequence. Replaces
 * paged_decode_attention + _split_decode_attention (babyvllm/kernels/paged_attn.py:259-346)
 * and its three kernels (paged_attn.py:9-251).
 *
 * q [B, H, D]; block_tables int32 [B, >= max_blocks] (row stride bt_stride);
 * seq_lens int32 [B]; out [B, H, D] bf16. Row b attends keys 0..seq_lens[b]-1
 * (at most max_blocks pages); a row with seq_len 0 outputs zeros.
 * (num_splits, blocks_per_split) is the flash-decoding plan
 * (decode_split_plan, babyvllm/kernels/decode_split.py:48-79): split s covers
 * pages [s·bps, (s+1)·bps), the last split runs to the row's last page.
 * `workspace` must hold bvllm_decode_workspace_bytes() bytes when that is > 0.
 * `waves` is the number of 64-lane waves per single-pass work-group: 0 (the
 * library's choice) or 4.
 * Bits: a row that fits in one split gives the same output from the single
 * pass and from any split plan, and a plan sized for a longer context (a graph
 * bucket) gives the same output as one sized for the live lengths.
 */
BVLLM_API int bvllm_paged_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                       const void* k_cache, const void* v_cache,
                       int64_t cache_stride_block, int64_t cache_stride_tok, int64_t cache_stride_head,
                       int32_t num_blocks,
                       const int32_t* block_tables, int64_t bt_stride, int32_t max_blocks,
                       const int32_t* seq_lens, float scale,
                       void* out, int64_t out_stride_b, int64_t out_stride_h,
                       void* workspace, int32_t num_splits, int32_t blocks_per_split,
                       int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                       int32_t head_dim, int32_t block_size, int32_t waves, void* stream);

/*
 * bvllm_paged_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under hipGraph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference: its
 * decode allocates the split scratch through torch on every call
 * (babyvllm/kernels/paged_attn.py:317-320).
 *
 * Same arguments, kernels and results as bvllm_paged_decode; the split
 * partials go to a static device array of BVLLM_NOALLOC_SCRATCH_BYTES per GPU,
 * owned by the library until the process ends. The call allocates and frees
 * nothing. A launch whose bvllm_decode_workspace_bytes() exceeds that size is
 * rejected with BVLLM_ERROR_SCRATCH_LIMIT before anything is launched.
 * Every call on one GPU shares that GPU's array: calls that overlap in time on
 * one GPU (different streams, or different host threads) race and must not be
 * issued; calls ordered on one stream are fine. Nothing in the array needs to
 * start at zero: every launch writes each partial it later reads.
 */
#define BVLLM_NOALLOC_SCRATCH_BYTES (32ll << 20)
#define BVLLM_ERROR_SCRATCH_LIMIT 10001
BVLLM_API int bvllm_paged_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                         const void* k_cache, const void* v_cache,
                                         int64_t cache_stride_block, int64_t cache_stride_tok,
                                         int64_t cache_stride_head, int32_t num_blocks,
                                         const int32_t* block_tables, int64_t bt_stride, int32_t max_blocks,
                                         const int32_t* seq_lens, float scale,
                                         void* out, int64_t out_stride_b, int64_t out_stride_h,
                                         int32_t num_splits, int32_t blocks_per_split,
                                         int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                         int32_t head_dim, int32_t block_size, int32_t waves, void* stream);

/*
 * Varlen paged prefill attention. Replaces paged_prefill_attention
 * (babyvllm/kernels/paged_prefill.py:104-146, kernel :6-101).
 *
 * q [T, H, D] holds the query rows of num_seqs sequences back to back:
 * sequence s owns rows query_start_loc[s] .. query_start_loc[s+1]-1 (int32 [S+1]).
 * Row i of sequence s sits at position context_lens[s] + i and attends keys
 * 0 .. context_lens[s] + i (and < seq_lens[s]) read from the cache through
 * block_tables[s]. K/V of the new tokens must already be in the cache.
 * max_query_len bounds every sequence's query count (it sizes the grid).
 * single_query_seqs is the number of sequences with exactly one query token
 * (decode rows of a mixed step), or -1 if the caller does not know it; when it
 * is not 0 those sequences run on the decode kernel (a second launch on the
 * same stream), which splits a row's pages over the waves of a work-group.
 * Passing 0 when such sequences exist is allowed: the prefill kernel then
 * computes them too.
 */
BVLLM_API int bvllm_paged_prefill(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                        const void* k_cache, const void* v_cache,
                        int64_t cache_stride_block, int64_t cache_stride_tok, int64_t cache_stride_head,
                        int32_t num_blocks,
                        const int32_t* block_tables, int64_t bt_stride, int32_t max_blocks,
                        const int32_t* query_start_loc, const int32_t* seq_lens,
                        const int32_t* context_lens, float scale,
                        void* out, int64_t out_stride_t, int64_t out_stride_h,
                        int32_t num_seqs, int32_t num_tokens, int32_t max_query_len,
                        int32_t single_query_seqs,
                        int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                        int32_t block_size, void* stream);

/*
 * Tuning switch for experiments and tests (no counterpart in the reference):
 * sets process-wide knob `knob` to `value` (0 = the library's default) and
 * returns the previous value, or -1 for an unknown knob. Knobs: 0 decode split
 * mode (default: four waves per split of at most 32 pages, two per longer
 * split, or per group of 4 splits when the plan groups them, two only while
 * the groups are at most one per compute unit; 1 one wave per split, 2 one
 * wave per group, 3 two waves per group, 4 two waves per split), 1 prefill
 * column blocks per work-group (tables of at most 8 pages), 2 decode wave
 * order (1 split units fastest), 3 decode single pass on streaming waves (1),
 * 4 decode page loads of the streaming waves without the nontemporal hint
 * (1), 5 aligned RoPE + append on the per-chunk kernel instead of the
 * per-row kernel (1), 6 short prefill grids on the single key walk instead of
 * the in-work-group key split (1). Knobs 0-5 change no result bit (a NaN's
 * payload aside); knob 6 changes the prefill's summation order (both paths
 * within the same tolerance of the reference).
 */
BVLLM_API int bvllm_set_tuning(int32_t knob, int32_t value);

/*
 * Greedy sampling: out[r] = argmax(logits[r, :]) for rows r < rows. Replaces
 * greedy_argmax (babyvllm/kernels/argmax.py:41-56) and its two kernels
 * (argmax.py:14-38). logits [rows, vocab] with unit column stride and row
 * stride row_stride elements, bf16 (logits_fp32 = 0) or fp32 (1); out int64.
 * Ties go to the lowest index and NaN beats every number, as torch.argmax.
 * `workspace` must hold bvllm_argmax_workspace_bytes(rows, vocab) bytes.
 */
BVLLM_API int64_t bvllm_argmax_workspace_bytes(int32_t rows, int32_t vocab);
BVLLM_API int bvllm_greedy_argmax(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab,
                        int32_t logits_fp32, void* workspace, int64_t* out, void* stream);

/*
 * Residual add + RMSNorm over rows of `hidden` bf16 elements. Replaces
 * fused_add_rms_norm (babyvllm/kernels/layernorm.py:46-83, kernel :5-43).
 * If residual is non-NULL: x = bf16(input + residual), written back to
 * residual; else x = input. out = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w),
 * weight [hidden] bf16 (weight_fp32 = 0) or fp32 (1). Strides in elements.
 */
BVLLM_API int bvllm_fused_add_rms_norm(const void* input, int64_t input_stride, void* residual,
                             int64_t residual_stride, const void* weight, int32_t weight_fp32,
                             void* out, int64_t out_stride, int32_t rows, int32_t hidden, float eps,
                             void* stream);

/*
 * out[r, c] = bf16(silu(gate_up[r, c]) * gate_up[r, d + c]), silu in fp32.
 * Replaces fused_silu_mul (babyvllm/kernels/activation.py:44-65, kernel :5-42).
 * gate_up [rows, 2d] and out [rows, d] bf16, contiguous.
 */
BVLLM_API int bvllm_silu_mul(const void* gate_up, int64_t rows, int32_t d, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BABYVLLM_AMD_H */
