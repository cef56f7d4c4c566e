/* lvattn: MI355X (gfx950) continuous-batching attention path -- the C ABI.
 *
 * Every entry point takes plain device pointers, element strides and sizes, enqueues its kernels on `stream`
 * (a hipStream_t passed as void*; NULL is the default stream), never synchronises the host, never allocates,
 * and returns LV_OK or an error status whose message lv_last_error() returns (thread-local). No C++ exception
 * crosses the ABI. Buffers are owned by the caller. Strides are in elements, not bytes.
 *
 * Element formats: LV_DTYPE_BF16 and LV_DTYPE_F16 for attention; the store kernels copy bytes and take any
 * element size.
 */
#ifndef LVATTN_H_
#define LVATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LV_OK 0
#define LV_EINVAL 1 /* bad argument: shape, stride, alignment or size */
#define LV_EHIP 2   /* a HIP runtime call or kernel launch failed */

#define LV_DTYPE_BF16 0
#define LV_DTYPE_F16 1

#define LV_SCHEDULE_AUTO 0
#define LV_SCHEDULE_SERIAL 1
#define LV_SCHEDULE_OVERLAP 2

#define LV_ABI_VERSION 9

/* The last error message of the calling thread ("" if none). */
const char* lv_last_error(void);

/* LV_ABI_VERSION of the built library. */
int lv_abi_version(void);

/* ---------------------------------------------------------------------------------------------------------
 * Ragged-batch packing. Replaces the host packing of ModelRunner.prepare_batch
 * (lean_vllm/engine/model_runner.py:356-446, context dict :448-462) with one kernel.
 *
 * Inputs, in scheduler order, one entry per row: num_cached[B], num_new[B] (int32), and the rows' block lists
 * as CSR: blk_indptr[B+1], blk_ids[blk_indptr[B]] (int32). query_len is the length whose rows lead the batch
 * (decode_query_len, model_runner.py:51-63). table_width = the longest list; num_tokens = sum(num_new).
 * Outputs, in batch order (rows of length query_len first, scheduler order kept within each group):
 *   order[B]            batch row -> scheduler row
 *   cu_seqlens_q[B+1]   int32 prefix sums of num_new
 *   cu_seqlens_k[B+1]   int32 prefix sums of num_cached + num_new
 *   positions[T]        int64, num_cached + offset within the row
 *   slot_mapping[<=T]   int32, block_list[pos / bs] * bs + pos % bs, only for rows whose list is non-empty
 *                       (compacted, as model_runner.py:442-445)
 *   context_lens[B]     int32 num_cached + num_new
 *   block_tables[B*W]   int32 block lists padded with -1 (may be NULL when table_width == 0)
 * Optional, for steps that gather logits rows (model_runner.py:424-430): num_logits[B] (scheduler order) is the
 * number of logits rows each row samples -- its drafts + 1, or 0 for a chunk that does not sample (at most its
 * num_new); then
 *   logits_indices[L]   int64, L = sum(num_logits): for each sampling row in scheduler order, the last
 *                       num_logits token rows of its chunk, cu_seqlens_q[b+1] - n .. cu_seqlens_q[b+1] - 1
 * (both NULL to skip).
 * num_back[B] (optional, scheduler order, may be NULL): drafts of the previous step that were rejected, per row;
 * the row's tokens start that many positions before num_cached (ModelRunner._move_back, model_runner.py:527-551:
 * positions, slots, context lengths and cu_seqlens_k follow; host-side lengths computed from num_cached remain
 * upper bounds, as in the reference).
 * A token whose page lies past its row's block list gets slot -1 (stores nothing).
 * flags: 0, or LV_PACK_DENSE_SLOTS for a step replayed in a captured graph of fixed size: slot_mapping then has
 * one entry per token, -1 for the tokens of rows without a block list (model_runner.py:597-602 pads a graph's
 * rows that way). Such a padding row is given num_cached = -num_new, so its context length is 0.
 * Limit: num_rows <= LV_PACK_MAX_ROWS. */
#define LV_PACK_MAX_ROWS 4096
#define LV_PACK_DENSE_SLOTS 1
int lv_pack(const int32_t* num_cached, const int32_t* num_new, const int32_t* blk_indptr, const int32_t* blk_ids,
            int32_t num_rows, int32_t query_len, int32_t block_size, int32_t table_width, int32_t num_tokens,
            int32_t* order, int32_t* cu_seqlens_q, int32_t* cu_seqlens_k, int64_t* positions,
            int32_t* slot_mapping, int32_t* context_lens, int32_t* block_tables, const int32_t* num_logits,
            int64_t* logits_indices, const int32_t* num_back, int32_t flags, void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * Scatter new keys/values into the paged cache. Replaces AttentionBackend.store_kvcache
 * (lean_vllm/attention/abstract.py:107-116; Triton store_kvcache_kernel, lean_vllm/attention/triton_cache.py:9-37,58-81).
 * key/value: [T, Hkv, D] with unit dim stride and head stride D; row strides key_stride_t / value_stride_t.
 * Caches: logical (block, token, head, dim) addressed by their strides (an HND cache's transposed view works),
 * unit dim stride. slot_mapping[T]: slot = block * block_size + offset; -1 skips the token. Bit-exact copy. */
int lv_store_kvcache(const void* key, const void* value, int64_t key_stride_t, int64_t value_stride_t,
                     int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim, void* k_cache, void* v_cache,
                     int64_t cache_stride_block, int64_t cache_stride_token, int64_t cache_stride_head,
                     int32_t block_size, const int32_t* slot_mapping, int32_t elem_bytes, void* stream);

/* Scatter MLA latents [T, dim] (row stride latent_stride_t, unit dim stride) into a cache whose token rows are
 * `dim` elements apart (cache.view(-1, dim)[slot] = latent[t]); -1 skips. Replaces
 * AttentionBackend.store_latents (lean_vllm/attention/abstract.py:178-185; triton_cache.py:39-55,84-91). */
int lv_store_latents(const void* latent, int64_t latent_stride_t, int32_t num_tokens, int32_t dim, void* cache,
                     const int32_t* slot_mapping, int32_t elem_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * Paged attention over a step: pure decode, chunked prefill, or a mixed batch in one kernel.
 * Replaces AttentionBackend.decode / prefill / forward for this backend (lean_vllm/attention/abstract.py:118-176;
 * math of TorchAttention.decode/prefill, lean_vllm/attention/torch_backend.py:62-103).
 *
 * q: [T, Hq, D] (strides q_stride_t, q_stride_h; unit dim stride). out: same shape, own strides.
 * Caches as lv_store_kvcache, with 64 * cache_stride_token * 2 below 2^30 (a token row under 16 MiB).
 * block_tables: [B, *] int32 with row stride table_stride.
 * cu_seqlens_q: [B+1], or NULL for one query per row (decode; T == B).
 * Key length of row b: seqlens_k[b] if seqlens_k is non-NULL, else cu_seqlens_k[b+1] - cu_seqlens_k[b].
 * Query j of a row with lq queries and lk keys sees keys 0 .. lk-lq+j (bottom-right causal).
 * A row with no keys gets a zero output.
 * max_seqlen_k (at most 2^30) bounds every row's key length (block-table width * block_size will do); it sizes the
 * split-K grid so a captured graph needs no length read back. num_tokens is T (it sizes the work list).
 * workspace: caller-owned device memory of at least lv_paged_attention_workspace_bytes(...) bytes for the same
 * arguments; its contents need no initialisation.
 * schedule (a step with prompt rows): LV_SCHEDULE_OVERLAP runs the prompt tiles on part of the CUs beside the
 * decode rows' streaming (a second stream, joined back into `stream` by events); LV_SCHEDULE_SERIAL runs the
 * prompt tiles on the whole GPU, then the decode rows -- the faster choice when the decode rows' bytes take less
 * time than the prompt tiles' MFMA work (e.g. a step of prompts only). LV_SCHEDULE_AUTO overlaps. The result is
 * the same either way.
 * prompt_workgroups (overlap only): how many CUs run a prompt workgroup beside the decode rows; 0 picks 44% of
 * them. Other values are clamped to [44%, three quarters] of the CUs and rounded down to a multiple of 8 (each
 * kv head's prompt items then stay on one XCD). A step heavy in prompt tiles ends sooner with more.
 * flags: 0, or LV_ATTN_REUSE_PLAN for the later layers of a step: the workspace already holds the work list a previous
 * call planned for this step (the same rows, lengths, shape and max_seqlen_k, through the same cu_seqlens_q /
 * seqlens_k / cu_seqlens_k pointers, whose contents have not changed since), so the plan launch is skipped -- the
 * per-step plan the reference's backends cache in context.attn_metadata (lean_vllm/attention/flash_backend.py:16-20,
 * 157-160). The library honours the flag only if the last plan it made in this workspace was for the same shape and
 * pointers, and plans again otherwise; unchanged contents are the caller's promise. Besides the list, a plan zeroes
 * the counters of the persistent decode grid and of the split rows' in-kernel merges; every completed call leaves
 * them at zero again, so a later layer finds them as the plan left them. */
#define LV_ATTN_REUSE_PLAN 1
/* flags, also: LV_ATTN_PROMPTS_ONLY -- every row of the step has more than one query (the caller's host lengths say
 * so), so no decode launch and no split-K merge are made. Needs cu_seqlens_q and max_seqlen_q > 1. */
#define LV_ATTN_PROMPTS_ONLY 2
size_t lv_paged_attention_workspace_bytes(int32_t num_rows, int32_t num_tokens, int32_t num_heads,
                                          int32_t num_kv_heads, int32_t head_dim, int32_t max_seqlen_k,
                                          int32_t decode_only);
int lv_paged_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
                       const void* v_cache, int64_t cache_stride_block, int64_t cache_stride_token,
                       int64_t cache_stride_head, int32_t block_size, const int32_t* block_tables,
                       int64_t table_stride, const int32_t* cu_seqlens_q, const int32_t* seqlens_k,
                       const int32_t* cu_seqlens_k, int32_t num_rows, int32_t num_tokens, int32_t num_heads,
                       int32_t num_kv_heads, int32_t head_dim, float scale, int32_t max_seqlen_q,
                       int32_t max_seqlen_k, void* out, int64_t out_stride_t, int64_t out_stride_h,
                       void* workspace, size_t workspace_bytes, int32_t schedule, int32_t prompt_workgroups,
                       int32_t flags, int32_t dtype, void* stream);

/* Which kernels lv_paged_attention / lv_paged_attention_static launch for a step of this shape: the host-side
 * decision those calls make, reported without launching anything (it reads the device's CU count and the kernels'
 * occupancy, so it needs the device current). No counterpart in the reference, whose backends launch third-party
 * kernels; for callers and tests that check which path a step takes (the per-step plan of
 * lean_vllm/attention/flash_backend.py:141-182 is the nearest analogue). Arguments as lv_paged_attention's, plus
 * has_cu_seqlens_q (whether cu_seqlens_q would be non-NULL). A step with no rows or tokens reports no kernels.
 * two_streams = 1: the decode items run on the library's second stream beside the prompt launch (if that stream
 * cannot be created, the call runs the two serially instead, with the same results). */
#define LV_KERNEL_NONE 0
#define LV_KERNEL_DECODE_LIST 1    /* one workgroup per decode item of the work list */
#define LV_KERNEL_DECODE_BESIDE 2  /* persistent grid taking decode items by ticket, beside prompt_overlap */
#define LV_KERNEL_DECODE_GRID 3    /* one workgroup per (row, kv head, head group), unsplit; no work list (> 4096 rows) */
#define LV_KERNEL_PROMPT_LIST 4    /* one workgroup per prompt item, on the whole GPU */
#define LV_KERNEL_PROMPT_OVERLAP 5 /* persistent prompt workgroups on part of the CUs, beside the decode items */
#define LV_KERNEL_MIXED_SMALL 6    /* prompt and decode items of a small mixed step in one launch */
typedef struct lv_launch_info {
  int32_t decode_kernel;      /* LV_KERNEL_*: the launch running the decode items */
  int32_t decode_workgroups;  /* its grid (a bound: workgroups past the planned items exit at once) */
  int32_t prompt_kernel;      /* LV_KERNEL_*: the launch running the prompt items (MIXED_SMALL: the same launch) */
  int32_t prompt_workgroups;
  int32_t kv_heads_per_item;  /* 1, or 2: a decode item reads two adjacent kv heads of each token */
  int32_t two_streams;
  int32_t keys_per_split;     /* keys per decode item */
  int32_t max_splits;         /* the most decode items one row is split into */
  int32_t splitk_merge;       /* 1: rows are split over several items; each row's last split to finish merges
                                 them (log-sum-exp) inside the decode launch */
} lv_launch_info;
int lv_paged_attention_launch_info(int32_t num_rows, int32_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
                                   int32_t head_dim, int32_t block_size, int64_t cache_stride_head,
                                   int32_t has_cu_seqlens_q, int32_t max_seqlen_q, int32_t max_seqlen_k,
                                   int32_t schedule, int32_t prompt_workgroups, int32_t flags, int32_t dtype,
                                   lv_launch_info* info);

/* The same step with no workspace argument and no allocation of any kind. No counterpart in the reference: for
 * callers that cannot call hipMalloc -- code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation. The work list, its counters and the split-K partials live in a static device array of
 * LV_STATIC_WORKSPACE_BYTES that each GPU the library runs on holds until the process ends; a step needing more
 * (lv_paged_attention_workspace_bytes larger than that; the split-K sizing keeps steps of up to 4096 rows at any
 * context length under 9 MiB) is refused with LV_EINVAL. The kernels clear what must start at zero themselves
 * (the plan kernel zeroes the persistent grid's ticket and the split rows' merge counters), so no memset is recorded
 * into a captured graph. Every call
 * on one GPU shares that GPU's array, which keeps the last call's contents: calls that overlap on one GPU (two
 * streams, two host threads, or a graph replay beside an eager call) race. Results equal lv_paged_attention's for
 * the same arguments. Set-up: the first call on a device resolves the array's address there and creates the
 * device's second stream and its two fork/join events (which lv_paged_attention creates at its first overlapped
 * step); no device memory is allocated, and later calls create nothing. A caller that captures graphs makes one
 * call on each device before capturing. */
#define LV_STATIC_WORKSPACE_BYTES (16u << 20)
int lv_paged_attention_static(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
                              const void* v_cache, int64_t cache_stride_block, int64_t cache_stride_token,
                              int64_t cache_stride_head, int32_t block_size, const int32_t* block_tables,
                              int64_t table_stride, const int32_t* cu_seqlens_q, const int32_t* seqlens_k,
                              const int32_t* cu_seqlens_k, int32_t num_rows, int32_t num_tokens, int32_t num_heads,
                              int32_t num_kv_heads, int32_t head_dim, float scale, int32_t max_seqlen_q,
                              int32_t max_seqlen_k, void* out, int64_t out_stride_t, int64_t out_stride_h,
                              int32_t schedule, int32_t prompt_workgroups, int32_t flags, int32_t dtype,
                              void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * Attention over packed keys (no pages). Replaces AttentionBackend.prefill without block tables and
 * AttentionBackend.varlen_with_lse (lean_vllm/attention/abstract.py:148-164,187-204; math of TorchAttention.prefill
 * and varlen_with_lse, lean_vllm/attention/torch_backend.py:62-91): the warmup prefill and MLA prefill chunks.
 *
 * q: [T, Hq, head_dim_qk], k: [Tk, Hkv, head_dim_qk], v: [Tk, Hkv, head_dim_v], each with its own token and head
 * strides (elements) and unit dim stride, 64 * token stride * 2 below 2^30; rows given by cu_seqlens_q /
 * cu_seqlens_k [num_rows + 1] (device).
 * causal != 0: query j of a row with lq queries and lk keys sees keys 0 .. lk - lq + j; else all of its row's keys.
 * out: [T, Hq, head_dim_v]. lse (optional, may be NULL): fp32 [T, Hq] natural log-sum-exp of each query row's
 * scaled scores (-inf for a row with no keys). max_seqlen_q bounds every row's query count (it sizes the grid).
 * (head_dim_qk, head_dim_v) in {(64, 64), (128, 128), (192, 128), (192, 192)}. No workspace. */
int lv_varlen_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k, int64_t k_stride_t,
                        int64_t k_stride_h, const void* v, int64_t v_stride_t, int64_t v_stride_h,
                        const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t num_rows, int32_t num_heads,
                        int32_t num_kv_heads, int32_t head_dim_qk, int32_t head_dim_v, float scale, int32_t causal,
                        int32_t max_seqlen_q, void* out, int64_t out_stride_t, int64_t out_stride_h, float* lse,
                        int64_t lse_stride_t, int64_t lse_stride_h, int32_t dtype, void* stream);

/* MLA prefill over cached context in one call. Replaces the sequence MLAAttention._prefill runs for a step whose
 * cached keys form one chunk (lean_vllm/layers/attention.py:280-316): varlen_with_lse over the new tokens (causal),
 * varlen_with_lse over the expanded context keys (unmasked), then merge_attention_ of the two -- the same
 * attention, computed as one softmax per query over [context keys; new keys] with no partial outputs.
 *
 * As lv_varlen_attention with causal = 1, plus each row's context keys ctx_k: [Tc, Hkv, head_dim_qk], ctx_v:
 * [Tc, Hkv, head_dim_v] (token and head strides in elements, token strides bounded as k's, unit dim stride), rows
 * given by cu_seqlens_ctx [num_rows + 1] (device; a row may have none). Every query of a row sees all of its
 * context keys, then its own keys under the causal mask. lse (optional) is over both. No workspace. */
int lv_varlen_context_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k,
                                int64_t k_stride_t, int64_t k_stride_h, const void* v, int64_t v_stride_t,
                                int64_t v_stride_h, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                const void* ctx_k, int64_t ctx_k_stride_t, int64_t ctx_k_stride_h, const void* ctx_v,
                                int64_t ctx_v_stride_t, int64_t ctx_v_stride_h, const int32_t* cu_seqlens_ctx,
                                int32_t num_rows, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim_qk,
                                int32_t head_dim_v, float scale, int32_t max_seqlen_q, void* out,
                                int64_t out_stride_t, int64_t out_stride_h, float* lse, int64_t lse_stride_t,
                                int64_t lse_stride_h, int32_t dtype, void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * MLA absorbed decode. Replaces AttentionBackend.mla_decode (lean_vllm/attention/abstract.py:206-219; math of
 * TorchAttention.mla_decode, lean_vllm/attention/torch_backend.py:105-119; FlashMLA in the FlashMLA backend,
 * lean_vllm/attention/flashmla_backend.py:52-68).
 *
 * Each of num_rows rows has queries_per_row queries, its last positions: query j of a row with L = context_lens[b]
 * cached latents sees latents 0 .. L - queries_per_row + j. The latents are one key head shared by all num_heads
 * query heads; the values are their leading v_dim entries.
 * q: [num_rows * queries_per_row, num_heads, latent_dim] (strides q_stride_t, q_stride_h; unit dim stride), row b's
 * queries consecutive. latent_cache: [blocks, block_size, latent_dim] with block stride cache_stride_block and token
 * stride cache_stride_token (elements), unit dim stride. block_tables: [num_rows, *] int32, row stride table_stride.
 * out: [num_rows * queries_per_row, num_heads, v_dim]. latent_dim must be 576 and v_dim 512 (DeepSeek's
 * kv_lora_rank 512 + rope 64). max_seqlen_k bounds every row's latent count and sizes the split grid.
 * workspace: at least lv_mla_decode_workspace_bytes(...) bytes for the same arguments; no initialisation needed. */
size_t lv_mla_decode_workspace_bytes(int32_t num_rows, int32_t queries_per_row, int32_t num_heads,
                                     int32_t max_seqlen_k);
int lv_mla_decode(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* latent_cache,
                  int64_t cache_stride_block, int64_t cache_stride_token, int32_t block_size,
                  const int32_t* block_tables, int64_t table_stride, const int32_t* context_lens, int32_t num_rows,
                  int32_t queries_per_row, int32_t num_heads, int32_t latent_dim, int32_t v_dim, float scale,
                  int32_t max_seqlen_k, void* out, int64_t out_stride_t, int64_t out_stride_h, void* workspace,
                  size_t workspace_bytes, int32_t dtype, void* stream);

/* ---------------------------------------------------------------------------------------------------------
 * Merge two partial attentions over disjoint key sets by log-sum-exp. Replaces merge_attention_
 * (lean_vllm/attention/merge.py:18-28; Triton merge_attn_states_kernel, lean_vllm/attention/triton_merge.py:14-82).
 * o_*: [T, H, D] (unit dim stride, own token/head strides), lse_*: [T, H] fp32 natural log (own strides).
 * Writes out (may alias o_a) and overwrites lse_a with the merged lse. */
int lv_merge_attn_states(void* out, int64_t out_stride_t, int64_t out_stride_h, const void* o_a,
                         int64_t oa_stride_t, int64_t oa_stride_h, float* lse_a, int64_t lsea_stride_t,
                         int64_t lsea_stride_h, const void* o_b, int64_t ob_stride_t, int64_t ob_stride_h,
                         const float* lse_b, int64_t lseb_stride_t, int64_t lseb_stride_h, int32_t num_tokens,
                         int32_t num_heads, int32_t head_dim, int32_t dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LVATTN_H_ */
