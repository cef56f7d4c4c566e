// Ragged-batch packing on the GPU: per-row (num_cached, num_new, block list) -> the step's attention metadata.
//
// One kernel. Every workgroup first rebuilds the row-level prefix sums in LDS (the rows are few: a few thousand
// ints), then fills its share of the per-token outputs (positions, slot_mapping) and of the padded block table.
// Workgroup 0 also writes the row-level outputs. No grid-wide synchronisation, no atomics, no host read back.
// The integer arithmetic mirrors ModelRunner.prepare_batch (lean_vllm/engine/model_runner.py:367-446).
// num_logits[s] <= num_new[s] is the caller's contract (a row samples at most its own token rows).
// num_back (optional): per scheduler row, drafts of the previous step that were rejected; the row's tokens start
// that many positions earlier (ModelRunner._move_back, model_runner.py:527-551, applied before any output is
// formed, so positions, slots, context lengths and cu_seqlens_k all follow).
// A token whose page lies past its row's block list gets slot -1 (stores nothing) rather than another row's page.
#include "lv_common.h"

namespace lv {

constexpr int kPackThreads = kScanThreads;
constexpr int kPackMaxRows = 4096;  // LDS holds seven (rows + 1)-int arrays (112 KB)

__global__ __launch_bounds__(kPackThreads) void pack_kernel(
    const int32_t* __restrict__ num_cached, const int32_t* __restrict__ num_new, const int32_t* __restrict__ indptr,
    const int32_t* __restrict__ blk_ids, int32_t rows, int32_t query_len, int32_t bs, int32_t width, int32_t tokens,
    int32_t* __restrict__ order, int32_t* __restrict__ cu_q_out, int32_t* __restrict__ cu_k_out,
    int64_t* __restrict__ positions, int32_t* __restrict__ slots, int32_t* __restrict__ context_lens,
    int32_t* __restrict__ tables, const int32_t* __restrict__ num_logits, int64_t* __restrict__ logits,
    const int32_t* __restrict__ num_back, bool dense_slots) {
  __shared__ int src[kPackMaxRows];       // batch row -> scheduler row
  __shared__ int cu_q[kPackMaxRows + 1];  // token offsets, batch order
  __shared__ int cu_s[kPackMaxRows + 1];  // slot_mapping offsets (rows with a block list only), batch order
  __shared__ int row_of[kPackMaxRows];    // scheduler row -> batch row (logits only)
  __shared__ int wave_tot[kPackThreads / 64 + 1];
  __shared__ int s_cached[kPackMaxRows];    // the per-row inputs, staged once: every later read is from LDS
  __shared__ int s_new[kPackMaxRows];
  __shared__ int s_ptr[kPackMaxRows + 1];
  const int tid = threadIdx.x;

  // 0. Stage the row inputs (their loads all issued before any is used).
  for (int i = tid; i <= rows; i += kPackThreads) {
    s_ptr[i] = indptr[i];
    if (i < rows) {
      s_cached[i] = num_cached[i] - (num_back ? num_back[i] : 0);
      s_new[i] = num_new[i];
    }
  }
  __syncthreads();

  // 1. Stable partition: rows of query_len first, scheduler order kept in each group (model_runner.py:367-374).
  for (int i = tid; i < rows; i += kPackThreads) cu_q[i] = s_new[i] == query_len ? 1 : 0;
  __syncthreads();
  block_scan(cu_q, rows, wave_tot);
  const int leading = cu_q[rows];
  for (int i = tid; i < rows; i += kPackThreads) {
    const int before = cu_q[i];  // leading rows before i
    const bool lead = s_new[i] == query_len;
    src[lead ? before : leading + (i - before)] = i;
  }
  __syncthreads();

  // 2. Row prefix sums in batch order (model_runner.py:393-397).
  for (int r = tid; r < rows; r += kPackThreads) {
    const int s = src[r];
    cu_q[r] = s_new[s];
    cu_s[r] = dense_slots || s_ptr[s + 1] > s_ptr[s] ? s_new[s] : 0;
  }
  __syncthreads();
  block_scan(cu_q, rows, wave_tot);
  block_scan(cu_s, rows, wave_tot);

  // 3. Row-level outputs, from one workgroup (cu_seqlens_k last, once cu_q is free to reuse).
  if (blockIdx.x == 0) {
    for (int r = tid; r < rows; r += kPackThreads) {
      const int s = src[r];
      order[r] = s;
      cu_q_out[r] = cu_q[r];
      context_lens[r] = s_cached[s] + s_new[s];
    }
    if (tid == 0) cu_q_out[rows] = cu_q[rows];
  }

  // 4. Per-token outputs (model_runner.py:398-400, :440-445).
  const int stride = gridDim.x * kPackThreads;
  for (int t = blockIdx.x * kPackThreads + tid; t < tokens; t += stride) {
    int lo = 0, hi = rows - 1;  // last row whose start <= t
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (cu_q[mid] <= t) lo = mid; else hi = mid - 1;
    }
    const int r = lo, s = src[r];
    const int offset = t - cu_q[r];
    const int pos = s_cached[s] + offset;  // a position fits 32 bits (num_cached and num_new are int32)
    positions[t] = pos;
    const int list = s_ptr[s], len = s_ptr[s + 1] - list;
    if (len > 0) {
      const int page = pos / bs;
      const int64_t block = page < len ? blk_ids[list + page] : -1;
      slots[cu_s[r] + offset] = block < 0 ? -1 : (int32_t)(block * bs + (pos - page * bs));
    } else if (dense_slots) {
      slots[cu_s[r] + offset] = -1;  // a padding row of a captured step: its tokens store nothing
    }
  }

  // 5. Padded block tables (model_runner.py:437-439).
  const int cells = rows * width;  // the table's int32 cells (the caller's tensor: under 2^31)
  for (int e = blockIdx.x * kPackThreads + tid; e < cells; e += stride) {
    const int r = e / width, j = e - r * width;
    const int s = src[r];
    const int list = s_ptr[s], len = s_ptr[s + 1] - list;
    tables[e] = j < len ? blk_ids[list + j] : -1;
  }

  // 6. logits_indices (model_runner.py:424-430), in workgroup 0: the sampling rows in scheduler order, each the
  // last num_logits[s] token rows of its chunk (its drafts, then the next token).
  if (blockIdx.x == 0 && num_logits) {
    __syncthreads();  // this workgroup's tokens are done with cu_s
    for (int i = tid; i < rows; i += kPackThreads) cu_s[i] = s_new[i] == query_len ? 1 : 0;
    __syncthreads();
    block_scan(cu_s, rows, wave_tot);
    for (int i = tid; i < rows; i += kPackThreads) {
      const int before = cu_s[i];
      row_of[i] = s_new[i] == query_len ? before : leading + (i - before);
    }
    __syncthreads();
    for (int i = tid; i < rows; i += kPackThreads) cu_s[i] = num_logits[i];
    __syncthreads();
    block_scan(cu_s, rows, wave_tot);
    for (int s = tid; s < rows; s += kPackThreads) {
      const int n = num_logits[s];
      const int64_t first = (int64_t)cu_q[row_of[s] + 1] - n;
      for (int j = 0; j < n; ++j) logits[cu_s[s] + j] = first + j;
    }
  }

  // 7. cu_seqlens_k (model_runner.py:395-397), in workgroup 0, reusing cu_q's LDS now that its tokens are done.
  if (blockIdx.x == 0) {
    __syncthreads();
    for (int r = tid; r < rows; r += kPackThreads) {
      const int s = src[r];
      cu_q[r] = s_cached[s] + s_new[s];
    }
    __syncthreads();
    block_scan(cu_q, rows, wave_tot);
    for (int r = tid; r <= rows; r += kPackThreads) cu_k_out[r] = cu_q[r];
  }
}

}  // namespace lv

using namespace lv;

extern "C" int lv_pack(const int32_t* num_cached, const int32_t* num_new, const int32_t* blk_indptr,
                       const int32_t* blk_ids, int32_t num_rows, int32_t query_len, int32_t block_size,
                       int32_t table_width, int32_t num_tokens, int32_t* order, int32_t* cu_seqlens_q,
                       int32_t* cu_seqlens_k, int64_t* positions, int32_t* slot_mapping, int32_t* context_lens,
                       int32_t* block_tables, const int32_t* num_logits, int64_t* logits_indices,
                       const int32_t* num_back, int32_t flags, void* stream) {
  LV_REQUIRE(num_rows > 0 && num_rows <= kPackMaxRows, "pack: %d rows; 1 to %d are supported", num_rows,
             kPackMaxRows);
  LV_REQUIRE(block_size > 0, "pack: block_size must be positive, got %d", block_size);
  LV_REQUIRE(table_width >= 0 && num_tokens >= 0, "pack: negative table width or token count");
  LV_REQUIRE((int64_t)num_rows * table_width <= INT32_MAX, "pack: a %d x %d block table exceeds 2^31 cells", num_rows,
             table_width);
  LV_REQUIRE(num_cached && num_new && blk_indptr && order && cu_seqlens_q && cu_seqlens_k && context_lens,
             "pack: null row pointer");
  LV_REQUIRE(num_tokens == 0 || positions, "pack: null positions");
  LV_REQUIRE(table_width == 0 || (block_tables && blk_ids && slot_mapping), "pack: null table pointer");
  LV_REQUIRE(!num_logits || logits_indices, "pack: num_logits given without logits_indices");
  LV_REQUIRE((flags & ~LV_PACK_DENSE_SLOTS) == 0, "pack: unknown flags 0x%x", flags);
  const bool dense = (flags & LV_PACK_DENSE_SLOTS) != 0;
  LV_REQUIRE(!dense || num_tokens == 0 || slot_mapping, "pack: dense slots need slot_mapping");
  const int64_t work = (int64_t)num_tokens + (int64_t)num_rows * table_width;
  int grid = (int)((work + kPackThreads * 4 - 1) / (kPackThreads * 4));
  grid = grid < 1 ? 1 : (grid > 64 ? 64 : grid);
  hipLaunchKernelGGL(pack_kernel, dim3(grid), dim3(kPackThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     num_cached, num_new, blk_indptr, blk_ids, num_rows, query_len, block_size, table_width,
                     num_tokens, order, cu_seqlens_q, cu_seqlens_k, positions, slot_mapping, context_lens,
                     block_tables, num_logits, logits_indices, num_back, dense);
  LV_LAUNCH_CHECK("pack_kernel");
  return LV_OK;
}
