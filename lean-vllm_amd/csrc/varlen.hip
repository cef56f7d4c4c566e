// Attention over packed (unpaged) keys: lean-vLLM's prefill without block tables and varlen_with_lse.
//
// Rows are given by cu_seqlens_q / cu_seqlens_k over packed q [T, Hq, DQK], k [Tk, Hkv, DQK], v [Tk, Hkv, DV].
// Every row runs the MFMA prompt item of attn_common.h; the grid covers (kv head, row, tile of query positions)
// for the longest row and items past a row's queries return at once, so no work list or workspace is needed.
// Math: TorchAttention.prefill without tables and TorchAttention.varlen_with_lse
// (lean_vllm/attention/torch_backend.py:62-91), bottom-right causal or unmasked, plus the natural log-sum-exp of
// every query row ([T, Hq]; -inf for a row with no keys).
#include "attn_common.h"

namespace lv {

// Keys are packed, so every 64-key tile is contiguous: tiles stream through an LDS ring. Up to 128-wide q.k two
// 4-wave workgroups fit a CU; the 192-wide tiles (an 88 KB stage pair) run one workgroup per CU of 8 waves (256
// query rows per item, two waves per SIMD, each staged tile serving twice the rows).
template <int DQK, int DV>
struct VarlenCfg {
  static constexpr int kPerCu = DQK <= 128 ? 2 : 1;  // workgroups per CU
  static constexpr int kRing = 2;  // a third stage for the one-per-CU tiles measured 6% slower
  static constexpr int kSmem = kRing * PromptSmem<DQK, DV>::kBytes;
  static constexpr int kWaves = kPerCu == 2 ? 4 : 8;        // waves per workgroup
  static constexpr int kRows = 32 * kWaves;                  // (position, head) query rows per item
};

constexpr int kXcds = 8;  // workgroups are dealt round-robin over the XCDs by their linear index

// XCDs that share one (kv head, row) group's query tiles: 1 when there are at least as many groups as XCDs, else
// enough that every XCD gets a share (a group's tiles dealt every S-th to each of S virtual groups).
__host__ __device__ inline int xcds_per_group(int groups) {
  return groups >= kXcds ? 1 : (kXcds + groups - 1) / groups;
}

// Items (kv head, row, query tile) are dealt to the XCDs in contiguous ranges of (kv head, row) groups: the query
// tiles of one (row, kv head), which read the same key and value tiles, share an L2 instead of fetching them once
// per XCD. Workgroup b runs on XCD b % 8 and is that XCD's (b / 8)-th workgroup. Unmasked, every query tile of a row
// walks all its keys: an XCD's items go out group by group, so a group's tiles run together and read each key tile
// once from memory (query tiles outermost cost 1.5x the time on DeepSeek-V2-Lite's prefix chunks). Causal, query
// tile t walks t + 1 tiles' worth of keys: the items go out by descending query tile, then group, so the long ones
// start first and the short ones fill the tail (0.67x the time of group order on its 1536-token chunks). With
// context keys (CTX) every query tile walks the whole context first: items go out group by group, as unmasked ones,
// the longest query tile of each group first. With fewer groups than XCDs (a few rows of few kv heads), each group
// is split into S = xcds_per_group virtual groups, every S-th query tile each, so that no XCD idles; each of the S
// XCDs then reads the group's key and value tiles.
template <typename T, int DQK, int DV, bool CTX>
__global__ __launch_bounds__((64 * VarlenCfg<DQK, DV>::kWaves), (VarlenCfg<DQK, DV>::kPerCu)) void varlen_kernel(
    AttnParams p, int32_t qtiles) {
  using Cfg = VarlenCfg<DQK, DV>;
  __shared__ __attribute__((aligned(16))) char smem[Cfg::kSmem];
  const int groups = p.rows * p.hkv;  // (kv head, row) groups
  const int S = xcds_per_group(groups);
  const int vgroups = groups * S, nq = (qtiles + S - 1) / S;  // virtual groups and their query tiles
  const int x = blockIdx.x % kXcds, k = blockIdx.x / kXcds;
  const int v0 = x * (vgroups / kXcds) + min(x, vgroups % kXcds);  // this XCD's first virtual group
  const int nv = vgroups / kXcds + (x < vgroups % kXcds ? 1 : 0);   // and its number of them
  if (k >= nv * nq) return;  // the grid is rounded up to whole XCD rounds
  const int qi = CTX ? nq - 1 - k % nq : p.causal ? nq - 1 - k / nv : k % nq;
  const int v = v0 + (CTX || !p.causal ? k / nq : k % nv);
  const int g = v / S, qt = v - g * S + S * qi;
  if (qt >= qtiles) return;  // a virtual group's last tile past the row's (S does not divide qtiles)
  const int kvh = g / p.rows, row = g - kvh * p.rows;
  prefill_item<T, DQK, DV, true, false, Cfg::kRing, Cfg::kWaves, CTX>(p, row, qt, kvh, smem);
}

// Query tiles per row of at most max_seqlen_q queries, for a (q.k, v) width pair; 0 for unsupported widths.
static int64_t varlen_qtiles(int dqk, int dv, int group, int max_seqlen_q) {
  int rows = 0;
  if (dqk == 64 && dv == 64) rows = VarlenCfg<64, 64>::kRows;
  else if (dqk == 128 && dv == 128) rows = VarlenCfg<128, 128>::kRows;
  else if (dqk == 192 && dv == 128) rows = VarlenCfg<192, 128>::kRows;
  else if (dqk == 192 && dv == 192) rows = VarlenCfg<192, 192>::kRows;
  if (rows == 0 || group > rows) return 0;
  const int qp = rows / group;
  return ((int64_t)max_seqlen_q + qp - 1) / qp;
}

// Threads per workgroup for a (q.k, v) width pair; 0 for unsupported widths.
static int varlen_threads(int dqk, int dv) {
  if (dqk == 64 && dv == 64) return 64 * VarlenCfg<64, 64>::kWaves;
  if (dqk == 128 && dv == 128) return 64 * VarlenCfg<128, 128>::kWaves;
  if (dqk == 192 && dv == 128) return 64 * VarlenCfg<192, 128>::kWaves;
  if (dqk == 192 && dv == 192) return 64 * VarlenCfg<192, 192>::kWaves;
  return 0;
}

// Workgroups of a launch over `groups` (kv head, row) groups of `qtiles` query tiles: each XCD gets a whole number
// of virtual groups, ceil(virtual groups / 8) times their query tiles.
static int64_t varlen_grid(int64_t groups, int64_t qtiles) {
  const int S = xcds_per_group((int)std::min<int64_t>(groups, kXcds));
  return (groups * S + kXcds - 1) / kXcds * ((qtiles + S - 1) / S) * kXcds;
}

template <typename T, int DQK, int DV>
static void launch_one(const AttnParams& p, int qtiles, hipStream_t st) {
  const dim3 grid((uint32_t)varlen_grid((int64_t)p.rows * p.hkv, qtiles)), block(64 * VarlenCfg<DQK, DV>::kWaves);
  if (p.cu_ctx)
    hipLaunchKernelGGL((varlen_kernel<T, DQK, DV, true>), grid, block, 0, st, p, qtiles);
  else
    hipLaunchKernelGGL((varlen_kernel<T, DQK, DV, false>), grid, block, 0, st, p, qtiles);
}

template <typename T>
static int launch_varlen(const AttnParams& p, int dqk, int dv, int qtiles, hipStream_t st) {
  if (dqk == 64 && dv == 64)
    launch_one<T, 64, 64>(p, qtiles, st);
  else if (dqk == 128 && dv == 128)
    launch_one<T, 128, 128>(p, qtiles, st);
  else if (dqk == 192 && dv == 128)
    launch_one<T, 192, 128>(p, qtiles, st);
  else if (dqk == 192 && dv == 192)
    launch_one<T, 192, 192>(p, qtiles, st);
  else {
    set_error("varlen_attention: head dims (q.k %d, v %d) are not (64, 64), (128, 128), (192, 128) or (192, 192)",
              dqk, dv);
    return LV_EINVAL;
  }
  LV_LAUNCH_CHECK("varlen_kernel");
  return LV_OK;
}

}  // namespace lv

using namespace lv;

// Both entry points: without context keys (ctx_k null) or with them.
static int varlen_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k, int64_t k_stride_t,
                            int64_t k_stride_h, const void* v, int64_t v_stride_t, int64_t v_stride_h,
                            const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, const void* ctx_k,
                            int64_t ctx_k_stride_t, int64_t ctx_k_stride_h, const void* ctx_v, int64_t ctx_v_stride_t,
                            int64_t ctx_v_stride_h, const int32_t* cu_seqlens_ctx, int32_t num_rows, int32_t num_heads,
                            int32_t num_kv_heads, int32_t head_dim_qk, int32_t head_dim_v, float scale, int32_t causal,
                            int32_t max_seqlen_q, void* out, int64_t out_stride_t, int64_t out_stride_h, float* lse,
                            int64_t lse_stride_t, int64_t lse_stride_h, int32_t dtype, void* stream) {
  LV_REQUIRE(dtype == LV_DTYPE_BF16 || dtype == LV_DTYPE_F16, "varlen_attention: dtype %d is not bf16 or fp16",
             dtype);
  LV_REQUIRE(num_rows >= 0 && max_seqlen_q >= 0, "varlen_attention: negative row count or max_seqlen_q");
  if (num_rows == 0 || max_seqlen_q == 0) return LV_OK;
  LV_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
             "varlen_attention: %d query heads do not group over %d key heads", num_heads, num_kv_heads);
  LV_REQUIRE(num_heads / num_kv_heads <= kPrefillRows, "varlen_attention: query group %d exceeds %d",
             num_heads / num_kv_heads, kPrefillRows);
  LV_REQUIRE(q && k && v && out && cu_seqlens_q && cu_seqlens_k, "varlen_attention: null tensor pointer");
  LV_REQUIRE(scale > 0.f, "varlen_attention: the softmax scale must be positive, got %g", (double)scale);
  LV_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(out, 16) && (q_stride_t * 2) % 16 == 0 &&
                 (q_stride_h * 2) % 16 == 0 && (k_stride_t * 2) % 16 == 0 && (k_stride_h * 2) % 16 == 0 &&
                 (v_stride_t * 2) % 16 == 0 && (v_stride_h * 2) % 16 == 0 && (out_stride_t * 2) % 8 == 0 &&
                 (out_stride_h * 2) % 8 == 0,
             "varlen_attention: tensors and their strides must be 16-byte aligned");
  // Lanes address the rows of a 64-key tile with 32-bit byte offsets, as 24-bit products (key row times token
  // stride).
  auto row_stride_ok = [](int64_t st) { return st >= 0 && (int64_t)kPrefillKeys * st * 2 < ((int64_t)1 << 30); };
  LV_REQUIRE(row_stride_ok(k_stride_t) && row_stride_ok(v_stride_t), "varlen_attention: key token stride %lld or "
             "value token stride %lld is negative or too large", (long long)k_stride_t, (long long)v_stride_t);
  if (cu_seqlens_ctx) {
    LV_REQUIRE(ctx_k && ctx_v, "varlen_context_attention: null context key or value pointer");
    LV_REQUIRE(row_stride_ok(ctx_k_stride_t) && row_stride_ok(ctx_v_stride_t), "varlen_context_attention: context "
               "token stride %lld or %lld is negative or too large", (long long)ctx_k_stride_t,
               (long long)ctx_v_stride_t);
    LV_REQUIRE(aligned(ctx_k, 16) && aligned(ctx_v, 16) && (ctx_k_stride_t * 2) % 16 == 0 &&
                   (ctx_k_stride_h * 2) % 16 == 0 && (ctx_v_stride_t * 2) % 16 == 0 &&
                   (ctx_v_stride_h * 2) % 16 == 0,
               "varlen_context_attention: context keys, values and their strides must be 16-byte aligned");
  }
  AttnParams p{};
  p.q = (const char*)q;
  p.q_st = q_stride_t * 2;
  p.q_sh = q_stride_h * 2;
  p.k_cache = (const char*)k;
  p.v_cache = (const char*)v;
  p.c_st = k_stride_t * 2;
  p.c_sh = k_stride_h * 2;
  p.v_st = v_stride_t * 2;
  p.v_sh = v_stride_h * 2;
  p.paged = false;
  p.causal = causal != 0;
  p.bs = FastDiv::make(1);
  p.cu_q = cu_seqlens_q;
  p.cu_k = cu_seqlens_k;
  p.rows = num_rows;
  p.hq = num_heads;
  p.hkv = num_kv_heads;
  p.group = num_heads / num_kv_heads;
  p.qgroups = 1;
  p.scale_log2 = scale * kLog2e;
  p.out = (char*)out;
  p.o_st = out_stride_t * 2;
  p.o_sh = out_stride_h * 2;
  p.lse = lse;
  p.lse_st = lse_stride_t;
  p.lse_sh = lse_stride_h;
  if (cu_seqlens_ctx) {
    p.ctx_k = (const char*)ctx_k;
    p.ctx_v = (const char*)ctx_v;
    p.cx_st = ctx_k_stride_t * 2;
    p.cx_sh = ctx_k_stride_h * 2;
    p.cv_st = ctx_v_stride_t * 2;
    p.cv_sh = ctx_v_stride_h * 2;
    p.cu_ctx = cu_seqlens_ctx;
  }
  const int64_t qtiles = varlen_qtiles(head_dim_qk, head_dim_v, p.group, max_seqlen_q);
  LV_REQUIRE(qtiles > 0, "varlen_attention: head dims (q.k %d, v %d) are not (64, 64), (128, 128), (192, 128) or "
             "(192, 192)", head_dim_qk, head_dim_v);
  const int64_t wgs = varlen_grid((int64_t)num_rows * num_kv_heads, qtiles);
  LV_REQUIRE(fits_one_launch(wgs, varlen_threads(head_dim_qk, head_dim_v)),
             "varlen_attention: %d rows x %d kv heads x %lld query tiles need %lld workgroups, more than one launch "
             "holds", num_rows, num_kv_heads, (long long)qtiles, (long long)wgs);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  return dtype == LV_DTYPE_BF16 ? launch_varlen<BF16>(p, head_dim_qk, head_dim_v, (int)qtiles, st)
                                : launch_varlen<F16>(p, head_dim_qk, head_dim_v, (int)qtiles, st);
}

extern "C" int lv_varlen_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k,
                                   int64_t k_stride_t, int64_t k_stride_h, const void* v, int64_t v_stride_t,
                                   int64_t v_stride_h, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                   int32_t num_rows, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim_qk,
                                   int32_t head_dim_v, float scale, int32_t causal, int32_t max_seqlen_q, void* out,
                                   int64_t out_stride_t, int64_t out_stride_h, float* lse, int64_t lse_stride_t,
                                   int64_t lse_stride_h, int32_t dtype, void* stream) {
  return varlen_attention(q, q_stride_t, q_stride_h, k, k_stride_t, k_stride_h, v, v_stride_t, v_stride_h,
                          cu_seqlens_q, cu_seqlens_k, nullptr, 0, 0, nullptr, 0, 0, nullptr, num_rows, num_heads,
                          num_kv_heads, head_dim_qk, head_dim_v, scale, causal, max_seqlen_q, out, out_stride_t,
                          out_stride_h, lse, lse_stride_t, lse_stride_h, dtype, stream);
}

extern "C" int lv_varlen_context_attention(
    const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k, int64_t k_stride_t, int64_t k_stride_h,
    const void* v, int64_t v_stride_t, int64_t v_stride_h, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
    const void* ctx_k, int64_t ctx_k_stride_t, int64_t ctx_k_stride_h, const void* ctx_v, int64_t ctx_v_stride_t,
    int64_t ctx_v_stride_h, const int32_t* cu_seqlens_ctx, int32_t num_rows, int32_t num_heads, int32_t num_kv_heads,
    int32_t head_dim_qk, int32_t head_dim_v, float scale, int32_t max_seqlen_q, void* out, int64_t out_stride_t,
    int64_t out_stride_h, float* lse, int64_t lse_stride_t, int64_t lse_stride_h, int32_t dtype, void* stream) {
  LV_REQUIRE(cu_seqlens_ctx, "varlen_context_attention: cu_seqlens_ctx is null");
  return varlen_attention(q, q_stride_t, q_stride_h, k, k_stride_t, k_stride_h, v, v_stride_t, v_stride_h,
                          cu_seqlens_q, cu_seqlens_k, ctx_k, ctx_k_stride_t, ctx_k_stride_h, ctx_v, ctx_v_stride_t,
                          ctx_v_stride_h, cu_seqlens_ctx, num_rows, num_heads, num_kv_heads, head_dim_qk, head_dim_v,
                          scale, 1, max_seqlen_q, out, out_stride_t, out_stride_h, lse, lse_stride_t, lse_stride_h,
                          dtype, stream);
}
