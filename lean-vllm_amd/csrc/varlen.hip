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

// Keys are packed, so every 64-key tile is contiguous: tiles stream through an LDS ring. Two workgroups fit a CU
// up to 128-wide q.k; wider tiles take one (and its registers).
template <int DQK, int DV>
struct VarlenCfg {
  static constexpr int kRing = 2;
  static constexpr int kSmem = (kRing > 0 ? kRing : 1) * PromptSmem<DQK, DV>::kBytes;
  static constexpr int kWaves = kSmem <= 80 * 1024 && DQK <= 128 ? 2 : 1;
};

constexpr int kXcds = 8;  // workgroups are dealt round-robin over the XCDs by their linear index

// Item w = (kv head, row, query tile), query tiles innermost. Workgroup b (on XCD b % 8) takes item
// start(b % 8) + b / 8, so each XCD runs a contiguous range of items: the query tiles of one (row, kv head),
// which read the same key and value tiles, share an L2 instead of fetching them once per XCD.
template <typename T, int DQK, int DV>
__global__ __launch_bounds__(256, (VarlenCfg<DQK, DV>::kWaves)) void varlen_kernel(AttnParams p, int32_t qtiles) {
  __shared__ __attribute__((aligned(16))) char smem[VarlenCfg<DQK, DV>::kSmem];
  const int n = gridDim.x, b = blockIdx.x, x = b % kXcds;
  const int w = x * (n / kXcds) + min(x, n % kXcds) + b / kXcds;
  const int per_head = p.rows * qtiles;
  const int kvh = w / per_head, rest = w - kvh * per_head;
  const int row = rest / qtiles, qt = rest - row * qtiles;
  prefill_item<T, DQK, DV, true, false, VarlenCfg<DQK, DV>::kRing>(p, row, qt, kvh, smem);
}

template <typename T>
static int launch_varlen(const AttnParams& p, int dqk, int dv, int qtiles, hipStream_t st) {
  const dim3 grid(p.rows * qtiles * p.hkv);
  if (dqk == 64 && dv == 64)
    hipLaunchKernelGGL((varlen_kernel<T, 64, 64>), grid, dim3(256), 0, st, p, qtiles);
  else if (dqk == 128 && dv == 128)
    hipLaunchKernelGGL((varlen_kernel<T, 128, 128>), grid, dim3(256), 0, st, p, qtiles);
  else if (dqk == 192 && dv == 128)
    hipLaunchKernelGGL((varlen_kernel<T, 192, 128>), grid, dim3(256), 0, st, p, qtiles);
  else if (dqk == 192 && dv == 192)
    hipLaunchKernelGGL((varlen_kernel<T, 192, 192>), grid, dim3(256), 0, st, p, qtiles);
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

extern "C" int lv_varlen_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k,
                                   int64_t k_stride_t, int64_t k_stride_h, const void* v, int64_t v_stride_t,
                                   int64_t v_stride_h, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                   int32_t num_rows, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim_qk,
                                   int32_t head_dim_v, float scale, int32_t causal, int32_t max_seqlen_q, void* out,
                                   int64_t out_stride_t, int64_t out_stride_h, float* lse, int64_t lse_stride_t,
                                   int64_t lse_stride_h, int32_t dtype, void* stream) {
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
  const int qp = kPrefillRows / p.group;
  const int64_t qtiles = (max_seqlen_q + qp - 1) / qp;
  LV_REQUIRE(qtiles * num_rows * num_kv_heads < ((int64_t)1 << 31), "varlen_attention: grid too large");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  return dtype == LV_DTYPE_BF16 ? launch_varlen<BF16>(p, head_dim_qk, head_dim_v, (int)qtiles, st)
                                : launch_varlen<F16>(p, head_dim_qk, head_dim_v, (int)qtiles, st);
}
