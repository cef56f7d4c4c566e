// Two partial attentions over disjoint key sets, merged by their natural log-sum-exp:
//   M = max(lse_a, lse_b), w_x = exp(lse_x - M), o = (w_a o_a + w_b o_b) / (w_a + w_b), lse = M + log(w_a + w_b).
// The formula of lean_vllm/attention/triton_merge.py:34-49 (equivalently merge.py:8-15), in fp32.
// One wave per (token, head); each lane handles D/64 elements.
#include "lv_common.h"

namespace lv {

template <typename T>
__global__ __launch_bounds__(64) void merge_states_kernel(char* __restrict__ out, int64_t out_st, int64_t out_sh,
                                                          const char* __restrict__ oa, int64_t oa_st, int64_t oa_sh,
                                                          float* __restrict__ lse_a, int64_t la_st, int64_t la_sh,
                                                          const char* __restrict__ ob, int64_t ob_st, int64_t ob_sh,
                                                          const float* __restrict__ lse_b, int64_t lb_st,
                                                          int64_t lb_sh, int32_t head_dim) {
  using E = Elem<T>;
  const int64_t t = blockIdx.x;
  const int h = blockIdx.y;
  const float la = lse_a[t * la_st + h * la_sh];
  const float lb = lse_b[t * lb_st + h * lb_sh];
  const float m = fmaxf(la, lb);
  const float wa = expf(la - m), wb = expf(lb - m);
  const float total = wa + wb;
  const uint16_t* pa = reinterpret_cast<const uint16_t*>(oa + t * oa_st + h * oa_sh);
  const uint16_t* pb = reinterpret_cast<const uint16_t*>(ob + t * ob_st + h * ob_sh);
  uint16_t* po = reinterpret_cast<uint16_t*>(out + t * out_st + h * out_sh);
  // Read everything before writing: out may alias o_a.
  constexpr int kMaxPer = 8;  // head_dim <= 512
  float o[kMaxPer];
  int n = 0;
  for (int d = threadIdx.x; d < head_dim && n < kMaxPer; d += 64, ++n) {
    const float a = E::lo((uint32_t)pa[d]);
    const float b = E::lo((uint32_t)pb[d]);
    o[n] = (a * wa + b * wb) / total;
  }
  __syncthreads();
  n = 0;
  for (int d = threadIdx.x; d < head_dim && n < kMaxPer; d += 64, ++n)
    po[d] = (uint16_t)(E::pack(o[n], 0.f) & 0xffffu);
  if (threadIdx.x == 0) lse_a[t * la_st + h * la_sh] = m + logf(total);
}

}  // namespace lv

using namespace lv;

extern "C" int lv_merge_attn_states(void* out, int64_t out_stride_t, int64_t out_stride_h, const void* o_a,
                                    int64_t oa_stride_t, int64_t oa_stride_h, float* lse_a, int64_t lsea_stride_t,
                                    int64_t lsea_stride_h, const void* o_b, int64_t ob_stride_t, int64_t ob_stride_h,
                                    const float* lse_b, int64_t lseb_stride_t, int64_t lseb_stride_h,
                                    int32_t num_tokens, int32_t num_heads, int32_t head_dim, int32_t dtype,
                                    void* stream) {
  LV_REQUIRE(dtype == LV_DTYPE_BF16 || dtype == LV_DTYPE_F16, "merge_attn_states: dtype %d is not bf16 or fp16",
             dtype);
  LV_REQUIRE(num_tokens >= 0 && num_heads > 0 && head_dim > 0 && head_dim <= 512,
             "merge_attn_states: bad sizes T=%d H=%d D=%d", num_tokens, num_heads, head_dim);
  if (num_tokens == 0) return LV_OK;
  LV_REQUIRE(out && o_a && lse_a && o_b && lse_b, "merge_attn_states: null pointer");
  const dim3 grid(num_tokens, num_heads);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t e = 2;
  if (dtype == LV_DTYPE_BF16)
    hipLaunchKernelGGL(merge_states_kernel<BF16>, grid, dim3(64), 0, s, (char*)out, out_stride_t * e,
                       out_stride_h * e, (const char*)o_a, oa_stride_t * e, oa_stride_h * e, lse_a, lsea_stride_t,
                       lsea_stride_h, (const char*)o_b, ob_stride_t * e, ob_stride_h * e, lse_b, lseb_stride_t,
                       lseb_stride_h, head_dim);
  else
    hipLaunchKernelGGL(merge_states_kernel<F16>, grid, dim3(64), 0, s, (char*)out, out_stride_t * e,
                       out_stride_h * e, (const char*)o_a, oa_stride_t * e, oa_stride_h * e, lse_a, lsea_stride_t,
                       lsea_stride_h, (const char*)o_b, ob_stride_t * e, ob_stride_h * e, lse_b, lseb_stride_t,
                       lseb_stride_h, head_dim);
  LV_LAUNCH_CHECK("merge_states_kernel");
  return LV_OK;
}
