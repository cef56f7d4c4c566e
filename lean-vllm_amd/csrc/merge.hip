// Two partial attentions over disjoint key sets, merged by their natural log-sum-exp:
//   M = max(lse_a, lse_b), w_x = exp(lse_x - M), o = (w_a o_a + w_b o_b) / (w_a + w_b), lse = M + log(w_a + w_b).
// The formula of lean_vllm/attention/triton_merge.py:34-49 (equivalently merge.py:8-15), in fp32.
// One wave per (token, head), each lane D/64 elements; 16-byte lanes when every row and stride allows (below).
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

// The same merge, 16 bytes per lane: D / 8 lanes per (token, head) row, whole rows per workgroup. Every thread
// reads its row's lse values and its 16 bytes of both partials before any thread writes (out and lse_a may alias
// the inputs).
template <typename T>
__global__ __launch_bounds__(256) void merge_states_vec_kernel(char* __restrict__ out, int64_t out_st,
                                                               int64_t out_sh, const char* __restrict__ oa,
                                                               int64_t oa_st, int64_t oa_sh, float* __restrict__ lse_a,
                                                               int64_t la_st, int64_t la_sh,
                                                               const char* __restrict__ ob, int64_t ob_st,
                                                               int64_t ob_sh, const float* __restrict__ lse_b,
                                                               int64_t lb_st, int64_t lb_sh, int32_t rows,
                                                               int32_t heads, int32_t lanes_per_row) {
  using E = Elem<T>;
  const int rows_per_block = blockDim.x / lanes_per_row;
  const int r = threadIdx.x / lanes_per_row, chunk = threadIdx.x - r * lanes_per_row;
  const int64_t row = (int64_t)blockIdx.x * rows_per_block + r;
  const bool live = row < rows;
  const int64_t t = live ? row / heads : 0;
  const int h = live ? (int)(row - t * heads) : 0;
  float m = 0.f, wa = 0.f, wb = 0.f;
  u32x4 a = {0, 0, 0, 0}, b = {0, 0, 0, 0};
  if (live) {
    const float la = lse_a[t * la_st + h * la_sh];
    const float lb = lse_b[t * lb_st + h * lb_sh];
    m = fmaxf(la, lb);
    wa = expf(la - m);
    wb = expf(lb - m);
    a = ld16(oa + t * oa_st + h * oa_sh + chunk * 16);
    b = ld16(ob + t * ob_st + h * ob_sh + chunk * 16);
  }
  __syncthreads();
  if (!live) return;
  const float inv = 1.f / (wa + wb);
  u32x4 o;
#pragma unroll
  for (int w = 0; w < 4; ++w)
    o[w] = E::pack((E::lo(a[w]) * wa + E::lo(b[w]) * wb) * inv, (E::hi(a[w]) * wa + E::hi(b[w]) * wb) * inv);
  st16(out + t * out_st + h * out_sh + chunk * 16, o);
  if (chunk == 0) lse_a[t * la_st + h * la_sh] = m + logf(wa + wb);
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
  LV_REQUIRE(fits_one_launch(num_tokens, 64) && num_heads < 65536,
             "merge_attn_states: %d tokens x %d heads need a grid larger than one launch holds", num_tokens, num_heads);
  const dim3 grid(num_tokens, num_heads);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t e = 2;
  const bool vec = head_dim % 8 == 0 && head_dim / 8 <= 256 && aligned(out, 16) && aligned(o_a, 16) &&
                   aligned(o_b, 16) && (out_stride_t * e) % 16 == 0 && (out_stride_h * e) % 16 == 0 &&
                   (oa_stride_t * e) % 16 == 0 && (oa_stride_h * e) % 16 == 0 && (ob_stride_t * e) % 16 == 0 &&
                   (ob_stride_h * e) % 16 == 0;
  if (vec) {
    const int lpr = head_dim / 8;
    const int rpb = 256 / lpr;
    const int64_t rows = (int64_t)num_tokens * num_heads;
    const int64_t blocks = (rows + rpb - 1) / rpb;
    LV_REQUIRE(rows < ((int64_t)1 << 31) && fits_one_launch(blocks, rpb * lpr), "merge_attn_states: too many rows");
    if (dtype == LV_DTYPE_BF16)
      hipLaunchKernelGGL(merge_states_vec_kernel<BF16>, dim3((uint32_t)blocks), dim3(rpb * lpr), 0, s, (char*)out,
                         out_stride_t * e, out_stride_h * e, (const char*)o_a, oa_stride_t * e, oa_stride_h * e,
                         lse_a, lsea_stride_t, lsea_stride_h, (const char*)o_b, ob_stride_t * e, ob_stride_h * e,
                         lse_b, lseb_stride_t, lseb_stride_h, (int32_t)rows, num_heads, lpr);
    else
      hipLaunchKernelGGL(merge_states_vec_kernel<F16>, dim3((uint32_t)blocks), dim3(rpb * lpr), 0, s, (char*)out,
                         out_stride_t * e, out_stride_h * e, (const char*)o_a, oa_stride_t * e, oa_stride_h * e,
                         lse_a, lsea_stride_t, lsea_stride_h, (const char*)o_b, ob_stride_t * e, ob_stride_h * e,
                         lse_b, lseb_stride_t, lseb_stride_h, (int32_t)rows, num_heads, lpr);
    LV_LAUNCH_CHECK("merge_states_vec_kernel");
    return LV_OK;
  }
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
