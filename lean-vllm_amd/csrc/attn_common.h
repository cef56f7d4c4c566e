// Shared by the paged and the packed-key attention kernels: launch parameters and the prompt item (MFMA).
#pragma once

#include "lv_common.h"

namespace lv {

constexpr int kPrefillKeys = 64;  // keys per prompt tile
constexpr int kPrefillRows = 64;  // (position, head) query rows per prompt item, 16 per wave

struct AttnParams {
  const char* q;
  int64_t q_st, q_sh;  // bytes
  const char* k_cache;  // paged: the key cache; packed: keys [Tk, Hkv, DQK]
  const char* v_cache;  // paged: the value cache; packed: values [Tk, Hkv, DV]
  int64_t c_sb, c_st, c_sh;  // bytes: key page / row / head strides (page stride unused when packed)
  int64_t v_st, v_sh;        // bytes: value row / head strides (a paged cache: equal to c_st / c_sh)
  bool paged;                // keys through block tables, else packed by cu_k
  int32_t causal;            // bottom-right causal mask, else every query sees its row's keys
  FastDiv bs;                // tokens per page
  const int32_t* tables;
  int64_t t_stride;  // elements
  const int32_t* cu_q;
  const int32_t* lens_k;
  const int32_t* cu_k;
  int32_t rows, hq, hkv, group, qgroups;
  float scale_log2;  // softmax scale * log2(e): scores live in the exp2 domain
  char* out;
  int64_t o_st, o_sh;  // bytes
  float* lse;          // optional natural log-sum-exp of prompt rows [T, Hq]
  int64_t lse_st, lse_sh;  // elements
  int32_t split;       // S: keys per decode item
  int32_t max_splits;
  float* part_o;    // [rows][hq][max_splits][D] normalised partial outputs
  float* part_lse;  // [rows][hq][max_splits] log2-sum-exp2 of the partials
  const int2* items;
  const int32_t* n_items;
};

__device__ inline int key_len(const AttnParams& p, int row) {
  return p.lens_k ? p.lens_k[row] : p.cu_k[row + 1] - p.cu_k[row];
}

// ---------------------------------------------------------------------------------------------------------
// Prompt item: (row, tile of query positions, kv head). The 64 (position, head) query rows of one GQA group
// (16 per wave) run against 64-key tiles staged row-major in LDS, the next tile's K/V loads in flight in
// registers meanwhile. S^T = K Q^T and O^T += V^T P^T on MFMA 16x16x32 with fp32 accumulation; the V^T
// operands come from the row-major value tile by the transposing LDS read. Online softmax per query row;
// bottom-right causal mask (query j of a row with lq queries and lk keys sees keys 0 .. lk - lq + j) unless
// p.causal is 0. DQK: q.k width; DV: value width.

template <int DQK, int DV>
struct PromptSmem {
  static constexpr int kKRow = DQK + 8;   // key tile row pitch, elements: conflict-free operand reads
  static constexpr int kVRow = DV + 16;   // value tile row pitch, elements: conflict-free transposing reads
  static constexpr int kBytes = kPrefillKeys * (kKRow + kVRow) * 2;
};

template <typename T, int DQK, int DV>
__device__ void prefill_item(const AttnParams& p, int row, int qtile, int kvh, char* smem) {
  using E = Elem<T>;
  constexpr int KS = DQK / 32;  // MFMA k-steps over the q.k width
  constexpr int DB = DV / 16;   // 16-dim blocks of the output
  constexpr int KROW = PromptSmem<DQK, DV>::kKRow;
  constexpr int VROW = PromptSmem<DQK, DV>::kVRow;
  constexpr int KCH = DQK / 8, VCH = DV / 8;  // 16-byte chunks per key / value row
  constexpr int KCHUNKS = kPrefillKeys * KCH;
  constexpr int PER = kPrefillKeys * (KCH + VCH) / 256;  // chunks each thread stages per tile
  static_assert(kPrefillKeys * (KCH + VCH) % 256 == 0, "tile chunks split evenly over 256 threads");
  static_assert(DQK % 32 == 0 && DV % 16 == 0, "MFMA tile widths");
  uint16_t* ks = reinterpret_cast<uint16_t*>(smem);  // [64 keys][KROW]
  uint16_t* vs = ks + kPrefillKeys * KROW;            // [64 keys][VROW]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, j4 = lane >> 4;
  const int G = p.group;
  const int qp = kPrefillRows / G;  // positions per item
  const int q0 = p.cu_q[row], lq = p.cu_q[row + 1] - q0;
  const int lk = key_len(p, row);
  const int p0 = qtile * qp;
  if (p0 >= lq) return;  // a grid sized for the longest row

  const int mrow = wave * 16 + n;
  const int qi = p0 + mrow / G;
  const int head = kvh * G + mrow % G;
  const bool qvalid = mrow < qp * G && qi < lq;
  u32x4 qb[KS];
#pragma unroll
  for (int k = 0; k < KS; ++k)
    qb[k] = qvalid ? ld16(p.q + (int64_t)(q0 + qi) * p.q_st + head * p.q_sh + (int64_t)(32 * k + 8 * j4) * 2)
                   : u32x4{0, 0, 0, 0};
  // This query row sees keys < lim; the item needs keys < kmax.
  const int lim = qvalid && p.causal ? lk - lq + qi + 1 : lk;
  const int kmax = p.causal ? min(lk, lk - lq + min(p0 + qp, lq)) : lk;

  float mrun = -INFINITY, lrun = 0.f;
  f32x4 o[DB];
#pragma unroll
  for (int b = 0; b < DB; ++b) o[b] = f32x4{0, 0, 0, 0};

  const int32_t* table = p.tables + (int64_t)row * p.t_stride;
  const int kbase = p.paged ? 0 : p.cu_k[row];
  // Byte offset of key row j of this kv head in the key (v = false) or value (v = true) source.
  auto row_off = [&](int j, bool v) -> int64_t {
    const int64_t st = v ? p.v_st : p.c_st, sh = v ? p.v_sh : p.c_sh;
    if (p.paged) {
      const int pg = (int)p.bs.div(j);
      return (int64_t)table[pg] * p.c_sb + (int64_t)(j - pg * (int)p.bs.d) * st + (int64_t)kvh * sh;
    }
    return (int64_t)(kbase + j) * st + (int64_t)kvh * sh;
  };
  // Keys past the row are staged as zeros: their weight is 0 and 0 * NaN must not happen.
  auto fetch = [&](int kt, u32x4 (&st)[PER]) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = tid + 256 * i;
      const bool isv = c >= KCHUNKS;
      const int cc = isv ? c - KCHUNKS : c;
      const int key = isv ? cc / VCH : cc / KCH;
      const int part = isv ? cc - key * VCH : cc - key * KCH;
      const int jk = kt + key;
      st[i] = jk < lk ? ld16((isv ? p.v_cache : p.k_cache) + row_off(jk, isv) + part * 16) : u32x4{0, 0, 0, 0};
    }
  };
  auto stash = [&](const u32x4 (&st)[PER]) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = tid + 256 * i;
      const bool isv = c >= KCHUNKS;
      const int cc = isv ? c - KCHUNKS : c;
      const int key = isv ? cc / VCH : cc / KCH;
      const int part = isv ? cc - key * VCH : cc - key * KCH;
      st16(reinterpret_cast<char*>(isv ? vs + key * VROW + part * 8 : ks + key * KROW + part * 8), st[i]);
    }
  };

  u32x4 stage[PER];
  if (kmax > 0) fetch(0, stage);
  for (int kt = 0; kt < kmax; kt += kPrefillKeys) {
    __syncthreads();  // the previous tile's operand reads are done
    stash(stage);
    __syncthreads();
    if (kt + kPrefillKeys < kmax) fetch(kt + kPrefillKeys, stage);

    // S^T (keys x query rows): lane holds keys kt + 16 kb + 4 j4 + r of query row n.
    f32x4 st[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      st[kb] = f32x4{0, 0, 0, 0};
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(ks + (kb * 16 + n) * KROW + 32 * k + 8 * j4);
        st[kb] = E::mfma16x16x32(a, qb[k], st[kb]);
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kt + kb * 16 + 4 * j4 + r;
        const float s = key < lim ? st[kb][r] * p.scale_log2 : -INFINITY;
        st[kb][r] = s;
        mx = fmaxf(mx, s);
      }
    mx = xor32_max(xor16_max(mx));
    const float mnew = fmaxf(mrun, mx);
    const float mref = mnew == -INFINITY ? 0.f : mnew;
    const float alpha = fast_exp2(mrun - mref);
    mrun = mnew;
    float psum = 0.f;
    u32x4 pb[2];  // P^T operands: k slots 8 j4 .. 8 j4 + 7 = keys 32 h + 4 j4 + 0..3, then 32 h + 16 + 4 j4 + 0..3
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float pr[8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pr[r] = fast_exp2(st[2 * h][r] - mref);
        pr[4 + r] = fast_exp2(st[2 * h + 1][r] - mref);
      }
#pragma unroll
      for (int r = 0; r < 8; ++r) psum += pr[r];
#pragma unroll
      for (int w = 0; w < 4; ++w) pb[h][w] = E::pack(pr[2 * w], pr[2 * w + 1]);
    }
    lrun = lrun * alpha + psum;
    // V^T operand rows (dims) 16 b + n; transposing reads of rows 32 h + 4 j4 + (n >> 2) (+ 16), dims + 4 (n & 3).
    const uint16_t* vrow = vs + (4 * j4 + (n >> 2)) * VROW + 4 * (n & 3);
#pragma unroll
    for (int b = 0; b < DB; ++b) {
      o[b] *= alpha;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const u32x2 lo = lds_read_tr16(vrow + 32 * h * VROW + 16 * b);
        const u32x2 hi = lds_read_tr16(vrow + (32 * h + 16) * VROW + 16 * b);
        o[b] = E::mfma16x16x32(u32x4{lo[0], lo[1], hi[0], hi[1]}, pb[h], o[b]);
      }
    }
  }

  lrun = xor32_sum(xor16_sum(lrun));
  if (qvalid) {
    const float inv = lrun > 0.f ? 1.f / lrun : 0.f;
    char* dst = p.out + (int64_t)(q0 + qi) * p.o_st + head * p.o_sh;
#pragma unroll
    for (int b = 0; b < DB; ++b) {
      const u32x2 packed = {E::pack(o[b][0] * inv, o[b][1] * inv), E::pack(o[b][2] * inv, o[b][3] * inv)};
      *reinterpret_cast<u32x2*>(dst + (int64_t)(b * 16 + 4 * j4) * 2) = packed;
    }
    if (p.lse && j4 == 0)
      p.lse[(int64_t)(q0 + qi) * p.lse_st + (int64_t)head * p.lse_sh] =
          lrun > 0.f ? (mrun + fast_log2(lrun)) * kLn2 : -INFINITY;
  }
}

}  // namespace lv
