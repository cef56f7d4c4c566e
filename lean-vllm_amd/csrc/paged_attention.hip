// Paged attention for a continuous-batching step on gfx950: pure decode, chunked prefill, or both in one launch.
//
// Work items (one workgroup of 4 waves each):
//   decode item  = (row, split, kv head or pair of kv heads, query-head group): a row with one query, keys
//                  [split*S, (split+1)*S). Streaming, bandwidth-bound: each wave takes every 4th tile of the
//                  range; a token's head row (D elements) is spread over 16 lanes as 16-byte loads (the two head
//                  rows of a pair, adjacent in the cache, over 32); q.k by v_dot2 with a DPP butterfly inside the
//                  16-lane row; online softmax per tile; p.v on the VALU in fp32. The four waves and, for long
//                  rows, the splits are merged by log-sum-exp (a row's splits by whichever finishes last).
//   prompt item  = (row, q tile, kv head): a row with several queries; the MFMA tile of attn_common.h.
// Launches read a work list built on the device by plan_kernel from the key lengths (and cu_seqlens_q), longest
// work first; its workspace also holds the split rows' partials and their merge counters.
//
// Math: TorchAttention.decode / prefill (lean_vllm/attention/torch_backend.py:62-103,159-181): query head h reads
// key head h / (Hq/Hkv); query j of a row with lq queries and lk keys sees keys 0..lk-lq+j.
#include <algorithm>
#include <mutex>

#include "attn_common.h"

namespace lv {

constexpr int kTile = 16;          // decode tokens per tile; block sizes are multiples of 16, so a tile sits in one block
constexpr int kWaves = 4;          // waves per workgroup
constexpr int kPlanMaxRows = 4096;  // rows of a step with prompts (the work-list scan lives in LDS)

constexpr int kPromptRing = 2;        // LDS stages of the prompt tiles' ring
constexpr int kOverlapCusPct = 44;    // percent of the CUs that hold a prompt workgroup in a mixed step by default
constexpr int kOverlapCusMaxPct = 75;  // at most this percent when the caller sizes the prompt share
constexpr int kDecodeWgs = 2;         // persistent decode workgroups per CU outside the overlap
constexpr int kOverlapDecodeWgs = 3;  // persistent decode workgroups per CU beside a mixed step's prompt workgroups
                                      // (at most: pair items at D = 128 fit two)
constexpr int kSplitTarget = 4096;    // decode items (x kv heads x query-head groups) a split-K grid aims for
constexpr int kMinSplit = 256;        // keys per decode item at least
constexpr int kSmallStepRounds = 8;   // a mixed step of at most this many GPU-fulls of workgroups is one launch

// ---------------------------------------------------------------------------------------------------------
// Decode item.
//
// Lane layout (D = 128): 16 lanes hold one token's head row, 16 bytes (8 dims) each. With one kv head per item
// (HP = 1) the wave's 4 lane groups take 4 tokens at a time, 4 times per 16-token tile; with a pair (HP = 2) lanes
// 0-31 take one token's two head rows (512 contiguous bytes of an NHD token row) and lanes 32-63 the next token's.
// Scores stay in raw q.k units; the softmax scale (positive) and log2(e) are folded into the exp2 argument. The
// running max is uniform over the lanes of a head, so rescaling the accumulators is a branch taken only when a
// tile raises some head's max. p.v runs as 2-term dot products over token pairs with p in
// the 16-bit format of the cache (fp32 accumulation), as the MFMA path does with its probability tiles.

// Reduce over the lane groups of a wave that hold different tokens of one head (lanes i, i + LPH, i + 2 LPH, ...;
// LPH lanes hold a token's piece of the item's head rows).
template <int LPH>
__device__ inline float groups_max(float x) {
  static_assert(LPH == 8 || LPH == 16 || LPH == 32, "8, 16 or 32 lanes per token piece");
  if constexpr (LPH == 8) x = vmax(x, dpp_ror8(x));  // lanes i and i ^ 8 of each 16-lane row
  if constexpr (LPH <= 16) x = xor16_max(x);
  return xor32_max(x);
}
template <int LPH>
__device__ inline float groups_sum(float x) {
  static_assert(LPH == 8 || LPH == 16 || LPH == 32, "8, 16 or 32 lanes per token piece");
  if constexpr (LPH == 8) x += dpp_ror8(x);
  if constexpr (LPH <= 16) x = xor16_sum(x);
  return xor32_sum(x);
}

// A split row's partials pass between workgroups that may run on different XCDs, whose L2 caches are not coherent
// with each other. They are stored and loaded as device-scope relaxed atomics (global_store / global_load with sc1:
// written through to memory, read past the L2), so neither side needs a whole-L2 writeback or invalidate.
__device__ __forceinline__ void coherent_store(float* ptr, float v) {
  __hip_atomic_store(ptr, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coherent_load(const float* ptr) {
  return __hip_atomic_load(ptr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Merge of a split row's partial outputs for dims d0 .. d0 + PER - 1 of query head `head`, written to the output row
// `tok`: o = sum_s 2^(lse_s - M) o_s / sum_s 2^(lse_s - M). The partials are read kMergeBatch splits at a time, every
// load of a batch issued before the first is used, with the max and the sums carried from batch to batch (a long
// row's 32 splits are two round trips to memory, not 64). Each output element's arithmetic depends only on its own
// head and dim, so any spread of the elements over threads gives the same bits.
constexpr int kMergeBatch = 16;
template <typename T, int D, int PER>
__device__ __forceinline__ void merge_split_partials(const AttnParams& p, int row, int tok, int head, int nsplit,
                                                     int d0) {
  using E = Elem<T>;
  static_assert(PER == 1 || PER == 2, "one or two dims per thread");
  const int64_t slot0 = ((int64_t)row * p.hq + head) * p.max_splits;
  float m = -INFINITY, den = 0.f, o[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) o[e] = 0.f;
  for (int s0 = 0; s0 < nsplit; s0 += kMergeBatch) {
    float ls[kMergeBatch], x[kMergeBatch][PER];
#pragma unroll
    for (int i = 0; i < kMergeBatch; ++i) {
      ls[i] = -INFINITY;
#pragma unroll
      for (int e = 0; e < PER; ++e) x[i][e] = 0.f;
      if (s0 + i < nsplit) {  // uniform over the threads of a row
        ls[i] = coherent_load(p.part_lse + slot0 + s0 + i);
        const float* src = p.part_o + (slot0 + s0 + i) * D;
#pragma unroll
        for (int e = 0; e < PER; ++e) x[i][e] = coherent_load(src + d0 + e);
      }
    }
    float bm = m;
#pragma unroll
    for (int i = 0; i < kMergeBatch; ++i) bm = fmaxf(bm, ls[i]);
    if (bm == -INFINITY) continue;
    const float alpha = fast_exp2(m - bm);  // 0 while m is -inf
    den *= alpha;
#pragma unroll
    for (int e = 0; e < PER; ++e) o[e] *= alpha;
#pragma unroll
    for (int i = 0; i < kMergeBatch; ++i) {
      const float w = fast_exp2(ls[i] - bm);  // 0 past the last split
      den += w;
#pragma unroll
      for (int e = 0; e < PER; ++e) o[e] = fmaf(w, x[i][e], o[e]);
    }
    m = bm;
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  char* dst = p.out + tok * p.o_st + head * p.o_sh + (int64_t)d0 * 2;
  if constexpr (PER == 2) {
    *reinterpret_cast<uint32_t*>(dst) = E::pack(o[0] * inv, o[1] * inv);
  } else {
    *reinterpret_cast<uint16_t*>(dst) = (uint16_t)(E::pack(o[0] * inv, 0.f) & 0xffffu);
  }
}

// publish (persistent launches): thread 0 stores publish_value there before the item's merge barrier, and the
// barrier is met even by an item with nothing to do, so the whole workgroup reads the value after the call.
template <typename T, int D, int GS, int HP, int US = 0>
__device__ void decode_item(const AttnParams& p, int row, int split, int kvh, int qg, char* smem,
                            int* publish = nullptr, int publish_value = 0) {
  using E = Elem<T>;
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static_assert(HP == 1 || HP == 2, "one or two kv heads per item");
  constexpr int LPT = D / 8;      // lanes per token head row, 16 bytes each
  constexpr int LPH = LPT * HP;   // lanes per token piece: the item's HP head rows, adjacent in a token's NHD row
  constexpr int TPI = 64 / LPH;   // tokens per wave step
  constexpr int KT = US > 0 ? TPI * US : kTile / HP;  // tokens per wave tile
  constexpr int U = KT / TPI;     // load steps per wave tile
  static_assert(U % 2 == 0, "token pairs");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = lane / LPH, hs = (lane / LPT) % HP, part = lane % LPT;

  const int lk = key_len(p, row);
  const int kbeg = split * p.split;
  // Past the row's end (the grid is sized for the longest row), or past the bound the caller gave.
  const bool valid = !((split > 0 && kbeg >= lk) || split >= p.max_splits);
  if (!valid && !publish) return;
  const int kend = valid ? min(lk, kbeg + p.split) : kbeg;
  const int nsplit = min((lk + p.split - 1) / p.split, p.max_splits);
  const int tok = p.cu_q ? p.cu_q[row] : row;
  const int head0 = (kvh + hs) * p.group + qg * GS;  // this lane's query heads (kvh: the item's first kv head)
  const float c = p.scale_log2;

  u32x4 qv[GS];
#pragma unroll
  for (int g = 0; g < GS; ++g) qv[g] = ld16(p.q + tok * p.q_st + (head0 + g) * p.q_sh + part * 16);

  float m[GS], l[GS], acc[GS][8];
#pragma unroll
  for (int g = 0; g < GS; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }

  // Byte offset of this lane's 16 bytes of step u inside a tile (tile rows are p.c_st apart; fits 32 bits).
  uint32_t loff[U];
#pragma unroll
  for (int u = 0; u < U; ++u) loff[u] = (uint32_t)((u * TPI + grp) * p.c_st + hs * p.c_sh + part * 16);
  const int32_t* table = p.tables + (int64_t)row * p.t_stride;

  // Page numbers come through the scalar cache, once per page this wave enters: a vector load of the table would
  // be waited for in order with the K/V loads already in flight.
  int cached_pg = -1;
  int64_t cached_base = 0;
  auto tile_base = [&](int t0) {
    const int pg = (int)p.bs.div(t0);
    if (pg != cached_pg) {
      cached_pg = pg;
      cached_base = (int64_t)sload(table + pg) * p.c_sb + (int64_t)kvh * p.c_sh;
    }
    return cached_base + (int64_t)(t0 - pg * (int)p.bs.d) * p.c_st;
  };
  auto load_rows = [&](const char* cache, int64_t base, u32x4 (&x)[U]) {
    const char* b = cache + base;
#pragma unroll
    for (int u = 0; u < U; ++u) x[u] = ld16_stream(b + loff[u]);
  };
  // Scores of a tile -> online-softmax update -> probabilities packed in token pairs, per query head.
  auto qk = [&](int t0, const u32x4 (&kv)[U], uint32_t (&pp)[GS][U / 2]) {
    float s[U][GS];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int g = 0; g < GS; ++g) {
        float d = E::dot2(qv[g][0], kv[u][0], 0.f);
#pragma unroll
        for (int w = 1; w < 4; ++w) d = E::dot2(qv[g][w], kv[u][w], d);
        s[u][g] = group_sum<LPT>(d);
      }
    if (t0 + KT > kend) {  // wave-uniform: the row's last tile; tokens past it get no weight
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool in = t0 + u * TPI + grp < kend;
#pragma unroll
        for (int g = 0; g < GS; ++g) s[u][g] = in ? s[u][g] : -INFINITY;
      }
    }
    float mt[GS];
    int grow = 0;
#pragma unroll
    for (int g = 0; g < GS; ++g) {
      float x = s[0][g];
#pragma unroll
      for (int u = 1; u < U; ++u) x = vmax(x, s[u][g]);
      mt[g] = groups_max<LPH>(x);  // finite: every tile holds a token in range
      grow |= mt[g] > m[g];
    }
    // One kv head per item: the max is wave-uniform. Two: each head's lanes hold their own, and a lane whose max did
    // not grow rescales by 1.
    if (HP == 1 ? __builtin_amdgcn_readfirstlane(grow) != 0 : __builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
      for (int g = 0; g < GS; ++g) {
        const float mn = vmax(m[g], mt[g]);
        const float alpha = fast_exp2((m[g] - mn) * c);
        m[g] = mn;
        l[g] *= alpha;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] *= alpha;
      }
    }
#pragma unroll
    for (int g = 0; g < GS; ++g) {
      const float mc = m[g] * c;
#pragma unroll
      for (int u = 0; u < U; u += 2) {
        const float p0 = fast_exp2(fmaf(s[u][g], c, -mc));
        const float p1 = fast_exp2(fmaf(s[u + 1][g], c, -mc));
        l[g] += p0 + p1;
        pp[g][u / 2] = E::pack(p0, p1);
      }
    }
  };
  // acc += p . V over the tile: value rows of token pairs interleaved per dim, 2-term dot products.
  auto pv = [&](int t0, u32x4 (&vv)[U], const uint32_t (&pp)[GS][U / 2]) {
    if (t0 + KT > kend) {  // values past the range may be NaN: zero them (their p is 0)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool in = t0 + u * TPI + grp < kend;
#pragma unroll
        for (int w = 0; w < 4; ++w) vv[u][w] = in ? vv[u][w] : 0u;
      }
    }
#pragma unroll
    for (int u = 0; u < U; u += 2)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t lo = __builtin_amdgcn_perm(vv[u + 1][w], vv[u][w], 0x05040100u);
        const uint32_t hi = __builtin_amdgcn_perm(vv[u + 1][w], vv[u][w], 0x07060302u);
#pragma unroll
        for (int g = 0; g < GS; ++g) {
          acc[g][2 * w] = E::dot2(pp[g][u / 2], lo, acc[g][2 * w]);
          acc[g][2 * w + 1] = E::dot2(pp[g][u / 2], hi, acc[g][2 * w + 1]);
        }
      }
  };

  constexpr int kStride = KT * kWaves;
  int t0 = kbeg + KT * wave;
  if (t0 < kend) {
    // Staggered: the next tile's keys load during this tile's p.v, its values during its own q.k.
    u32x4 kv[U], vv[U];
    uint32_t pp[GS][U / 2];
    int64_t base = tile_base(t0);
    load_rows(p.k_cache, base, kv);
    load_rows(p.v_cache, base, vv);
    while (true) {
      qk(t0, kv, pp);
      const int t1 = t0 + kStride;
      int64_t next = 0;
      if (t1 < kend) {
        next = tile_base(t1);
        load_rows(p.k_cache, next, kv);
      }
      pv(t0, vv, pp);
      if (t1 >= kend) break;
      load_rows(p.v_cache, next, vv);
      t0 = t1;
    }
  }

  // Sum the token groups of the wave (they share m); m moves to the log2 domain of the merges.
#pragma unroll
  for (int g = 0; g < GS; ++g) {
    l[g] = groups_sum<LPH>(l[g]);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = groups_sum<LPH>(acc[g][e]);
    m[g] *= c;
  }
  // Merge the waves through LDS: wm/wl [kWaves][HG], wacc [kWaves][HG][D] for the item's HG = HP GS query heads
  // (lanes of token group 0 hold their head's sums).
  constexpr int HG = HP * GS;
  float* wm = reinterpret_cast<float*>(smem);
  float* wl = wm + kWaves * HG;
  float* wacc = wl + kWaves * HG;
  if (lane < LPH) {
#pragma unroll
    for (int g = 0; g < GS; ++g) {
      const int hg = wave * HG + hs * GS + g;
#pragma unroll
      for (int e = 0; e < 8; ++e) wacc[hg * D + part * 8 + e] = acc[g][e];
      if (part == 0) {
        wm[hg] = m[g];
        wl[hg] = l[g];
      }
    }
  }
  if (publish && threadIdx.x == 0) *publish = publish_value;
  __syncthreads();
  if (!valid) return;
  // One thread per 8 output elements.
  for (int c = threadIdx.x; c < HG * D / 8; c += blockDim.x) {
    const int g = c / (D / 8), d0 = (c % (D / 8)) * 8;  // g: query head of the item, hs-major
    float mmax = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mmax = fmaxf(mmax, wm[w * HG + g]);
    float o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float den = 0.f;
    if (mmax != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float wt = fast_exp2(wm[w * HG + g] - mmax);
        den += wt * wl[w * HG + g];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] += wt * wacc[(w * HG + g) * D + d0 + e];
      }
      const float inv = 1.f / den;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] *= inv;
    }
    const int head = (kvh + g / GS) * p.group + qg * GS + g % GS;
    if (nsplit <= 1) {
      u32x4 packed;
#pragma unroll
      for (int w = 0; w < 4; ++w) packed[w] = E::pack(o[2 * w], o[2 * w + 1]);
      st16(p.out + tok * p.o_st + head * p.o_sh + (int64_t)d0 * 2, packed);
    } else {
      const int64_t slot = ((int64_t)row * p.hq + head) * p.max_splits + split;
      float* dst = p.part_o + slot * D + d0;
#pragma unroll
      for (int e = 0; e < 8; ++e) coherent_store(dst + e, o[e]);
      if (d0 == 0) coherent_store(p.part_lse + slot, mmax == -INFINITY ? -INFINITY : mmax + fast_log2(den));
    }
  }
  // A split row: the split that counts in last merges the item's heads. Each wave waits until its partial stores
  // are complete (written through to memory) before the barrier that precedes the count, so every split's partials
  // are in memory before its count; the merger reads them past its L2 after its own count has returned.
  if (nsplit > 1 && p.merge_count) {
    __shared__ int s_last;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int32_t* count = p.merge_count + (row * (p.hkv / HP) + kvh / HP) * p.qgroups + qg;
    if (threadIdx.x == 0)
      s_last = __hip_atomic_fetch_add(count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nsplit - 1;
    __syncthreads();
    if (s_last) {
      for (int c = threadIdx.x; c < HG * D / 2; c += blockDim.x) {
        const int g = c / (D / 2), d0 = (c % (D / 2)) * 2;
        merge_split_partials<T, D, 2>(p, row, tok, (kvh + g / GS) * p.group + qg * GS + g % GS, nsplit, d0);
      }
      // Back to zero for the next layer on this plan.
      if (threadIdx.x == 0) __hip_atomic_store(count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------
// Kernels.

template <int D, int GS, int HP>
struct SmemBytes {
  static constexpr int kDecode = kWaves * HP * GS * (D + 2) * 4;
};

// Work-list kernels. blockIdx.x walks the device work list with the query-head groups innermost, so workgroups
// are dispatched in list order (longest first). The list holds a step's prompt items first (n_items[1] of them),
// then its decode items (n_items[0] in all). Decode items run in decode_list_kernel at the decode item's register
// budget; prompt items in prompt_list_kernel, whose MFMA tile needs more registers and LDS.
template <typename T, int D, int GS, int HP, int US = 0>
__global__ __launch_bounds__(256) void decode_list_kernel(AttnParams p) {
  __shared__ __attribute__((aligned(16))) char smem[SmemBytes<D, GS, HP>::kDecode];
  const int ny = p.hkv / HP * p.qgroups;
  const int bx = blockIdx.x / ny, by = blockIdx.x - bx * ny;
  const int kh = by / p.qgroups, qg = by - kh * p.qgroups;
  const int i = bx + p.n_items[1];
  if (i >= p.n_items[0]) return;
  const int2 it = p.items[i];
  decode_item<T, D, GS, HP, US>(p, it.x, it.y, kh * HP, qg, smem);
}

// Decode items of the work list on a persistent grid beside a mixed step's prompt workgroups: each workgroup takes
// items by ticket (an atomic counter the plan kernel zeroes), in list order, so the longest still go first. A
// fixed number of workgroups per CU lets the prompt workgroups stay resident beside them (outside the overlap,
// one workgroup per item measured as fast or faster). The next ticket is drawn at the start of an item and
// published at its merge barrier; the merge alternates between two LDS buffers, so one barrier per item suffices.
// The last workgroup to finish puts the ticket and the exit count back to zero, so the next layer of the step can
// run on the same plan without a plan launch: every workgroup's ticket draws have returned (their values were
// read) before it counts itself out, so no draw can follow the reset.
template <typename T, int D, int GS, int HP, int US = 0>
__device__ __forceinline__ void decode_persistent(const AttnParams& p) {
  __shared__ __attribute__((aligned(16))) char smem[2][SmemBytes<D, GS, HP>::kDecode];
  __shared__ int s_ticket[2];
  const int ny = p.hkv / HP * p.qgroups;
  const int first = p.n_items[1];
  const int total = (p.n_items[0] - first) * ny;
  if (threadIdx.x == 0) s_ticket[0] = atomicAdd(p.ticket, 1);
  __syncthreads();
  int f = __builtin_amdgcn_readfirstlane(s_ticket[0]);
  for (int k = 0; f < total; ++k) {
    int next = 0;
    if (threadIdx.x == 0) next = atomicAdd(p.ticket, 1);
    const int bx = f / ny, by = f - bx * ny;
    const int kh = by / p.qgroups, qg = by - kh * p.qgroups;
    const int2 it = p.items[first + bx];
    decode_item<T, D, GS, HP, US>(p, it.x, it.y, kh * HP, qg, smem[k & 1], &s_ticket[(k + 1) & 1], next);
    f = __builtin_amdgcn_readfirstlane(s_ticket[(k + 1) & 1]);
  }
  if (threadIdx.x == 0 && atomicAdd(p.ticket + 1, 1) == (int)gridDim.x - 1) {
    atomicExch(p.ticket, 0);
    atomicExch(p.ticket + 1, 0);
  }
}

// Load steps of a wave tile: pair items at D = 128 hold 16-token wave tiles (8 load steps, twice the bytes in
// flight per wave of the 8-token tile, about 210 registers); other shapes keep the kTile / HP default.
template <int D, int HP>
constexpr int kWideSteps = HP == 2 && D == 128 ? 8 : 0;

// Beside a mixed step's prompt workgroups (one per CU; a prompt wave takes 193 registers, allocated as 200) the
// decode workgroups share each SIMD's 512 registers per lane: one pair-item workgroup at D = 128 (210) beside a
// prompt wave and two on the other CUs; the smaller items of other shapes (131 or fewer) two beside a prompt wave
// and three on the others. The grid asks for up to three per CU, as many as fit alone.
template <typename T, int D, int GS, int HP>
__global__ __launch_bounds__(256, 2) void decode_beside_kernel(AttnParams p) {
  decode_persistent<T, D, GS, HP, kWideSteps<D, HP>>(p);
}

// TP: pages per 64-key prompt tile. TP > 0 (pages of a multiple of 64 keys, or of 32 or 16): the tiles stream
// through an LDS ring of kPromptRing stages; TP = 0 (other page sizes): through registers.
template <int TP>
constexpr int kRingOf = TP > 0 ? kPromptRing : 0;

template <typename T, int D, int TP>
__global__ __launch_bounds__(256, 2) void prompt_list_kernel(AttnParams p) {
  constexpr int RING = kRingOf<TP>;
  __shared__ __attribute__((aligned(16))) char smem[(RING > 0 ? RING : 1) * PromptSmem<D, D, (TP > 1)>::kBytes];
  const int bx = blockIdx.x / p.hkv, kvh = blockIdx.x - bx * p.hkv;
  if (bx >= p.n_items[1]) return;
  const int2 it = p.items[bx];
  prefill_item<T, D, D, true, false, RING, 4, false, (TP > 0 ? TP : 1)>(p, it.x, -1 - it.y, kvh, smem);
}

// Prompt items of a mixed step, run at the same time as its decode items: one workgroup per CU, each walking the
// prompt items blockIdx.x, + gridDim.x, ... in list order. Its LDS request (padded at launch, so the compiler still
// budgets registers for 2 waves per SIMD) leaves room for no second one, and the decode workgroups take the CU's
// remaining registers: the MFMA work of the prompt tiles hides under the decode rows' memory streaming.
constexpr int kOverlapLds = 84 * 1024;
template <typename T, int D, int TP>
__global__ __launch_bounds__(256, 2) void prompt_overlap_kernel(AttnParams p) {
  constexpr int RING = kRingOf<TP>;
  __shared__ __attribute__((aligned(16))) char smem[(RING > 0 ? RING : 1) * PromptSmem<D, D, (TP > 1)>::kBytes];
  // The prompt tiles are the step's critical path beside the decode waves, which need few issue slots: the prompt
  // waves win the SIMD's issue arbitration (1% on the Qwen3-8B mixed step; favouring the decode waves costs 15%).
  __builtin_amdgcn_s_setprio(1);
  const int n = p.n_items[1] * p.hkv;
  for (int f = blockIdx.x; f < n; f += gridDim.x) {
    const int bx = f / p.hkv, kvh = f - bx * p.hkv;
    const int2 it = p.items[bx];
    prefill_item<T, D, D, true, true, RING, 4, false, (TP > 0 ? TP : 1)>(p, it.x, -1 - it.y, kvh, smem);
    __syncthreads();  // the next item restages the LDS tiles
  }
}

// A small mixed step in one launch: workgroups [0, prompt_wgs) take the prompt items (one per item and kv head, the
// longest first), the rest the decode items in list order. Dispatched in that order, the prompt workgroups start
// first and the decode workgroups stream through the slots they leave, as in the overlapped schedule but without a
// second stream, its events and one launch: for steps of a few hundred rows, whose launch sequence is a large share
// of their time.
template <typename T, int D, int GS, int TP, int HP>
__global__ __launch_bounds__(256, 2) void mixed_small_kernel(AttnParams p, int32_t prompt_wgs) {
  constexpr int RING = kRingOf<TP>;
  static_assert(SmemBytes<D, GS, HP>::kDecode <= (RING > 0 ? RING : 1) * PromptSmem<D, D, (TP > 1)>::kBytes,
                "LDS for both");
  __shared__ __attribute__((aligned(16))) char smem[(RING > 0 ? RING : 1) * PromptSmem<D, D, (TP > 1)>::kBytes];
  const int b = blockIdx.x;
  if (b < prompt_wgs) {
    const int bx = b / p.hkv, kvh = b - bx * p.hkv;
    if (bx >= p.n_items[1]) return;
    const int2 it = p.items[bx];
    prefill_item<T, D, D, true, false, RING, 4, false, (TP > 0 ? TP : 1)>(p, it.x, -1 - it.y, kvh, smem);
  } else {
    const int ny = p.hkv / HP * p.qgroups;
    const int f = b - prompt_wgs, bx = f / ny, by = f - bx * ny;
    const int kh = by / p.qgroups, qg = by - kh * p.qgroups;
    const int i = bx + p.n_items[1];
    if (i >= p.n_items[0]) return;
    const int2 it = p.items[i];
    decode_item<T, D, GS, HP>(p, it.x, it.y, kh * HP, qg, smem);
  }
}

// Decode of more rows than the planner holds: blockIdx.x is (row, split), blockIdx.y the query-head group. Such a
// step is planned unsplit (max_splits 1): a split row's partials need the merge counters of a work list.
template <typename T, int D, int GS, int HP>
__global__ __launch_bounds__(256) void decode_grid_kernel(AttnParams p) {
  __shared__ __attribute__((aligned(16))) char smem[SmemBytes<D, GS, HP>::kDecode];
  const int kh = blockIdx.y / p.qgroups, qg = blockIdx.y % p.qgroups;
  decode_item<T, D, GS, HP>(p, blockIdx.x / p.max_splits, blockIdx.x % p.max_splits, kh * HP, qg, smem);
}

constexpr int kLenBuckets = 64;
// Bucket of a split of `keys` keys out of `split`: longer splits get smaller buckets (dispatched first).
__device__ inline int len_bucket(int keys, int split) {
  const int b = (int)(((int64_t)(split - keys) * kLenBuckets) / split);
  return b < kLenBuckets - 1 ? b : kLenBuckets - 1;
}

// Work list of a step, longest work first: prompt items (row, -1 - tile), then every full decode split (row, s),
// then each decode row's last split (row, n - 1) by decreasing key count (counting sort over length buckets).
// In-order dispatch of that list approximates longest-processing-time scheduling, so the launch ends with short
// items instead of a tail of full ones. A prompt row's tiles go last tile first (most keys) when the prompt items
// have the GPU to themselves (last_first: a step of prompts, or the serial schedule): the Qwen3-8B chunks 5-6%
// faster than first tile first. Beside the decode rows (the overlapped schedule) the order made no measurable
// difference, and the first tile goes first there as before. The split rows' merge counters start at zero.
__global__ __launch_bounds__(kScanThreads) void plan_kernel(const int32_t* __restrict__ cu_q,
                                                            const int32_t* __restrict__ lens_k,
                                                            const int32_t* __restrict__ cu_k, int32_t rows,
                                                            int32_t split, int32_t qp, int32_t max_items,
                                                            int32_t last_first, int2* __restrict__ items,
                                                            int32_t* __restrict__ n_items,
                                                            int32_t* __restrict__ merge_count, int32_t n_merge) {
  __shared__ int pre[kPlanMaxRows + 1];
  __shared__ int full[kPlanMaxRows + 1];
  __shared__ int bucket[kLenBuckets + 1];
  __shared__ int wave_tot[kScanThreads / 64 + 1];
  const int tid = threadIdx.x;
  for (int b = tid; b <= kLenBuckets; b += kScanThreads) bucket[b] = 0;
  for (int i = tid; i < n_merge; i += kScanThreads) merge_count[i] = 0;
  __syncthreads();
  for (int r = tid; r < rows; r += kScanThreads) {
    const int lq = cu_q ? cu_q[r + 1] - cu_q[r] : 1;
    const int lk = lens_k ? lens_k[r] : cu_k[r + 1] - cu_k[r];
    pre[r] = lq > 1 ? (lq + qp - 1) / qp : 0;
    full[r] = 0;
    if (lq == 1) {
      const int n = lk > 0 ? (lk + split - 1) / split : 1;
      full[r] = n - 1;
      atomicAdd(&bucket[len_bucket(lk - (n - 1) * split, split)], 1);
    }
  }
  __syncthreads();
  if (tid < kLenBuckets) {  // wave 0: the bucket counts to offsets (one bucket per lane)
    static_assert(kLenBuckets == 64, "one wave scans the buckets");
    const int v = bucket[tid];
    const int x = wave_incl_scan(v);
    bucket[tid] = x - v;
    if (tid == kLenBuckets - 1) bucket[kLenBuckets] = x;
  }
  block_scan(pre, rows, wave_tot);  // its barriers also publish the bucket offsets
  block_scan(full, rows, wave_tot);
  const int npre = pre[rows], nfull = full[rows], npart = bucket[kLenBuckets];
  for (int r = tid; r < rows; r += kScanThreads) {
    for (int i = pre[r]; i < pre[r + 1]; ++i)
      if (i < max_items) items[i] = make_int2(r, -1 - (last_first ? pre[r + 1] - 1 - i : i - pre[r]));
    for (int i = full[r]; i < full[r + 1]; ++i)
      if (npre + i < max_items) items[npre + i] = make_int2(r, i - full[r]);
    const int lq = cu_q ? cu_q[r + 1] - cu_q[r] : 1;
    if (lq == 1) {
      const int lk = lens_k ? lens_k[r] : cu_k[r + 1] - cu_k[r];
      const int n = lk > 0 ? (lk + split - 1) / split : 1;
      const int pos = npre + nfull + atomicAdd(&bucket[len_bucket(lk - (n - 1) * split, split)], 1);
      if (pos < max_items) items[pos] = make_int2(r, n - 1);
    }
  }
  if (tid == 0) {
    n_items[0] = min(npre + nfull + npart, max_items);
    n_items[1] = min(npre, max_items);
    n_items[2] = 0;  // the persistent decode launch's ticket counter
    n_items[3] = 0;  // and its count of workgroups done
  }
}

// ---------------------------------------------------------------------------------------------------------
// Host side.

struct Shape {
  int32_t split, max_splits, max_items, max_prompt_items, max_decode_items, gs;
  int64_t merges;  // split rows' merge counters (rows x kv heads x query-head groups), listed steps only
  size_t items_off, count_off, lse_off, o_off, merge_off, bytes;
};

static int pick_gs(int group) {
  if (group % 4 == 0) return 4;
  if (group % 2 == 0) return 2;
  return 1;
}

static Shape plan_shape(int32_t rows, int32_t tokens, int32_t hq, int32_t hkv, int32_t d, int32_t max_k,
                        bool listed) {
  Shape s{};
  const int group = hq / hkv;
  s.gs = pick_gs(group);
  const int64_t units = (int64_t)rows * hkv * (group / s.gs);
  const int64_t keys = max_k > 0 ? max_k : 1;
  // Keys per decode item: enough items to fill the chip several times over, at least 256 keys each. Rows split only
  // in a listed step (whose workspace holds the merge counters); a step of more rows has units beyond the target
  // anyway.
  const int64_t target = kSplitTarget;
  int64_t split = kMinSplit;
  while (split < keys && (!listed || units * ((keys + split - 1) / split) > target)) split *= 2;
  s.split = (int32_t)split;
  s.max_splits = (int32_t)((keys + split - 1) / split);
  const int qp = kPrefillRows / (group > 0 ? group : 1);
  // In 64 bits, saturated: a count past INT32_MAX is far past what one launch holds (check_grids refuses it).
  auto sat = [](int64_t x) { return (int32_t)std::min<int64_t>(x, INT32_MAX); };
  s.max_prompt_items = listed ? sat(((int64_t)tokens + qp - 1) / qp + rows) : 0;
  s.max_decode_items = listed ? sat((int64_t)rows * s.max_splits) : 0;
  s.max_items = sat((int64_t)s.max_prompt_items + s.max_decode_items);
  size_t off = 0;
  s.items_off = off;
  off += (size_t)s.max_items * sizeof(int2);
  off = (off + 255) / 256 * 256;
  s.count_off = off;
  off += 256;
  const size_t parts = s.max_splits > 1 ? (size_t)rows * hq * s.max_splits : 0;
  s.lse_off = off;
  off += parts * sizeof(float);
  off = (off + 255) / 256 * 256;
  s.o_off = off;
  off += parts * d * sizeof(float);
  off = (off + 255) / 256 * 256;
  s.merges = listed && s.max_splits > 1 ? (int64_t)rows * hkv * (group / s.gs) : 0;
  s.merge_off = off;
  off += (size_t)s.merges * sizeof(int32_t);
  s.bytes = off;
  return s;
}

// A second stream per device and the fork/join events that tie it to the caller's stream, created on first use.
// The mutex makes each call's record / wait / launch sequence atomic against calls from other host threads that
// share the device's second stream.
struct SideStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  std::mutex lock;
};
static SideStream* side_stream() {
  static SideStream side[64];
  static std::mutex create;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  SideStream& s = side[dev];
  std::lock_guard<std::mutex> g(create);
  if (!s.stream) {  // default priority, non-blocking with respect to the legacy stream
    hipStream_t st = nullptr;
    hipEvent_t f = nullptr, j = nullptr;
    if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) return nullptr;
    if (hipEventCreateWithFlags(&f, hipEventDisableTiming) != hipSuccess) {
      (void)hipStreamDestroy(st);
      return nullptr;
    }
    if (hipEventCreateWithFlags(&j, hipEventDisableTiming) != hipSuccess) {
      (void)hipEventDestroy(f);
      (void)hipStreamDestroy(st);
      return nullptr;
    }
    s.fork = f;
    s.join = j;
    s.stream = st;
  }
  return &s;
}

// Workgroups of kernel K (256 threads) that one CU holds at once, from its register and LDS needs (cached per
// kernel and device).
template <auto K>
static int resident_per_cu() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cached[dev] > 0) return cached[dev];
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, K, 256, 0) != hipSuccess || n <= 0) n = 1;
  cached[dev] = n;
  return n;
}

// The kernels of one call, decided on the host from the step's shape (the same decision for a launch and for
// lv_paged_attention_launch_info).
struct StepKind {
  bool listed;        // the step's items come from a device work list (at most kPlanMaxRows rows)
  bool mixed;         // some row has more than one query
  bool overlap;       // the caller's schedule lets prompt tiles run beside the decode items
  bool prompts_only;  // the caller says every row has more than one query
  int prompt_wgs;     // the caller's prompt share of the CUs in an overlap (0: the default)
};
struct Route {
  int hp = 1;                                    // kv heads per decode item
  int decode = LV_KERNEL_NONE, decode_grid = 0;  // the launch running the decode items, its workgroups
  int prompt = LV_KERNEL_NONE, prompt_grid = 0;  // the launch running the prompt items (MIXED_SMALL: the same one)
  bool two_streams = false;                      // decode items on the second stream beside prompt_overlap_kernel
  bool merge = false;                            // rows split over items, merged by their last split
};

// CUs that hold a prompt workgroup in an overlapped step: the caller's count clamped to [default, max] and
// rounded down to a multiple of 8, or the default share for 0; never more than there are prompt items.
static int prompt_grid(const Shape& s, const AttnParams& p, int requested) {
  const int cus = device_cus();
  const int lo = std::max(8, cus * kOverlapCusPct / 100 / 8 * 8), hi = std::max(lo, cus * kOverlapCusMaxPct / 100);
  const int n = requested > 0 ? std::min(hi, std::max(lo, requested / 8 * 8)) : lo;
  return std::min(s.max_prompt_items * p.hkv, n);
}

// The route of a step:
// - a step of prompts: its prompt items one workgroup each on the whole GPU;
// - more rows than the work list holds (decode only): one workgroup per (row, split, item head group), no list;
// - a mixed step under the overlapped schedule whose workgroups (bounds: prompt bounds past a row's queries exit at
//   once) fill the GPU at most kSmallStepRounds times: prompt and decode items in one launch (mixed_small_kernel);
// - a larger one: prompt items on a persistent share of the CUs, decode items beside them on a second stream, on the
//   persistent ticket grid where the item bound gives each of its workgroups at least eight items (else one
//   workgroup per item: few short items finish sooner all at once than in rounds);
// - otherwise (the serial schedule, or decode only): the prompt items on the whole GPU if any, then the decode items
//   one workgroup each. Outside the overlap one workgroup per item measured as fast as the persistent grid or faster
//   (Qwen3-8B batch-256 decode of kv-head pairs 0.727 against 0.771 ms, same box, medians of 3).
template <typename T, int D, int GS, int TP, int HP>
static Route route_of(const AttnParams& p, const Shape& s, const StepKind& k) {
  Route r;
  r.hp = HP;
  const int ny = p.hkv / HP * p.qgroups;
  const int cus = device_cus();
  const int64_t pw = k.listed && k.mixed ? (int64_t)s.max_prompt_items * p.hkv : 0;
  const int64_t dw = k.listed ? (int64_t)s.max_decode_items * ny : (int64_t)p.rows * p.max_splits * ny;
  r.merge = p.max_splits > 1 && !k.prompts_only;
  if (k.prompts_only) {
    r.prompt = LV_KERNEL_PROMPT_LIST;
    r.prompt_grid = (int)pw;
  } else if (!k.listed) {
    r.decode = LV_KERNEL_DECODE_GRID;
    r.decode_grid = (int)dw;
  } else if (k.mixed && k.overlap &&
             pw + dw <= (int64_t)kSmallStepRounds * resident_per_cu<mixed_small_kernel<T, D, GS, TP, HP>>() * cus) {
    r.prompt = r.decode = LV_KERNEL_MIXED_SMALL;
    r.prompt_grid = (int)pw;
    r.decode_grid = (int)dw;
  } else if (k.mixed && k.overlap) {
    r.two_streams = true;
    r.prompt = LV_KERNEL_PROMPT_OVERLAP;
    r.prompt_grid = prompt_grid(s, p, k.prompt_wgs);
    const int grid = std::min(kOverlapDecodeWgs, resident_per_cu<decode_beside_kernel<T, D, GS, HP>>()) * cus;
    r.decode = dw >= 8 * (int64_t)grid ? LV_KERNEL_DECODE_BESIDE : LV_KERNEL_DECODE_LIST;
    r.decode_grid = r.decode == LV_KERNEL_DECODE_BESIDE ? grid : (int)dw;
  } else {
    if (k.mixed) {
      r.prompt = LV_KERNEL_PROMPT_LIST;
      r.prompt_grid = (int)pw;
    }
    r.decode = LV_KERNEL_DECODE_LIST;
    r.decode_grid = (int)dw;
  }
  return r;
}

// The decode launch of a route on `stream`.
template <typename T, int D, int GS, int HP>
static void launch_decode(const AttnParams& p, const Route& r, hipStream_t stream) {
  if (r.decode == LV_KERNEL_DECODE_BESIDE)
    hipLaunchKernelGGL((decode_beside_kernel<T, D, GS, HP>), dim3(r.decode_grid), dim3(256), 0, stream, p);
  else if (r.decode == LV_KERNEL_DECODE_GRID)
    hipLaunchKernelGGL((decode_grid_kernel<T, D, GS, HP>), dim3(p.rows * p.max_splits, p.hkv / HP * p.qgroups),
                       dim3(256), 0, stream, p);
  else if (r.decode == LV_KERNEL_DECODE_LIST)
    hipLaunchKernelGGL((decode_list_kernel<T, D, GS, HP, kWideSteps<D, HP>>), dim3(r.decode_grid), dim3(256), 0,
                       stream, p);
}

// A step's kernels after the plan. An overlapped mixed step forks the decode items onto the device's second stream
// and joins it back into `stream` with events; if the second stream cannot be set up, or the fork's record or wait
// fails before anything is launched, the step runs serially instead (the same results). A failure after the decode
// launch leaves the two streams unordered and is returned as LV_EHIP. With `info` set nothing is launched: the
// route is reported instead.
template <typename T, int D, int GS, int TP, int HP>
static int launch(const AttnParams& p, const Shape& s, const StepKind& k, hipStream_t stream, Route* info) {
  const Route r = route_of<T, D, GS, TP, HP>(p, s, k);
  if (info) {
    *info = r;
    return LV_OK;
  }
  if (r.prompt == LV_KERNEL_MIXED_SMALL) {
    hipLaunchKernelGGL((mixed_small_kernel<T, D, GS, TP, HP>), dim3(r.prompt_grid + r.decode_grid), dim3(256), 0,
                       stream, p, (int32_t)r.prompt_grid);
    LV_LAUNCH_CHECK("mixed_small_kernel");
  } else {
    SideStream* side = r.two_streams ? side_stream() : nullptr;
    bool forked = false;
    if (side) {
      // Decode items go to the second stream first, then the prompt items to the caller's stream: the prompt
      // workgroups (one per CU) are dispatched as soon as the plan ends, the decode workgroups fill the rest.
      std::lock_guard<std::mutex> g(side->lock);
      if (hipEventRecord(side->fork, stream) == hipSuccess &&
          hipStreamWaitEvent(side->stream, side->fork, 0) == hipSuccess) {
        forked = true;
        launch_decode<T, D, GS, HP>(p, r, side->stream);
        LV_LAUNCH_CHECK("decode kernel beside the prompt tiles");
        LV_HIP_CHECK(hipEventRecord(side->join, side->stream));
        constexpr int pad = std::max(0, kOverlapLds - std::max(1, kRingOf<TP>) * PromptSmem<D, D, (TP > 1)>::kBytes);
        hipLaunchKernelGGL((prompt_overlap_kernel<T, D, TP>), dim3(r.prompt_grid), dim3(256), pad, stream, p);
        LV_LAUNCH_CHECK("prompt_overlap_kernel");
        LV_HIP_CHECK(hipStreamWaitEvent(stream, side->join, 0));
      } else {
        (void)hipGetLastError();  // the failed record or wait: fall back to the serial schedule
      }
    }
    if (!forked) {
      if (r.prompt != LV_KERNEL_NONE)  // the serial schedule (or its fallback): prompt items on the whole GPU
        hipLaunchKernelGGL((prompt_list_kernel<T, D, TP>), dim3(s.max_prompt_items * p.hkv), dim3(256), 0, stream,
                           p);
      if (r.decode != LV_KERNEL_NONE) {
        Route serial = r;
        if (serial.decode == LV_KERNEL_DECODE_BESIDE) {  // the fallback: one workgroup per item
          serial.decode = LV_KERNEL_DECODE_LIST;
          serial.decode_grid = s.max_decode_items * (p.hkv / HP) * p.qgroups;
        }
        launch_decode<T, D, GS, HP>(p, serial, stream);
      }
      LV_LAUNCH_CHECK("paged attention kernels");
    }
  }
  return LV_OK;
}

// Pages per 64-key prompt tile for the LDS ring: 1 for pages of a multiple of 64 keys, 2 or 4 for pages of 32 or
// 16; 0 (register staging) for any other size.
static int tile_pages(int block_size) {
  if (block_size % kPrefillKeys == 0) return 1;
  if (block_size == 32) return 2;
  if (block_size == 16) return 4;
  return 0;
}

template <typename T, int D, int GS, int HP>
static int launch_tp(const AttnParams& p, const Shape& s, const StepKind& k, hipStream_t stream, Route* info) {
  switch (tile_pages((int)p.bs.d)) {
    case 1: return launch<T, D, GS, 1, HP>(p, s, k, stream, info);
    case 2: return launch<T, D, GS, 2, HP>(p, s, k, stream, info);
    case 4: return launch<T, D, GS, 4, HP>(p, s, k, stream, info);
    default: return launch<T, D, GS, 0, HP>(p, s, k, stream, info);
  }
}

// Decode items of a streaming step take two kv heads where the step has an even number: a token's two head rows are
// adjacent in the NHD cache, so each 64-lane load covers 512-byte pieces of token rows instead of 256-byte ones (a
// math-free stream of 512-byte pieces at a 2 KB stride reads 7.15 TB/s on an MI355X, of 256-byte pieces
// 6.5-6.7 TB/s). The split of a row's keys stays as planned, so such items are half as many and twice as long;
// steps of fewer than kPairItems one-head items per CU (a few short rows, latency-bound) keep one head per item.
// A lane addresses the second head's row with a 32-bit offset (the head stride) inside its tile, so pairs also need
// a head stride under 2^30 bytes.
constexpr int kPairItems = 8;
template <typename T, int D, int GS>
static int launch_hp(const AttnParams& p, const Shape& s, const StepKind& k, hipStream_t stream, Route* info) {
  const int64_t items = (int64_t)(k.listed ? s.max_decode_items : p.rows * p.max_splits) * p.hkv * p.qgroups;
  if (p.hkv % 2 == 0 && p.c_sh >= 0 && p.c_sh < ((int64_t)1 << 30) && items >= (int64_t)kPairItems * device_cus())
    return launch_tp<T, D, GS, 2>(p, s, k, stream, info);
  return launch_tp<T, D, GS, 1>(p, s, k, stream, info);
}

template <typename T, int D>
static int launch_gs(const AttnParams& p, int gs, const Shape& s, const StepKind& k, hipStream_t stream,
                     Route* info) {
  if (gs == 4) return launch_hp<T, D, 4>(p, s, k, stream, info);
  if (gs == 2) return launch_hp<T, D, 2>(p, s, k, stream, info);
  return launch_hp<T, D, 1>(p, s, k, stream, info);
}

template <typename T>
static int launch_d(const AttnParams& p, int d, int gs, const Shape& s, const StepKind& k, hipStream_t stream,
                    Route* info) {
  switch (d) {
    case 64: return launch_gs<T, 64>(p, gs, s, k, stream, info);
    case 128: return launch_gs<T, 128>(p, gs, s, k, stream, info);
    default: set_error("paged_attention: head_dim %d is not 64 or 128", d); return LV_EINVAL;
  }
}

// ---------------------------------------------------------------------------------------------------------
// The workspace of lv_paged_attention_static: a file-scope device array (each GPU that loads the library holds its
// own copy until the process ends). Host code must not pass the array's name to a kernel -- in host code it is a
// stand-in, not a device address; its address on the current device comes from hipGetSymbolAddress, resolved once
// per device and kept. The same set-up creates the device's second stream and its fork/join events, so that no
// later call creates anything.
static __device__ __align__(256) char scratch[LV_STATIC_WORKSPACE_BYTES];

static void* scratch_on_current_device() {
  static void* addr[64];
  static std::mutex lock;
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("paged_attention_static: hipGetDevice failed: %s", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= 64) {
    set_error("paged_attention_static: device %d is past the 64 devices served", dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> g(lock);
  if (!addr[dev]) {
    void* ptr = nullptr;
    const hipError_t r = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (r != hipSuccess || !ptr) {
      set_error("paged_attention_static: hipGetSymbolAddress of the static workspace failed on device %d: %s", dev,
                hipGetErrorString(r));
      return nullptr;
    }
    if (!side_stream()) {
      set_error("paged_attention_static: the second stream of device %d could not be created", dev);
      return nullptr;
    }
    addr[dev] = ptr;
  }
  return addr[dev];
}

// What a work list was planned for, per workspace: a caller's request to reuse the plan already in a workspace
// (LV_ATTN_REUSE_PLAN, for the later layers of a step) is honoured only if the workspace's last plan was made for the
// same rows, shape and row-length arrays; otherwise the call plans again.
struct PlanSig {
  const void* ws = nullptr;
  const int32_t *cu_q = nullptr, *lens = nullptr, *cu_k = nullptr;
  int64_t rows = 0, tokens = 0, max_k = 0, split = 0, qp = 0, max_items = 0, bytes = 0;
  bool mixed = false, last_first = false;
  bool operator==(const PlanSig& o) const {
    return ws == o.ws && cu_q == o.cu_q && lens == o.lens && cu_k == o.cu_k && rows == o.rows &&
           tokens == o.tokens && max_k == o.max_k && split == o.split && qp == o.qp && max_items == o.max_items &&
           bytes == o.bytes && mixed == o.mixed && last_first == o.last_first;
  }
};
constexpr int kPlanRecords = 32;
static std::mutex g_plan_lock;
static PlanSig g_plans[kPlanRecords];

// True if a caller asks to reuse the plan in `sig`'s workspace and that workspace's last plan is the one `sig`
// describes.
static bool plan_is_current(const PlanSig& sig, bool reuse) {
  if (!reuse) return false;
  std::lock_guard<std::mutex> g(g_plan_lock);
  for (int i = 0; i < kPlanRecords; ++i)
    if (g_plans[i].ws == sig.ws) return g_plans[i] == sig;
  return false;
}

// Records what workspace `ws` now holds: the plan `sig` (after its launch was accepted), or nothing (sig null: a
// call that failed after choosing to plan, whose list may never be written).
static void record_plan(const void* ws, const PlanSig* sig) {
  std::lock_guard<std::mutex> g(g_plan_lock);
  int slot = -1;
  for (int i = 0; i < kPlanRecords; ++i)
    if (g_plans[i].ws == ws) slot = i;
  if (!sig) {
    if (slot >= 0) g_plans[slot] = PlanSig{};
    return;
  }
  if (slot < 0) {  // a new workspace: take a free record, else the first
    slot = 0;
    for (int i = 0; i < kPlanRecords; ++i)
      if (!g_plans[i].ws) {
        slot = i;
        break;
      }
  }
  g_plans[slot] = *sig;
}

// The checks on a step's shape and options, shared by the call and the launch-info query.
static int check_shape(int32_t num_rows, int32_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
                       int32_t head_dim, int32_t block_size, bool has_cu_q, int32_t max_seqlen_q,
                       int32_t max_seqlen_k, int32_t schedule, int32_t prompt_workgroups, int32_t flags,
                       int32_t dtype) {
  LV_REQUIRE(dtype == LV_DTYPE_BF16 || dtype == LV_DTYPE_F16, "paged_attention: dtype %d is not bf16 or fp16",
             dtype);
  LV_REQUIRE(num_rows >= 0 && num_tokens >= 0, "paged_attention: negative row or token count");
  LV_REQUIRE(schedule == LV_SCHEDULE_AUTO || schedule == LV_SCHEDULE_SERIAL || schedule == LV_SCHEDULE_OVERLAP,
             "paged_attention: unknown schedule %d", schedule);
  LV_REQUIRE(prompt_workgroups >= 0, "paged_attention: negative prompt_workgroups %d", prompt_workgroups);
  LV_REQUIRE((flags & ~(LV_ATTN_REUSE_PLAN | LV_ATTN_PROMPTS_ONLY)) == 0, "paged_attention: unknown flags 0x%x",
             flags);
  LV_REQUIRE(!(flags & LV_ATTN_PROMPTS_ONLY) || (has_cu_q && max_seqlen_q > 1),
             "paged_attention: LV_ATTN_PROMPTS_ONLY needs cu_seqlens_q and max_seqlen_q > 1");
  if (num_rows == 0 || num_tokens == 0) return LV_OK;
  LV_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
             "paged_attention: %d query heads do not group over %d key heads", num_heads, num_kv_heads);
  LV_REQUIRE(num_heads / num_kv_heads <= kPrefillRows, "paged_attention: query group %d exceeds %d",
             num_heads / num_kv_heads, kPrefillRows);
  LV_REQUIRE(head_dim == 64 || head_dim == 128, "paged_attention: head_dim %d is not 64 or 128", head_dim);
  LV_REQUIRE(block_size > 0 && block_size % kTile == 0, "paged_attention: block_size %d is not a multiple of %d",
             block_size, kTile);
  LV_REQUIRE(has_cu_q || num_tokens == num_rows, "paged_attention: without cu_seqlens_q, T (%d) must equal B (%d)",
             num_tokens, num_rows);
  LV_REQUIRE(max_seqlen_k >= 0 && max_seqlen_k <= (1 << 30), "paged_attention: max_seqlen_k %d is negative or above "
             "2^30 keys", max_seqlen_k);
  LV_REQUIRE(!(has_cu_q && max_seqlen_q > 1) || num_rows <= kPlanMaxRows,
             "paged_attention: a step with prompts holds at most %d rows, got %d", kPlanMaxRows, num_rows);
  return LV_OK;
}

static StepKind step_kind(int32_t num_rows, bool has_cu_q, int32_t max_seqlen_q, int32_t schedule,
                          int32_t prompt_workgroups, int32_t flags) {
  StepKind k;
  k.mixed = has_cu_q && max_seqlen_q > 1;
  k.listed = num_rows <= kPlanMaxRows;
  k.overlap = schedule != LV_SCHEDULE_SERIAL;
  k.prompts_only = (flags & LV_ATTN_PROMPTS_ONLY) != 0;
  k.prompt_wgs = prompt_workgroups;
  return k;
}

// A launch counts its work-items (workgroups x 256) in 32 bits: the step's largest grid must stay below that.
static int check_grids(const Shape& s, int32_t num_rows, int32_t num_heads, int32_t num_kv_heads) {
  // Split rows are merged through the work list's counters: a step without the list must not split.
  LV_REQUIRE(s.max_splits == 1 || s.merges > 0, "paged_attention: %d rows split over %d items without a work list",
             num_rows, s.max_splits);
  const int64_t prompt = (int64_t)s.max_prompt_items * num_kv_heads;
  const int64_t decode = std::max<int64_t>(s.max_decode_items, (int64_t)num_rows * s.max_splits) * num_heads;
  LV_REQUIRE(fits_one_launch(prompt + decode, 256),
             "paged_attention: the step needs %lld + %lld workgroups, more than one launch holds", (long long)prompt,
             (long long)decode);
  return LV_OK;
}

// The shape part of a step's parameters (what the route depends on).
static void shape_params(AttnParams& p, const Shape& s, int32_t num_rows, int32_t num_heads, int32_t num_kv_heads,
                         int32_t block_size, int64_t cache_stride_head) {
  p.bs = FastDiv::make((uint32_t)block_size);
  p.c_sh = cache_stride_head * 2;
  p.rows = num_rows;
  p.hq = num_heads;
  p.hkv = num_kv_heads;
  p.group = num_heads / num_kv_heads;
  p.qgroups = p.group / s.gs;
  p.split = s.split;
  p.max_splits = s.max_splits;
}

// One step, with the workspace given (workspace != nullptr or an empty shape) or, for static_ws, the device's
// static workspace.
static int paged_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
                           const void* v_cache, int64_t cache_stride_block, int64_t cache_stride_token,
                           int64_t cache_stride_head, int32_t block_size, const int32_t* block_tables,
                           int64_t table_stride, const int32_t* cu_seqlens_q, const int32_t* seqlens_k,
                           const int32_t* cu_seqlens_k, int32_t num_rows, int32_t num_tokens, int32_t num_heads,
                           int32_t num_kv_heads, int32_t head_dim, float scale, int32_t max_seqlen_q,
                           int32_t max_seqlen_k, void* out, int64_t out_stride_t, int64_t out_stride_h,
                           void* workspace, size_t workspace_bytes, bool static_ws, int32_t schedule,
                           int32_t prompt_workgroups, int32_t flags, int32_t dtype, void* stream) {
  const int rc0 = check_shape(num_rows, num_tokens, num_heads, num_kv_heads, head_dim, block_size,
                              cu_seqlens_q != nullptr, max_seqlen_q, max_seqlen_k, schedule, prompt_workgroups,
                              flags, dtype);
  if (rc0 != LV_OK || num_rows == 0 || num_tokens == 0) return rc0;
  LV_REQUIRE(q && k_cache && v_cache && out && block_tables, "paged_attention: null tensor pointer");
  LV_REQUIRE(seqlens_k || cu_seqlens_k, "paged_attention: neither key lengths nor cu_seqlens_k given");
  // 16-byte rows: q, out and cache head rows are read and written as 16-byte vectors.
  LV_REQUIRE(aligned(q, 16) && aligned(out, 16) && aligned(k_cache, 16) && aligned(v_cache, 16) &&
                 (q_stride_t * 2) % 16 == 0 && (q_stride_h * 2) % 16 == 0 && (out_stride_t * 2) % 16 == 0 &&
                 (out_stride_h * 2) % 16 == 0 && (cache_stride_block * 2) % 16 == 0 &&
                 (cache_stride_token * 2) % 16 == 0 && (cache_stride_head * 2) % 16 == 0,
             "paged_attention: tensors and their strides must be 16-byte aligned");
  // Lanes address their rows inside a 16-token decode tile or a 64-key prompt tile with 32-bit byte offsets, the
  // prompt tile's as 24-bit products (key row times token stride).
  LV_REQUIRE(cache_stride_token >= 0 && (int64_t)kPrefillKeys * cache_stride_token * 2 < (int64_t)1 << 30,
             "paged_attention: cache token stride %lld is negative or too large", (long long)cache_stride_token);
  LV_REQUIRE(scale > 0.f, "paged_attention: the softmax scale must be positive, got %g", (double)scale);
  const StepKind kind = step_kind(num_rows, cu_seqlens_q != nullptr, max_seqlen_q, schedule, prompt_workgroups, flags);
  const Shape s = plan_shape(num_rows, num_tokens, num_heads, num_kv_heads, head_dim, max_seqlen_k, kind.listed);
  const int rg = check_grids(s, num_rows, num_heads, num_kv_heads);
  if (rg != LV_OK) return rg;
  if (static_ws) {
    LV_REQUIRE(s.bytes <= (size_t)LV_STATIC_WORKSPACE_BYTES,
               "paged_attention_static: this step needs %zu bytes of workspace; the static workspace holds %zu "
               "(LV_STATIC_WORKSPACE_BYTES): call lv_paged_attention with a workspace instead",
               s.bytes, (size_t)LV_STATIC_WORKSPACE_BYTES);
    workspace = scratch_on_current_device();
    if (!workspace) return LV_EHIP;
    workspace_bytes = LV_STATIC_WORKSPACE_BYTES;
  }
  LV_REQUIRE(workspace_bytes >= s.bytes && (s.bytes == 0 || workspace),
             "paged_attention: workspace of %zu bytes given, %zu needed", workspace_bytes, s.bytes);
  LV_REQUIRE(aligned(workspace, 256), "paged_attention: workspace must be 256-byte aligned");

  AttnParams p{};
  shape_params(p, s, num_rows, num_heads, num_kv_heads, block_size, cache_stride_head);
  p.q = (const char*)q;
  p.q_st = q_stride_t * 2;
  p.q_sh = q_stride_h * 2;
  p.k_cache = (const char*)k_cache;
  p.v_cache = (const char*)v_cache;
  p.c_sb = cache_stride_block * 2;
  p.c_st = cache_stride_token * 2;
  p.v_st = p.c_st;
  p.v_sh = p.c_sh;
  p.paged = true;
  p.causal = 1;
  p.tables = block_tables;
  p.t_stride = table_stride;
  p.cu_q = cu_seqlens_q;
  p.lens_k = seqlens_k;
  p.cu_k = cu_seqlens_k;
  p.scale_log2 = scale * kLog2e;
  p.out = (char*)out;
  p.o_st = out_stride_t * 2;
  p.o_sh = out_stride_h * 2;
  char* ws = (char*)workspace;
  p.part_lse = s.max_splits > 1 ? reinterpret_cast<float*>(ws + s.lse_off) : nullptr;
  p.part_o = s.max_splits > 1 ? reinterpret_cast<float*>(ws + s.o_off) : nullptr;
  p.items = kind.listed ? reinterpret_cast<const int2*>(ws + s.items_off) : nullptr;
  p.n_items = kind.listed ? reinterpret_cast<const int32_t*>(ws + s.count_off) : nullptr;
  p.ticket = kind.listed ? reinterpret_cast<int32_t*>(ws + s.count_off) + 2 : nullptr;
  p.merge_count = s.merges > 0 ? reinterpret_cast<int32_t*>(ws + s.merge_off) : nullptr;

  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int qp = kPrefillRows / p.group;
  PlanSig sig;
  sig.ws = workspace;
  sig.cu_q = kind.mixed ? cu_seqlens_q : nullptr;
  sig.lens = seqlens_k;
  sig.cu_k = cu_seqlens_k;
  sig.rows = num_rows;
  sig.tokens = num_tokens;
  sig.max_k = max_seqlen_k;
  sig.split = s.split;
  sig.qp = qp;
  sig.max_items = s.max_items;
  sig.bytes = (int64_t)s.bytes;
  sig.mixed = kind.mixed;
  sig.last_first = kind.prompts_only || !kind.overlap;  // prompt items with the GPU to themselves: last tile first
  bool planned = false;
  if (kind.listed && !plan_is_current(sig, (flags & LV_ATTN_REUSE_PLAN) != 0)) {
    record_plan(workspace, nullptr);  // until this plan's launch is accepted, the workspace holds no plan
    hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kScanThreads), 0, st, kind.mixed ? cu_seqlens_q : nullptr,
                       seqlens_k, cu_seqlens_k, num_rows, s.split, qp, s.max_items, (int32_t)sig.last_first,
                       reinterpret_cast<int2*>(ws + s.items_off), reinterpret_cast<int32_t*>(ws + s.count_off),
                       p.merge_count, (int32_t)s.merges);
    LV_LAUNCH_CHECK("plan_kernel");
    planned = true;
  }
  const int rc = dtype == LV_DTYPE_BF16 ? launch_d<BF16>(p, head_dim, s.gs, s, kind, st, nullptr)
                                        : launch_d<F16>(p, head_dim, s.gs, s, kind, st, nullptr);
  if (rc != LV_OK) {
    // A failed launch may leave the persistent grid's ticket unreset: the next call on this workspace plans again.
    record_plan(workspace, nullptr);
    return rc;
  }
  if (planned) record_plan(workspace, &sig);
  return LV_OK;
}

}  // namespace lv

using namespace lv;

extern "C" size_t lv_paged_attention_workspace_bytes(int32_t num_rows, int32_t num_tokens, int32_t num_heads,
                                                     int32_t num_kv_heads, int32_t head_dim, int32_t max_seqlen_k,
                                                     int32_t decode_only) {
  if (num_rows <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads || max_seqlen_k < 0 ||
      max_seqlen_k > (1 << 30))
    return 0;
  const bool mixed = decode_only == 0;
  const bool listed = mixed || num_rows <= kPlanMaxRows;
  return plan_shape(num_rows, num_tokens, num_heads, num_kv_heads, head_dim, max_seqlen_k, listed).bytes;
}

extern "C" int lv_paged_attention_launch_info(int32_t num_rows, int32_t num_tokens, int32_t num_heads,
                                              int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                              int64_t cache_stride_head, int32_t has_cu_seqlens_q,
                                              int32_t max_seqlen_q, int32_t max_seqlen_k, int32_t schedule,
                                              int32_t prompt_workgroups, int32_t flags, int32_t dtype,
                                              lv_launch_info* info) {
  LV_REQUIRE(info, "paged_attention_launch_info: info is null");
  *info = lv_launch_info{};
  const int rc0 = check_shape(num_rows, num_tokens, num_heads, num_kv_heads, head_dim, block_size,
                              has_cu_seqlens_q != 0, max_seqlen_q, max_seqlen_k, schedule, prompt_workgroups, flags,
                              dtype);
  if (rc0 != LV_OK || num_rows == 0 || num_tokens == 0) return rc0;
  const StepKind kind = step_kind(num_rows, has_cu_seqlens_q != 0, max_seqlen_q, schedule, prompt_workgroups, flags);
  const Shape s = plan_shape(num_rows, num_tokens, num_heads, num_kv_heads, head_dim, max_seqlen_k, kind.listed);
  const int rg = check_grids(s, num_rows, num_heads, num_kv_heads);
  if (rg != LV_OK) return rg;
  AttnParams p{};
  shape_params(p, s, num_rows, num_heads, num_kv_heads, block_size, cache_stride_head);
  Route r;
  const int rc = dtype == LV_DTYPE_BF16 ? launch_d<BF16>(p, head_dim, s.gs, s, kind, nullptr, &r)
                                        : launch_d<F16>(p, head_dim, s.gs, s, kind, nullptr, &r);
  if (rc != LV_OK) return rc;
  info->decode_kernel = r.decode;
  info->decode_workgroups = r.decode_grid;
  info->prompt_kernel = r.prompt;
  info->prompt_workgroups = r.prompt_grid;
  info->kv_heads_per_item = r.hp;
  info->two_streams = r.two_streams;
  info->keys_per_split = s.split;
  info->max_splits = s.max_splits;
  info->splitk_merge = r.merge;
  return LV_OK;
}

extern "C" int lv_paged_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
                                  const void* v_cache, int64_t cache_stride_block, int64_t cache_stride_token,
                                  int64_t cache_stride_head, int32_t block_size, const int32_t* block_tables,
                                  int64_t table_stride, const int32_t* cu_seqlens_q, const int32_t* seqlens_k,
                                  const int32_t* cu_seqlens_k, int32_t num_rows, int32_t num_tokens,
                                  int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float scale,
                                  int32_t max_seqlen_q, int32_t max_seqlen_k, void* out, int64_t out_stride_t,
                                  int64_t out_stride_h, void* workspace, size_t workspace_bytes, int32_t schedule,
                                  int32_t prompt_workgroups, int32_t flags, int32_t dtype, void* stream) {
  return paged_attention(q, q_stride_t, q_stride_h, k_cache, v_cache, cache_stride_block, cache_stride_token,
                         cache_stride_head, block_size, block_tables, table_stride, cu_seqlens_q, seqlens_k,
                         cu_seqlens_k, num_rows, num_tokens, num_heads, num_kv_heads, head_dim, scale, max_seqlen_q,
                         max_seqlen_k, out, out_stride_t, out_stride_h, workspace, workspace_bytes, false, schedule,
                         prompt_workgroups, flags, dtype, stream);
}

extern "C" int lv_paged_attention_static(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
                                         const void* v_cache, int64_t cache_stride_block, int64_t cache_stride_token,
                                         int64_t cache_stride_head, int32_t block_size, const int32_t* block_tables,
                                         int64_t table_stride, const int32_t* cu_seqlens_q, const int32_t* seqlens_k,
                                         const int32_t* cu_seqlens_k, int32_t num_rows, int32_t num_tokens,
                                         int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float scale,
                                         int32_t max_seqlen_q, int32_t max_seqlen_k, void* out, int64_t out_stride_t,
                                         int64_t out_stride_h, int32_t schedule, int32_t prompt_workgroups,
                                         int32_t flags, int32_t dtype, void* stream) {
  return paged_attention(q, q_stride_t, q_stride_h, k_cache, v_cache, cache_stride_block, cache_stride_token,
                         cache_stride_head, block_size, block_tables, table_stride, cu_seqlens_q, seqlens_k,
                         cu_seqlens_k, num_rows, num_tokens, num_heads, num_kv_heads, head_dim, scale, max_seqlen_q,
                         max_seqlen_k, out, out_stride_t, out_stride_h, nullptr, 0, true, schedule, prompt_workgroups,
                         flags, dtype, stream);
}
