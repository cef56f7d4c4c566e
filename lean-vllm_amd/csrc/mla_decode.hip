// MLA absorbed decode on gfx950: each row's last queries attend its paged latents as one key head shared by all
// query heads; values are the latents' leading v_dim entries.
//
// Math of TorchAttention.mla_decode (lean_vllm/attention/torch_backend.py:105-119), called by
// MLAAttention._decode_latents (lean_vllm/layers/attention.py:319-335) with q = [q_nope W_UK_T | q_pe] of width
// 576 (kv_lora_rank 512 + rope 64) and v_dim 512: query j of a row with lq queries and L cached latents sees
// latents 0 .. L - lq + j.
//
// Two schedules, both streaming latents from HBM straight into an LDS ring (global_load_lds_dwordx4):
//   balanced runs (mla_run_kernel)  pages a multiple of 16 latents: the units' 16-latent stages, end to end, are cut
//                                   into equal runs, one per workgroup; units cut by run boundaries are merged by
//                                   log-sum-exp in mla_run_merge_kernel.
//   split schedule (mla_decode_dma_kernel)  other page sizes, or more units than the runs' in-kernel scan holds:
//                                   one workgroup per (row, split of <= 4096 latents, query, 16-head tile); split
//                                   rows are merged by log-sum-exp in mla_merge_kernel.
// Per 16-latent stage: S^T = Lat Q^T (16 latents x 16 heads, K = 576) on MFMA 16x16x32, the online softmax per
// head, and O^T += V^T P^T (512 dims x 16 heads) on MFMA 16x16x16 with V^T operands from gfx950's transposing LDS
// read (ds_read_b64_tr_b16).
#include <algorithm>

#include "lv_common.h"

namespace lv {

constexpr int kLatent = 576;              // latent width served: kv_lora_rank 512 + rope 64
constexpr int kVDim = 512;                // value width: the latents' leading entries
constexpr int kMlaPitch = kLatent + 16;   // LDS row pitch in elements (1184 bytes): conflict-free operand reads and
                                          // transposing reads (a 1168-byte pitch halves the latter's rate)
constexpr int kLatChunks = kLatent / 8;   // 16-byte chunks per latent row

constexpr int kMlaMaxSplit = 4096;        // latents per work item at most
constexpr int kMlaMaxBlocks = kMlaMaxSplit / 16 + 2;  // pages one work item touches at most (pages >= 16 latents)

constexpr int kMlaSplitStages = 4;    // ring depth of the split schedule
constexpr int kMlaSplitTarget = 4096;  // split-schedule items (x queries x head tiles) a grid aims for

struct MlaParams {
  const char* q;
  int64_t q_st, q_sh;  // bytes
  const char* cache;
  int64_t c_sb, c_st;  // bytes
  FastDiv bs;  // latents per page
  const int32_t* tables;
  int64_t t_stride;  // elements
  const int32_t* lens;
  int32_t rows, lq, heads, htiles;
  float scale_log2;
  char* out;
  int64_t o_st, o_sh;  // bytes
  int32_t split, max_splits;
  float* part_o;    // split schedule: [rows * lq][heads][max_splits][kVDim]; runs: [runs][2][16][kVDim]
  float* part_lse;  // split schedule: [rows * lq][heads][max_splits]; runs: [runs][2][16]; log2 domain
  int32_t units;    // runs: (row, query, 16-head tile) units
  int32_t* prefix;  // runs: [units + 2] stage prefix over units, then the stage total and the run length
};

// ---------------------------------------------------------------------------------------------------------
// Split schedule: latents move from HBM straight into LDS (global_load_lds_dwordx4), a ring of kMlaSplitStages
// 16-latent stages with all but one in flight while one is consumed; no registers stage data. Each wave computes
// the stage's whole S^T (16 latents x 16 heads, K = 576) from LDS, then O^T for its 128 output dims with MFMA
// 16x16x16 whose V^T operands come from one transposing LDS read each. One unfenced barrier per stage; every wait
// on the stage loads is an explicit vmcnt.

constexpr int kDmaTile = 16;                            // latents per stage
constexpr int kDmaRowSlots = kLatChunks + 2;            // 16-byte slots per LDS row (two pad slots: pitch 1184 B)
constexpr int kDmaStageSlots = kDmaTile * kDmaRowSlots;  // 1184
constexpr int kDmaInstr = (kDmaStageSlots + 63) / 64;   // 64-lane loads per stage: 19, 5 per wave (4 for wave 3)
constexpr int kDmaStageElems = kDmaStageSlots * 8;
static_assert(kDmaRowSlots * 8 == kMlaPitch, "one LDS row pitch for both variants");
static_assert(kDmaInstr == 19, "the stage waits count 5 loads for waves 0-2 and 4 for wave 3");

// Wait until at most `ahead` (<= 6) stages of this wave's loads (5 per stage, 4 for wave 3) are outstanding, then meet
// the other waves. No fence: the stage's LDS writes are exactly the loads waited for, and a fence would wait for
// the stages still in flight as well.
#define LV_WAIT_BARRIER(N) asm volatile("s_waitcnt vmcnt(" #N ")\n\ts_barrier" ::: "memory")
__device__ __forceinline__ void dma_stage_barrier(int ahead, int wave) {
  if (wave < 3) {
    switch (ahead) {
      case 0: LV_WAIT_BARRIER(0); break;
      case 1: LV_WAIT_BARRIER(5); break;
      case 2: LV_WAIT_BARRIER(10); break;
      case 3: LV_WAIT_BARRIER(15); break;
      case 4: LV_WAIT_BARRIER(20); break;
      case 5: LV_WAIT_BARRIER(25); break;
      default: LV_WAIT_BARRIER(30); break;
    }
  } else {
    switch (ahead) {
      case 0: LV_WAIT_BARRIER(0); break;
      case 1: LV_WAIT_BARRIER(4); break;
      case 2: LV_WAIT_BARRIER(8); break;
      case 3: LV_WAIT_BARRIER(12); break;
      case 4: LV_WAIT_BARRIER(16); break;
      case 5: LV_WAIT_BARRIER(20); break;
      default: LV_WAIT_BARRIER(24); break;
    }
  }
}
#undef LV_WAIT_BARRIER

// STAGES: ring depth (STAGES - 1 stages in flight while one is consumed; at most 4). ONE_PAGE: block_size is a
// multiple of 16, so a stage (16 latents starting at a multiple of 16) lies in one page: one page lookup per
// stage, every lane's load a fixed offset from it.
template <typename T, int STAGES, bool ONE_PAGE>
__global__ __launch_bounds__(256) void mla_decode_dma_kernel(MlaParams p) {
  static_assert(STAGES >= 2 && STAGES <= 4, "the stage waits cover up to three stages in flight");
  using E = Elem<T>;
  __shared__ __attribute__((aligned(16))) uint16_t ring[STAGES * kDmaStageElems];
  __shared__ int64_t page_off[kMlaMaxBlocks];
  const int row = blockIdx.x / p.max_splits, split = blockIdx.x % p.max_splits;
  const int qj = blockIdx.y / p.htiles, ht = blockIdx.y % p.htiles;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;

  const int lk = p.lens[row] - p.lq + qj + 1;  // latents this query sees
  const int kbeg = split * p.split;
  if ((split > 0 && kbeg >= lk) || split >= p.max_splits) return;
  const int kend = min(lk, kbeg + p.split);
  const int nsplit = lk > 0 ? min((lk + p.split - 1) / p.split, p.max_splits) : 0;
  const int tokq = row * p.lq + qj;
  const int head = ht * 16 + n;
  const bool hvalid = head < p.heads;
  const float c = p.scale_log2;

  // Q^T operand over the whole latent: lane holds dims 32 s + 8 g .. + 7 of head n.
  u32x4 qb[18];
  {
    const char* qrow = p.q + tokq * p.q_st + (int64_t)head * p.q_sh;
#pragma unroll
    for (int s = 0; s < 18; ++s) qb[s] = hvalid ? ld16(qrow + (int64_t)(32 * s + 8 * g) * 2) : u32x4{0, 0, 0, 0};
  }
  const int page0 = kend > kbeg ? (int)p.bs.div(kbeg) : 0;
  const int npages = kend > kbeg ? (int)p.bs.div(kend - 1) - page0 + 1 : 0;
  {
    const int32_t* table = p.tables + (int64_t)row * p.t_stride + page0;
    for (int i = tid; i < npages; i += 256) page_off[i] = (int64_t)table[i] * p.c_sb;
  }
  // This wave's loads j = wave + 4 i (i < 5) of a stage's 19: slot 64 j + lane is 16-byte chunk `part` of latent
  // row r of the stage. Slots 74 r + 72 and 74 r + 73 of row r are LDS padding, filled with copies of chunk 71.
  int lrow[5], lpart[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    const int slot = min(64 * (wave + 4 * i) + lane, kDmaStageSlots - 1);
    lrow[i] = slot / kDmaRowSlots;
    lpart[i] = min(slot - lrow[i] * kDmaRowSlots, kLatChunks - 1) * 16;
  }
  __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0): q is in registers before the stage loads are counted
  __syncthreads();

  // Stage load of latents t0 .. t0 + 15; latents at or past kend load a latent of the range instead (finite
  // values; their weight is 0).
  auto fill = [&](int t0, uint16_t* stage) {
    const int last = kend - 1 - t0;  // rows past it are clamped
    int64_t base = 0;
    if (ONE_PAGE) {
      const int pg = (int)p.bs.div(t0);
      const int64_t po = page_off[pg - page0];
      // Uniform: move it to scalar registers. The low half is widened unsigned (offsets reach past 2 GiB).
      base = (int64_t)((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)po) |
                       ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(po >> 32)) << 32));
      base += (int64_t)(t0 - pg * (int)p.bs.d) * p.c_st;
    }
#pragma unroll
    for (int i = 0; i < 5; ++i) {
      const int j = wave + 4 * i;
      if (j < kDmaInstr && 64 * j + lane < kDmaStageSlots) {
        const int r = min(lrow[i], last);
        if (ONE_PAGE) {
          lds_dma16(p.cache + base, (uint32_t)(r * (int)p.c_st + lpart[i]), lds_addr(stage + 64 * 8 * j));
        } else {
          const int tok = t0 + r;
          const int pg = (int)p.bs.div(tok);
          lds_dma16(p.cache + page_off[pg - page0] + (int64_t)(tok - pg * (int)p.bs.d) * p.c_st + lpart[i],
                    lds_addr(stage + 64 * 8 * j));
        }
      }
    }
  };

  float m = -INFINITY, lsum = 0.f;
  f32x4 o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = f32x4{0, 0, 0, 0};

  const int ntiles = kend > kbeg ? (kend - kbeg + kDmaTile - 1) / kDmaTile : 0;
  for (int t = 0; t < STAGES - 1 && t < ntiles; ++t) fill(kbeg + t * kDmaTile, ring + t * kDmaStageElems);
  for (int it = 0; it < ntiles; ++it) {
    const int t0 = kbeg + it * kDmaTile;
    dma_stage_barrier(min(STAGES - 2, ntiles - 1 - it), wave);  // stage `it` has landed for every wave
    const bool refill = it + STAGES - 1 < ntiles;
    // Refill the stage read last iteration (every wave has passed the barrier, so its reads are done), then
    // consume this one.
    auto step = [&](uint16_t* next, const uint16_t* stage) {
      if (refill) fill(t0 + (STAGES - 1) * kDmaTile, next);
      f32x4 sc = {0, 0, 0, 0};  // latents t0 + 4 g + r of head n
      const uint16_t* arow = stage + n * kMlaPitch + 8 * g;
#pragma unroll
      for (int s = 0; s < 18; ++s) sc = E::mfma16x16x32(*reinterpret_cast<const u32x4*>(arow + 32 * s), qb[s], sc);
      if (t0 + kDmaTile > kend) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[r] = t0 + 4 * g + r < kend ? sc[r] : -INFINITY;
      }
      float mx = vmax(vmax(sc[0], sc[1]), vmax(sc[2], sc[3]));
      mx = xor32_max(xor16_max(mx));
      if (__any(mx > m && (m == -INFINITY || (mx - m) * c > kRescaleSlack))) {
        const float mn = vmax(m, mx);
        const float alpha = m == -INFINITY ? 0.f : fast_exp2((m - mn) * c);
        m = mn;
        lsum *= alpha;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] *= alpha;
      }
      const float mc = m * c;
      float pr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) pr[r] = fast_exp2(fmaf(sc[r], c, -mc));
      lsum += (pr[0] + pr[1]) + (pr[2] + pr[3]);
      const u32x2 pb = {E::pack(pr[0], pr[1]), E::pack(pr[2], pr[3])};
      const uint16_t* v = stage + (4 * g + (n >> 2)) * kMlaPitch + 128 * wave + 4 * (n & 3);
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = E::mfma16x16x16(lds_read_tr16(v + 16 * j), pb, o[j]);
    };
    step(ring + ((it + STAGES - 1) % STAGES) * kDmaStageElems, ring + (it % STAGES) * kDmaStageElems);
  }

  lsum = xor32_sum(xor16_sum(lsum));
  if (!hvalid) return;
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  if (nsplit <= 1) {
    char* dst = p.out + tokq * p.o_st + (int64_t)head * p.o_sh;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int d = 128 * wave + 16 * j + 4 * g;
      const u32x2 v = {E::pack(o[j][0] * inv, o[j][1] * inv), E::pack(o[j][2] * inv, o[j][3] * inv)};
      *reinterpret_cast<u32x2*>(dst + d * 2) = v;
    }
  } else {
    const int64_t slot = ((int64_t)tokq * p.heads + head) * p.max_splits + split;
    float* dst = p.part_o + slot * kVDim;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int d = 128 * wave + 16 * j + 4 * g;
      *reinterpret_cast<f32x4*>(dst + d) = o[j] * inv;
    }
    if (wave == 0 && g == 0) p.part_lse[slot] = lsum > 0.f ? m * c + fast_log2(lsum) : -INFINITY;
  }
}

// ---------------------------------------------------------------------------------------------------------
// Balanced schedule over equal runs of stages, for pages whose size is a multiple of 16 latents.
//
// Unit u = (row, query j, 16-head tile), u = (row * lq + j) * htiles + tile, needs T_u = ceil(L_u / 16) stages
// of 16 latents (L_u latents seen). Laid end to end (prefix P_u) the units' stages are cut into equal runs, one
// per workgroup of a grid that fills the GPU once; every workgroup streams its run through the LDS ring of the
// kernel above, each unit it enters preceded by one stage holding that unit's 16 query rows (the same 16 x 576
// shape as a latent stage). A unit that lies wholly inside one run is finished in place. A unit cut by run
// boundaries leaves (o / l, log2 l + m) per head in slot 0 (the run's first unit) or slot 1 (its last unit) of
// every run it touches, and mla_run_merge_kernel combines them; that kernel also writes the zero output of units
// that see no latents. Every run does equal work, whatever the spread of row lengths, and partials are written
// only where a row crosses a run boundary.
//
// Each stage's work (the score MFMAs, their exchange, the softmax, P.V) runs between two barriers of one
// workgroup. On DeepSeek-V2-Lite's step, two workgroups per CU with a two-stage ring (one stage in flight while one
// is consumed) stream fastest. That is 5% faster than three per CU: their extra runs cut more units, and each cut
// leaves partials to write and merge. It is 3% faster than two per CU with three stages. One workgroup with five or
// eight stages is 40% slower.

constexpr int kRunMin = 16;          // stages per run at least (256 latents)
constexpr int kRunStages = 2;        // ring depth of a run
constexpr int kRunsPerCU = 2;        // run workgroups per CU
constexpr int kRunMaxUnits = 8192;   // units the in-kernel scan serves

__device__ __forceinline__ int unit_latents(const MlaParams& p, int u) {
  const int tq = u / p.htiles;  // row * lq + j
  const int row = tq / p.lq, qj = tq - row * p.lq;
  return p.lens[row] - p.lq + qj + 1;
}

__device__ __forceinline__ int unit_latents_uniform(const MlaParams& p, int u) {
  const int tq = u / p.htiles;
  const int row = tq / p.lq, qj = tq - row * p.lq;
  return sload(p.lens + row) - p.lq + qj + 1;
}

__device__ __forceinline__ int unit_stages(const MlaParams& p, int u) {
  const int lk = unit_latents(p, u);
  return lk > 0 ? (lk + kDmaTile - 1) / kDmaTile : 0;
}

// Position in a run's stage sequence: unit u (prefix pu, tu stages, lk latents), next tile t (-1: its query). The
// unit's query row tq and head tile ht, its block-table row, and the cache page of the last tile loaded are kept
// here, so a stage's loads need no division and at most one page lookup per page.
struct RunCursor {
  int u, pu, tu, lk, t;
  int tq, ht, pg;
  const int32_t* table;
  const char* page;
  bool done;
};

template <typename T, int STAGES>
__global__ __launch_bounds__(256) void mla_run_kernel(MlaParams p) {
  static_assert(STAGES >= 2 && STAGES <= 8, "the stage waits cover up to seven stages in flight");
  using E = Elem<T>;
  __shared__ __attribute__((aligned(16))) uint16_t ring[STAGES * kDmaStageElems];
  __shared__ f32x4 spart[4][64];  // each wave's partial S^T of the stage
  __shared__ int wave_tot[4];
  __shared__ int first[2];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const float c = p.scale_log2;

  // Stage counts over units; thread tid sums units [ulo, uhi). Exclusive scan of those sums across the block.
  const int per_thread = (p.units + 255) / 256;
  const int ulo = min(tid * per_thread, p.units), uhi = min(ulo + per_thread, p.units);
  int local = 0;
  for (int u = ulo; u < uhi; ++u) local += unit_stages(p, u);
  int x = local;
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) wave_tot[wave] = x;
  __syncthreads();
  int excl = x - local, total = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    excl += w < wave ? wave_tot[w] : 0;
    total += wave_tot[w];
  }
  total = __builtin_amdgcn_readfirstlane(total);
  const int per = max((total + (int)gridDim.x - 1) / (int)gridDim.x, kRunMin);
  if (blockIdx.x == 0) {  // the prefix, for the merge
    int run = excl;
    for (int u = ulo; u < uhi; ++u) {
      p.prefix[u] = run;
      run += unit_stages(p, u);
    }
    if (tid == 0) {
      p.prefix[p.units] = total;
      p.prefix[p.units + 1] = per;
    }
  }
  const int start = blockIdx.x * per;
  if (start >= total) return;
  const int end = min(start + per, total);
  if (local > 0 && excl <= start && start < excl + local) {
    int u = ulo, acc = excl;
    for (int tu = unit_stages(p, u); acc + tu <= start; tu = unit_stages(p, u)) {
      acc += tu;
      ++u;
    }
    first[0] = u;
    first[1] = acc;
  }
  __syncthreads();

  // Both cursors walk the same sequence: for each unit, its query stage, then its tiles inside [start, end).
  auto enter = [&](RunCursor& r, int u, int pu) {
    int lk = unit_latents_uniform(p, u);
    while (lk <= 0) lk = unit_latents_uniform(p, ++u);  // units without latents hold no stages
    r.u = u;
    r.pu = pu;
    r.lk = lk;
    r.tu = (lk + kDmaTile - 1) / kDmaTile;
    r.t = -1;
    r.tq = u / p.htiles;
    r.ht = u - r.tq * p.htiles;
    r.table = p.tables + (int64_t)(r.tq / p.lq) * p.t_stride;
    r.pg = -1;
    r.page = nullptr;
    r.done = false;
  };
  auto advance = [&](RunCursor& r) {
    if (r.t < 0) {
      r.t = max(start, r.pu) - r.pu;
    } else if (r.pu + r.t + 1 == end) {
      r.done = true;
    } else if (r.t + 1 == r.tu) {
      enter(r, r.u + 1, r.pu + r.tu);
    } else {
      ++r.t;
    }
  };
  RunCursor prod, cons;
  enter(prod, __builtin_amdgcn_readfirstlane(first[0]), __builtin_amdgcn_readfirstlane(first[1]));
  cons = prod;

  // This wave's loads j = wave + 4 i (i < 5) of a stage's 19: slot 64 j + lane is 16-byte chunk `part` of row r
  // (latent or head) of the stage. Slots 74 r + 72 and 74 r + 73 of row r are LDS padding, filled with copies of
  // chunk 71.
  int lrow[5], lpart[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    const int slot = min(64 * (wave + 4 * i) + lane, kDmaStageSlots - 1);
    lrow[i] = slot / kDmaRowSlots;
    lpart[i] = min(slot - lrow[i] * kDmaRowSlots, kLatChunks - 1) * 16;
  }
  // Query stage: head ht 16 + r of the unit's token (heads past the last load the last head; not written).
  // Latent stage: latents t0 .. t0 + 15 of the row, one page (the page size is a multiple of 16); latents at
  // or past lk load latent lk - 1 instead (finite values; their weight is 0).
  auto fill = [&](RunCursor& r, uint16_t* stage) {
    if (r.t < 0) {
      const char* qrow = p.q + r.tq * p.q_st;
#pragma unroll
      for (int i = 0; i < 5; ++i) {
        const int j = wave + 4 * i;
        if (j < kDmaInstr && 64 * j + lane < kDmaStageSlots)
          lds_dma16(qrow + (int64_t)min(r.ht * 16 + lrow[i], p.heads - 1) * p.q_sh + lpart[i],
                    lds_addr(stage + 64 * 8 * j));
      }
    } else {
      const int t0 = r.t * kDmaTile;
      const int pg = (int)p.bs.div(t0);
      if (pg != r.pg) {
        r.pg = pg;
        r.page = p.cache + (int64_t)sload(r.table + pg) * p.c_sb;
      }
      const char* base = r.page + (int64_t)(t0 - pg * (int)p.bs.d) * p.c_st;
      const int last = r.lk - 1 - t0;
#pragma unroll
      for (int i = 0; i < 5; ++i) {
        const int j = wave + 4 * i;
        if (j < kDmaInstr && 64 * j + lane < kDmaStageSlots)
          lds_dma16(base, (uint32_t)(min(lrow[i], last) * (int)p.c_st + lpart[i]), lds_addr(stage + 64 * 8 * j));
      }
    }
  };

  // S^T = Lat Q^T over K = 576 is split over the waves: wave w takes MFMA k-steps [s0, s0 + ns) of the 18.
  const int s0 = wave < 2 ? 5 * wave : 4 * wave + 2, ns = wave < 2 ? 5 : 4;
  u32x4 qb[5];
  float m = -INFINITY, lsum = 0.f;
  f32x4 o[8];
  int issued = 0;
  for (; issued < STAGES - 1 && !prod.done; ++issued) {
    fill(prod, ring + issued * kDmaStageElems);
    advance(prod);
  }
  for (int k = 0; !cons.done; ++k) {
    dma_stage_barrier(issued - k - 1, wave);  // stage k has landed for every wave
    // Refill the slot read last iteration (every wave has passed the barrier, so its reads are done).
    if (!prod.done) {
      fill(prod, ring + (issued % STAGES) * kDmaStageElems);
      advance(prod);
      ++issued;
    }
    const uint16_t* stage = ring + (k % STAGES) * kDmaStageElems;
    if (cons.t < 0) {
      // Q^T operand of this wave's k-steps: lane holds dims 32 (s0 + i) + 8 g .. + 7 of head n.
      const uint16_t* qs = stage + n * kMlaPitch + 32 * s0 + 8 * g;
#pragma unroll
      for (int i = 0; i < 5; ++i)
        if (i < ns) qb[i] = *reinterpret_cast<const u32x4*>(qs + 32 * i);
      m = -INFINITY;
      lsum = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = f32x4{0, 0, 0, 0};
      advance(cons);
      continue;
    }
    const int t0 = cons.t * kDmaTile;
    f32x4 sc = {0, 0, 0, 0};  // latents t0 + 4 g + r of head n
    const uint16_t* arow = stage + n * kMlaPitch + 32 * s0 + 8 * g;
#pragma unroll
    for (int i = 0; i < 5; ++i)
      if (i < ns) sc = E::mfma16x16x32(*reinterpret_cast<const u32x4*>(arow + 32 * i), qb[i], sc);
    // Sum the four partials, in the same order in every wave (every wave then holds the same S^T). The barrier
    // waits for LDS only: the stage loads in flight are not waited for.
    spart[wave][lane] = sc;
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    sc = (spart[0][lane] + spart[1][lane]) + (spart[2][lane] + spart[3][lane]);
    if (t0 + kDmaTile > cons.lk) {
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[r] = t0 + 4 * g + r < cons.lk ? sc[r] : -INFINITY;
    }
    float mx = vmax(vmax(sc[0], sc[1]), vmax(sc[2], sc[3]));
    mx = xor32_max(xor16_max(mx));
    if (__any(mx > m && (m == -INFINITY || (mx - m) * c > kRescaleSlack))) {
      const float mn = vmax(m, mx);
      const float alpha = m == -INFINITY ? 0.f : fast_exp2((m - mn) * c);
      m = mn;
      lsum *= alpha;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] *= alpha;
    }
    const float mc = m * c;
    float pr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pr[r] = fast_exp2(fmaf(sc[r], c, -mc));
    lsum += (pr[0] + pr[1]) + (pr[2] + pr[3]);
    const u32x2 pb = {E::pack(pr[0], pr[1]), E::pack(pr[2], pr[3])};
    const uint16_t* v = stage + (4 * g + (n >> 2)) * kMlaPitch + 128 * wave + 4 * (n & 3);
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = E::mfma16x16x16(lds_read_tr16(v + 16 * j), pb, o[j]);

    if (cons.t + 1 == cons.tu || cons.pu + cons.t + 1 == end) {  // the unit's last stage in this run
      const float l = xor32_sum(xor16_sum(lsum));
      const int tq = cons.tq, head = cons.ht * 16 + n;
      const float inv = 1.f / l;  // l > 0: each of the run's stages of the unit holds a latent in range
      if (head < p.heads) {
        if (cons.pu >= start && cons.pu + cons.tu <= end) {
          char* dst = p.out + tq * p.o_st + (int64_t)head * p.o_sh;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int d = 128 * wave + 16 * j + 4 * g;
            const u32x2 val = {E::pack(o[j][0] * inv, o[j][1] * inv), E::pack(o[j][2] * inv, o[j][3] * inv)};
            *reinterpret_cast<u32x2*>(dst + d * 2) = val;
          }
        } else {
          const int slot = (blockIdx.x * 2 + (cons.pu <= start ? 0 : 1)) * 16 + n;
          float* dst = p.part_o + (int64_t)slot * kVDim;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int d = 128 * wave + 16 * j + 4 * g;
            *reinterpret_cast<f32x4*>(dst + d) = o[j] * inv;
          }
          if (wave == 0 && g == 0) p.part_lse[slot] = m * c + fast_log2(l);
        }
      }
    }
    advance(cons);
  }
}

// Finish units cut by run boundaries (log-sum-exp over the runs that touched them) and zero the output of units
// that see no latents; units finished in place are left alone. Block (unit, head of its tile), 64 threads.
template <typename T>
__global__ __launch_bounds__(64) void mla_run_merge_kernel(MlaParams p) {
  using E = Elem<T>;
  const int u = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int tq = u / p.htiles, head = (u - tq * p.htiles) * 16 + h;
  if (head >= p.heads) return;
  const int pu = p.prefix[u], tu = p.prefix[u + 1] - pu, per = p.prefix[p.units + 1];
  constexpr int PER = kVDim / 64;
  float o[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) o[e] = 0.f;
  if (tu > 0) {
    const int b0 = pu / per, b1 = (pu + tu - 1) / per;
    if (b0 == b1) return;
    // The runs' partials, kRunMergeBatch at a time with every load of a batch issued before the first is used;
    // the max and the sums carry from batch to batch.
    constexpr int kRunMergeBatch = 4;
    float m = -INFINITY, den = 0.f;
    for (int c0 = b0; c0 <= b1; c0 += kRunMergeBatch) {
      float ls[kRunMergeBatch];
      f32x4 x[kRunMergeBatch][PER / 4];
#pragma unroll
      for (int i = 0; i < kRunMergeBatch; ++i) {
        const int b = c0 + i;
        ls[i] = -INFINITY;
#pragma unroll
        for (int e = 0; e < PER / 4; ++e) x[i][e] = f32x4{0, 0, 0, 0};
        if (b <= b1) {  // wave-uniform
          const int slot = (b * 2 + (b == b0 && pu != b0 * per ? 1 : 0)) * 16 + h;
          ls[i] = p.part_lse[slot];
          const f32x4* src = reinterpret_cast<const f32x4*>(p.part_o + (int64_t)slot * kVDim + lane * PER);
#pragma unroll
          for (int e = 0; e < PER / 4; ++e) x[i][e] = src[e];
        }
      }
      float bm = m;
#pragma unroll
      for (int i = 0; i < kRunMergeBatch; ++i) bm = fmaxf(bm, ls[i]);
      if (bm == -INFINITY) continue;
      const float alpha = fast_exp2(m - bm);  // 0 while m is -inf
      den *= alpha;
#pragma unroll
      for (int e = 0; e < PER; ++e) o[e] *= alpha;
#pragma unroll
      for (int i = 0; i < kRunMergeBatch; ++i) {
        const float w = fast_exp2(ls[i] - bm);  // 0 past the last run
        den += w;
#pragma unroll
        for (int e = 0; e < PER / 4; ++e)
#pragma unroll
          for (int r = 0; r < 4; ++r) o[4 * e + r] = fmaf(w, x[i][e][r], o[4 * e + r]);
      }
      m = bm;
    }
    const float inv = den > 0.f ? 1.f / den : 0.f;
#pragma unroll
    for (int e = 0; e < PER; ++e) o[e] *= inv;
  }
  u32x4 packed;
#pragma unroll
  for (int w = 0; w < 4; ++w) packed[w] = E::pack(o[2 * w], o[2 * w + 1]);
  *reinterpret_cast<u32x4*>(p.out + tq * p.o_st + (int64_t)head * p.o_sh + lane * PER * 2) = packed;
}

// Combine a split query's partials: o = sum_s 2^(lse_s - M) o_s / sum_s 2^(lse_s - M).
template <typename T>
__global__ __launch_bounds__(64) void mla_merge_kernel(MlaParams p) {
  using E = Elem<T>;
  const int tokq = blockIdx.x, head = blockIdx.y, lane = threadIdx.x;
  const int row = tokq / p.lq, qj = tokq - row * p.lq;
  const int lk = p.lens[row] - p.lq + qj + 1;
  const int nsplit = lk > 0 ? min((lk + p.split - 1) / p.split, p.max_splits) : 0;
  if (nsplit <= 1) return;
  const int64_t slot0 = ((int64_t)tokq * p.heads + head) * p.max_splits;
  float mmax = -INFINITY;
  for (int s = 0; s < nsplit; ++s) mmax = fmaxf(mmax, p.part_lse[slot0 + s]);
  constexpr int PER = kVDim / 64;
  float o[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) o[e] = 0.f;
  float den = 0.f;
  if (mmax != -INFINITY) {
    for (int s = 0; s < nsplit; ++s) {
      const float w = fast_exp2(p.part_lse[slot0 + s] - mmax);
      den += w;
      const f32x4* src = reinterpret_cast<const f32x4*>(p.part_o + (slot0 + s) * kVDim + lane * PER);
#pragma unroll
      for (int e = 0; e < PER / 4; ++e) {
        const f32x4 x = src[e];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[4 * e + r] = fmaf(w, x[r], o[4 * e + r]);
      }
    }
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  u32x4 packed;
#pragma unroll
  for (int w = 0; w < 4; ++w) packed[w] = E::pack(o[2 * w] * inv, o[2 * w + 1] * inv);
  *reinterpret_cast<u32x4*>(p.out + tokq * p.o_st + (int64_t)head * p.o_sh + lane * PER * 2) = packed;
}

struct MlaShape {
  int32_t split, max_splits;  // split schedule
  int32_t runs, units;        // run schedule: workgroups, units
  size_t lse_off, o_off, prefix_off, bytes;
};


template <typename T>
static void launch_dma(const MlaParams& p, bool one_page, dim3 grid, hipStream_t st) {
  if (one_page)
    hipLaunchKernelGGL((mla_decode_dma_kernel<T, kMlaSplitStages, true>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((mla_decode_dma_kernel<T, kMlaSplitStages, false>), grid, dim3(256), 0, st, p);
}

static MlaShape mla_shape(int32_t rows, int32_t lq, int32_t heads, int32_t max_k) {
  MlaShape s{};
  const int64_t units = (int64_t)rows * lq * ((heads + 15) / 16);
  const int64_t keys = max_k > 0 ? max_k : 1;
  // Split schedule (pages not a multiple of 16 latents, or too many units for the in-kernel scan).
  int64_t split = 256;
  while (split < kMlaMaxSplit && split < keys && units * ((keys + split - 1) / split) > kMlaSplitTarget)
    split *= 2;
  s.split = (int32_t)split;
  s.max_splits = (int32_t)((keys + split - 1) / split);
  const size_t parts = s.max_splits > 1 ? (size_t)rows * lq * heads * s.max_splits : 0;
  // Run schedule: two workgroups per CU, fewer when the stages cannot fill runs of kRunMin.
  const int64_t stages = units * ((keys + kDmaTile - 1) / kDmaTile);
  s.units = (int32_t)std::min<int64_t>(units, INT32_MAX);
  s.runs = (int32_t)std::max<int64_t>(
      1, std::min<int64_t>(kRunsPerCU * device_cus(), (stages + kRunMin - 1) / kRunMin));
  const size_t run_parts = (size_t)s.runs * 2 * 16;
  const size_t nparts = std::max(parts, run_parts);
  s.lse_off = 0;
  s.o_off = (nparts * sizeof(float) + 255) / 256 * 256;
  s.prefix_off = s.o_off + nparts * kVDim * sizeof(float);
  s.bytes = s.prefix_off + (size_t)(units + 2) * sizeof(int32_t);
  return s;
}

template <typename T>
static void launch_runs(const MlaParams& p, int runs, hipStream_t st) {
  hipLaunchKernelGGL((mla_run_kernel<T, kRunStages>), dim3(runs), dim3(256), 0, st, p);
  hipLaunchKernelGGL(mla_run_merge_kernel<T>, dim3(p.units, 16), dim3(64), 0, st, p);
}

}  // namespace lv

using namespace lv;

extern "C" size_t lv_mla_decode_workspace_bytes(int32_t num_rows, int32_t queries_per_row, int32_t num_heads,
                                                int32_t max_seqlen_k) {
  if (num_rows <= 0 || queries_per_row <= 0 || num_heads <= 0) return 0;
  return mla_shape(num_rows, queries_per_row, num_heads, max_seqlen_k).bytes;
}

extern "C" int lv_mla_decode(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* latent_cache,
                             int64_t cache_stride_block, int64_t cache_stride_token, int32_t block_size,
                             const int32_t* block_tables, int64_t table_stride, const int32_t* context_lens,
                             int32_t num_rows, int32_t queries_per_row, int32_t num_heads, int32_t latent_dim,
                             int32_t v_dim, float scale, int32_t max_seqlen_k, void* out, int64_t out_stride_t,
                             int64_t out_stride_h, void* workspace, size_t workspace_bytes, int32_t dtype,
                             void* stream) {
  LV_REQUIRE(dtype == LV_DTYPE_BF16 || dtype == LV_DTYPE_F16, "mla_decode: dtype %d is not bf16 or fp16", dtype);
  LV_REQUIRE(num_rows >= 0 && queries_per_row > 0 && num_heads > 0, "mla_decode: bad sizes B=%d Lq=%d H=%d",
             num_rows, queries_per_row, num_heads);
  LV_REQUIRE(latent_dim == kLatent && v_dim == kVDim, "mla_decode: latent %d / values %d; %d / %d are served",
             latent_dim, v_dim, kLatent, kVDim);
  if (num_rows == 0) return LV_OK;
  LV_REQUIRE(block_size >= 16, "mla_decode: block_size must be at least 16, got %d", block_size);
  LV_REQUIRE(q && latent_cache && block_tables && context_lens && out, "mla_decode: null tensor pointer");
  LV_REQUIRE(max_seqlen_k >= 0, "mla_decode: negative max_seqlen_k");
  LV_REQUIRE(scale > 0.f, "mla_decode: the softmax scale must be positive, got %g", (double)scale);
  LV_REQUIRE(aligned(q, 16) && aligned(out, 16) && aligned(latent_cache, 16) && (q_stride_t * 2) % 16 == 0 &&
                 (q_stride_h * 2) % 16 == 0 && (out_stride_t * 2) % 16 == 0 && (out_stride_h * 2) % 16 == 0 &&
                 (cache_stride_block * 2) % 16 == 0 && (cache_stride_token * 2) % 16 == 0,
             "mla_decode: tensors and their strides must be 16-byte aligned");
  const MlaShape s = mla_shape(num_rows, queries_per_row, num_heads, max_seqlen_k);
  LV_REQUIRE(workspace_bytes >= s.bytes && (s.bytes == 0 || workspace),
             "mla_decode: workspace of %zu bytes given, %zu needed", workspace_bytes, s.bytes);
  LV_REQUIRE(aligned(workspace, 256), "mla_decode: workspace must be 256-byte aligned");
  LV_REQUIRE(fits_one_launch((int64_t)num_rows * s.max_splits, 256) &&
                 fits_one_launch((int64_t)num_rows * queries_per_row, 64) &&
                 (int64_t)queries_per_row * ((num_heads + 15) / 16) < 65536,
             "mla_decode: %d rows x %d queries x %d splits need a grid larger than one launch holds", num_rows,
             queries_per_row, s.max_splits);

  MlaParams p{};
  p.q = (const char*)q;
  p.q_st = q_stride_t * 2;
  p.q_sh = q_stride_h * 2;
  p.cache = (const char*)latent_cache;
  p.c_sb = cache_stride_block * 2;
  p.c_st = cache_stride_token * 2;
  p.bs = FastDiv::make((uint32_t)block_size);
  p.tables = block_tables;
  p.t_stride = table_stride;
  p.lens = context_lens;
  p.rows = num_rows;
  p.lq = queries_per_row;
  p.heads = num_heads;
  p.htiles = (num_heads + 15) / 16;
  p.scale_log2 = scale * kLog2e;
  p.out = (char*)out;
  p.o_st = out_stride_t * 2;
  p.o_sh = out_stride_h * 2;
  p.split = s.split;
  p.max_splits = s.max_splits;
  char* ws = (char*)workspace;
  p.part_lse = s.max_splits > 1 ? reinterpret_cast<float*>(ws + s.lse_off) : nullptr;
  p.part_o = s.max_splits > 1 ? reinterpret_cast<float*>(ws + s.o_off) : nullptr;

  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool one_page = block_size % kDmaTile == 0 && p.c_st * kDmaTile < ((int64_t)1 << 31);
  // The run schedule counts stages in 32 bits on the device.
  const int64_t stage_bound = (int64_t)s.units * (((int64_t)std::max(max_seqlen_k, 1) + kDmaTile - 1) / kDmaTile);
  if (one_page && s.units <= kRunMaxUnits && stage_bound < ((int64_t)1 << 30)) {
    p.units = s.units;
    p.part_lse = reinterpret_cast<float*>(ws + s.lse_off);
    p.part_o = reinterpret_cast<float*>(ws + s.o_off);
    p.prefix = reinterpret_cast<int32_t*>(ws + s.prefix_off);
    if (dtype == LV_DTYPE_BF16)
      launch_runs<BF16>(p, s.runs, st);
    else
      launch_runs<F16>(p, s.runs, st);
    LV_LAUNCH_CHECK("mla_run_kernel");
    return LV_OK;
  }
  const dim3 grid(num_rows * s.max_splits, queries_per_row * p.htiles);
  if (dtype == LV_DTYPE_BF16)
    launch_dma<BF16>(p, one_page, grid, st);
  else
    launch_dma<F16>(p, one_page, grid, st);
  LV_LAUNCH_CHECK("mla_decode_dma_kernel");
  if (s.max_splits > 1) {
    const dim3 mgrid(num_rows * queries_per_row, num_heads);
    if (dtype == LV_DTYPE_BF16)
      hipLaunchKernelGGL(mla_merge_kernel<BF16>, mgrid, dim3(64), 0, st, p);
    else
      hipLaunchKernelGGL(mla_merge_kernel<F16>, mgrid, dim3(64), 0, st, p);
    LV_LAUNCH_CHECK("mla_merge_kernel");
  }
  return LV_OK;
}
