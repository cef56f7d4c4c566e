// Shared by the paged and the packed-key attention kernels: launch parameters and the prompt item (MFMA).
#pragma once

#include "lv_common.h"

namespace lv {

constexpr int kPrefillKeys = 64;  // keys per prompt tile
constexpr int kPrefillRows = 128;  // (position, head) query rows per prompt item, 32 per wave

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
  const int32_t* n_items;  // [0]: list length, [1]: prompt items at its head
  int32_t* ticket;         // next decode item of a persistent launch (zeroed by the plan kernel)
  // Split rows (listed steps only): per (row, item head group), the count of its splits that have written their
  // partials (zeroed by the plan kernel); the last to arrive merges them and puts the count back to zero.
  int32_t* merge_count;
  // Packed keys only: a row's context keys, seen unmasked before the row's own keys (prefill_item's CTX).
  const char* ctx_k;  // [Tc, Hkv, DQK]
  const char* ctx_v;  // [Tc, Hkv, DV]
  int64_t cx_st, cx_sh, cv_st, cv_sh;  // bytes: context key / value row and head strides
  const int32_t* cu_ctx;               // [rows + 1]
};

__device__ inline int key_len(const AttnParams& p, int row) {
  return p.lens_k ? p.lens_k[row] : p.cu_k[row + 1] - p.cu_k[row];
}

// ---------------------------------------------------------------------------------------------------------
// Prompt item: (row, tile of query positions, kv head). The 32 WAVES (position, head) query rows of one GQA group (32
// per wave, as two 16-row MFMA blocks that share every K and V operand read) run against 64-key tiles staged
// row-major in LDS, the next tile's K/V loads in flight in registers meanwhile. S^T = K Q^T and O^T += V^T P^T on
// MFMA 16x16x32 with fp32 accumulation; the V^T operands come from the row-major value tile by the transposing
// LDS read. Online softmax per query row with the scale folded into the exp2 argument. The causal mask (query j of
// a row with lq queries and lk keys sees keys 0 .. lk - lq + j; none if p.causal is 0) is applied only on tiles
// that cross it. DQK: q.k width; DV: value width.
// The row max, in at most two passes over the item's tiles:
// - held (the first pass; bf16 only, whose P operands hold the fp32 range): taken from the item's first tile and
//   held, so later tiles compute no max and never rescale. Every query row sees its first tile's keys (key 0, or
//   the context keys, come first), so on ordinary data a row's first-tile max sits within a few log2 units of its
//   final one. After the last tile every row sum must be finite and below kHeldLimit (all probabilities <=
//   2^kHeldSlack); otherwise (scores that rose far above a row's first tile, or non-finite ones) the workgroup
//   makes the second pass;
// - running (the second pass): replaced only when a tile raises it by more than kRescaleSlack (log2 units), so
//   rescaling the accumulators is rare and probabilities stay <= 2^kRescaleSlack.

// Stage tiles are row-major, laid out so that the operand reads (row = lane % 16, one 16-byte chunk per lane) and the
// transposing value reads (rows 4 j4 + n / 4, 8 bytes per lane) meet no bank conflicts on gfx950. Its LDS (64 banks
// of 4 bytes) serves a 16-byte read in passes over lanes {0-7, 16-23}, {8-15, 24-31}, ... and an 8-byte read over
// lanes {0-31}, {32-63}; counter probes confirm the model (row pitches of 72 and 104 dwords conflict-free; 68, 76,
// 80, 100 and 108 two-way). Two layouts meet it:
// - padded (SWZ false): a 32-byte pad per row (pitch 8 mod 16 dwords), the pad slots loaded with copies of the row's
//   last chunk; every read offset is a compile-time immediate;
// - swizzled (SWZ true): no padding, chunk c of row r at position c ^ 2 (r mod 8) for rows of 16 chunks, c ^ (r mod 8)
//   for rows of 8 or 24. A 64-lane load then covers whole key rows, so on pages of 16 or 32 keys each load stays in
//   one page; the reads take per-lane offsets (measured 1.6% slower on one-page tiles, so those keep the pads).
template <int DQK, int DV, bool SWZ = false>
struct PromptSmem {
  static constexpr int kKRow = SWZ ? DQK : DQK + 16;  // key tile row pitch, elements
  static constexpr int kVRow = SWZ ? DV : DV + 16;    // value tile row pitch, elements
  static constexpr int kBytes = kPrefillKeys * (kKRow + kVRow) * 2;
};

// Position of 16-byte chunk c in a stage row r of CH chunks (an involution: it also maps a position to its chunk).
template <int CH, bool SWZ>
__device__ __forceinline__ int swz(int r, int c) {
  static_assert(CH == 8 || CH == 16 || CH == 24, "rows of 8, 16 or 24 chunks");
  if constexpr (!SWZ) return c;
  return c ^ (CH == 16 ? 2 * (r & 7) : (r & 7));
}

// PREFETCH: the next tile's K/V loads are in flight in registers while this tile is consumed (more registers).
// OPAQUE_TID: for a caller that runs items in a loop; the thread index is hidden from the optimiser, so per-lane
// offsets are recomputed per item rather than hoisted out of the loop and spilled.
// RING > 0: tiles go straight from memory into a ring of RING LDS stages (smem holds RING * PromptSmem::kBytes),
// RING - 1 in flight while one is consumed, one barrier per tile; for keys whose 64-key tiles each lie in one page
// (unpaged, or pages a multiple of 64). The caller picks it; the register path serves every other page size.
// WAVES: waves of the workgroup (blockDim.x == 64 WAVES), each taking 32 query rows; an item is 32 WAVES rows, so
// with 8 waves every staged K/V tile serves twice the rows of a 4-wave item.
// CTX (packed keys, RING > 0): the row's context keys (p.ctx_k / p.ctx_v, rows p.cu_ctx) come first, every one
// visible to every query, then the row's own keys under the mask above -- one softmax over both, as the attention
// over [context; own keys] with the mask aligned to the end.
// TP (paged keys, RING > 0): pages per 64-key tile -- 1 for pages of a multiple of 64 keys (one lookup per page,
// kept across the page's tiles), 2 or 4 for pages of 32 or 16 keys (the tile's pages looked up at every fill, each
// lane loading from its key's page).
template <typename T, int DQK, int DV, bool PREFETCH = true, bool OPAQUE_TID = false, int RING = 0, int WAVES = 4,
          bool CTX = false, int TP = 1>
__device__ void prefill_item(const AttnParams& p, int row, int qtile, int kvh, char* smem) {
  using E = Elem<T>;
  constexpr int KS = DQK / 32;  // MFMA k-steps over the q.k width
  constexpr int DB = DV / 16;   // 16-dim blocks of the output
  constexpr bool SWZ = TP > 1;  // the swizzled stage layout (pages of 16 or 32 keys)
  constexpr int KROW = PromptSmem<DQK, DV, SWZ>::kKRow;
  constexpr int VROW = PromptSmem<DQK, DV, SWZ>::kVRow;
  constexpr int KCH = DQK / 8, VCH = DV / 8;  // 16-byte chunks per key / value row
  constexpr int KCHUNKS = kPrefillKeys * KCH;
  constexpr int NT = 64 * WAVES;                        // threads
  constexpr int ROWS = 32 * WAVES;                      // (position, head) query rows per item
  constexpr int KPER = KCHUNKS / NT;                    // key chunks each thread stages per tile
  constexpr int PER = kPrefillKeys * (KCH + VCH) / NT;  // all chunks each thread stages per tile
  static_assert(WAVES == 4 || WAVES == 8, "4 or 8 waves");
  static_assert(RING > 0 || (KCHUNKS % NT == 0 && kPrefillKeys * (KCH + VCH) % NT == 0),
                "tile chunks split over the threads");
  static_assert(DQK % 32 == 0 && DV % 16 == 0, "MFMA tile widths");
  static_assert(!CTX || RING > 0, "context keys stream through the LDS ring");
  static_assert((TP == 1 || TP == 2 || TP == 4) && (TP == 1 || (RING > 0 && !CTX)), "pages per 64-key tile");
  int tid = threadIdx.x;
  if (OPAQUE_TID) asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, j4 = lane >> 4;
  const int G = p.group;
  const int qp = ROWS / G;  // positions per item
  const int q0 = p.cu_q[row], lq = p.cu_q[row + 1] - q0;
  const int lk = key_len(p, row);
  const int p0 = qtile * qp;
  if (p0 >= lq) return;  // a grid sized for the longest row
  const float c = p.scale_log2;

  // Two 16-row query blocks per wave: rows 32 wave + 16 nb + n.
  int qi[2], head[2], lim[2];
  bool qvalid[2];
  u32x4 qb[2][KS];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int mrow = wave * 32 + nb * 16 + n;
    qi[nb] = p0 + mrow / G;
    head[nb] = kvh * G + mrow % G;
    qvalid[nb] = mrow < qp * G && qi[nb] < lq;
    lim[nb] = qvalid[nb] && p.causal ? lk - lq + qi[nb] + 1 : lk;  // this query row sees keys < lim
#pragma unroll
    for (int k = 0; k < KS; ++k)
      qb[nb][k] = qvalid[nb] ? ld16(p.q + (int64_t)(q0 + qi[nb]) * p.q_st + head[nb] * p.q_sh +
                                    (int64_t)(32 * k + 8 * j4) * 2)
                             : u32x4{0, 0, 0, 0};
  }
  const int kmax = p.causal ? min(lk, lk - lq + min(p0 + qp, lq)) : lk;  // keys the item needs
  int lc = 0, cbase = 0;  // the row's context keys
  if constexpr (CTX) {
    cbase = p.cu_ctx[row];
    lc = p.cu_ctx[row + 1] - cbase;
  }
  const int nc = (lc + kPrefillKeys - 1) / kPrefillKeys;                  // context tiles
  const int ntiles = nc + (kmax + kPrefillKeys - 1) / kPrefillKeys;       // all tiles of the item

  float m[2], l[2];  // raw-score max (held or running) and row sums
  f32x4 o[2][DB];

  // Staging: chunk i of this thread is key key_of(i) (a tile row), 16-byte part part_of(i).
  auto key_of = [&](int i) { return i < KPER ? (tid + NT * i) / KCH : (tid + NT * i - KCHUNKS) / VCH; };
  auto part_of = [&](int i) {
    return i < KPER ? (tid + NT * i) % KCH : (tid + NT * i - KCHUNKS) % VCH;
  };
  const int32_t* table = p.tables + (int64_t)row * p.t_stride;
  const int kbase = p.paged ? 0 : p.cu_k[row];
  const bool one_page = !p.paged || p.bs.d % kPrefillKeys == 0;  // every tile lies in one page
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
    const bool tail = kt + kPrefillKeys > lk;
    if (one_page) {
      const char* kb = p.k_cache + row_off(kt, false);
      const char* vb = p.v_cache + row_off(kt, true);
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int key = key_of(i);
        const char* src = i < KPER ? kb + (int64_t)key * p.c_st : vb + (int64_t)key * p.v_st;
        st[i] = !tail || kt + key < lk ? ld16(src + part_of(i) * 16) : u32x4{0, 0, 0, 0};
      }
    } else {
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int jk = kt + key_of(i);
        st[i] = jk < lk ? ld16((i < KPER ? p.k_cache : p.v_cache) + row_off(jk, i >= KPER) + part_of(i) * 16)
                        : u32x4{0, 0, 0, 0};
      }
    }
  };
  auto stash = [&](uint16_t* ks, uint16_t* vs, const u32x4 (&st)[PER]) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int key = key_of(i), part = part_of(i);
      uint16_t* dst =
          i < KPER ? ks + key * KROW + swz<KCH, SWZ>(key, part) * 8 : vs + key * VROW + swz<VCH, SWZ>(key, part) * 8;
      st16(reinterpret_cast<char*>(dst), st[i]);
    }
  };

  // Swizzled element offsets of this lane's operand reads inside a stage row, the same for every tile: the key chunk
  // of k-step k (row 16 kb + n, chunk 4 k + j4), and the value half-chunk of output block b (rows 32 h + 4 j4 + n / 4
  // (+ 16), dims 16 b + 4 (n % 4) .. + 3).
  // (Padded layout: 32 k + 8 j4 and 16 b + 4 (n % 4), offsets the compiler folds into the reads' immediates.)
  int kpos[SWZ ? KS : 1], vpos[SWZ ? DB : 1];
  if constexpr (SWZ) {
#pragma unroll
    for (int k = 0; k < KS; ++k) kpos[k] = 8 * swz<KCH, SWZ>(n, 4 * k + j4);
#pragma unroll
    for (int b = 0; b < DB; ++b)
      vpos[b] = 8 * swz<VCH, SWZ>(4 * j4 + (n >> 2), 2 * b + ((n & 3) >> 1)) + 4 * (n & 1);
  }

  // One 64-key tile (keys kt .. kt + 63 of its source) from the K/V tile in LDS at ks / vs: scores, mask (query row
  // nb sees keys < l[nb]), online softmax, P.V. first: the item's first tile; running: the second pass (both
  // wave-uniform).
  auto consume = [&](int kt, const int (&lm)[2], const uint16_t* ks, const uint16_t* vs, bool first, bool running) {
    // S^T (keys x query rows): st[kb][nb] lane holds keys kt + 16 kb + 4 j4 + r of query row (nb, n).
    f32x4 st[4][2];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) st[kb][nb] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < KS; ++k)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(ks + (kb * 16 + n) * KROW +
                                                         (SWZ ? kpos[SWZ ? k : 0] : 32 * k + 8 * j4));
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) st[kb][nb] = E::mfma16x16x32(a, qb[nb][k], st[kb][nb]);
      }
    // Mask only a tile that crosses some row's last key (wave-uniform test).
    if (__any(kt + kPrefillKeys > lm[0] || kt + kPrefillKeys > lm[1])) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = kt + kb * 16 + 4 * j4 + r;
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) st[kb][nb][r] = key < lm[nb] ? st[kb][nb][r] : -INFINITY;
        }
    }
    if (first || running) {  // held: only the first tile takes a max
      float mx[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        float x = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
          x = vmax(x, vmax(vmax(st[kb][nb][0], st[kb][nb][1]), vmax(st[kb][nb][2], st[kb][nb][3])));
        mx[nb] = xor32_max(xor16_max(x));  // over the row's 64 keys of this tile
      }
      if (!running) {  // the held max: nothing is accumulated yet
        m[0] = mx[0];
        m[1] = mx[1];
      } else {
        const bool grow = (mx[0] > m[0] && (m[0] == -INFINITY || (mx[0] - m[0]) * c > kRescaleSlack)) ||
                          (mx[1] > m[1] && (m[1] == -INFINITY || (mx[1] - m[1]) * c > kRescaleSlack));
        if (__any(grow)) {
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) {
            const float mn = vmax(m[nb], mx[nb]);
            const float alpha = m[nb] == -INFINITY ? 0.f : fast_exp2((m[nb] - mn) * c);
            m[nb] = mn;
            l[nb] *= alpha;
#pragma unroll
            for (int b = 0; b < DB; ++b) o[nb][b] *= alpha;
          }
        }
      }
    }
    // P^T operands: k slots 8 j4 .. 8 j4 + 7 = keys 32 h + 4 j4 + 0..3, then 32 h + 16 + 4 j4 + 0..3.
    u32x4 pb[2][2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const float mc = m[nb] == -INFINITY ? 0.f : m[nb] * c;  // a row with no key yet: every score is -inf
      float psum = 0.f;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float pr[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pr[r] = fast_exp2(fmaf(st[2 * h][nb][r], c, -mc));
          pr[4 + r] = fast_exp2(fmaf(st[2 * h + 1][nb][r], c, -mc));
        }
#pragma unroll
        for (int r = 0; r < 8; ++r) psum += pr[r];
#pragma unroll
        for (int w = 0; w < 4; ++w) pb[nb][h][w] = E::pack(pr[2 * w], pr[2 * w + 1]);
      }
      l[nb] += psum;
    }
    // V^T operand rows (dims) 16 b + n; transposing reads of rows 32 h + 4 j4 + (n >> 2) (+ 16), dims + 4 (n & 3).
    const uint16_t* vrow = vs + (4 * j4 + (n >> 2)) * VROW + (SWZ ? 0 : 4 * (n & 3));
#pragma unroll
    for (int b = 0; b < DB; ++b)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int vb = SWZ ? vpos[SWZ ? b : 0] : 16 * b;
        const u32x2 lo = lds_read_tr16(vrow + 32 * h * VROW + vb);
        const u32x2 hi = lds_read_tr16(vrow + (32 * h + 16) * VROW + vb);
        const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) o[nb][b] = E::mfma16x16x32(a, pb[nb][h], o[nb][b]);
      }
  };

  // A pass over the item's tiles, with the held max (RUNNING false) or the running one.
  auto run_pass = [&](auto running_tag) {
  constexpr bool running = decltype(running_tag)::value;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    m[nb] = -INFINITY;
    l[nb] = 0.f;
#pragma unroll
    for (int b = 0; b < DB; ++b) o[nb][b] = f32x4{0, 0, 0, 0};
  }
  if constexpr (RING > 0) {
    // Stage layout: 64 key rows of KJ 16-byte slots, then 64 value rows of VJ (KCH / VCH chunks, plus two pad slots
    // in the padded layout, which hold copies of the row's last chunk). 64-lane load j covers slots 64 j .. 64 j + 63
    // (of the key rows for j < KJ, else of the value rows); lane l of it loads the chunk that belongs at its slot.
    // Wave w issues j = w, w + WAVES, ... Keys at or past lk load key lk - 1 instead (finite values; their weight is
    // 0).
    constexpr int KJ = KCH + (SWZ ? 0 : 2), VJ = VCH + (SWZ ? 0 : 2);
    constexpr int NJ = KJ + VJ;  // loads per stage
    // this wave's loads per stage: waves < NJ % WAVES take HI
    constexpr int CNT_HI = (NJ + WAVES - 1) / WAVES, CNT_LO = NJ / WAVES;
    constexpr int kStageElems = PromptSmem<DQK, DV, SWZ>::kBytes / 2;
    static_assert(KROW == KJ * 8 && VROW == VJ * 8, "pitches");
    static_assert(RING >= 2 && RING <= 3, "one or two tiles in flight");
    uint16_t* ring = reinterpret_cast<uint16_t*>(smem);
    const bool hi = wave < NJ % WAVES || NJ % WAVES == 0;
    // Stages fill in key order, so the page of the last fill is kept: one page-table lookup per page, shared by
    // the key and value sources (a page of 256 keys holds four tiles).
    int cached_pg = -1;
    int64_t page_off = 0;  // the cached page's byte offset in either cache
    // Tile t of the item: context tile t (t < nc), else the row's keys from (t - nc) 64.
    auto fill = [&](int t, uint16_t* stage) {
      const bool in_ctx = CTX && t < nc;
      const int kt = (in_ctx ? t : t - nc) * kPrefillKeys;
      const int last = (in_ctx ? lc : lk) - 1 - kt;
      const int64_t kst = in_ctx ? p.cx_st : p.c_st, vst = in_ctx ? p.cv_st : p.v_st;
      // Load j of this wave: chunk position slot of the key (isk) or value rows; its key row and source chunk.
      auto source = [&](int j, bool& isk, int& key, int& chunk) {
        isk = j < KJ;  // wave-uniform
        const int slot = 64 * (isk ? j : j - KJ) + lane;
        const int kkey = slot / KJ, vkey = slot / VJ;
        key = isk ? kkey : vkey;
        chunk = isk ? swz<KCH, SWZ>(kkey, min(slot - kkey * KJ, KCH - 1))
                    : swz<VCH, SWZ>(vkey, min(slot - vkey * VJ, VCH - 1));
      };
      if constexpr (TP > 1) {
        // Pages of BS = 64 / TP keys. A load's 64 lanes cover 64 / KCH (or 64 / VCH) consecutive keys inside one page
        // (those past the row's end load its last key, on the same page), so each load has a wave-uniform page: the
        // tile's TP page numbers (clamped to the row's last page) come in with one scalar wait.
        constexpr int BS = kPrefillKeys / TP;
        static_assert(SWZ && kPrefillKeys / KCH <= BS && kPrefillKeys / VCH <= BS, "a load within one page");
        const int pg_last = (lk - 1) / BS;
        const int32_t* pp[TP];
#pragma unroll
        for (int q = 0; q < TP; ++q) pp[q] = table + min(t * TP + q, pg_last);
        int pg[TP];
        sload_n<TP>(pp, pg);
#pragma unroll
        for (int i = 0; i < (NJ + WAVES - 1) / WAVES; ++i) {
          const int j = wave + WAVES * i;
          if (NJ % WAVES == 0 || i < NJ / WAVES || j < NJ) {
            bool isk;
            int key, chunk;
            source(j, isk, key, chunk);
            const int first = min((isk ? j : j - KJ) * (kPrefillKeys / (isk ? KJ : VJ)), last);
            const int q = first / BS;  // wave-uniform
            int page = pg[0];
#pragma unroll
            for (int qq = 1; qq < TP; ++qq) page = q == qq ? pg[qq] : page;
            const char* base = (isk ? p.k_cache : p.v_cache) + (int64_t)page * p.c_sb + kvh * (isk ? p.c_sh : p.v_sh);
            const uint32_t off = __umul24(min(key, last) - q * BS, (uint32_t)(isk ? p.c_st : p.v_st)) + chunk * 16;
            lds_dma16<false>(base, off, lds_addr(stage + 64 * 8 * j));  // tiles other query tiles read again
          }
        }
        return;
      }
      int64_t koff, voff;  // wave-uniform byte offsets of key kt of this kv head
      if (in_ctx) {
        koff = (int64_t)(cbase + kt) * p.cx_st + kvh * p.cx_sh;
        voff = (int64_t)(cbase + kt) * p.cv_st + kvh * p.cv_sh;
      } else if (p.paged) {
        const int pg = (int)p.bs.div(kt);
        if (pg != cached_pg) {
          cached_pg = pg;
          page_off = (int64_t)sload(table + pg) * p.c_sb;
        }
        const int in_page = kt - pg * (int)p.bs.d;
        koff = page_off + (int64_t)in_page * p.c_st + kvh * p.c_sh;
        voff = page_off + (int64_t)in_page * p.v_st + kvh * p.v_sh;
      } else {
        koff = (int64_t)(kbase + kt) * p.c_st + kvh * p.c_sh;
        voff = (int64_t)(kbase + kt) * p.v_st + kvh * p.v_sh;
      }
      const char* kb = (in_ctx ? p.ctx_k : p.k_cache) + koff;
      const char* vb = (in_ctx ? p.ctx_v : p.v_cache) + voff;
      // Branch-free where it can be: every wave issues NJ / WAVES loads (when WAVES does not divide NJ, the first
      // NJ % WAVES waves one more), each picking its source by selects rather than branches.
#pragma unroll
      for (int i = 0; i < (NJ + WAVES - 1) / WAVES; ++i) {
        const int j = wave + WAVES * i;
        if (NJ % WAVES == 0 || i < NJ / WAVES || j < NJ) {
          const bool isk = j < KJ;  // wave-uniform: a load of key rows, else of value rows
          const int slot = 64 * (isk ? j : j - KJ) + lane;
          const int kkey = slot / KJ, vkey = slot / VJ;
          const int key = isk ? kkey : vkey;
          const int chunk = isk ? min(slot - kkey * KJ, KCH - 1) : min(slot - vkey * VJ, VCH - 1);
          const uint32_t off = __umul24(min(key, last), (uint32_t)(isk ? kst : vst)) + chunk * 16;
          lds_dma16<false>(isk ? kb : vb, off, lds_addr(stage + 64 * 8 * j));  // tiles other query tiles read again
        }
      }
    };
    // q must be in registers before the stage loads are counted. Reading q here makes the compiler wait for its
    // loads now, outside the loop; otherwise its own wait lands at q's first use inside the loop, where it would
    // also wait for every stage in flight.
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int k = 0; k < KS; ++k) asm volatile("" ::"v"(qb[nb][k]));
    int issued = 0;
    for (; issued < RING - 1 && issued < ntiles; ++issued) fill(issued, ring + issued * kStageElems);
    for (int it = 0; it < ntiles; ++it) {
      // This wave's loads of tile `it` have landed when only the later tiles' are outstanding; the barrier makes
      // every wave's visible and frees the slot read last iteration.
      const int ahead = issued - it - 1;
      if (ahead == 0) vm_wait_barrier<0>();
      else if (ahead == 1) { if (hi) vm_wait_barrier<CNT_HI>(); else vm_wait_barrier<CNT_LO>(); }
      else { if (hi) vm_wait_barrier<2 * CNT_HI>(); else vm_wait_barrier<2 * CNT_LO>(); }
      if (issued < ntiles) {
        fill(issued, ring + (issued % RING) * kStageElems);
        ++issued;
      }
      const uint16_t* ks = ring + (it % RING) * kStageElems;
      const bool in_ctx = CTX && it < nc;  // a context tile: every query sees its keys < lc
      const int lcur[2] = {in_ctx ? lc : lim[0], in_ctx ? lc : lim[1]};
      consume((in_ctx ? it : it - nc) * kPrefillKeys, lcur, ks, ks + kPrefillKeys * KROW, it == 0, running);
    }
  } else {
    uint16_t* ks = reinterpret_cast<uint16_t*>(smem);  // [64 keys][KROW]
    uint16_t* vs = ks + kPrefillKeys * KROW;            // [64 keys][VROW]
    u32x4 stage[PER];
    if (PREFETCH && kmax > 0) fetch(0, stage);
    for (int kt = 0; kt < kmax; kt += kPrefillKeys) {
      if (!PREFETCH) fetch(kt, stage);
      __syncthreads();  // the previous tile's operand reads are done
      stash(ks, vs, stage);
      __syncthreads();
      if (PREFETCH && kt + kPrefillKeys < kmax) fetch(kt + kPrefillKeys, stage);
      consume(kt, lim, ks, vs, kt == 0, running);
    }
  }
  };
  // The held pass, for bf16 on one-page and multi-page LDS rings of up to 128-wide values. fp16 P operands overflow
  // past 65504 (2^16), far below the 2^64 that the row sums bound; the register-staged tiles (other page sizes) and
  // 192-wide values have no registers to spare for it; 8-wave items over context keys (MLA prefill in one call)
  // measured 2.4% slower with it (without context keys, as the reference layer's two calls run, 7.8% faster). Those
  // make one running pass.
  constexpr bool kHeld = std::is_same<T, BF16>::value && RING > 0 && DV <= 128 && (WAVES == 4 || !CTX);
  if constexpr (kHeld) {
    run_pass(std::false_type{});
    // Held rows: every sum finite and below kHeldLimit (false for a NaN sum), and every accumulator finite (a value
    // of magnitude past 2^63 times a probability near 2^64 would overflow where the running max does not).
    bool held = true;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      bool fin = true;
#pragma unroll
      for (int b = 0; b < DB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) fin = fin && __builtin_isfinite(o[nb][b][r]);
      held = held && (!qvalid[nb] || (xor32_sum(xor16_sum(l[nb])) < kHeldLimit && fin));
    }
    // Every wave has consumed its last tile here, so the stages are free for a second pass.
    if (__syncthreads_or(!held)) run_pass(std::true_type{});
  } else {
    run_pass(std::true_type{});
  }

#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const float lsum = xor32_sum(xor16_sum(l[nb]));
    if (!qvalid[nb]) continue;
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    char* dst = p.out + (int64_t)(q0 + qi[nb]) * p.o_st + head[nb] * p.o_sh;
#pragma unroll
    for (int b = 0; b < DB; ++b) {
      const u32x2 packed = {E::pack(o[nb][b][0] * inv, o[nb][b][1] * inv),
                            E::pack(o[nb][b][2] * inv, o[nb][b][3] * inv)};
      *reinterpret_cast<u32x2*>(dst + (int64_t)(b * 16 + 4 * j4) * 2) = packed;
    }
    if (p.lse && j4 == 0)
      p.lse[(int64_t)(q0 + qi[nb]) * p.lse_st + (int64_t)head[nb] * p.lse_sh] =
          lsum > 0.f ? (m[nb] * c + fast_log2(lsum)) * kLn2 : -INFINITY;
  }
}

}  // namespace lv
