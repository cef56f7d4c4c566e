// store_kvcache / store_latents: scatter this step's new rows into the paged cache by slot.
//
// Four tokens per workgroup. Each thread copies VEC-byte pieces of the tokens' key and value rows to
// (block, offset, head) addressed through the cache's own strides, so NHD caches and HND caches seen through a
// transposed view take the same kernel. Slot -1 leaves the cache untouched. The copy is bit-exact: bytes move,
// nothing is converted.
#include "lv_common.h"

namespace lv {

// An empty use of x in registers: whatever computes x must have happened here.
template <typename X>
__device__ __forceinline__ void keep_live(const X& x) {
  if constexpr (sizeof(X) == 16) {
    asm volatile("" ::"v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]));
  } else if constexpr (sizeof(X) == 8) {
    asm volatile("" ::"v"(x[0]), "v"(x[1]));
  } else {
    asm volatile("" ::"v"((uint32_t)x));
  }
}

template <int VEC>
struct Piece;
template <> struct Piece<16> { typedef u32x4 type; };
template <> struct Piece<8> { typedef u32x2 type; };
template <> struct Piece<4> { typedef uint32_t type; };
template <> struct Piece<2> { typedef uint16_t type; };
template <> struct Piece<1> { typedef uint8_t type; };

// kStoreTokens tokens per workgroup; each thread copies one piece of their key or value rows (blockIdx.y picks
// the thread's share of the pieces when a row pair has more than 256). The source rows do not depend on the slots,
// so every load -- the pieces, and each wave's four slots, one per lane -- is issued before the first wait: one
// round trip to memory before the stores, not two.
constexpr int kStoreTokens = 4;
template <int VEC>
__global__ __launch_bounds__(256) void store_kv_kernel(const char* __restrict__ key, const char* __restrict__ value,
                                                       int64_t key_row, int64_t value_row, int32_t pieces_per_head,
                                                       int32_t pieces_per_row, char* __restrict__ k_cache,
                                                       char* __restrict__ v_cache, int64_t sb, int64_t st, int64_t sh,
                                                       int32_t block_size, const int32_t* __restrict__ slots,
                                                       int32_t tokens) {
  typedef typename Piece<VEC>::type P;
  const int t0 = blockIdx.x * kStoreTokens;
  const int n = min(kStoreTokens, tokens - t0);  // tokens of this workgroup
  // Every thread runs to the end, so lanes 0-3 of each wave load the slots; threads past the row pair copy piece 0
  // without storing it.
  const bool active = blockIdx.y * blockDim.x + threadIdx.x < 2 * pieces_per_row;
  const int i = active ? blockIdx.y * blockDim.x + threadIdx.x : 0;
  // Pieces [0, pieces_per_row) are the key row, the rest the value row.
  const bool is_v = i >= pieces_per_row;
  const int j = is_v ? i - pieces_per_row : i;
  const int head = j / pieces_per_head;
  const int within = j - head * pieces_per_head;
  const int64_t dst = head * sh + (int64_t)within * VEC;
  const int64_t row = is_v ? value_row : key_row;
  const char* src = (is_v ? value : key) + (int64_t)j * VEC + (int64_t)t0 * row;
  char* cache = is_v ? v_cache : k_cache;
  // No branch between the loads: a last workgroup's missing tokens read its first token again (slot -1 below).
  P piece[kStoreTokens];
#pragma unroll
  for (int k = 0; k < kStoreTokens; ++k) piece[k] = *reinterpret_cast<const P*>(src + (k < n ? k : 0) * row);
  const int lane = threadIdx.x & 63;
  const int mine = slots[t0 + (lane % kStoreTokens < n ? lane % kStoreTokens : 0)];  // lane k: token k's slot
  // The pieces are needed here, before the branches on the slots: the compiler would otherwise sink a piece's load
  // into its store's branch, after the wait for the slots.
#pragma unroll
  for (int k = 0; k < kStoreTokens; ++k) keep_live(piece[k]);
  // Every slot is read out before the first store: a wait for the slot load after a store would wait for the
  // store too (stores count in the same counter).
  int slot[kStoreTokens];
#pragma unroll
  for (int k = 0; k < kStoreTokens; ++k) {
    slot[k] = k < n ? __builtin_amdgcn_readlane(mine, k) : -1;  // tokens past the last: nothing stored
    asm volatile("" ::"s"(slot[k]));
  }
#pragma unroll
  for (int k = 0; k < kStoreTokens; ++k)
    if (active && slot[k] >= 0)  // slot -1: nothing stored
      *reinterpret_cast<P*>(cache + (int64_t)(slot[k] / block_size) * sb + (int64_t)(slot[k] % block_size) * st +
                            dst) = piece[k];
}

// One latent per workgroup; each thread copies one piece (blockIdx.y picks the thread's share of the pieces when a
// latent has more than 128). The piece and the slot are loaded together, as vector loads, before the first wait.
template <int VEC>
__global__ __launch_bounds__(128) void store_latent_kernel(const char* __restrict__ latent, int64_t latent_row,
                                                           int32_t pieces, int64_t cache_row,
                                                           char* __restrict__ cache,
                                                           const int32_t* __restrict__ slots) {
  typedef typename Piece<VEC>::type P;
  const int t = blockIdx.x;
  const int i = blockIdx.y * blockDim.x + threadIdx.x;
  if (i >= pieces) return;
  const P piece = *reinterpret_cast<const P*>(latent + (int64_t)t * latent_row + (int64_t)i * VEC);
  int zero;  // 0, in a vector register: the slot load is then a vector load, counted in order with the piece load
  asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
  const int slot = __builtin_amdgcn_readfirstlane(slots[t + zero]);
  keep_live(piece);
  if (slot < 0) return;
  *reinterpret_cast<P*>(cache + (int64_t)slot * cache_row + (int64_t)i * VEC) = piece;
}

// Widest piece (16, 8, 4, 2 or 1 bytes) that divides every byte offset and pointer involved.
static int piece_bytes(std::initializer_list<int64_t> offsets, std::initializer_list<const void*> ptrs) {
  for (int vec : {16, 8, 4, 2}) {
    bool ok = true;
    for (int64_t o : offsets) ok = ok && (o % vec == 0);
    for (const void* p : ptrs) ok = ok && aligned(p, vec);
    if (ok) return vec;
  }
  return 1;
}

}  // namespace lv

using namespace lv;

extern "C" int lv_store_kvcache(const void* key, const void* value, int64_t key_stride_t, int64_t value_stride_t,
                                int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim, void* k_cache,
                                void* v_cache, int64_t cache_stride_block, int64_t cache_stride_token,
                                int64_t cache_stride_head, int32_t block_size, const int32_t* slot_mapping,
                                int32_t elem_bytes, void* stream) {
  LV_REQUIRE(num_tokens >= 0 && num_kv_heads > 0 && head_dim > 0, "store_kvcache: bad sizes T=%d H=%d D=%d",
             num_tokens, num_kv_heads, head_dim);
  LV_REQUIRE(block_size > 0, "store_kvcache: block_size must be positive, got %d", block_size);
  LV_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8,
             "store_kvcache: element size %d is not 1, 2, 4 or 8 bytes", elem_bytes);
  if (num_tokens == 0) return LV_OK;
  LV_REQUIRE(key && value && k_cache && v_cache && slot_mapping, "store_kvcache: null pointer");
  const int64_t eb = elem_bytes;
  const int64_t head_bytes = (int64_t)head_dim * eb;
  const int64_t row_bytes = head_bytes * num_kv_heads;
  const int vec = piece_bytes({head_bytes, key_stride_t * eb, value_stride_t * eb, cache_stride_block * eb,
                               cache_stride_token * eb, cache_stride_head * eb},
                              {key, value, k_cache, v_cache});
  const int32_t pph = (int32_t)(head_bytes / vec);
  const int32_t ppr = (int32_t)(row_bytes / vec);
  const int threads = ppr * 2 >= 256 ? 256 : ((ppr * 2 + 63) / 64) * 64;
  const int shares = (ppr * 2 + threads - 1) / threads;
  const int64_t blocks = ((int64_t)num_tokens + kStoreTokens - 1) / kStoreTokens;
  LV_REQUIRE(fits_one_launch(blocks, threads), "store_kvcache: %d tokens need a grid larger than one launch holds",
             num_tokens);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
#define LV_STORE_LAUNCH(V)                                                                                     \
  hipLaunchKernelGGL(store_kv_kernel<V>, dim3((uint32_t)blocks, shares),                                      \
                     dim3(threads), 0,                                                                         \
                     s, (const char*)key, (const char*)value, key_stride_t * eb, value_stride_t * eb, pph, ppr,  \
                     (char*)k_cache, (char*)v_cache, cache_stride_block * eb, cache_stride_token * eb,           \
                     cache_stride_head * eb, block_size, slot_mapping, num_tokens)
  switch (vec) {
    case 16: LV_STORE_LAUNCH(16); break;
    case 8: LV_STORE_LAUNCH(8); break;
    case 4: LV_STORE_LAUNCH(4); break;
    case 2: LV_STORE_LAUNCH(2); break;
    default: LV_STORE_LAUNCH(1); break;
  }
#undef LV_STORE_LAUNCH
  LV_LAUNCH_CHECK("store_kv_kernel");
  return LV_OK;
}

extern "C" int lv_store_latents(const void* latent, int64_t latent_stride_t, int32_t num_tokens, int32_t dim,
                                void* cache, const int32_t* slot_mapping, int32_t elem_bytes, void* stream) {
  LV_REQUIRE(num_tokens >= 0 && dim > 0, "store_latents: bad sizes T=%d dim=%d", num_tokens, dim);
  LV_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8,
             "store_latents: element size %d is not 1, 2, 4 or 8 bytes", elem_bytes);
  if (num_tokens == 0) return LV_OK;
  LV_REQUIRE(latent && cache && slot_mapping, "store_latents: null pointer");
  const int64_t eb = elem_bytes;
  const int64_t row = (int64_t)dim * eb;
  const int vec = piece_bytes({row, latent_stride_t * eb}, {latent, cache});
  const int32_t pieces = (int32_t)(row / vec);
  LV_REQUIRE(fits_one_launch(num_tokens, 128) && (pieces + 127) / 128 < 65536,
             "store_latents: %d tokens of %d bytes need a grid larger than one launch holds", num_tokens, (int)row);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
#define LV_LATENT_LAUNCH(V)                                                                                    \
  hipLaunchKernelGGL(store_latent_kernel<V>, dim3(num_tokens, (pieces + 127) / 128), dim3(128), 0, s,          \
                     (const char*)latent,                                                                      \
                     latent_stride_t * eb, pieces, row, (char*)cache, slot_mapping)
  switch (vec) {
    case 16: LV_LATENT_LAUNCH(16); break;
    case 8: LV_LATENT_LAUNCH(8); break;
    case 4: LV_LATENT_LAUNCH(4); break;
    case 2: LV_LATENT_LAUNCH(2); break;
    default: LV_LATENT_LAUNCH(1); break;
  }
#undef LV_LATENT_LAUNCH
  LV_LAUNCH_CHECK("store_latent_kernel");
  return LV_OK;
}
