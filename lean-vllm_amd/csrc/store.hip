// store_kvcache / store_latents: scatter this step's new rows into the paged cache by slot.
//
// Four tokens per workgroup. Each thread copies VEC-byte pieces of the tokens' key and value rows to
// (block, offset, head) addressed through the cache's own strides, so NHD caches and HND caches seen through a
// transposed view take the same kernel. Slot -1 leaves the cache untouched. The copy is bit-exact: bytes move,
// nothing is converted.
#include "lv_common.h"

namespace lv {

template <int VEC>
struct Piece;
template <> struct Piece<16> { typedef u32x4 type; };
template <> struct Piece<8> { typedef u32x2 type; };
template <> struct Piece<4> { typedef uint32_t type; };
template <> struct Piece<2> { typedef uint16_t type; };
template <> struct Piece<1> { typedef uint8_t type; };

// kStoreTokens tokens per workgroup: their slots, then every piece of theirs that a thread copies, are loaded
// before the first is used, so a workgroup waits for two round trips to memory, not two per token.
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
  int64_t base[kStoreTokens];  // cache byte offset of each token's (block, offset)
  bool keep[kStoreTokens];     // slot -1, or past the last token: nothing stored
#pragma unroll
  for (int k = 0; k < kStoreTokens; ++k) {
    const int slot = t0 + k < tokens ? slots[t0 + k] : -1;
    keep[k] = slot >= 0;
    base[k] = keep[k] ? (int64_t)(slot / block_size) * sb + (int64_t)(slot % block_size) * st : 0;
  }
  // Pieces [0, pieces_per_row) are the key row, the rest the value row.
  for (int i = threadIdx.x; i < 2 * pieces_per_row; i += blockDim.x) {
    const bool is_v = i >= pieces_per_row;
    const int j = is_v ? i - pieces_per_row : i;
    const int head = j / pieces_per_head;
    const int within = j - head * pieces_per_head;
    const int64_t dst = head * sh + (int64_t)within * VEC;
    const char* src = (is_v ? value : key) + (int64_t)j * VEC;
    const int64_t row = is_v ? value_row : key_row;
    char* cache = is_v ? v_cache : k_cache;
    P piece[kStoreTokens];
#pragma unroll
    for (int k = 0; k < kStoreTokens; ++k)
      if (keep[k]) piece[k] = *reinterpret_cast<const P*>(src + (int64_t)(t0 + k) * row);
#pragma unroll
    for (int k = 0; k < kStoreTokens; ++k)
      if (keep[k]) *reinterpret_cast<P*>(cache + base[k] + dst) = piece[k];
  }
}

template <int VEC>
__global__ __launch_bounds__(128) void store_latent_kernel(const char* __restrict__ latent, int64_t latent_row,
                                                           int32_t pieces, int64_t cache_row,
                                                           char* __restrict__ cache,
                                                           const int32_t* __restrict__ slots) {
  typedef typename Piece<VEC>::type P;
  const int t = blockIdx.x;
  const int slot = slots[t];
  if (slot < 0) return;
  const char* src = latent + (int64_t)t * latent_row;
  char* dst = cache + (int64_t)slot * cache_row;
  for (int i = threadIdx.x; i < pieces; i += blockDim.x)
    *reinterpret_cast<P*>(dst + (int64_t)i * VEC) = *reinterpret_cast<const P*>(src + (int64_t)i * VEC);
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
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
#define LV_STORE_LAUNCH(V)                                                                                     \
  hipLaunchKernelGGL(store_kv_kernel<V>, dim3((num_tokens + kStoreTokens - 1) / kStoreTokens), dim3(threads), 0, \
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
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
#define LV_LATENT_LAUNCH(V)                                                                                    \
  hipLaunchKernelGGL(store_latent_kernel<V>, dim3(num_tokens), dim3(128), 0, s, (const char*)latent,           \
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
