// Shared helpers for the lvattn HIP kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <string>

#include "lvattn.h"

namespace lv {

// ---------------------------------------------------------------------------------------------------------
// Errors: every C entry point returns a status and leaves a message in a thread-local string.

void set_error(const char* fmt, ...);
const char* last_error();

#define LV_REQUIRE(cond, ...)                 \
  do {                                        \
    if (!(cond)) {                            \
      ::lv::set_error(__VA_ARGS__);           \
      return LV_EINVAL;                       \
    }                                         \
  } while (0)

#define LV_HIP_CHECK(expr)                                                              \
  do {                                                                                  \
    hipError_t lv_err_ = (expr);                                                        \
    if (lv_err_ != hipSuccess) {                                                        \
      ::lv::set_error("%s failed: %s", #expr, hipGetErrorString(lv_err_));              \
      return LV_EHIP;                                                                   \
    }                                                                                   \
  } while (0)

#define LV_LAUNCH_CHECK(name)                                                           \
  do {                                                                                  \
    hipError_t lv_err_ = hipGetLastError();                                             \
    if (lv_err_ != hipSuccess) {                                                        \
      ::lv::set_error("launch of %s failed: %s", name, hipGetErrorString(lv_err_));     \
      return LV_EHIP;                                                                   \
    }                                                                                   \
  } while (0)

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// A launch counts the work-items along each grid dimension (workgroups x threads along it) in 32 bits.
inline bool fits_one_launch(int64_t workgroups, int64_t threads) {
  return workgroups >= 0 && workgroups * threads < ((int64_t)1 << 32);
}

// ---------------------------------------------------------------------------------------------------------
// Vector types and element conversion.

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4v __attribute__((ext_vector_type(4)));

struct BF16 {};  // tag types for the two 16-bit element formats
struct F16 {};

template <typename T> struct Elem;

template <> struct Elem<BF16> {
  // Two packed elements -> two floats.
  __device__ static inline float lo(uint32_t x) { return __uint_as_float(x << 16); }
  __device__ static inline float hi(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }
  // acc + a.x*b.x + a.y*b.y, fp32 accumulation.
  __device__ static inline float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), acc, false);
  }
  // Two floats -> packed pair, round to nearest even.
  __device__ static inline uint32_t pack(float a, float b) {
    bf16x2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
  __device__ static inline f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  __device__ static inline f32x4 mfma16x16x16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4v, a), __builtin_bit_cast(i16x4v, b), c,
                                                     0, 0, 0);
  }
};

template <> struct Elem<F16> {
  __device__ static inline float lo(uint32_t x) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(x & 0xffffu));
  }
  __device__ static inline float hi(uint32_t x) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(x >> 16)); }
  __device__ static inline float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), acc, false);
  }
  __device__ static inline uint32_t pack(float a, float b) {
    f16x2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
  __device__ static inline f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
  __device__ static inline f32x4 mfma16x16x16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0,
                                                 0);
  }
};

// ---------------------------------------------------------------------------------------------------------
// Wave-level reductions. DPP within a row of 16 lanes; cross-row through the LDS crossbar (ds_bpermute).

__device__ inline float dpp_xor1(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xB1, 0xf, 0xf, false));
}
__device__ inline float dpp_xor2(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4E, 0xf, 0xf, false));
}
__device__ inline float dpp_half_mirror(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x141, 0xf, 0xf, false));
}
__device__ inline float dpp_mirror(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x140, 0xf, 0xf, false));
}

// Lane (i + 8) mod 16 of the same 16-lane row.
__device__ inline float dpp_ror8(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false));
}

// Sum over aligned groups of N lanes (N = 4, 8 or 16); every lane of a group ends with the group's sum.
template <int N>
__device__ inline float group_sum(float x) {
  static_assert(N == 4 || N == 8 || N == 16, "group of 4, 8 or 16 lanes");
  x += dpp_xor1(x);
  x += dpp_xor2(x);
  if constexpr (N >= 8) x += dpp_half_mirror(x);
  if constexpr (N >= 16) x += dpp_mirror(x);
  return x;
}

__device__ inline float shfl_xor(float x, int mask) { return __shfl_xor(x, mask, 64); }

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ inline float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// ---------------------------------------------------------------------------------------------------------
// Division of non-negative 31-bit integers by a divisor fixed at launch (Granlund and Montgomery, "Division by
// invariant integers using multiplication", 1994): q = (umulhi(n, m) + n) >> s with s = ceil(log2 d) and
// m = floor(2^32 (2^s - d) / d) + 1. Exact for 0 <= n < 2^31, 1 <= d < 2^31.
struct FastDiv {
  uint32_t d, m, s;
  static FastDiv make(uint32_t d) {
    uint32_t s = 0;
    while ((1ull << s) < d) ++s;
    const uint64_t m = ((((uint64_t)1 << s) - d) << 32) / d + 1;
    return FastDiv{d, (uint32_t)m, s};
  }
  __device__ __host__ inline uint32_t div(uint32_t n) const {
#ifdef __HIP_DEVICE_COMPILE__
    const uint32_t hi = __umulhi(n, m);
#else
    const uint32_t hi = (uint32_t)(((uint64_t)n * m) >> 32);
#endif
    return (hi + n) >> s;
  }
};

// ---------------------------------------------------------------------------------------------------------
// Global memory.

__device__ inline u32x4 ld16(const char* ptr) { return *reinterpret_cast<const u32x4*>(ptr); }
// Streaming load of cache rows that this launch reads once: the non-temporal hint keeps them from displacing
// reusable lines in L2 and the Infinity Cache (about 7.0 vs 6.2 TB/s for a plain streaming read on MI355X).
__device__ inline u32x4 ld16_stream(const char* ptr) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ptr));
}
__device__ inline void st16(char* ptr, u32x4 v) { *reinterpret_cast<u32x4*>(ptr) = v; }

// Transposing LDS read (ds_read_b64_tr_b16): each group of 16 lanes reads a 4 x 16 tile of 16-bit values, lane
// 4 * row + quad addressing 4 consecutive elements of one row; lane i of the group receives column i (4 values,
// one per row) -- the operand layout of an MFMA whose reduction runs along the tile's rows.
typedef short i16x4 __attribute__((ext_vector_type(4)));

__device__ inline u32x2 lds_read_tr16(const uint16_t* p) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  return __builtin_bit_cast(u32x2, v);
}

// ---------------------------------------------------------------------------------------------------------
// Cross-row lane exchange.

// Maximum of two scores, NaN-propagating (IEEE maximum): gfx950's v_maximum3_f32, which the compiler also fuses
// into three-input maxima. fmaxf (maxNum) must first quiet a signalling NaN in every operand that is not a known
// arithmetic result (an MFMA output, a lane swap), one extra instruction per operand. For scores the two agree:
// a NaN score makes the row's output NaN either way.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Sum / max over lanes i and i ^ 16, and over lanes i and i ^ 32, with gfx950's cross-row swaps (no LDS round trip).
__device__ inline float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Inclusive prefix sum over the 64 lanes of a wave.
__device__ inline int wave_incl_scan(int x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  return x;
}

// Exclusive prefix sum of a[0, n) in LDS, in place, by a block of kScanThreads threads; a[n] receives the total.
// wave_tot holds kScanThreads / 64 ints of LDS. Every thread of the block must call it, after a barrier that follows
// the last write of a[] (a thread's chunk holds entries other threads wrote once n > kScanThreads). Each thread scans its
// chunk, each wave its threads' chunk totals; every thread then sums the wave totals before its own (16 broadcast
// LDS reads, issued together) instead of one thread scanning them in sequence between two more barriers.
constexpr int kScanThreads = 1024;
__device__ inline void block_scan(int* a, int n, int* wave_tot) {
  const int tid = threadIdx.x;
  const int per = (n + kScanThreads - 1) / kScanThreads;
  const int lo = min(tid * per, n), hi = min(lo + per, n);
  int local = 0;
  for (int i = lo; i < hi; ++i) local += a[i];
  const int lane = tid & 63, wave = tid >> 6;
  const int x = wave_incl_scan(local);  // inclusive scan of the chunk totals across the wave
  if (lane == 63) wave_tot[wave] = x;
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kScanThreads / 64; ++w) {
    const int v = wave_tot[w];
    before += w < wave ? v : 0;
    total += v;
  }
  int run = before + x - local;  // exclusive prefix of this thread's chunk
  for (int i = lo; i < hi; ++i) {
    const int v = a[i];
    a[i] = run;
    run += v;
  }
  if (tid == 0) a[n] = total;
  __syncthreads();
}

constexpr float kLog2e = 1.4426950408889634f;
// log2 units by which an online softmax's running max may trail the true max before the accumulators are
// rescaled: probabilities then stay below 2^kRescaleSlack, well inside bf16 / fp16 and fp32 range.
constexpr float kRescaleSlack = 8.f;
// An online softmax may instead hold a row's max from its first key tile: later scores up to kHeldSlack log2 units
// above it give probabilities up to 2^kHeldSlack, exact in fp32 and in bf16 P operands (not fp16, whose range ends
// at 65504). A row sum below
// kHeldLimit (= 2^kHeldSlack, finite) shows that every probability of the row stayed in that range.
constexpr float kHeldSlack = 64.f;
constexpr float kHeldLimit = 18446744073709551616.f;
constexpr float kLn2 = 0.6931471805599453f;

// Compute units of the current device (cached per device; 256 on MI355X). Host code.
inline int device_cus() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64 && cached[dev] > 0) return cached[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (dev < 64) cached[dev] = cus;
  return cus;
}

// ---------------------------------------------------------------------------------------------------------
// Loads straight from global memory into LDS (global_load_lds_dwordx4), for staging rings.

typedef __attribute__((address_space(3))) void lds_void_t;

// STREAM: rows this launch reads once (non-temporal, as ld16_stream); otherwise cached, for tiles that other
// workgroups read again.

// One 16-byte load per lane from base + off into LDS at lds_base + 16 lane (lds_base wave-uniform, set through
// M0). Issued as inline assembly so that the compiler, which cannot tell which LDS bytes the load writes, adds no
// wait-for-every-load before later LDS reads; the kernel waits for these loads itself (vmcnt).
template <bool STREAM = true>
__device__ __forceinline__ void lds_dma16(const char* base, uint32_t off, uint32_t lds_base) {
  if (STREAM)
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(off), "s"(base),
                 "s"(lds_base)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base),
                 "s"(lds_base)
                 : "memory", "m0");
}

// As above, from a per-lane address.
template <bool STREAM = true>
__device__ __forceinline__ void lds_dma16(const char* src, uint32_t lds_base) {
  if (STREAM)
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src),
                 "s"(lds_base)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_base)
                 : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_void_t*)p;
}

// Load of a wave-uniform int through the scalar cache. For tables this kernel only reads: the compiler would use
// a vector load here (the kernel's stores might alias), and its wait for that load would also wait for every
// latent load in flight.
__device__ __forceinline__ int sload(const int32_t* ptr) {
  int v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(ptr));
  return v;
}

// N such loads (2 or 4) issued together, then one wait.
template <int N>
__device__ __forceinline__ void sload_n(const int32_t* const (&ptr)[N], int (&v)[N]) {
  static_assert(N == 2 || N == 4, "2 or 4 loads");
  if constexpr (N == 2) {
    asm volatile("s_load_dword %0, %2, 0x0\n\ts_load_dword %1, %3, 0x0\n\ts_waitcnt lgkmcnt(0)"
                 : "=&s"(v[0]), "=&s"(v[1])
                 : "s"(ptr[0]), "s"(ptr[1]));
  } else {
    asm volatile(
        "s_load_dword %0, %4, 0x0\n\ts_load_dword %1, %5, 0x0\n\ts_load_dword %2, %6, 0x0\n\t"
        "s_load_dword %3, %7, 0x0\n\ts_waitcnt lgkmcnt(0)"
        : "=&s"(v[0]), "=&s"(v[1]), "=&s"(v[2]), "=&s"(v[3])
        : "s"(ptr[0]), "s"(ptr[1]), "s"(ptr[2]), "s"(ptr[3]));
  }
}

// Wait until at most N of this wave's vector-memory operations are outstanding, then meet the other waves. No
// fence: a staging ring's LDS writes are exactly the loads waited for, and a fence would also wait for the stages
// still in flight.
template <int N>
__device__ __forceinline__ void vm_wait_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

}  // namespace lv
