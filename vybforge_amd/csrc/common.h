// Shared device helpers and host plumbing for libvybdq (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <atomic>
#include <string>

#include "vybdq.h"

namespace vybdq {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

// ---- host: error state ----------------------------------------------------------------

int set_error(int code, const std::string &msg);
int check_launch(const char *what);  // hipGetLastError after a launch
// a launch-plan override from the environment, only when VYBDQ_TUNING is set (else null)
const char *tuning_env(const char *name);
inline hipStream_t as_stream(uint64_t s) { return reinterpret_cast<hipStream_t>(s); }

// Raise a kernel's dynamic-LDS limit to `bytes` once per device: `done` is the caller's static mask
// of devices already raised (one per kernel instantiation; atomic, so host threads may race here).
inline int ensure_lds_limit(const void *fn, int bytes, std::atomic<uint64_t> &done, const char *what) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return set_error(VYBDQ_ERR_HIP, std::string(what) + ": no current HIP device");
  const uint64_t bit = uint64_t(1) << dev;
  if (done.load(std::memory_order_relaxed) & bit) return VYBDQ_OK;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) return set_error(VYBDQ_ERR_HIP, std::string(what) + ": LDS attribute: " + hipGetErrorString(e));
  done.fetch_or(bit, std::memory_order_relaxed);
  return VYBDQ_OK;
}

// Resident workgroups per CU of a kernel at `lds` bytes of dynamic LDS: queried once per device and
// LDS size; `cache` is the caller's static per-device word ((lds << 8) | count, 0 = not queried).
inline int resident_per_cu(const void *fn, int threads, size_t lds, std::atomic<int64_t> (&cache)[64], int &per_cu,
                           const char *what) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return set_error(VYBDQ_ERR_HIP, std::string(what) + ": no current HIP device");
  const int64_t key = static_cast<int64_t>(lds) << 8;
  const int64_t have = cache[dev].load(std::memory_order_relaxed);
  if ((have & ~int64_t(0xff)) == key && (have & 0xff) > 0) {
    per_cu = static_cast<int>(have & 0xff);
    return VYBDQ_OK;
  }
  int nb = 0;
  const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, threads, lds);
  if (e != hipSuccess) return set_error(VYBDQ_ERR_HIP, std::string(what) + ": occupancy: " + hipGetErrorString(e));
  per_cu = nb < 1 ? 1 : (nb > 255 ? 255 : nb);
  cache[dev].store(key | per_cu, std::memory_order_relaxed);
  return VYBDQ_OK;
}

// Compute units of the current device (cached per device; 256 if the query fails).
inline int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

#define VYBDQ_REQUIRE(cond, code, msg)                                                     \
  do {                                                                                     \
    if (!(cond)) return ::vybdq::set_error((code), std::string(__func__) + ": " + (msg));  \
  } while (0)

inline bool dt_valid_in(int dt) { return dt == VYBDQ_F32 || dt == VYBDQ_F16 || dt == VYBDQ_BF16; }
inline bool dt_valid_out(int dt) { return dt_valid_in(dt) || dt == VYBDQ_F64; }
inline int dt_size(int dt) { return dt == VYBDQ_F64 ? 8 : dt == VYBDQ_F32 ? 4 : 2; }

// ---- device: DPP lane permutations (update_dpp controls) -------------------------------

constexpr int DPP_QUAD_XOR1 = 0xB1;     // quad_perm [1, 0, 3, 2]
constexpr int DPP_QUAD_XOR2 = 0x4E;     // quad_perm [2, 3, 0, 1]
constexpr int DPP_ROW_MIRROR = 0x140;   // lane i <- lane 15 - i of its row
constexpr int DPP_HALF_MIRROR = 0x141;  // lane i <- lane 7 - i of its half-row
constexpr int DPP_BCAST15 = 0x142;      // row r <- lane 15 of row r - 1
constexpr int DPP_BCAST31 = 0x143;      // rows 2, 3 <- lane 31
constexpr int DPP_ROW_SHL = 0x100;     // + n: lane i <- lane i + n of its row (n = 1..15)
constexpr int DPP_ROW_SHR = 0x110;     // + n: lane i <- lane i - n of its row

// ---- device: element load/store -------------------------------------------------------

// A device address read from memory (a parameter-block word) as a pointer into global memory.
// Through a plain integer-to-pointer cast the compiler cannot tell global from LDS and emits flat
// loads, which also count against lgkmcnt: every LDS wait would then wait for them as well.
template <class T>
__device__ __forceinline__ T *gptr(int64_t a) {
  return (T *)(T __attribute__((address_space(1))) *)a;
}

// Direct global -> LDS load of 16 bytes per lane: lane L's 16 bytes at src go to LDS dst + 16 L
// (dst wave-uniform). Issued from asm, so the compiler does not track it: it inserts no waits of
// its own for it (its direct-to-LDS bookkeeping merges conservatively at loop heads and would drain
// every load there), the caller waits for it by vmcnt explicitly, and the compiler's own waits for
// loads issued before it only grow longer. One wait state between the M0 write and the load.
__device__ __forceinline__ void lds_dma16(const void *src, const void *dst) {
  const uint32_t l = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void *)dst)));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(l) : "memory", "m0");
}

// The same with a wave-uniform base address (scalar registers) and a 32-bit lane byte offset: one
// offset register per load instead of a 64-bit address pair.
__device__ __forceinline__ void lds_dma16_s(const void *base, uint32_t off, const void *dst) {
  const uint32_t l = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void *)dst)));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(l)
               : "memory", "m0");
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// float32 -> bfloat16, round to nearest even (NaN kept quiet)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

template <int DT>
__device__ __forceinline__ float load_elem(const void *p, int64_t i) {
  if constexpr (DT == VYBDQ_F32) return static_cast<const float *>(p)[i];
  else if constexpr (DT == VYBDQ_F16) return static_cast<float>(static_cast<const _Float16 *>(p)[i]);
  else return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
}

// Store y (+ residual of the same type). F64 keeps the reference's f64-output mode
// (rgemv.vyb:359-366): the f32 accumulator is widened, then the f64 residual is added.
template <int DT>
__device__ __forceinline__ void store_elem(void *p, const void *rs, int64_t i, float v) {
  if constexpr (DT == VYBDQ_F64) {
    double d = static_cast<double>(v);
    if (rs) d += static_cast<const double *>(rs)[i];
    static_cast<double *>(p)[i] = d;
  } else if constexpr (DT == VYBDQ_F32) {
    if (rs) v += static_cast<const float *>(rs)[i];
    static_cast<float *>(p)[i] = v;
  } else if constexpr (DT == VYBDQ_F16) {
    if (rs) v += static_cast<float>(static_cast<const _Float16 *>(rs)[i]);
    static_cast<_Float16 *>(p)[i] = static_cast<_Float16>(v);
  } else {
    if (rs) v += bf16_to_f32(static_cast<const uint16_t *>(rs)[i]);
    static_cast<uint16_t *>(p)[i] = f32_to_bf16(v);
  }
}

__device__ __forceinline__ float half_bits_to_f32(uint32_t bits16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}

// Block scale for the largest |x| of a block: with ex its biased float32 exponent
// (2^(ex - 127) <= amax < 2^(ex - 126)), the block is staged as x * 2^-e, e = ex - 141, which brings
// its largest value into [2^14, 2^15): no overflow for large activations, no fp16 subnormals for
// small ones (a power of two: exact). e is clamped to [-100, 113] (beyond that the block is still
// representable, if less precisely); all-zero blocks stay unscaled. Returns 2^e, writes 2^-e.
__device__ __forceinline__ float block_scale(float amax, float &inv) {
  const int ex = static_cast<int>((__float_as_uint(amax) >> 23) & 0xffu);
  if (ex == 0) {
    inv = 1.0f;
    return 1.0f;
  }
  int e = ex - 141;
  e = e < -100 ? -100 : (e > 113 ? 113 : e);
  inv = __uint_as_float(static_cast<uint32_t>(127 - e) << 23);
  return __uint_as_float(static_cast<uint32_t>(127 + e) << 23);
}

}  // namespace vybdq

// Dispatch a runtime dtype to a template parameter.
#define VYBDQ_DISPATCH_IN(dt, NAME, ...)                                                    \
  switch (dt) {                                                                            \
    case VYBDQ_F32: { constexpr int NAME = VYBDQ_F32; __VA_ARGS__; } break;                \
    case VYBDQ_F16: { constexpr int NAME = VYBDQ_F16; __VA_ARGS__; } break;                \
    default: { constexpr int NAME = VYBDQ_BF16; __VA_ARGS__; } break;                      \
  }

#define VYBDQ_DISPATCH_OUT(dt, NAME, ...)                                                   \
  switch (dt) {                                                                            \
    case VYBDQ_F32: { constexpr int NAME = VYBDQ_F32; __VA_ARGS__; } break;                \
    case VYBDQ_F16: { constexpr int NAME = VYBDQ_F16; __VA_ARGS__; } break;                \
    case VYBDQ_BF16: { constexpr int NAME = VYBDQ_BF16; __VA_ARGS__; } break;              \
    default: { constexpr int NAME = VYBDQ_F64; __VA_ARGS__; } break;                       \
  }
