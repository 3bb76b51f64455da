// Library plumbing (error state) and the decode-only q4_0 / Q8_0 kernels.
#include "common.h"

namespace vybdq {

static thread_local std::string g_last_error = "no error";

int set_error(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(VYBDQ_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  return VYBDQ_OK;
}

// The launch-plan overrides (VYBDQ_GEMV_PLAN, VYBDQ_MMQ_PLAN, VYBDQ_MOE_*, VYBDQ_EXL3_SPLITS) are
// read only when VYBDQ_TUNING was set when the library first needed one; otherwise no launch
// reads the environment.
const char *tuning_env(const char *name) {
  static const bool enabled = [] {
    const char *t = getenv("VYBDQ_TUNING");
    return t && t[0] && t[0] != '0';
  }();
  return enabled ? getenv(name) : nullptr;
}

// ---- decode-only kernels ----------------------------------------------------------------
// One thread per 8 consecutive output elements of one block (4 threads per block): the
// thread loads the block scale and its 4 quant bytes, decodes exactly (fp16 d times a small
// integer is exact in f32) and stores 8 outputs.

template <int ORDER, int ODT>
__global__ void __launch_bounds__(256) k_dequant_q4_0(const uint8_t *__restrict__ W,
                                                      void *__restrict__ out, int64_t nblocks) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t b = t >> 2;
  const int part = static_cast<int>(t & 3);
  if (b >= nblocks) return;
  const uint8_t *blk = W + b * 18;
  const float d = half_bits_to_f32(blk[0] | (static_cast<uint32_t>(blk[1]) << 8));
  float v[8];
  int e0;
  if constexpr (ORDER == VYBDQ_Q4_GGML) {
    // elements 8*part .. 8*part+7: part 0,1 -> low nibbles of qs[0..15]; 2,3 -> high nibbles
    const int byte0 = (part & 1) * 8;
    const int sh = (part >> 1) * 4;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = d * static_cast<float>(((blk[2 + byte0 + i] >> sh) & 15) - 8);
    e0 = part * 8;
  } else {
    // elements 8*part .. +7 = both nibbles of qs[4*part .. 4*part+3]
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint8_t q = blk[2 + part * 4 + i];
      v[2 * i] = d * static_cast<float>((q & 15) - 8);
      v[2 * i + 1] = d * static_cast<float>((q >> 4) - 8);
    }
    e0 = part * 8;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) store_elem<ODT>(out, nullptr, b * 32 + e0 + i, v[i]);
}

template <int ODT>
__global__ void __launch_bounds__(256) k_dequant_q8_0(const uint8_t *__restrict__ W,
                                                      void *__restrict__ out, int64_t nblocks) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t b = t >> 2;
  const int part = static_cast<int>(t & 3);
  if (b >= nblocks) return;
  const uint8_t *blk = W + b * 34;
  const float d = half_bits_to_f32(blk[0] | (static_cast<uint32_t>(blk[1]) << 8));
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int8_t q = static_cast<int8_t>(blk[2 + part * 8 + i]);
    store_elem<ODT>(out, nullptr, b * 32 + part * 8 + i, d * static_cast<float>(q));
  }
}

static inline unsigned grid_for(int64_t threads, int bs) {
  return static_cast<unsigned>((threads + bs - 1) / bs);
}

}  // namespace vybdq

using namespace vybdq;

extern "C" int vybdq_abi_version(void) { return VYBDQ_ABI_VERSION; }

extern "C" const char *vybdq_last_error(void) { return g_last_error.c_str(); }

extern "C" int vybdq_dequant_q4_0(uint64_t W, uint64_t out, int64_t nblocks, int order,
                                  int out_dt, uint64_t stream) {
  VYBDQ_REQUIRE(W && out, VYBDQ_ERR_ARG, "null buffer");
  VYBDQ_REQUIRE(nblocks >= 0, VYBDQ_ERR_SHAPE, "nblocks < 0");
  VYBDQ_REQUIRE(order == VYBDQ_Q4_GGML || order == VYBDQ_Q4_INTERLEAVED, VYBDQ_ERR_ARG,
                "unknown q4_0 order");
  VYBDQ_REQUIRE(out_dt == VYBDQ_F32 || out_dt == VYBDQ_F16 || out_dt == VYBDQ_F64, VYBDQ_ERR_ARG,
                "out_dt must be F32, F16 or F64");
  if (nblocks == 0) return VYBDQ_OK;
  const auto *w = reinterpret_cast<const uint8_t *>(W);
  void *o = reinterpret_cast<void *>(out);
  const unsigned g = grid_for(nblocks * 4, 256);
  hipStream_t s = as_stream(stream);
#define LAUNCH(ORD, ODT) hipLaunchKernelGGL((k_dequant_q4_0<ORD, ODT>), dim3(g), dim3(256), 0, s, w, o, nblocks)
  if (order == VYBDQ_Q4_GGML) {
    if (out_dt == VYBDQ_F32) LAUNCH(VYBDQ_Q4_GGML, VYBDQ_F32);
    else if (out_dt == VYBDQ_F16) LAUNCH(VYBDQ_Q4_GGML, VYBDQ_F16);
    else LAUNCH(VYBDQ_Q4_GGML, VYBDQ_F64);
  } else {
    if (out_dt == VYBDQ_F32) LAUNCH(VYBDQ_Q4_INTERLEAVED, VYBDQ_F32);
    else if (out_dt == VYBDQ_F16) LAUNCH(VYBDQ_Q4_INTERLEAVED, VYBDQ_F16);
    else LAUNCH(VYBDQ_Q4_INTERLEAVED, VYBDQ_F64);
  }
#undef LAUNCH
  return check_launch("vybdq_dequant_q4_0");
}

extern "C" int vybdq_dequant_q8_0(uint64_t W, uint64_t out, int64_t nblocks, int out_dt,
                                  uint64_t stream) {
  VYBDQ_REQUIRE(W && out, VYBDQ_ERR_ARG, "null buffer");
  VYBDQ_REQUIRE(nblocks >= 0, VYBDQ_ERR_SHAPE, "nblocks < 0");
  VYBDQ_REQUIRE(out_dt == VYBDQ_F32 || out_dt == VYBDQ_F16 || out_dt == VYBDQ_F64, VYBDQ_ERR_ARG,
                "out_dt must be F32, F16 or F64");
  if (nblocks == 0) return VYBDQ_OK;
  const auto *w = reinterpret_cast<const uint8_t *>(W);
  void *o = reinterpret_cast<void *>(out);
  const unsigned g = grid_for(nblocks * 4, 256);
  hipStream_t s = as_stream(stream);
  if (out_dt == VYBDQ_F32) hipLaunchKernelGGL((k_dequant_q8_0<VYBDQ_F32>), dim3(g), dim3(256), 0, s, w, o, nblocks);
  else if (out_dt == VYBDQ_F16) hipLaunchKernelGGL((k_dequant_q8_0<VYBDQ_F16>), dim3(g), dim3(256), 0, s, w, o, nblocks);
  else hipLaunchKernelGGL((k_dequant_q8_0<VYBDQ_F64>), dim3(g), dim3(256), 0, s, w, o, nblocks);
  return check_launch("vybdq_dequant_q8_0");
}
