// Q8 activation quantizer (xq8 semantics), gfx950.
//
// Per 32-value block of a row: a = max|x| (half-wave xor-shuffle max: a wave64 covers two
// blocks, lanes 0-31 and 32-63), d = a / 127 (correctly rounded float32 division),
// iv = 127 / a (0 for an all-zero block), q = saturate_s8(round_half_even(x * iv)).
// Replaces xq8 (native/kernels/rgemv7.vyb:195-214), whose 32-lane warp_max becomes the
// 32-lane half of a wave64 here.
#include "common.h"

namespace vybdq {

template <int XDT>
__global__ void __launch_bounds__(256) k_quant_q8(const void *__restrict__ X, int8_t *__restrict__ Xq,
                                                  float *__restrict__ Xs, int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const float x = i < total ? load_elem<XDT>(X, i) : 0.f;
  float a = fabsf(x);
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 64));
  const float d = a / 127.0f;
  const float iv = a > 0.f ? 127.0f / a : 0.f;
  if (i < total) {
    float r = __builtin_rintf(x * iv);
    r = fminf(fmaxf(r, -128.f), 127.f);
    Xq[i] = static_cast<int8_t>(static_cast<int>(r));
    if ((i & 31) == 0) Xs[i >> 5] = d;
  }
}

}  // namespace vybdq

using namespace vybdq;

extern "C" int vybdq_quant_q8_act(uint64_t X, uint64_t Xq, uint64_t Xs, int64_t M, int64_t K, int x_dt,
                                  uint64_t stream) {
  VYBDQ_REQUIRE(X && Xq && Xs, VYBDQ_ERR_ARG, "null buffer");
  VYBDQ_REQUIRE(dt_valid_in(x_dt), VYBDQ_ERR_ARG, "x_dt must be F32, F16 or BF16");
  VYBDQ_REQUIRE(M >= 0 && K >= 0 && K % 32 == 0, VYBDQ_ERR_SHAPE, "K must be a multiple of 32");
  const int64_t total = M * K;
  if (total == 0) return VYBDQ_OK;
  VYBDQ_REQUIRE((Xs & 3) == 0, VYBDQ_ERR_ALIGN, "Xs must be 4-byte aligned");
  const unsigned grid = static_cast<unsigned>((total + 255) / 256);
  hipStream_t s = as_stream(stream);
  const void *x = reinterpret_cast<const void *>(X);
  auto *q = reinterpret_cast<int8_t *>(Xq);
  auto *d = reinterpret_cast<float *>(Xs);
  VYBDQ_DISPATCH_IN(x_dt, XDT, hipLaunchKernelGGL((k_quant_q8<XDT>), dim3(grid), dim3(256), 0, s, x, q, d, total));
  return check_launch("vybdq_quant_q8_act");
}
