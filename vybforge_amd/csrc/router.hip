// MoE router logits: Y[t, e] = sum_h X[t, h] * W[e, h] in float64, gfx950. Replaces the
// reference's router GEMM (native/glm53/glm_engine.vyb:2728-2745: the bf16 gate weight widened to
// float64, then a float64 matmul). Each product is rounded, then added (no contraction); with
// f32 / f16 / bf16 activations every product is exact in float64 (at most 48 significant bits),
// so only the summation order separates this from any other float64 GEMM. The order: one workgroup per
// row e, wave q of 4 sums the contiguous quarter [q H/4, (q+1) H/4) (H % 32 == 0), lane l the
// elements q H/4 + 512 k + 8 l + j in (k, j) order; the 64 lane sums fold as s_l + s_(l xor d),
// d = 32 .. 1; the 4 wave sums add as ((w0 + w1) + w2) + w3. A lane reads 8 consecutive weights
// and activations per step (16-B loads for 16-bit types), x straight from L2.
#include "common.h"

namespace vybdq {

// 8 consecutive elements from i (a multiple of 8) as float64
template <int DT>
__device__ __forceinline__ void load8(const void *p, int64_t i, double (&v)[8]) {
  if constexpr (DT == VYBDQ_F64) {
    const double *q = static_cast<const double *>(p) + i;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = q[j];
  } else if constexpr (DT == VYBDQ_F32) {
    const f4 *q = reinterpret_cast<const f4 *>(static_cast<const float *>(p) + i);
    const f4 a = q[0], b = q[1];
#pragma unroll
    for (int j = 0; j < 4; ++j) { v[j] = a[j]; v[4 + j] = b[j]; }
  } else {
    const u4 r = *reinterpret_cast<const u4 *>(static_cast<const uint16_t *>(p) + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = r[j];
      if constexpr (DT == VYBDQ_F16) {
        v[2 * j] = half_bits_to_f32(w & 0xffffu);
        v[2 * j + 1] = half_bits_to_f32(w >> 16);
      } else {
        v[2 * j] = __uint_as_float(w << 16);
        v[2 * j + 1] = __uint_as_float(w & 0xffff0000u);
      }
    }
  }
}

// TT tokens per pass over the row: the row's weights are loaded once per pass and every token keeps
// its own accumulator, so each (t, e) sum runs in exactly the order above; one barrier per pass.
// The grid is (expert rows, token tiles of TT): workgroup (e, y) runs tokens y TT .. y TT + TT - 1.
template <int XDT, int WDT, int TT>
__global__ void __launch_bounds__(256) k_router_logits(const void *__restrict__ X, const void *__restrict__ W,
                                                       void *__restrict__ Y, int ydt, int64_t T, int64_t E,
                                                       int64_t H) {
#pragma clang fp contract(off)
  __shared__ double wsum[2][4][TT];
  const int q = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t e = blockIdx.x;
  const int64_t Hq = H / 4;
  const int64_t h0 = q * Hq;
  int par = 0;
  for (int64_t t0 = static_cast<int64_t>(blockIdx.y) * TT; t0 < T; t0 += static_cast<int64_t>(TT) * gridDim.y, par ^= 1) {
    double acc[TT];
#pragma unroll
    for (int u = 0; u < TT; ++u) acc[u] = 0.0;
    for (int64_t k = 8 * lane; k < Hq; k += 512) {
      double wv[8];
      load8<WDT>(W, e * H + h0 + k, wv);
#pragma unroll
      for (int u = 0; u < TT; ++u) {
        const int64_t t = t0 + u < T ? t0 + u : T - 1;  // past T: a valid row, never stored
        double xv[8];
        load8<XDT>(X, t * H + h0 + k, xv);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[u] = acc[u] + xv[j] * wv[j];  // a product, then a sum (no contraction)
      }
    }
#pragma unroll
    for (int u = 0; u < TT; ++u) {
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) acc[u] = acc[u] + __shfl_xor(acc[u], off, 64);
    }
    if (lane == 0) {
#pragma unroll
      for (int u = 0; u < TT; ++u) wsum[par][q][u] = acc[u];
    }
    // the two halves of wsum alternate between passes, so one barrier per pass suffices
    __syncthreads();
    if (threadIdx.x < TT && t0 + threadIdx.x < T) {
      const int u = threadIdx.x;
      const double y = ((wsum[par][0][u] + wsum[par][1][u]) + wsum[par][2][u]) + wsum[par][3][u];
      const int64_t t = t0 + u;
      if (ydt == VYBDQ_F64) static_cast<double *>(Y)[t * E + e] = y;
      else static_cast<float *>(Y)[t * E + e] = static_cast<float>(y);
    }
  }
}

template <int WDT>
static void launch_router(int x_dt, dim3 grid, hipStream_t s, const void *x, const void *w, void *y, int y_dt,
                          int64_t T, int64_t E, int64_t H) {
#define RL(XDT, TT) hipLaunchKernelGGL((k_router_logits<XDT, WDT, TT>), grid, dim3(256), 0, s, x, w, y, y_dt, T, E, H)
#define RX(XDT) \
  do { if (T <= 4) RL(XDT, 1); else if (T <= 64) RL(XDT, 4); else RL(XDT, 16); } while (0)
  switch (x_dt) {
    case VYBDQ_F64: RX(VYBDQ_F64); break;
    case VYBDQ_F32: RX(VYBDQ_F32); break;
    case VYBDQ_F16: RX(VYBDQ_F16); break;
    default: RX(VYBDQ_BF16); break;
  }
#undef RX
#undef RL
}

}  // namespace vybdq

using namespace vybdq;

extern "C" int vybdq_router_logits(uint64_t X, int x_dt, uint64_t W, int w_dt, uint64_t Y, int y_dt, int64_t T,
                                   int64_t E, int64_t H, uint64_t stream) {
  VYBDQ_REQUIRE(X && W && Y, VYBDQ_ERR_ARG, "null X, W or Y");
  VYBDQ_REQUIRE(dt_valid_out(x_dt), VYBDQ_ERR_ARG, "x_dt must be F32, F16, BF16 or F64");
  VYBDQ_REQUIRE(dt_valid_in(w_dt), VYBDQ_ERR_ARG, "w_dt must be F32, F16 or BF16");
  VYBDQ_REQUIRE(y_dt == VYBDQ_F32 || y_dt == VYBDQ_F64, VYBDQ_ERR_ARG, "y_dt must be F32 or F64");
  VYBDQ_REQUIRE(T >= 0 && E >= 1 && E < (int64_t(1) << 31) && H >= 32 && H % 32 == 0, VYBDQ_ERR_SHAPE,
                "need E >= 1 and H a positive multiple of 32");
  VYBDQ_REQUIRE((X & 15) == 0 && (W & 15) == 0, VYBDQ_ERR_ALIGN, "X and W must be 16-byte aligned");
  if (T == 0) return VYBDQ_OK;
  hipStream_t s = as_stream(stream);
  // token tiles (measured at 256 x 6144): one token each up to 4 tokens, 4 up to 64 (1024
  // workgroups at 16 tokens), 16 above; one pass per workgroup up to 65535 tiles
  const int64_t tt = T <= 4 ? 1 : T <= 64 ? 4 : 16;
  const int64_t tiles = (T + tt - 1) / tt;
  const dim3 grid(static_cast<unsigned>(E), static_cast<unsigned>(tiles < 65535 ? tiles : 65535));
  const void *x = reinterpret_cast<const void *>(X), *w = reinterpret_cast<const void *>(W);
  void *y = reinterpret_cast<void *>(Y);
  VYBDQ_DISPATCH_IN(w_dt, WDT, launch_router<WDT>(x_dt, grid, s, x, w, y, y_dt, T, E, H));
  return check_launch("vybdq_router_logits");
}
