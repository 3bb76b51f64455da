// Producer-side q8 activation quantization, gfx950: RMSNorm and SwiGLU that also write the q8
// copy (int8 + float32 scale per 32) of their float32 output, so the int8 GEMM / GEMV that
// consumes it needs no separate quantizer launch. Replaces rms_blkg with its Y8 output
// (VYB_RMSQ8, native/kernels/layer.vyb:989-1066) and silu32q (VYB_SWQ8, layer.vyb:1567-1590).
//
// Arithmetic follows the reference term by term in float64, with contraction off (every product
// and sum rounds separately, as written):
//  RMSNorm: thread t of 256 sums x[t]^2, x[t+256]^2, ... in index order; the partials fold
//    pairwise through LDS (strides 128 .. 1); v = S / N + eps; sqrt(v) by six Newton steps from
//    the bit-trick seed v * bits(0x5FE6EB50C7B537A9 - bits(v) / 2) for 1e-9 < v < 1e9, else 24
//    steps from y = v (native/kernels/vmath.vyb:75-83); y_i = x_i * r * w_i with r = 1 / sqrt(v).
//  SwiGLU: h = g * (1 / (1 + vexp(-g))) * u, vexp being the reference's own exp
//    (vmath.vyb:7-40: clamp to [-20, 20], n = z rounded half away from zero, degree-8
//    polynomial for 2^r summed left to right, times 2^n).
//  q8 copy: xq8 (rgemv7.vyb:195-214) of the float32 output: per 32 consecutive elements (a
//    32-lane half of a wave) a = max|x|, d = a / 127, q = sat_s8(rint(x * 127 / a)).
#include "common.h"

namespace vybdq {

template <int DT>
__device__ __forceinline__ double load_d(const void *p, int64_t i) {
  if constexpr (DT == VYBDQ_F64) return static_cast<const double *>(p)[i];
  else return static_cast<double>(load_elem<DT>(p, i));
}

__device__ __forceinline__ double sqrt_newton(double v) {
#pragma clang fp contract(off)
  if (v > 0.000000001 && v < 1000000000.0) {
    const long long bits = __double_as_longlong(v);
    double y = v * __longlong_as_double(6910469410427058089LL - bits / 2);
#pragma unroll
    for (int i = 0; i < 6; ++i) y = 0.5 * (y + v / y);
    return y;
  }
  if (v <= 0.0) return 0.0;
  double y = v;
  for (int i = 0; i < 24; ++i) y = 0.5 * (y + v / y);
  return y;
}

__device__ __forceinline__ double vexp_ref(double x) {
#pragma clang fp contract(off)
  double xt = x;
  if (xt > 20.0) xt = 20.0;
  if (xt < -20.0) xt = -20.0;
  const double z = xt * 1.4426950408889634;
  const double nf = z >= 0.0 ? trunc(z + 0.5) : trunc(z - 0.5);
  const double r = z - nf;
  const double r2 = r * r, r3 = r2 * r, r4 = r3 * r, r5 = r4 * r, r6 = r5 * r, r7 = r6 * r, r8 = r7 * r;
  double p = 1.0 + r * 0.6931471805599453;
  p = p + r2 * 0.2402265069591007;
  p = p + r3 * 0.05550410866482158;
  p = p + r4 * 0.009618129107628478;
  p = p + r5 * 0.001333355814642845;
  p = p + r6 * 0.0001540353039338161;
  p = p + r7 * 0.000015252733804059856;
  p = p + r8 * 0.0000013215486790144306;
  const int n = static_cast<int>(fmin(fmax(nf, -2048.0), 2048.0));
  return ldexp(p, n);  // n doublings or halvings: exact for the |n| <= 29 of a clamped argument
}

// q8 copy of one float32 value per lane; lanes 32k .. 32k+31 of the wave hold one 32-block
// (lanes without an element pass x = 0 and store nothing).
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ float dpp_max(float v) {
  const int t = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xf, false);
  return fmaxf(v, __builtin_bit_cast(float, t));  // lanes outside ROWS see 0 <= v
}

// max over each 32-lane half of the wave of a >= 0, in every lane (DPP steps on the VALU: the
// row maximum, then row 1 / 3 folds in row 0 / 2, then the halves' last lanes are read back)
__device__ __forceinline__ float half_wave_max(float a) {
  a = dpp_max<DPP_QUAD_XOR1>(a);
  a = dpp_max<DPP_QUAD_XOR2>(a);
  a = dpp_max<DPP_HALF_MIRROR>(a);
  a = dpp_max<DPP_ROW_MIRROR>(a);
  a = dpp_max<DPP_BCAST15, 0xa>(a);
  const float lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 31));
  const float hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 63));
  return (threadIdx.x & 32) ? hi : lo;
}

__device__ __forceinline__ void q8_store(float x, bool valid, int64_t i, int8_t *Xq, float *Xs) {
  const float a = half_wave_max(fabsf(x));
  const float d = a / 127.0f;
  const float iv = a > 0.f ? 127.0f / a : 0.f;
  if (valid) {
    float r = __builtin_rintf(x * iv);
    r = fminf(fmaxf(r, -128.f), 127.f);
    Xq[i] = static_cast<int8_t>(static_cast<int>(r));
    if ((i & 31) == 0) Xs[i >> 5] = d;
  }
}

template <int DT>
__device__ __forceinline__ void store_out(void *p, int dt, int64_t i, double v) {
  (void)sizeof(DT);
  if (dt == VYBDQ_F64) static_cast<double *>(p)[i] = v;
  else if (dt == VYBDQ_F32) static_cast<float *>(p)[i] = static_cast<float>(v);
  else if (dt == VYBDQ_F16) static_cast<_Float16 *>(p)[i] = static_cast<_Float16>(static_cast<float>(v));
  else static_cast<uint16_t *>(p)[i] = f32_to_bf16(static_cast<float>(v));
}

// One workgroup of 256 threads per row; thread t owns elements t + 256 c. C > 0: the row fits
// C elements per thread, whose x and w loads are all issued before the sum (kept in registers
// for the scale pass); C = 0: any N, loaded per iteration.
template <int XDT, int C>
__global__ void __launch_bounds__(256) k_rms_q8(const void *__restrict__ X, const void *__restrict__ W,
                                                void *__restrict__ Y, int ydt, float *__restrict__ Y32,
                                                int8_t *__restrict__ Xq, float *__restrict__ Xs, int64_t N,
                                                double eps) {
#pragma clang fp contract(off)
  __shared__ double part[256];
  __shared__ double rsh;
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t base = row * N;
  constexpr int CR = C > 0 ? C : 1;
  double xv[CR], wv[CR];
  double ss = 0.0;
  if constexpr (C > 0) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t d = t + 256 * c;
      xv[c] = d < N ? load_d<XDT>(X, base + d) : 0.0;
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t d = t + 256 * c;
      wv[c] = d < N ? load_d<XDT>(W, d) : 0.0;
    }
#pragma unroll
    for (int c = 0; c < C; ++c)
      if (t + 256 * c < N) ss = ss + xv[c] * xv[c];
  } else {
    for (int64_t d = t; d < N; d += 256) {
      const double v = load_d<XDT>(X, base + d);
      ss = ss + v * v;
    }
  }
  // pairwise fold: element i += element i + stride, strides 128 .. 1 (64 and below in wave 0)
  part[t] = ss;
  __syncthreads();
  if (t < 128) part[t] = part[t] + part[t + 128];
  __syncthreads();
  if (t < 64) {
    double sw = part[t] + part[t + 64];
#pragma unroll
    for (int st = 32; st > 0; st >>= 1) sw = sw + __shfl_down(sw, st, 64);
    if (t == 0) rsh = 1.0 / sqrt_newton(sw / static_cast<double>(N) + eps);
  }
  __syncthreads();
  const double r = rsh;
  auto emit = [&](int64_t d, bool valid, double y) {
    if (valid) {
      if (Y) store_out<0>(Y, ydt, base + d, y);
      if (Y32) Y32[base + d] = static_cast<float>(y);
    }
    if (Xq) q8_store(static_cast<float>(y), valid, base + d, Xq, Xs);
  };
  if constexpr (C > 0) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t d = t + 256 * c;
      emit(d, d < N, d < N ? xv[c] * r * wv[c] : 0.0);
    }
  } else {
    for (int64_t d0 = 0; d0 < N; d0 += 256) {
      const int64_t d = d0 + t;
      const bool valid = d < N;
      emit(d, valid, valid ? load_d<XDT>(X, base + d) * r * load_d<XDT>(W, d) : 0.0);
    }
  }
}

template <int GDT>
__global__ void __launch_bounds__(256) k_swiglu_q8(const void *__restrict__ G, const void *__restrict__ U,
                                                   void *__restrict__ H, int hdt, int8_t *__restrict__ Xq,
                                                   float *__restrict__ Xs, int64_t n) {
#pragma clang fp contract(off)
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const bool valid = i < n;
  double h = 0.0;
  if (valid) {
    const double g = load_d<GDT>(G, i), u = load_d<GDT>(U, i);
    const double sg = 1.0 / (1.0 + vexp_ref(0.0 - g));
    h = g * sg * u;
    if (H) store_out<0>(H, hdt, i, h);
  }
  if (Xq) q8_store(static_cast<float>(h), valid, i, Xq, Xs);
}

static bool dt_any(int dt) { return dt == VYBDQ_F32 || dt == VYBDQ_F16 || dt == VYBDQ_BF16 || dt == VYBDQ_F64; }

#define VYBDQ_DISPATCH_ANY(dt, NAME, ...)                                                   \
  switch (dt) {                                                                            \
    case VYBDQ_F64: { constexpr int NAME = VYBDQ_F64; __VA_ARGS__; } break;                \
    case VYBDQ_F32: { constexpr int NAME = VYBDQ_F32; __VA_ARGS__; } break;                \
    case VYBDQ_F16: { constexpr int NAME = VYBDQ_F16; __VA_ARGS__; } break;                \
    default: { constexpr int NAME = VYBDQ_BF16; __VA_ARGS__; } break;                      \
  }

}  // namespace vybdq

using namespace vybdq;

extern "C" int vybdq_rmsnorm_q8(uint64_t X, uint64_t W, uint64_t Y, uint64_t Y32, uint64_t Xq, uint64_t Xs,
                                int64_t M, int64_t N, double eps, int x_dt, int y_dt, uint64_t stream) {
  VYBDQ_REQUIRE(X && W, VYBDQ_ERR_ARG, "null X or W");
  VYBDQ_REQUIRE(dt_any(x_dt), VYBDQ_ERR_ARG, "x_dt must be F64, F32, F16 or BF16");
  VYBDQ_REQUIRE(!Y || dt_any(y_dt), VYBDQ_ERR_ARG, "y_dt must be F64, F32, F16 or BF16");
  VYBDQ_REQUIRE((Xq == 0) == (Xs == 0), VYBDQ_ERR_ARG, "Xq and Xs go together");
  VYBDQ_REQUIRE(Y || Y32 || Xq, VYBDQ_ERR_ARG, "no output");
  VYBDQ_REQUIRE(M >= 0 && M < (int64_t(1) << 31) && N >= 1, VYBDQ_ERR_SHAPE, "need 0 <= M < 2^31, N >= 1");
  VYBDQ_REQUIRE(!Xq || N % 32 == 0, VYBDQ_ERR_SHAPE, "the q8 copy needs N % 32 == 0");
  VYBDQ_REQUIRE(!Xs || (Xs & 3) == 0, VYBDQ_ERR_ALIGN, "Xs must be 4-byte aligned");
  if (M == 0) return VYBDQ_OK;
  hipStream_t s = as_stream(stream);
  const void *x = reinterpret_cast<const void *>(X), *w = reinterpret_cast<const void *>(W);
  void *y = reinterpret_cast<void *>(Y);
  auto *y32 = reinterpret_cast<float *>(Y32);
  auto *q = reinterpret_cast<int8_t *>(Xq);
  auto *d = reinterpret_cast<float *>(Xs);
  const int per = static_cast<int>((N + 255) / 256);
#define L(C) VYBDQ_DISPATCH_ANY(x_dt, XDT, hipLaunchKernelGGL((k_rms_q8<XDT, C>), dim3(static_cast<unsigned>(M)), \
                                                                dim3(256), 0, s, x, w, y, y_dt, y32, q, d, N, eps))
  if (per <= 4) { L(4); }
  else if (per <= 8) { L(8); }
  else if (per <= 16) { L(16); }
  else if (per <= 24) { L(24); }
  else if (per <= 32) { L(32); }
  else { L(0); }
#undef L
  return check_launch("vybdq_rmsnorm_q8");
}

extern "C" int vybdq_swiglu_q8(uint64_t G, uint64_t U, uint64_t H, uint64_t Xq, uint64_t Xs, int64_t n, int g_dt,
                               int h_dt, uint64_t stream) {
  VYBDQ_REQUIRE(G && U, VYBDQ_ERR_ARG, "null G or U");
  VYBDQ_REQUIRE(dt_any(g_dt), VYBDQ_ERR_ARG, "g_dt must be F64, F32, F16 or BF16");
  VYBDQ_REQUIRE(!H || dt_any(h_dt), VYBDQ_ERR_ARG, "h_dt must be F64, F32, F16 or BF16");
  VYBDQ_REQUIRE((Xq == 0) == (Xs == 0), VYBDQ_ERR_ARG, "Xq and Xs go together");
  VYBDQ_REQUIRE(H || Xq, VYBDQ_ERR_ARG, "no output");
  VYBDQ_REQUIRE(n >= 0, VYBDQ_ERR_SHAPE, "n < 0");
  VYBDQ_REQUIRE(!Xq || n % 32 == 0, VYBDQ_ERR_SHAPE, "the q8 copy needs n % 32 == 0");
  VYBDQ_REQUIRE(!Xs || (Xs & 3) == 0, VYBDQ_ERR_ALIGN, "Xs must be 4-byte aligned");
  if (n == 0) return VYBDQ_OK;
  hipStream_t s = as_stream(stream);
  const unsigned grid = static_cast<unsigned>((n + 255) / 256);
  const void *g = reinterpret_cast<const void *>(G), *u = reinterpret_cast<const void *>(U);
  void *h = reinterpret_cast<void *>(H);
  auto *q = reinterpret_cast<int8_t *>(Xq);
  auto *d = reinterpret_cast<float *>(Xs);
  VYBDQ_DISPATCH_ANY(g_dt, GDT,
      hipLaunchKernelGGL((k_swiglu_q8<GDT>), dim3(grid), dim3(256), 0, s, g, u, h, h_dt, q, d, n));
  return check_launch("vybdq_swiglu_q8");
}
