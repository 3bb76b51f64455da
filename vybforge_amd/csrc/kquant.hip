// Super-block decode (Q4_K, Q5_K, Q6_K, IQ2_S) and the type-id dequant dispatch, gfx950.
//
// One thread per 4 consecutive weights of a super-block (64 threads per super-block): the bytes
// are read directly (the decode is a gate, not a hot path). Every weight is exact before its
// final rounding: Q4_K/Q5_K d*sc*q (<= 22 significant bits) and dmin*m are exact products and the
// difference is rounded once (one fma); Q6_K d*sc*q has at most 24 significant bits, exact in
// float32. F64 output is the exact value, F32 its single rounding, F16 the rounding of the F32.
// Layouts: llama.cpp ggml-quants.c dequantize_row_q4_K / q5_K / q6_K as ported by the reference
// (native/kernels/q4k.vyb:9-70, native/tools/q5k_ref.py:40-65, native/gguf/q6k_verify.py:20-40).
#include "common.h"
#include "iq2s_grid.inc"

namespace vybdq {

__device__ __forceinline__ float f16_at(const uint8_t *p) {
  return half_bits_to_f32(static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8));
}

// get_scale_min_k4 on the scales[12] bytes at s
__device__ __forceinline__ void scale_min_bytes(const uint8_t *s, int j, int &sc, int &m) {
  if (j < 4) {
    sc = s[j] & 63;
    m = s[j + 4] & 63;
  } else {
    sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
    m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

template <int WT, typename T>
__device__ __forceinline__ T kq_value(const uint8_t *sb, int e) {
  if constexpr (WT == 22) {  // IQ2_S: group l = e / 8 of sub-block ib = e / 32, exact in float32
    const int ib = e >> 5, l = (e >> 3) & 3, j = e & 7, grp = 4 * ib + l;
    const int idx = sb[2 + grp] | (((sb[66 + ib] >> (2 * l)) & 3) << 8);
    const int g = static_cast<int>((kIq2sGrid[idx] >> (8 * j)) & 255);
    const int nib = l < 2 ? (sb[74 + ib] & 15) : (sb[74 + ib] >> 4);
    const T db = static_cast<T>(f16_at(sb)) * (static_cast<T>(0.5) + static_cast<T>(nib)) * static_cast<T>(0.25);
    const T v = db * static_cast<T>(g);
    return ((sb[34 + grp] >> j) & 1) ? -v : v;
  } else if constexpr (WT == 12 || WT == 13) {
    const int g = e >> 6, hi = (e >> 5) & 1, l = e & 31;
    int sc, m;
    scale_min_bytes(sb + 4, 2 * g + hi, sc, m);
    const uint8_t *qs = sb + (WT == 12 ? 16 : 48) + 32 * g;
    int q = hi ? (qs[l] >> 4) : (qs[l] & 15);
    if constexpr (WT == 13) q += ((sb[16 + l] >> (2 * g + hi)) & 1) << 4;
    const T d = static_cast<T>(f16_at(sb)), dmin = static_cast<T>(f16_at(sb + 2));
    if constexpr (sizeof(T) == 8) return fma(d * sc, static_cast<T>(q), -(dmin * m));
    else return fmaf(d * sc, static_cast<T>(q), -(dmin * m));
  } else {
    const int h = e >> 7, i = (e >> 5) & 3, l = e & 31;
    const uint8_t *ql = sb + 64 * h + (i & 1) * 32;
    const int nib = (i & 2) ? (ql[l] >> 4) : (ql[l] & 15);
    const int q = (nib | (((sb[128 + 32 * h + l] >> (2 * i)) & 3) << 4)) - 32;
    const int sc = static_cast<int8_t>(sb[192 + 8 * h + (l >> 4) + 2 * i]);
    const T d = static_cast<T>(f16_at(sb + 208));
    return d * static_cast<T>(sc) * static_cast<T>(q);
  }
}

template <int WT, int ODT>
__global__ void __launch_bounds__(256) k_dequant_kq(const uint8_t *__restrict__ W, void *__restrict__ out,
                                                    int64_t nsb) {
  constexpr int SB = WT == 12 ? 144 : WT == 13 ? 176 : WT == 22 ? 82 : 210;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= nsb * 64) return;
  const int64_t b = t >> 6;
  const int e0 = static_cast<int>(t & 63) * 4;
  const uint8_t *sb = W + b * SB;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t i = b * 256 + e0 + k;
    if constexpr (ODT == VYBDQ_F64) static_cast<double *>(out)[i] = kq_value<WT, double>(sb, e0 + k);
    else if constexpr (ODT == VYBDQ_F32) static_cast<float *>(out)[i] = kq_value<WT, float>(sb, e0 + k);
    else static_cast<_Float16 *>(out)[i] = static_cast<_Float16>(kq_value<WT, float>(sb, e0 + k));
  }
}

template <int WT>
static void launch_kq(const uint8_t *w, void *o, int64_t nsb, int out_dt, hipStream_t s) {
  const unsigned g = static_cast<unsigned>((nsb * 64 + 255) / 256);
  if (out_dt == VYBDQ_F32) hipLaunchKernelGGL((k_dequant_kq<WT, VYBDQ_F32>), dim3(g), dim3(256), 0, s, w, o, nsb);
  else if (out_dt == VYBDQ_F16) hipLaunchKernelGGL((k_dequant_kq<WT, VYBDQ_F16>), dim3(g), dim3(256), 0, s, w, o, nsb);
  else hipLaunchKernelGGL((k_dequant_kq<WT, VYBDQ_F64>), dim3(g), dim3(256), 0, s, w, o, nsb);
}

}  // namespace vybdq

using namespace vybdq;

extern "C" int vybdq_dequant(int wtype, uint64_t W, uint64_t out, int64_t n, int out_dt, uint64_t stream) {
  VYBDQ_REQUIRE(W && out, VYBDQ_ERR_ARG, "null buffer");
  VYBDQ_REQUIRE(n >= 0, VYBDQ_ERR_SHAPE, "n < 0");
  VYBDQ_REQUIRE(out_dt == VYBDQ_F32 || out_dt == VYBDQ_F16 || out_dt == VYBDQ_F64, VYBDQ_ERR_ARG,
                "out_dt must be F32, F16 or F64");
  if (wtype == 2 || wtype == 8) {
    VYBDQ_REQUIRE(n % 32 == 0, VYBDQ_ERR_SHAPE, "q4_0 / Q8_0: n must be a multiple of 32");
    return wtype == 2 ? vybdq_dequant_q4_0(W, out, n / 32, VYBDQ_Q4_GGML, out_dt, stream)
                      : vybdq_dequant_q8_0(W, out, n / 32, out_dt, stream);
  }
  VYBDQ_REQUIRE(wtype == 12 || wtype == 13 || wtype == 14 || wtype == 22, VYBDQ_ERR_ARG,
                "wtype must be 2 (q4_0), 8 (Q8_0), 12 (Q4_K), 13 (Q5_K), 14 (Q6_K) or 22 (IQ2_S)");
  VYBDQ_REQUIRE(n % 256 == 0, VYBDQ_ERR_SHAPE, "K-quants: n must be a multiple of 256");
  if (n == 0) return VYBDQ_OK;
  const auto *w = reinterpret_cast<const uint8_t *>(W);
  void *o = reinterpret_cast<void *>(out);
  hipStream_t s = as_stream(stream);
  if (wtype == 12) launch_kq<12>(w, o, n / 256, out_dt, s);
  else if (wtype == 13) launch_kq<13>(w, o, n / 256, out_dt, s);
  else if (wtype == 22) launch_kq<22>(w, o, n / 256, out_dt, s);
  else launch_kq<14>(w, o, n / 256, out_dt, s);
  return check_launch("vybdq_dequant");
}
