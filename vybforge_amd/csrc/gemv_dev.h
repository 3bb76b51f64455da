// Device helpers shared by the one-shot GEMV (gemv.hip) and the persistent chain (chain.hip):
// GGUF block formats, pair loads, quant unpack to fp16 pairs, the x stage and the pair dot.
#pragma once
#include "common.h"
#include <type_traits>

namespace vybdq {

enum { FMT_Q4_0 = 0, FMT_Q8_0 = 1, FMT_Q4_K = 2, FMT_Q5_K = 3, FMT_Q6_K = 4, FMT_IQ2_S = 5 };

// formats of 256-weight super-blocks (walked as four 64-weight units each)
template <int FMT> constexpr bool is_kquant() {
  return FMT == FMT_Q4_K || FMT == FMT_Q5_K || FMT == FMT_Q6_K || FMT == FMT_IQ2_S;
}

template <int FMT> struct Fmt;
template <> struct Fmt<FMT_Q4_0> {
  static constexpr int PAIR_BYTES = 36;
  static constexpr int PAIR_DWORDS = 9;
  static constexpr int QDW = 4;                 // quant dwords per block
  static constexpr int U = 4;                   // pairs per load batch (VGPR budget vs occupancy)
  static constexpr float CORR = 1032.0f;        // 1024 + 8
};
template <> struct Fmt<FMT_Q8_0> {
  static constexpr int PAIR_BYTES = 68;
  static constexpr int PAIR_DWORDS = 17;
  static constexpr int QDW = 8;
  static constexpr int U = 2;
  static constexpr float CORR = 1152.0f;        // 1024 + 128
};

struct Segs {
  const uint8_t *W[3];
  void *Y[3];
  const void *RS[3];
  int ydt[3];
  int64_t end[3];  // cumulative row ends
};

// Element i (0..2) of a three-entry kernel-argument array, chosen with selects: indexing the
// by-value array with a per-lane i would make the compiler fetch the argument block through
// vector memory loads, and the wait for them would delay the first weight load.
// The empty asm keeps the three values in scalar registers; without it the compiler folds the
// selects into one load through a selected address, which is the same memory access again.
template <class V>
__device__ __forceinline__ V pick3(const V (&a)[3], int i) {
  using B = typename std::conditional<sizeof(V) == 8, uint64_t, uint32_t>::type;
  static_assert(sizeof(V) == sizeof(B), "pick3: 4- or 8-byte values");
  B b0 = __builtin_bit_cast(B, a[0]), b1 = __builtin_bit_cast(B, a[1]), b2 = __builtin_bit_cast(B, a[2]);
  asm volatile("" : "+s"(b0), "+s"(b1), "+s"(b2));
  return __builtin_bit_cast(V, i == 0 ? b0 : (i == 1 ? b1 : b2));
}

// pick3 for pointers: the result is formed as an offset from a[0], so the compiler still sees
// a global-memory pointer (a pointer straight out of the asm would be generic: flat loads).
template <class V>
__device__ __forceinline__ V *pick3_ptr(V *const (&a)[3], int i) {
  uint64_t b0 = reinterpret_cast<uint64_t>(a[0]), b1 = reinterpret_cast<uint64_t>(a[1]),
           b2 = reinterpret_cast<uint64_t>(a[2]);
  asm volatile("" : "+s"(b0), "+s"(b1), "+s"(b2));
  const uint64_t d = (i == 0 ? b0 : (i == 1 ? b1 : b2)) - b0;  // byte distance from a[0] (mod 2^64)
  return (V *)((const char *)a[0] + d);
}

// LDS x stage, per X row m: pair p (64 fp16, natural order) at byte m*P*144 + 144*p (a 16-B pad
// per pair keeps the G lanes that read consecutive pairs on distinct banks); per 32-element block
// b = m*2P + (block of the row), sx[2b] = the sum of its staged fp16 values and sx[2b + 1] = its
// scale: the block's x values are scale * (staged values). For float32 / bf16 activations the
// scale is the power of two that brings the block's largest |x| into [2^14, 2^15) (block_scale),
// so activations of any magnitude stage without overflow or subnormals; fp16 activations stage
// as they are (scale 1). The dot products multiply the scale into the block's weight scale.
constexpr int XPAIR_STRIDE = 144;
constexpr int XSX_PER_PAIR = 4;                                  // floats of sx per pair (2 blocks)
constexpr int XSTAGE_PAIR_BYTES = XPAIR_STRIDE + 4 * XSX_PER_PAIR;  // LDS bytes per staged pair

// Raw x chunk (8 consecutive elements) -> registers: XW = 4 dwords for fp16/bf16, 8 for f32.
template <int XW>
__device__ __forceinline__ void load_x_chunk(const void *X, int64_t i, uint32_t (&r)[XW]) {
  if constexpr (XW == 8) {
    const u4 *p = reinterpret_cast<const u4 *>(static_cast<const float *>(X) + i);
    const u4 a = p[0], b = p[1];
    r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
    r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  } else {
    const u4 v = *reinterpret_cast<const u4 *>(static_cast<const uint16_t *>(X) + i);
    r[0] = v[0]; r[1] = v[1]; r[2] = v[2]; r[3] = v[3];
  }
}

// DPP lane exchange added to v: v + (the value of the lane that CTRL selects), on the VALU with
// no LDS round trip. Lanes of 16-lane rows outside ROWS add 0.
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ float dpp_add(float v) {
  const int t = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xf, false);
  return v + __builtin_bit_cast(float, t);
}

// Sum over each aligned group of G consecutive lanes (G = 8, 16, 32 or 64). After the quad swaps
// and the mirrors every lane of a 16-lane row holds its row's (or half-row's) sum; the
// broadcasts then fold rows together. The group total is in the group's last lane (G - 1).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(G == 4 || G == 8 || G == 16 || G == 32 || G == 64, "group size");
  v = dpp_add<DPP_QUAD_XOR1>(v);
  v = dpp_add<DPP_QUAD_XOR2>(v);
  if constexpr (G >= 8) v = dpp_add<DPP_HALF_MIRROR>(v);
  if constexpr (G >= 16) v = dpp_add<DPP_ROW_MIRROR>(v);
  if constexpr (G >= 32) v = dpp_add<DPP_BCAST15, 0xA>(v);  // rows 1, 3 += rows 0, 2
  if constexpr (G >= 64) v = dpp_add<DPP_BCAST31, 0x8>(v);  // row 3 += rows 0 + 1
  return v;
}

template <int CTRL>
__device__ __forceinline__ float dpp_max(float v) {
  const int t = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false);
  return fmaxf(v, __builtin_bit_cast(float, t));
}

// Convert a raw chunk to 4 fp16 pairs, store it at its LDS slot and reduce the block sums:
// chunk c holds x[8c .. 8c+7] (for every X row m, since K = 64 P), lives in pair c>>3 at
// (c>>3)*144 + (c&7)*16, and its 32-element block is c>>2. The 4 chunks of a block belong to 4
// consecutive threads, which combine their partial maxima and sums with two xor shuffles.
template <int XW>
__device__ __forceinline__ void stage_chunk(const uint32_t (&r)[XW], int xdt, int c, char *lds, float *sx) {
  uint32_t h[4];
  float scale = 1.0f;
  if constexpr (XW == 8) {
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(__uint_as_float(r[j])));
    amax = dpp_max<DPP_QUAD_XOR1>(amax);
    amax = dpp_max<DPP_QUAD_XOR2>(amax);
    float inv;
    scale = block_scale(amax, inv);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      h[j] = __builtin_bit_cast(uint32_t, h2{static_cast<_Float16>(__uint_as_float(r[2 * j]) * inv),
                                             static_cast<_Float16>(__uint_as_float(r[2 * j + 1]) * inv)});
  } else if (xdt == VYBDQ_BF16) {
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      amax = fmaxf(amax, fmaxf(fabsf(__uint_as_float(r[j] << 16)), fabsf(__uint_as_float(r[j] & 0xffff0000u))));
    amax = dpp_max<DPP_QUAD_XOR1>(amax);
    amax = dpp_max<DPP_QUAD_XOR2>(amax);
    float inv;
    scale = block_scale(amax, inv);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      h[j] = __builtin_bit_cast(uint32_t, h2{static_cast<_Float16>(__uint_as_float(r[j] << 16) * inv),
                                             static_cast<_Float16>(__uint_as_float(r[j] & 0xffff0000u) * inv)});
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) h[j] = r[j];
  }
  *reinterpret_cast<u4 *>(lds + (c >> 3) * XPAIR_STRIDE + (c & 7) * 16) = u4{h[0], h[1], h[2], h[3]};
  // block sum of the staged fp16 values: v_dot2 against (1, 1) adds two exact fp16 values per op
  const h2 ones = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) s = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, h[j]), ones, s, false);
  s = dpp_add<DPP_QUAD_XOR1>(s);
  s = dpp_add<DPP_QUAD_XOR2>(s);
  if ((c & 3) == 0) *reinterpret_cast<float2 *>(sx + 2 * (c >> 2)) = float2{s, scale};
}

// {sum, scale} of x block b (b = m*2P + block of the row)
__device__ __forceinline__ float2 x_block(const float *sx, int b) {
  return *reinterpret_cast<const float2 *>(sx + 2 * b);
}

typedef uint32_t u4a4 __attribute__((ext_vector_type(4), aligned(4)));

template <int FMT>
__device__ __forceinline__ void load_pair(const uint8_t *p, uint32_t (&dw)[Fmt<FMT>::PAIR_DWORDS]) {
  const u4a4 *v = reinterpret_cast<const u4a4 *>(p);
#pragma unroll
  for (int i = 0; i < Fmt<FMT>::PAIR_DWORDS / 4; ++i) {
    const u4a4 t = v[i];
    dw[4 * i + 0] = t[0];
    dw[4 * i + 1] = t[1];
    dw[4 * i + 2] = t[2];
    dw[4 * i + 3] = t[3];
  }
  dw[Fmt<FMT>::PAIR_DWORDS - 1] =
      reinterpret_cast<const uint32_t *>(p)[Fmt<FMT>::PAIR_DWORDS - 1];
}

// v_perm_b32 selectors: {S0 = 0x64646464, S1 = v} -> fp16 pair (0x6400 | v.byte a, 0x6400 | v.byte b)
constexpr uint32_t SEL_B01 = 0x04010400u;
constexpr uint32_t SEL_B23 = 0x04030402u;
constexpr uint32_t C64 = 0x64646464u;

// The 16 fp16 weight pairs (1024 + v_e, 1024 + v_e+1), e = 2i, of one block in element order.
template <int FMT, int ORDER>
__device__ __forceinline__ void unpack_block(const uint32_t (&q)[Fmt<FMT>::QDW], h2 (&wv)[16]) {
#pragma unroll
  for (int t = 0; t < Fmt<FMT>::QDW; ++t) {
    if constexpr (FMT == FMT_Q8_0) {
      const uint32_t u = q[t] ^ 0x80808080u;
      wv[2 * t] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(C64, u, SEL_B01));
      wv[2 * t + 1] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(C64, u, SEL_B23));
    } else {
      const uint32_t lo = q[t] & 0x0F0F0F0Fu;
      const uint32_t hi = (q[t] >> 4) & 0x0F0F0F0Fu;
      if constexpr (ORDER == VYBDQ_Q4_GGML) {
        // qs bytes 4t..4t+3: low nibbles = elements 4t..4t+3, high = 16+4t..16+4t+3
        wv[2 * t] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(C64, lo, SEL_B01));
        wv[2 * t + 1] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(C64, lo, SEL_B23));
        wv[8 + 2 * t] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(C64, hi, SEL_B01));
        wv[8 + 2 * t + 1] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(C64, hi, SEL_B23));
      } else {
        // byte s = (element 2s low, 2s+1 high): interleave low/high bytes first
        const uint32_t a = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // lo0 hi0 lo1 hi1
        const uint32_t b = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // lo2 hi2 lo3 hi3
        wv[4 * t] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(C64, a, SEL_B01));
        wv[4 * t + 1] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(C64, a, SEL_B23));
        wv[4 * t + 2] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(C64, b, SEL_B01));
        wv[4 * t + 3] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(C64, b, SEL_B23));
      }
    }
  }
}

// Dot products of one pair (two blocks) of one row with the M staged x rows.
template <int FMT, int ORDER, int M>
__device__ __forceinline__ void pair_dot(const uint32_t (&dw)[Fmt<FMT>::PAIR_DWORDS], const char *lds,
                                         const float *sx, int P, int p, float (&acc)[M]) {
  constexpr int QDW = Fmt<FMT>::QDW;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t q[QDW];
    float d;
    if (h == 0) {
#pragma unroll
      for (int t = 0; t < QDW; ++t) q[t] = __builtin_amdgcn_alignbit(dw[t + 1], dw[t], 16);
      d = half_bits_to_f32(dw[0] & 0xffffu);
    } else {
#pragma unroll
      for (int t = 0; t < QDW; ++t) q[t] = dw[QDW + 1 + t];
      d = half_bits_to_f32(dw[QDW] >> 16);
    }
    h2 wv[16];
    unpack_block<FMT, ORDER>(q, wv);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const u4 *xc = reinterpret_cast<const u4 *>(lds + m * P * XPAIR_STRIDE + p * XPAIR_STRIDE + 64 * h);
      float ps = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u4 xv = xc[c];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // copy the element to a scalar first: bit-casting a vector element expression
          // directly reads element 0 with this compiler
          const uint32_t xw = xv[j];
          ps = __builtin_amdgcn_fdot2(wv[4 * c + j], __builtin_bit_cast(h2, xw), ps, false);
        }
      }
      const float2 xb = x_block(sx, m * 2 * P + 2 * p + h);
      const float part = fmaf(-Fmt<FMT>::CORR, xb.x, ps);
      acc[m] = fmaf(d * xb.y, part, acc[m]);
    }
  }
}

}  // namespace vybdq

#include "kquant_dev.h"

namespace vybdq {

// Bytes of one packed row of P 64-weight units.
template <int FMT>
__host__ __device__ constexpr int64_t unit_row_bytes(int64_t P) {
  if constexpr (is_kquant<FMT>()) return (P / 4) * Fmt<FMT>::SB_BYTES;
  else return P * Fmt<FMT>::PAIR_BYTES;
}

// Unit p (weights 64p .. 64p+63) of the row at wrow: loads, then the dot with the staged x.
template <int FMT>
__device__ __forceinline__ void load_unit(const uint8_t *wrow, int p, uint32_t (&dw)[Fmt<FMT>::PAIR_DWORDS]) {
  if constexpr (is_kquant<FMT>()) load_unit_kq<FMT>(wrow, p, dw);
  else load_pair<FMT>(wrow + static_cast<int64_t>(p) * Fmt<FMT>::PAIR_BYTES, dw);
}

template <int FMT, int ORDER, int M>
__device__ __forceinline__ void unit_dot(const uint32_t (&dw)[Fmt<FMT>::PAIR_DWORDS], const char *lds,
                                         const float *sx, int P, int p, float (&acc)[M]) {
  if constexpr (is_kquant<FMT>()) unit_dot_kq<FMT, M>(dw, lds, sx, P, p, acc);
  else pair_dot<FMT, ORDER, M>(dw, lds, sx, P, p, acc);
}

}  // namespace vybdq
