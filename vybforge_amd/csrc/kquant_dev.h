// GGUF K-quant super-blocks (Q4_K, Q5_K, Q6_K) for the pair GEMV, gfx950.
//
// The GEMV walks a row in 64-weight units: unit p covers weights 64p .. 64p+63, i.e. the
// staged x pair p (the q4_0 pair layout: two 32-element blocks with their block sums). For the
// K-quants unit p is part (p & 3) of super-block p >> 2 (256 weights):
//   Q4_K (144 B: d, dmin, scales[12], qs[128]) / Q5_K (176 B: d, dmin, scales[12], qh[32],
//     qs[128]): unit g = sub-blocks 2g (low nibbles of qs[32g..32g+31], x block 0) and 2g+1
//     (high nibbles, x block 1); Q5_K adds bit 2g / 2g+1 of qh[l] as 16.
//     w = d*sc_j*q - dmin*m_j, so per block sum_k x_k w_k = d*sc_j*(dot - 1024*S) - dmin*m_j*S
//     with dot = sum x*(1024+q) (fp16 weights built by v_perm, v_dot2) and S the block's x sum.
//   Q6_K (210 B: ql[128], qh[64], scales[16] int8, d): half h = unit >> 1 of the super-block;
//     unit part A (p & 1 == 0) reads ql[64h .. 64h+31]: low nibbles are elements 128h + l,
//     high nibbles 128h + 64 + l; part B reads ql[64h+32 ..]: elements 128h + 32 + l and
//     128h + 96 + l; qh[32h + l] supplies 2 bits each (shift 0/4 for A, 2/6 for B). So A is
//     block 0 and B block 1 of x pairs 4sb + 2h and 4sb + 2h + 1. Weights are (1024 + q6) - 1056
//     = q - 32 in fp16 (exact), one scale per 16 weights.
// Q6_K super-blocks are 2-byte aligned only: the loads are dword-aligned windows and the
// re-alignment (v_alignbit by 0 or 16) happens at use, so nothing waits at load time.
// The layouts follow llama.cpp's ggml-quants.c, as ported by the reference
// (native/kernels/q4k.vyb:1-70, native/tools/q5k_ref.py:40-65, native/gguf/q6k_verify.py:20-40).
//   IQ2_S (82 B: d, qs[32] grid-index bytes, 32 sign bytes, qh[8], scales[8]): unit u = sub-blocks
//     2u, 2u+1 = groups 8u .. 8u+7 of 8 weights; group l takes grid entry
//     qs[8u+l] | ((qh[2u + l/4] >> 2(l%4)) & 3) << 8 (8 magnitudes 8/25/43, from the grid staged
//     in LDS), negated per the bits of sign byte 8u+l, scaled by d*(0.5 + 4-bit scale)/4 per 16.
#pragma once

#include "iq2s_grid.inc"

namespace vybdq {

template <> struct Fmt<FMT_Q4_K> {
  static constexpr int SB_BYTES = 144;
  static constexpr int PAIR_DWORDS = 12;  // header (d, dmin, scales) + 32 B of qs
};
template <> struct Fmt<FMT_Q5_K> {
  static constexpr int SB_BYTES = 176;
  static constexpr int PAIR_DWORDS = 20;  // header + qh[32] + 32 B of qs
};
// LDS of the IQ2_S tables behind the x stage and its block sums (16-B aligned): 1024 grid
// entries of 8 fp16 magnitudes, then 256 sign patterns as fp16 sign-bit masks, 16 B each
constexpr size_t kIq2sLdsBytes = (1024 + 256) * 16 + 16;
__device__ __forceinline__ u4 *iq2s_lds_grid(float *sx, int M, int P) {
  return reinterpret_cast<u4 *>(sx + ((XSX_PER_PAIR * M * P + 3) & ~3));  // sx is 16-B aligned
}

template <> struct Fmt<FMT_IQ2_S> {
  static constexpr int SB_BYTES = 82;
  static constexpr int PAIR_DWORDS = 10;  // index window 3 + sign window 3 + qh pair + scale pair + d + shift
};
template <> struct Fmt<FMT_Q6_K> {
  static constexpr int SB_BYTES = 210;
  static constexpr int PAIR_DWORDS = 23;  // ql window 9 + qh window 9 + scales window 3 + d + shift
};

// p rounded down to a 4-byte boundary by pointer arithmetic (an integer round trip would lose the
// pointer's address space, and loads through it would become flat loads)
template <int FMT>
__device__ __forceinline__ const uint32_t *dword_floor(const uint8_t *p) {
  return reinterpret_cast<const uint32_t *>(p - (reinterpret_cast<uintptr_t>(p) & 3));
}

template <int N>
__device__ __forceinline__ void load_dwords(const uint32_t *p, uint32_t *dw) {
  const u4a4 *v = reinterpret_cast<const u4a4 *>(p);
#pragma unroll
  for (int i = 0; i < N / 4; ++i) {
    const u4a4 t = v[i];
    dw[4 * i + 0] = t[0];
    dw[4 * i + 1] = t[1];
    dw[4 * i + 2] = t[2];
    dw[4 * i + 3] = t[3];
  }
#pragma unroll
  for (int i = (N / 4) * 4; i < N; ++i) dw[i] = p[i];
}

// Loads of unit p of the row at wrow (K-quants).
template <int FMT>
__device__ __forceinline__ void load_unit_kq(const uint8_t *wrow, int p, uint32_t (&dw)[Fmt<FMT>::PAIR_DWORDS]) {
  const uint8_t *sb = wrow + static_cast<int64_t>(p >> 2) * Fmt<FMT>::SB_BYTES;
  const int g = p & 3;
  if constexpr (FMT == FMT_Q4_K) {
    load_dwords<4>(reinterpret_cast<const uint32_t *>(sb), dw);
    load_dwords<8>(reinterpret_cast<const uint32_t *>(sb + 16 + 32 * g), dw + 4);
  } else if constexpr (FMT == FMT_Q5_K) {
    load_dwords<12>(reinterpret_cast<const uint32_t *>(sb), dw);  // header + qh
    load_dwords<8>(reinterpret_cast<const uint32_t *>(sb + 48 + 32 * g), dw + 12);
  } else if constexpr (FMT == FMT_IQ2_S) {
    // super-blocks are 2-byte aligned; both 8-byte windows sit 2 bytes past a dword boundary
    // exactly when the super-block starts on one
    load_dwords<3>(dword_floor<FMT>(sb + 2 + 8 * g), dw);
    load_dwords<3>(dword_floor<FMT>(sb + 34 + 8 * g), dw + 3);
    dw[6] = *reinterpret_cast<const uint16_t *>(sb + 66 + 2 * g);  // qh of sub-blocks 2g, 2g+1
    dw[7] = *reinterpret_cast<const uint16_t *>(sb + 74 + 2 * g);  // their scales
    dw[8] = *reinterpret_cast<const uint16_t *>(sb);                // d
    dw[9] = (reinterpret_cast<uintptr_t>(sb) & 2) ? 0u : 16u;
  } else {
    const int h = g >> 1, part = g & 1;
    const bool odd = (reinterpret_cast<uintptr_t>(sb) & 2) != 0;  // 2 bytes past a dword boundary
    load_dwords<9>(dword_floor<FMT>(sb + 64 * h + 32 * part), dw);
    load_dwords<9>(dword_floor<FMT>(sb + 128 + 32 * h), dw + 9);
    // scales[8h .. 8h+7]: the third dword is needed only when odd (an aligned super-block would
    // read 2 bytes past its end for h = 1), so aligned ones re-read the second
    const uint32_t *sc = dword_floor<FMT>(sb + 192 + 8 * h);
    dw[18] = sc[0];
    dw[19] = sc[1];
    dw[20] = sc[odd ? 2 : 1];
    dw[21] = *reinterpret_cast<const uint16_t *>(sb + 208);  // d
    dw[22] = odd ? 16u : 0u;
  }
}

// 6-bit scale and min of sub-block j (get_scale_min_k4) from the scale dwords s0, s1, s2.
__device__ __forceinline__ void scale_min_k4(uint32_t s0, uint32_t s1, uint32_t s2, int j, float &sc, float &mn) {
  const int o = 8 * (j & 3);
  uint32_t a, b;
  if (j < 4) {
    a = __builtin_amdgcn_ubfe(s0, o, 6);
    b = __builtin_amdgcn_ubfe(s1, o, 6);
  } else {
    a = __builtin_amdgcn_ubfe(s2, o, 4) | (__builtin_amdgcn_ubfe(s0, o + 6, 2) << 4);
    b = __builtin_amdgcn_ubfe(s2, o + 4, 4) | (__builtin_amdgcn_ubfe(s1, o + 6, 2) << 4);
  }
  sc = static_cast<float>(a);
  mn = static_cast<float>(b);
}

// sum over one 32-element x block of w * x for 16 fp16 weight pairs wv (element order)
__device__ __forceinline__ float block_dot(const h2 (&wv)[16], const char *xb) {
  const u4 *xc = reinterpret_cast<const u4 *>(xb);
  float ps = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const u4 xv = xc[c];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t xw = xv[j];
      ps = __builtin_amdgcn_fdot2(wv[4 * c + j], __builtin_bit_cast(h2, xw), ps, false);
    }
  }
  return ps;
}

// the same over the two 16-element halves separately (Q6_K: one scale per 16 weights)
__device__ __forceinline__ void block_dot16(const h2 (&wv)[16], const char *xb, float &p0, float &p1) {
  const u4 *xc = reinterpret_cast<const u4 *>(xb);
  p0 = 0.f;
  p1 = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const u4 xv = xc[c];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t xw = xv[j];
      if (c < 2) p0 = __builtin_amdgcn_fdot2(wv[4 * c + j], __builtin_bit_cast(h2, xw), p0, false);
      else p1 = __builtin_amdgcn_fdot2(wv[4 * c + j], __builtin_bit_cast(h2, xw), p1, false);
    }
  }
}

// fp16 pairs (1024 + b0, 1024 + b1), (1024 + b2, 1024 + b3) of the 4 bytes of v (each < 256)
__device__ __forceinline__ void bytes_to_h2(uint32_t v, h2 &a, h2 &b) {
  a = __builtin_bit_cast(h2, __builtin_amdgcn_perm(C64, v, SEL_B01));
  b = __builtin_bit_cast(h2, __builtin_amdgcn_perm(C64, v, SEL_B23));
}

template <int FMT, int M>
__device__ __forceinline__ void unit_dot_kq(const uint32_t (&dw)[Fmt<FMT>::PAIR_DWORDS], const char *lds,
                                            const float *sx, int P, int p, float (&acc)[M]) {
  const int g = p & 3;
  if constexpr (FMT == FMT_Q4_K || FMT == FMT_Q5_K) {
    constexpr int QS = FMT == FMT_Q4_K ? 4 : 12;  // first qs dword
    const float d = half_bits_to_f32(dw[0] & 0xffffu);
    const float dmin = half_bits_to_f32(dw[0] >> 16);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float sc, mn;
      scale_min_k4(dw[1], dw[2], dw[3], 2 * g + h, sc, mn);
      const float ds = d * sc, dm = dmin * mn;
      h2 wv[16];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        uint32_t v = h == 0 ? (dw[QS + t] & 0x0F0F0F0Fu) : ((dw[QS + t] >> 4) & 0x0F0F0F0Fu);
        if constexpr (FMT == FMT_Q5_K) v |= ((dw[4 + t] >> (2 * g + h)) & 0x01010101u) << 4;
        bytes_to_h2(v, wv[2 * t], wv[2 * t + 1]);
      }
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float ps = block_dot(wv, lds + m * P * XPAIR_STRIDE + p * XPAIR_STRIDE + 64 * h);
        const float2 xb = x_block(sx, m * 2 * P + 2 * p + h);
        acc[m] = fmaf(xb.y, fmaf(ds, fmaf(-1024.0f, xb.x, ps), -dm * xb.x), acc[m]);
      }
    }
  } else if constexpr (FMT == FMT_IQ2_S) {
    const uint32_t sh = dw[9];
    const uint32_t ix[2] = {__builtin_amdgcn_alignbit(dw[1], dw[0], sh), __builtin_amdgcn_alignbit(dw[2], dw[1], sh)};
    const uint32_t sg[2] = {__builtin_amdgcn_alignbit(dw[4], dw[3], sh), __builtin_amdgcn_alignbit(dw[5], dw[4], sh)};
    const float d = half_bits_to_f32(dw[8]) * 0.25f;
    const u4 *gridh = iq2s_lds_grid(const_cast<float *>(sx), M, P);  // [1024 grid][256 signs]
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const int ib = l >> 2, l2 = l & 3;
      const uint32_t idx = __builtin_amdgcn_ubfe(ix[l >> 2], 8 * (l & 3), 8) |
                           (__builtin_amdgcn_ubfe(dw[6], 8 * ib + 2 * l2, 2) << 8);
      const u4 e = gridh[idx];
      const u4 sm = gridh[1024 + __builtin_amdgcn_ubfe(sg[l >> 2], 8 * (l & 3), 8)];
      const float dl = d * (0.5f + static_cast<float>(__builtin_amdgcn_ubfe(dw[7], 8 * ib + 4 * (l2 >> 1), 4)));
      h2 wv[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t ek = e[k], sk = sm[k];  // vector elements to scalars before the bit casts
        wv[k] = __builtin_bit_cast(h2, ek ^ sk);
      }
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const u4 xv = *reinterpret_cast<const u4 *>(lds + m * P * XPAIR_STRIDE + p * XPAIR_STRIDE + 64 * ib + 16 * l2);
        float ps = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t xw = xv[k];
          ps = __builtin_amdgcn_fdot2(wv[k], __builtin_bit_cast(h2, xw), ps, false);
        }
        acc[m] = fmaf(dl * x_block(sx, m * 2 * P + 2 * p + ib).y, ps, acc[m]);
      }
    }
  } else {
    const int hf = g >> 1, part = g & 1;
    const uint32_t sh = dw[22];
    uint32_t ql[8], qh[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      ql[t] = __builtin_amdgcn_alignbit(dw[t + 1], dw[t], sh);
      qh[t] = __builtin_amdgcn_alignbit(dw[9 + t + 1], dw[9 + t], sh);
    }
    const uint32_t sc0 = __builtin_amdgcn_alignbit(dw[19], dw[18], sh);  // scales[8h + 0..3]
    const uint32_t sc1 = __builtin_amdgcn_alignbit(dw[20], dw[19], sh);  // scales[8h + 4..7]
    const float d = half_bits_to_f32(dw[21]);
    const h2 off = h2{static_cast<_Float16>(-1056.0f), static_cast<_Float16>(-1056.0f)};
    // nibble half 0: low nibbles (x pair 4sb + 2h, block part); 1: high nibbles (pair + 1)
#pragma unroll
    for (int nh = 0; nh < 2; ++nh) {
      const int hs = nh == 0 ? 2 * part : 4 + 2 * part;  // qh bit pair
      const uint32_t scw = nh == 0 ? sc0 : sc1;
      // scales of the two 16-element halves: bytes 2 part, 2 part + 1 of scw, signed
      const float s0 = static_cast<float>(static_cast<int8_t>(__builtin_amdgcn_ubfe(scw, 16 * part, 8)));
      const float s1 = static_cast<float>(static_cast<int8_t>(__builtin_amdgcn_ubfe(scw, 16 * part + 8, 8)));
      h2 wv[16];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t v = (nh == 0 ? (ql[t] & 0x0F0F0F0Fu) : ((ql[t] >> 4) & 0x0F0F0F0Fu)) |
                           (((qh[t] >> hs) & 0x03030303u) << 4);
        bytes_to_h2(v, wv[2 * t], wv[2 * t + 1]);
        wv[2 * t] = wv[2 * t] + off;
        wv[2 * t + 1] = wv[2 * t + 1] + off;
      }
      const int xp = (p & ~3) + 2 * hf + nh;  // x pair
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float p0, p1;
        block_dot16(wv, lds + m * P * XPAIR_STRIDE + xp * XPAIR_STRIDE + 64 * part, p0, p1);
        acc[m] = fmaf(d * x_block(sx, m * 2 * P + 2 * xp + part).y, fmaf(s0, p0, s1 * p1), acc[m]);
      }
    }
  }
}

}  // namespace vybdq
