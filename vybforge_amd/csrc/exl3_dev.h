// EXL3 4-bpw trellis device helpers shared by the fused GEMM (exl3.hip) and the grouped MoE
// experts (moe_exl3.hip): the lane windows of a 16x16 tile's stream, the mcg hash decode through
// the tile-slot composition table, and the 128-point FWHT across a wave. Format and decode:
// native/exl3/README.md:24-49, native/exl3/exl3_ref.py:1-120 (see exl3.hip's header).
#pragma once

#include "common.h"

namespace vybdq {

#include "exl3_slots.inc"

constexpr float kRScale = 0.08838834764831845f;  // 1/sqrt(128)

// bits [o, o+32) of the 192-bit lane window w[0..5] (o is a constant after unrolling)
__device__ __forceinline__ uint32_t win_extract(const uint32_t (&w)[6], int o) {
  const int i = o >> 5, s = o & 31;
  if (s == 0) return w[i];
  if (i == 5) return w[5] >> s;
  return __builtin_amdgcn_alignbit(w[i + 1], w[i], s);
}

// mcg hash of the 16-bit window in half HI of d (the other half is ignored): x = w * 0xCBAC1FED
// mod 2^32 from two full-rate 16 x 16-bit products, c = (w * 0xCBAC) << 16 (the multiply writes
// its low 16 bits to the high half through its SDWA destination select) and x = w * 0x1FED + c
// (v_mad_u32_u16, whose op_sel takes the window from either half). Written out because the
// compiler would merge the products into one quarter-rate 32-bit multiply, or shift and add
// separately.
template <bool HI>
__device__ __forceinline__ uint32_t mcg_hash(uint32_t d) {
  uint32_t c, x;
  if constexpr (HI) {
    asm("v_mul_u32_u24_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:DWORD"
        : "=v"(c) : "v"(d), "s"(0xCBACu));
    asm("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[1,0,0,0]" : "=v"(x) : "v"(d), "s"(0x1FEDu), "v"(c));
  } else {
    asm("v_mul_u32_u24_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:DWORD"
        : "=v"(c) : "v"(d), "s"(0xCBACu));
    asm("v_mad_u32_u16 %0, %1, %2, %3" : "=v"(x) : "v"(d), "s"(0x1FEDu), "v"(c));
  }
  return x;
}

// The mcg hash of a window (its low 16 bits; higher bits are ignored) up to the two fp16 halves
// (before they are added).
__device__ __forceinline__ uint32_t decode_window_halves(uint32_t w) {
  return (mcg_hash<false>(w) & 0x8FFF8FFFu) ^ 0x3B603B60u;
}

// Lane slot q's window hashed up to the two fp16 halves. A one-piece window at a 16-bit boundary
// is hashed straight from its stream dword; other one-piece windows are funnel-extracted without
// a mask (the hash reads only the low 16 bits); two-piece windows are assembled from their masks.
__device__ __forceinline__ uint32_t slot_halves(const uint32_t (&w)[6], int q) {
  const int o = kExl3SlotOff0[q];
  const bool one = kExl3SlotOff1[q] < 0 && kExl3SlotMask0[q] == 0xffffu;
  if (one && (o & 15) == 0) {
    const uint32_t x = (o & 16) ? mcg_hash<true>(w[o >> 5]) : mcg_hash<false>(w[o >> 5]);
    return (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
  }
  if (one) return decode_window_halves(win_extract(w, o));
  // A two-piece window whose first piece runs to the end of its stream dword and whose second
  // piece starts a dword is one funnel shift of those two dwords (the second above the first).
  const unsigned m0 = kExl3SlotMask0[q];
  const int n = __builtin_popcount(m0), o1 = kExl3SlotOff1[q];
  if (o1 >= 0 && m0 == (1u << n) - 1 && (o & 31) + n == 32 && ((o1 + n) & 31) == 0 &&
      kExl3SlotMask1[q] == (0xffffu & ~m0))
    return decode_window_halves(__builtin_amdgcn_alignbit(w[(o1 + n) >> 5], w[o >> 5], o & 31));
  uint32_t x = win_extract(w, o) & kExl3SlotMask0[q];
  if (kExl3SlotOff1[q] >= 0) x |= win_extract(w, kExl3SlotOff1[q]) & kExl3SlotMask1[q];
  return decode_window_halves(x);
}

// The 32 values of lane j: val[q] = row q of column j (q < 16), row q-16 of column j+8. Both
// halves of a hash lie in [0.125, 2), so their float32 sum is exact and one fp16 add rounds it as
// the reference's float32-sum-then-round does.
__device__ __forceinline__ void lane_decode(const uint32_t (&w)[6], _Float16 (&val)[32]) {
#pragma unroll
  for (int q = 0; q < 32; ++q) {
    const h2 v = __builtin_bit_cast(h2, slot_halves(w, q));
    val[q] = v[0] + v[1];
  }
}

// Load tile `tile`'s chunk for lane j (of the 8 lanes sharing it) and build the lane window.
__device__ __forceinline__ void lane_window(const uint16_t *__restrict__ trellis, int64_t tile, int j,
                                            uint32_t (&w)[6]) {
  const u4 c = *reinterpret_cast<const u4 *>(trellis + tile * 64 + 8 * j);
  w[0] = 0;  // stream dword 4j-2: no window reads it (checked by the generator)
  w[2] = c[0];
  w[3] = c[1];
  w[4] = c[2];
  w[5] = c[3];
  // stream dword 4j-1 = lane j-1's last chunk dword (lane 7's for j = 0)
  const int lane = threadIdx.x & 63;
  const int src = (lane & ~7) | ((lane - 1) & 7);
  w[1] = __shfl(c[3], src, 64);
}

// The lane window from an already loaded chunk c: dword 1 is lane j-1's last chunk dword (lane
// 7's for j = 0), taken by DPP row shifts (lane - 1, or lane + 7 for j = 0).
__device__ __forceinline__ void chunk_window(const u4 c, uint32_t (&w)[6]) {
  const int j = threadIdx.x & 7;
  const int prev = __builtin_amdgcn_update_dpp(0, static_cast<int>(c[3]), DPP_ROW_SHR + 1, 0xf, 0xf, false);
  const int wrap = __builtin_amdgcn_update_dpp(0, static_cast<int>(c[3]), DPP_ROW_SHL + 7, 0xf, 0xf, false);
  w[0] = 0;
  w[1] = static_cast<uint32_t>(j == 0 ? wrap : prev);
  w[2] = c[0];
  w[3] = c[1];
  w[4] = c[2];
  w[5] = c[3];
}

// One wave's LDS tile of decoded values for the matrix-core products: [128 columns][32 k] fp16,
// column stride kExl3WtStride bytes (five 16-B slots: 16 consecutive columns fall on distinct banks)
constexpr int kExl3WtStride = 80;
constexpr int kExl3WtBytes = 128 * kExl3WtStride;  // one wave's tile

// ---- 128-point FWHT across a wave (2 elements per lane) -------------------------------------

// The value of lane ^ M. M = 1, 2: a quad permutation; M = 4, 8: a row shift each way, picked by
// the lane's bit M (both on the VALU); M = 16, 32: ds_bpermute.
template <int M>
__device__ __forceinline__ float xor_lane(float v, bool upper) {
  const int b = __builtin_bit_cast(int, v);
  if constexpr (M == 1) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, b, DPP_QUAD_XOR1, 0xf, 0xf, false));
  } else if constexpr (M == 2) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, b, DPP_QUAD_XOR2, 0xf, 0xf, false));
  } else if constexpr (M == 4 || M == 8) {
    const int hi = __builtin_amdgcn_update_dpp(0, b, DPP_ROW_SHL + M, 0xf, 0xf, false);  // lane + M
    const int lo = __builtin_amdgcn_update_dpp(0, b, DPP_ROW_SHR + M, 0xf, 0xf, false);  // lane - M
    return __builtin_bit_cast(float, upper ? lo : hi);
  } else {
    return __shfl_xor(v, M, 64);
  }
}

template <int M>
__device__ __forceinline__ void fwht_stage(float &a0, float &a1, int lane) {
  const bool upper = (lane & M) != 0;
  const float p0 = xor_lane<M>(a0, upper), p1 = xor_lane<M>(a1, upper);
  a0 = upper ? p0 - a0 : a0 + p0;
  a1 = upper ? p1 - a1 : a1 + p1;
}

__device__ __forceinline__ void fwht128_wave(float &a0, float &a1) {
  const int lane = threadIdx.x & 63;
  float t0 = a0 + a1, t1 = a0 - a1;
  a0 = t0;
  a1 = t1;
  fwht_stage<1>(a0, a1, lane);
  fwht_stage<2>(a0, a1, lane);
  fwht_stage<4>(a0, a1, lane);
  fwht_stage<8>(a0, a1, lane);
  fwht_stage<16>(a0, a1, lane);
  fwht_stage<32>(a0, a1, lane);
}

}  // namespace vybdq
