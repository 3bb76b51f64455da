// Prefill GEMM on GGUF super-block rows (Q4_K, Q5_K, Q6_K, IQ2_S) with fp16 MFMA, gfx950.
//
// Y[m, n] = RS[m, n] + sum_k X[m, k] * W[n, k]   (W: rows of K/256 super-blocks, GGUF layout)
//
// The reference generates one prefill tile kernel per GGUF type and picks it by type id
// (native/host/ridge_decode.vyb:295-302, native/tools/gen_rpf.py:14-96,142-149); here the
// super-block types share one kernel body with a per-type unit decoder.
//
// Tile = 64 X rows x 64 weight rows, K step = one super-block (256 weights) per weight row.
// Each of the 256 threads decodes one 64-weight unit (unit g = tid & 3 of weight row tid >> 2) per
// step with the loads of the decode GEMV (kquant_dev.h: load_unit_kq, exact dword windows), into
// fp16 in LDS: every weight is computed exactly as the decode gate does (float32, one rounding,
// then one rounding to fp16: vybdq_dequant's F16 output). X chunks of 8 are converted to fp16
// into LDS. Each wave owns 16 of the 64 columns and runs v_mfma_f32_16x16x32_f16 over the four
// 16-row fragments. The next step's weight dwords and X chunks are loaded into registers before
// the MFMAs of the current step; the barriers carry no memory fence (the release fence of
// __syncthreads() would wait for those loads), only an explicit wait for this wave's LDS stores.
// Two workgroups share a CU (67.6 KB of LDS each). Units are ordered m-tile fastest, so the
// m-tiles that decode one weight tile run side by side and read it through the same L2.
// X is converted to fp16: activations must stay below 65504 in magnitude.
#include "gemv_dev.h"

#include <type_traits>

namespace vybdq {

constexpr int kKqBM = 64, kKqBN = 64, kKqBK = 256;
constexpr int kKqLda = kKqBK + 8;  // fp16 row stride in LDS (16-B pad: rows start on distinct banks)

typedef _Float16 kh8 __attribute__((ext_vector_type(8)));

struct KqArgs {
  const uint8_t *W;
  int64_t rowbytes;
  const void *X;
  int M, N, S;  // S: super-blocks per row (K / 256)
  int m_tiles;
  void *Y;
  int ydt;
  int64_t ldy;
  const void *RS;
};

template <int FMT> struct KqSb;
template <> struct KqSb<FMT_Q4_K> { static constexpr int BYTES = 144; };
template <> struct KqSb<FMT_Q5_K> { static constexpr int BYTES = 176; };
template <> struct KqSb<FMT_Q6_K> { static constexpr int BYTES = 210; };
template <> struct KqSb<FMT_IQ2_S> { static constexpr int BYTES = 82; };

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  return __builtin_bit_cast(uint32_t, h2{static_cast<_Float16>(a), static_cast<_Float16>(b)});
}

// 32 fp16 (16 packed pairs) -> LDS at dst (16-byte aligned)
__device__ __forceinline__ void store_run32(_Float16 *dst, const uint32_t (&v)[16]) {
  u4 *p = reinterpret_cast<u4 *>(dst);
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = u4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
}

// Decode unit g (64 weights) of the super-block whose windows dw holds into the weight row `row`
// of the LDS tile (element e of the super-block at row[e]).
template <int FMT>
__device__ __forceinline__ void kq_unit_to_lds(const uint32_t (&dw)[Fmt<FMT>::PAIR_DWORDS], int g, _Float16 *row) {
  if constexpr (FMT == FMT_Q4_K || FMT == FMT_Q5_K) {
    // sub-blocks 2g (low nibbles of qs[32g..]) and 2g+1 (high nibbles): elements 64g .. 64g+63;
    // w = d*sc*q - dmin*m as the decode gate computes it (one fma)
    constexpr int QS = FMT == FMT_Q4_K ? 4 : 12;
    const float d = half_bits_to_f32(dw[0] & 0xffffu);
    const float dmin = half_bits_to_f32(dw[0] >> 16);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float sc, mn;
      scale_min_k4(dw[1], dw[2], dw[3], 2 * g + h, sc, mn);
      const float ds = d * sc, dm = dmin * mn;
      uint32_t out[16];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        uint32_t v = h == 0 ? (dw[QS + t] & 0x0F0F0F0Fu) : ((dw[QS + t] >> 4) & 0x0F0F0F0Fu);
        if constexpr (FMT == FMT_Q5_K) v |= ((dw[4 + t] >> (2 * g + h)) & 0x01010101u) << 4;
        float w[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) w[b] = fmaf(ds, static_cast<float>((v >> (8 * b)) & 0xffu), -dm);
        out[2 * t] = pack_h2(w[0], w[1]);
        out[2 * t + 1] = pack_h2(w[2], w[3]);
      }
      store_run32(row + 64 * g + 32 * h, out);
    }
  } else if constexpr (FMT == FMT_Q6_K) {
    // unit g = (half hf, part): low nibbles of ql[64hf + 32part ..] are elements
    // 128hf + 32part + l, high nibbles 128hf + 64 + 32part + l; w = d*sc*(q - 32), exact in f32
    const int hf = g >> 1, part = g & 1;
    const uint32_t sh = dw[22];
    uint32_t ql[8], qh[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      ql[t] = __builtin_amdgcn_alignbit(dw[t + 1], dw[t], sh);
      qh[t] = __builtin_amdgcn_alignbit(dw[9 + t + 1], dw[9 + t], sh);
    }
    const uint32_t sc0 = __builtin_amdgcn_alignbit(dw[19], dw[18], sh);  // scales[8hf + 0..3]
    const uint32_t sc1 = __builtin_amdgcn_alignbit(dw[20], dw[19], sh);  // scales[8hf + 4..7]
    const float d = half_bits_to_f32(dw[21]);
#pragma unroll
    for (int nh = 0; nh < 2; ++nh) {
      const int hs = nh == 0 ? 2 * part : 4 + 2 * part;
      const uint32_t scw = nh == 0 ? sc0 : sc1;
      const float ds0 = d * static_cast<float>(static_cast<int8_t>(__builtin_amdgcn_ubfe(scw, 16 * part, 8)));
      const float ds1 = d * static_cast<float>(static_cast<int8_t>(__builtin_amdgcn_ubfe(scw, 16 * part + 8, 8)));
      uint32_t out[16];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t v = (nh == 0 ? (ql[t] & 0x0F0F0F0Fu) : ((ql[t] >> 4) & 0x0F0F0F0Fu)) |
                           (((qh[t] >> hs) & 0x03030303u) << 4);
        const float ds = t < 4 ? ds0 : ds1;  // elements 4t .. 4t+3: scale of the 16-element half
        float w[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) w[b] = ds * static_cast<float>(static_cast<int>((v >> (8 * b)) & 0xffu) - 32);
        out[2 * t] = pack_h2(w[0], w[1]);
        out[2 * t + 1] = pack_h2(w[2], w[3]);
      }
      store_run32(row + 128 * hf + 64 * nh + 32 * part, out);
    }
  } else {
    // IQ2_S unit g = groups 8g .. 8g+7 of 8 weights = elements 64g .. 64g+63; group l: grid entry
    // qs | 2 qh bits << 8, sign byte, scale d * (0.5 + 4-bit) / 4 per 16 weights (exact in f32)
    const uint32_t sh = dw[9];
    const uint32_t ix[2] = {__builtin_amdgcn_alignbit(dw[1], dw[0], sh), __builtin_amdgcn_alignbit(dw[2], dw[1], sh)};
    const uint32_t sg[2] = {__builtin_amdgcn_alignbit(dw[4], dw[3], sh), __builtin_amdgcn_alignbit(dw[5], dw[4], sh)};
    const float d = half_bits_to_f32(dw[8]) * 0.25f;
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      uint32_t out[16];
#pragma unroll
      for (int l2 = 0; l2 < 4; ++l2) {
        const uint32_t idx = __builtin_amdgcn_ubfe(ix[hb], 8 * l2, 8) | (__builtin_amdgcn_ubfe(dw[6], 8 * hb + 2 * l2, 2) << 8);
        const unsigned long long e = kIq2sGrid[idx];
        const uint32_t sgn = __builtin_amdgcn_ubfe(sg[hb], 8 * l2, 8);
        const float dl = d * (0.5f + static_cast<float>(__builtin_amdgcn_ubfe(dw[7], 8 * hb + 4 * (l2 >> 1), 4)));
        float w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float v = dl * static_cast<float>(static_cast<uint32_t>(e >> (8 * j)) & 0xffu);
          w[j] = ((sgn >> j) & 1u) ? -v : v;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) out[4 * l2 + j] = pack_h2(w[2 * j], w[2 * j + 1]);
      }
      store_run32(row + 64 * g + 32 * hb, out);
    }
  }
}

// 8 consecutive X elements (row offset off) -> 8 fp16 in a u4
template <int XDT> struct KqX { u4 r; };
template <> struct KqX<VYBDQ_F32> { u4 r[2]; };

template <int XDT>
__device__ __forceinline__ void kq_x_load(const void *X, int64_t off, KqX<XDT> &c) {
  if constexpr (XDT == VYBDQ_F32) {
    const u4 *p = reinterpret_cast<const u4 *>(static_cast<const float *>(X) + off);
    c.r[0] = p[0];
    c.r[1] = p[1];
  } else {
    c.r = *reinterpret_cast<const u4 *>(static_cast<const uint16_t *>(X) + off);
  }
}

template <int XDT>
__device__ __forceinline__ u4 kq_x_f16(const KqX<XDT> &c) {
  u4 o;
  if constexpr (XDT == VYBDQ_F16) {
    o = c.r;
  } else if constexpr (XDT == VYBDQ_BF16) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t v = c.r[j];
      o[j] = pack_h2(__uint_as_float(v << 16), __uint_as_float(v & 0xffff0000u));
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u4 &s = c.r[j >> 1];
      const uint32_t a = s[2 * (j & 1)], b = s[2 * (j & 1) + 1];
      o[j] = pack_h2(__uint_as_float(a), __uint_as_float(b));
    }
  }
  return o;
}

// One output tile (m-tile mt, n-tile nt); every thread of the workgroup calls it.
template <int FMT, int XDT>
__device__ __forceinline__ void kq_tile(const KqArgs &a, int mt, int nt, _Float16 *As, _Float16 *Bs) {
  constexpr int PD = Fmt<FMT>::PAIR_DWORDS;
  constexpr int XC = kKqBM * kKqBK / 8 / 256;  // X chunks of 8 per thread per step
  const int row0 = mt * kKqBM;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

  // decode task: weight row br of the tile, unit g of each super-block
  const int br = tid >> 2, g = tid & 3;
  const uint8_t *wrow = a.W + static_cast<int64_t>(nt * kKqBN + br) * a.rowbytes;
  // X task: chunk c = tid + 256 i: tile row c >> 5, k offset 8 (c & 31) within the step; rows
  // past M read row M - 1 (they feed only outputs that are never stored)
  int64_t xoff[XC];
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = tid + 256 * i;
    int r = row0 + (c >> 5);
    r = r < a.M ? r : a.M - 1;
    xoff[i] = static_cast<int64_t>(r) * a.S * kKqBK + 8 * (c & 31);
  }

  f4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = f4{0.f, 0.f, 0.f, 0.f};

  uint32_t dw[PD];
  KqX<XDT> xr[XC];
  load_unit_kq<FMT>(wrow, g, dw);
#pragma unroll
  for (int i = 0; i < XC; ++i) kq_x_load<XDT>(a.X, xoff[i], xr[i]);

  auto bar = [] {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS accesses are done
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
  };

  for (int s = 0; s < a.S; ++s) {
    kq_unit_to_lds<FMT>(dw, g, Bs + br * kKqLda);
#pragma unroll
    for (int i = 0; i < XC; ++i) {
      const int c = tid + 256 * i;
      *reinterpret_cast<u4 *>(As + (c >> 5) * kKqLda + 8 * (c & 31)) = kq_x_f16<XDT>(xr[i]);
    }
    if (s + 1 < a.S) {  // the next step's loads run under this step's MFMAs
      load_unit_kq<FMT>(wrow, 4 * (s + 1) + g, dw);
#pragma unroll
      for (int i = 0; i < XC; ++i) kq_x_load<XDT>(a.X, xoff[i] + static_cast<int64_t>(s + 1) * kKqBK, xr[i]);
    }
    bar();
#pragma unroll
    for (int kk = 0; kk < kKqBK / 32; ++kk) {
      const kh8 bf = *reinterpret_cast<const kh8 *>(Bs + (16 * wave + (lane & 15)) * kKqLda + 32 * kk + 8 * (lane >> 4));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const kh8 af = *reinterpret_cast<const kh8 *>(As + (16 * i + (lane & 15)) * kKqLda + 32 * kk + 8 * (lane >> 4));
        acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf, acc[i], 0, 0, 0);
      }
    }
    bar();
  }

  // acc[i][r] = C[row0 + 16 i + 4 (lane >> 4) + r][nt * 64 + 16 wave + (lane & 15)]
  const int64_t n = static_cast<int64_t>(nt) * kKqBN + 16 * wave + (lane & 15);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = row0 + 16 * i + 4 * (lane >> 4) + r;
      if (m >= a.M) continue;
      const int64_t idx = static_cast<int64_t>(m) * a.ldy + n;
      switch (a.ydt) {
        case VYBDQ_F32: store_elem<VYBDQ_F32>(a.Y, a.RS, idx, acc[i][r]); break;
        case VYBDQ_F16: store_elem<VYBDQ_F16>(a.Y, a.RS, idx, acc[i][r]); break;
        case VYBDQ_BF16: store_elem<VYBDQ_BF16>(a.Y, a.RS, idx, acc[i][r]); break;
        default: store_elem<VYBDQ_F64>(a.Y, a.RS, idx, acc[i][r]); break;
      }
    }
}

template <int FMT, int XDT>
__global__ void __launch_bounds__(256, 2) k_kq_gemm(KqArgs a) {
  __shared__ __attribute__((aligned(16))) _Float16 As[kKqBM * kKqLda];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[kKqBN * kKqLda];
  kq_tile<FMT, XDT>(a, blockIdx.x % a.m_tiles, blockIdx.x / a.m_tiles, As, Bs);
}

// The reference's set_gemm block (W@0 X@8 Y@16 S@24 N@32 K@40 LDY@48 RS@56; LDY >= 0: Y f64 of
// row stride LDY with the f64 residual RS, LDY < 0: Y f32 of row stride -LDY), every word read here
// when the launch runs; a persistent grid walks the tiles. Invalid words: nothing is written and
// bit 4 of *status is set.
template <int FMT, int XDT>
__global__ void __launch_bounds__(256, 2) k_kq_gemm_pb(const int64_t *__restrict__ pb, uint32_t *__restrict__ status) {
  __shared__ __attribute__((aligned(16))) _Float16 As[kKqBM * kKqLda];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[kKqBN * kKqLda];
  const int64_t W = pb[0], X = pb[1], Y = pb[2], M = pb[3], N = pb[4], K = pb[5], LDY = pb[6], RS = pb[7];
  const int64_t ldy = LDY < 0 ? -LDY : LDY;
  const bool ok = W && X && Y && M >= 1 && M < (1 << 24) && N >= 64 && N % 64 == 0 && N < (1 << 24) && K >= 256 &&
                  K % 256 == 0 && K < (1 << 24) && ldy >= N && (W & 3) == 0 && (X & 15) == 0;
  if (!ok) {
    if (blockIdx.x == 0 && threadIdx.x == 0) __hip_atomic_fetch_or(status, 4u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  KqArgs a{};
  a.W = gptr<const uint8_t>(W);
  a.S = static_cast<int>(K / 256);
  a.rowbytes = static_cast<int64_t>(a.S) * KqSb<FMT>::BYTES;
  a.X = gptr<const void>(X);
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.m_tiles = static_cast<int>((M + kKqBM - 1) / kKqBM);
  a.Y = gptr<void>(Y);
  a.ydt = LDY < 0 ? VYBDQ_F32 : VYBDQ_F64;
  a.ldy = ldy;
  a.RS = LDY < 0 ? nullptr : gptr<const void>(RS);
  const int units = a.m_tiles * (a.N / kKqBN);
  for (int u = blockIdx.x; u < units; u += gridDim.x) {
    kq_tile<FMT, XDT>(a, u % a.m_tiles, u / a.m_tiles, As, Bs);
    __builtin_amdgcn_s_barrier();  // the next tile's first LDS stores wait for this tile's last reads
  }
}

template <int FMT>
static int kq_launch(KqArgs &a, int xdt, hipStream_t s) {
  const unsigned grid = static_cast<unsigned>(a.m_tiles) * static_cast<unsigned>(a.N / kKqBN);
  VYBDQ_DISPATCH_IN(xdt, XDT, hipLaunchKernelGGL((k_kq_gemm<FMT, XDT>), dim3(grid), dim3(256), 0, s, a));
  return check_launch("super-block gemm");
}

template <int FMT>
static int kq_pb_launch(int xdt, const int64_t *pb, uint32_t *status, hipStream_t s) {
  const unsigned grid = static_cast<unsigned>(2 * device_cu_count());
  if (xdt == VYBDQ_F16) hipLaunchKernelGGL((k_kq_gemm_pb<FMT, VYBDQ_F16>), dim3(grid), dim3(256), 0, s, pb, status);
  else hipLaunchKernelGGL((k_kq_gemm_pb<FMT, VYBDQ_F32>), dim3(grid), dim3(256), 0, s, pb, status);
  return check_launch("p-block super-block gemm");
}

// The GEMM kind of vybdq_launch_pblock for wtype 12, 13, 14, 22 (pblock.hip); xdt F32 or F16.
int kq_gemm_pblock(int wtype, int xdt, const int64_t *pb, uint32_t *status, hipStream_t s) {
  switch (wtype) {
    case 12: return kq_pb_launch<FMT_Q4_K>(xdt, pb, status, s);
    case 13: return kq_pb_launch<FMT_Q5_K>(xdt, pb, status, s);
    case 14: return kq_pb_launch<FMT_Q6_K>(xdt, pb, status, s);
    default: return kq_pb_launch<FMT_IQ2_S>(xdt, pb, status, s);
  }
}

// Called by vybdq_gemm for wtype 12, 13, 14, 22 after its argument checks (K % 256 == 0,
// N % 64 == 0, W 4-byte aligned, X 16-byte aligned).
int kq_gemm(int wtype, const void *W, const void *X, int xdt, void *Y, int ydt, int64_t M, int64_t N, int64_t K,
            int64_t ldy, const void *RS, hipStream_t s) {
  KqArgs a{};
  a.W = static_cast<const uint8_t *>(W);
  a.X = X;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.S = static_cast<int>(K / 256);
  a.m_tiles = static_cast<int>((M + kKqBM - 1) / kKqBM);
  a.Y = Y;
  a.ydt = ydt;
  a.ldy = ldy;
  a.RS = RS;
  switch (wtype) {
    case 12: a.rowbytes = a.S * KqSb<FMT_Q4_K>::BYTES; return kq_launch<FMT_Q4_K>(a, xdt, s);
    case 13: a.rowbytes = a.S * KqSb<FMT_Q5_K>::BYTES; return kq_launch<FMT_Q5_K>(a, xdt, s);
    case 14: a.rowbytes = a.S * KqSb<FMT_Q6_K>::BYTES; return kq_launch<FMT_Q6_K>(a, xdt, s);
    default: a.rowbytes = a.S * KqSb<FMT_IQ2_S>::BYTES; return kq_launch<FMT_IQ2_S>(a, xdt, s);
  }
}

}  // namespace vybdq
