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

#include <cstdlib>
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

// Decode run h (0 or 1: 32 weights) of unit g (64 weights) of the super-block whose windows dw
// holds into 32 fp16 at dst (16-byte aligned); run_elem<FMT>(g, h) is the super-block element of
// dst[0]. Every weight is computed exactly as the decode gate does (float32, one rounding, then
// one rounding to fp16).
template <int FMT>
__device__ __forceinline__ int run_elem(int g, int h) {
  if constexpr (FMT == FMT_Q6_K) return 128 * (g >> 1) + 64 * h + 32 * (g & 1);
  else return 64 * g + 32 * h;
}

template <int FMT>
__device__ __forceinline__ void kq_run_to_lds(const uint32_t (&dw)[Fmt<FMT>::PAIR_DWORDS], int g, int h, _Float16 *dst) {
  uint32_t out[16];
  if constexpr (FMT == FMT_Q4_K || FMT == FMT_Q5_K) {
    // sub-block 2g + h (h = 0: low nibbles of qs[32g..], h = 1: high nibbles);
    // w = d*sc*q - dmin*m as the decode gate computes it (one fma)
    constexpr int QS = FMT == FMT_Q4_K ? 4 : 12;
    const float d = half_bits_to_f32(dw[0] & 0xffffu);
    const float dmin = half_bits_to_f32(dw[0] >> 16);
    float sc, mn;
    scale_min_k4(dw[1], dw[2], dw[3], 2 * g + h, sc, mn);
    const float ds = d * sc, dm = dmin * mn;
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
  } else if constexpr (FMT == FMT_Q6_K) {
    // unit g = (half hf, part): low nibbles of ql[64hf + 32part ..] (h = 0) are elements
    // 128hf + 32part + l, high nibbles (h = 1) 128hf + 64 + 32part + l; w = d*sc*(q - 32), exact
    // in f32
    const int part = g & 1;
    const uint32_t sh = dw[22];
    const int hs = h == 0 ? 2 * part : 4 + 2 * part;
    const uint32_t scw = __builtin_amdgcn_alignbit(dw[19 + h], dw[18 + h], sh);  // scales[8hf + 4h ..]
    const float d = half_bits_to_f32(dw[21]);
    const float ds0 = d * static_cast<float>(static_cast<int8_t>(__builtin_amdgcn_ubfe(scw, 16 * part, 8)));
    const float ds1 = d * static_cast<float>(static_cast<int8_t>(__builtin_amdgcn_ubfe(scw, 16 * part + 8, 8)));
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const uint32_t ql = __builtin_amdgcn_alignbit(dw[t + 1], dw[t], sh);
      const uint32_t qh = __builtin_amdgcn_alignbit(dw[9 + t + 1], dw[9 + t], sh);
      const uint32_t v = (h == 0 ? (ql & 0x0F0F0F0Fu) : ((ql >> 4) & 0x0F0F0F0Fu)) | (((qh >> hs) & 0x03030303u) << 4);
      const float ds = t < 4 ? ds0 : ds1;  // elements 4t .. 4t+3: scale of the 16-element half
      float w[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) w[b] = ds * static_cast<float>(static_cast<int>((v >> (8 * b)) & 0xffu) - 32);
      out[2 * t] = pack_h2(w[0], w[1]);
      out[2 * t + 1] = pack_h2(w[2], w[3]);
    }
  } else {
    // IQ2_S unit g = groups 8g .. 8g+7 of 8 weights = elements 64g .. 64g+63, run h = groups
    // 8g + 4h ..; group l: grid entry qs | 2 qh bits << 8, sign byte, scale d * (0.5 + 4-bit) / 4
    // per 16 weights (exact in f32)
    const uint32_t sh = dw[9];
    const uint32_t ix = __builtin_amdgcn_alignbit(dw[1 + h], dw[h], sh);
    const uint32_t sg = __builtin_amdgcn_alignbit(dw[4 + h], dw[3 + h], sh);
    const float d = half_bits_to_f32(dw[8]) * 0.25f;
#pragma unroll
    for (int l2 = 0; l2 < 4; ++l2) {
      const uint32_t idx = __builtin_amdgcn_ubfe(ix, 8 * l2, 8) | (__builtin_amdgcn_ubfe(dw[6], 8 * h + 2 * l2, 2) << 8);
      const unsigned long long e = kIq2sGrid[idx];
      const uint32_t sgn = __builtin_amdgcn_ubfe(sg, 8 * l2, 8);
      const float dl = d * (0.5f + static_cast<float>(__builtin_amdgcn_ubfe(dw[7], 8 * h + 4 * (l2 >> 1), 4)));
      float w[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float v = dl * static_cast<float>(static_cast<uint32_t>(e >> (8 * j)) & 0xffu);
        w[j] = ((sgn >> j) & 1u) ? -v : v;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) out[4 * l2 + j] = pack_h2(w[2 * j], w[2 * j + 1]);
    }
  }
  store_run32(dst, out);
}

// Decode unit g (64 weights) of the super-block whose windows dw holds into the weight row `row`
// of the LDS tile (element e of the super-block at row[e]).
template <int FMT>
__device__ __forceinline__ void kq_unit_to_lds(const uint32_t (&dw)[Fmt<FMT>::PAIR_DWORDS], int g, _Float16 *row) {
#pragma unroll
  for (int h = 0; h < 2; ++h) kq_run_to_lds<FMT>(dw, g, h, row + run_elem<FMT>(g, h));
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

// ---- 128-row tiles over fp16 X (Q6_K and IQ2_S from 96 rows; Q4_K and Q5_K from 96 rows with
// bf16 X and no workspace) -------------------------------------------------------------------
//
// Tile = 128 X rows x 64 weight rows, K step = 128 (half a super-block = four 32-weight runs).
// Four waves in a 2 x 2 grid each own 64 rows x 32 columns (4 x 2 accumulator fragments), so per
// 32-k slice a wave reads 6 operand fragments from LDS for 8 MFMAs (the 64-row tile above reads 5
// for 4); each weight is decoded once per 128 X rows. Thread t decodes run t % 4 of weight row
// t / 4; run-dependent choices are shift amounts and address offsets (no per-lane indexing of
// register arrays), and every address is a wave-uniform base plus a per-lane 32-bit offset that
// does not change from step to step. The run's
// weights are formed in fp16 arithmetic: Q6_K as fp16(d·sc) × (q − 32) (q − 32 exact from the
// 0x64vv bit pattern), IQ2_S as the grid's magnitude bytes (one 8-byte grid row per 8 weights)
// × fp16(d·(0.5 + s)/4) with the sign bits applied:
// each weight differs from the decode's fp16 value by at most the rounding of the scale and one
// product rounding. X is fp16: the caller's, or the workspace copy that x_rows_to_f16 made with
// a power-of-two scale per row (xscale), multiplied back into the outputs. Split K: each split
// writes f32 partials [split][M][N] to the workspace and k_kq_reduce sums them in split order and
// applies the epilogue. Three workgroups share a CU (52 KB of LDS each).
constexpr int kK2BM = 128, kK2BN = 64, kK2BK = 128;
constexpr int kK2Lda = kK2BK + 8;  // fp16 row stride in LDS (16-B pad)

struct Kq2Args {
  const uint8_t *W;      // weight rows, rowbytes apart
  uint32_t rowbytes;
  const _Float16 *X;     // [M][K] fp16
  const float *xscale;   // per X row (null: 1)
  int M, N, K;
  int S2;                // 128-k steps per row (K / 128)
  int m_tiles, n_tiles, splits, sps;
  int xcd;               // 1: workgroups of one XCD take consecutive units
  void *Y;
  int ydt;
  int64_t ldy;
  const void *RS;
  float *part;           // splits > 1: [splits][M][N] f32 partials
};

template <int FMT> struct K2Run;
// Q4_K / Q5_K run (sub-block j): the 16-byte head (d, dmin, 12 scale bytes), Q5_K the 32 high-bit
// bytes, and the 32 nibble bytes of qs[32 (j / 2) ..]
template <> struct K2Run<FMT_Q4_K> { static constexpr int DW = 12; };
template <> struct K2Run<FMT_Q5_K> { static constexpr int DW = 20; };
// IQ2_S run (sub-block j): its 4 grid-index bytes and 4 sign bytes as 2-dword windows, qh[j],
// scales[j], d
template <> struct K2Run<FMT_IQ2_S> { static constexpr int DW = 7; };

__device__ __forceinline__ uint32_t ld_u32(const uint8_t *base, uint32_t off) {
  return *reinterpret_cast<const uint32_t *>(base + off);
}
__device__ __forceinline__ uint32_t ld_u16(const uint8_t *base, uint32_t off) {
  return *reinterpret_cast<const uint16_t *>(base + off);
}

// Loads of run r of half hf for the super-block at sbase + o (sbase + 64 hf wave-uniform; o and
// the run's offsets within the super-block per lane, 32-bit, so every load is a scalar base plus
// a vector offset). Q6_K does not come here: its four row lanes share the super-block's loads
// (kq2_tile).
template <int FMT>
__device__ __forceinline__ void k2_load_run(const uint8_t *sbase, uint32_t o, int hf, int r,
                                            uint32_t (&d)[K2Run<FMT>::DW]) {
  static_assert(FMT != FMT_Q6_K, "Q6_K runs are loaded by the quad path of kq2_tile");
  if constexpr (FMT == FMT_Q4_K || FMT == FMT_Q5_K) {
    // 144 / 176-byte super-blocks keep every window dword aligned
    constexpr int QS = FMT == FMT_Q4_K ? 16 : 48;
    const uint32_t j = 4 * static_cast<uint32_t>(hf) + static_cast<uint32_t>(r);
    const u4a4 h = *reinterpret_cast<const u4a4 *>(sbase + o);
    const uint32_t qo = o + QS + 32 * (j >> 1);
    const u4a4 q0 = *reinterpret_cast<const u4a4 *>(sbase + qo), q1 = *reinterpret_cast<const u4a4 *>(sbase + qo + 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      d[i] = h[i];
      d[K2Run<FMT>::DW - 8 + i] = q0[i];
      d[K2Run<FMT>::DW - 4 + i] = q1[i];
    }
    if constexpr (FMT == FMT_Q5_K) {
      const u4a4 b0 = *reinterpret_cast<const u4a4 *>(sbase + o + 16), b1 = *reinterpret_cast<const u4a4 *>(sbase + o + 32);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        d[4 + i] = b0[i];
        d[8 + i] = b1[i];
      }
    }
  } else {
    // sub-block j = 4 hf + r; the index and sign windows start 2 bytes past o
    const uint32_t of = ((o + 2) & ~3u) + 4 * static_cast<uint32_t>(r);
    const uint8_t *ix = sbase + 16 * hf, *sg = sbase + 32 + 16 * hf;
    d[0] = ld_u32(ix, of);
    d[1] = ld_u32(ix, of + 4);
    d[2] = ld_u32(sg, of);
    d[3] = ld_u32(sg, of + 4);
    d[4] = *(sbase + 66 + 4 * hf + o + r);  // qh of sub-block j
    d[5] = *(sbase + 74 + 4 * hf + o + r);  // its two 4-bit scales
    d[6] = ld_u16(sbase, o);                 // d
  }
}

// 32 fp16 weights of the run (as 16 packed pairs) from its loads; sh = 16 when the lane's windows
// start 2 bytes past the dword they were loaded from
template <int FMT>
__device__ __forceinline__ void k2_decode_run(const uint32_t (&d)[K2Run<FMT>::DW], uint32_t sh, int r,
                                              uint32_t (&out)[16]) {
  static_assert(FMT != FMT_Q6_K, "Q6_K runs are decoded by the quad path of kq2_tile");
  if constexpr (FMT == FMT_Q4_K || FMT == FMT_Q5_K) {
    // run r of half hf is sub-block j = 4 hf + r; the caller passes r + 4 hf. w = fp16(d sc) q -
    // fp16(dmin m) by one packed fma per pair (q exact from the 0x64qq bit pattern)
    const uint32_t j = static_cast<uint32_t>(r);
    float sc, mn;
    scale_min_k4(d[1], d[2], d[3], static_cast<int>(j), sc, mn);
    const _Float16 dsh = static_cast<_Float16>(half_bits_to_f32(d[0] & 0xffffu) * sc);
    const _Float16 dmh = static_cast<_Float16>(-(half_bits_to_f32(d[0] >> 16) * mn));
    const h2 ds = {dsh, dsh}, dm = {dmh, dmh};
    const h2 bias = {static_cast<_Float16>(-1024.0f), static_cast<_Float16>(-1024.0f)};
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      uint32_t v = (d[K2Run<FMT>::DW - 8 + t] >> (4 * (j & 1u))) & 0x0F0F0F0Fu;
      if constexpr (FMT == FMT_Q5_K) v |= ((d[4 + t] >> j) & 0x01010101u) << 4;
      const h2 p0 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u)) + bias;
      const h2 p1 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u)) + bias;
      out[2 * t] = __builtin_bit_cast(uint32_t, p0 * ds + dm);
      out[2 * t + 1] = __builtin_bit_cast(uint32_t, p1 * ds + dm);
    }
  } else {
    const uint32_t ix = __builtin_amdgcn_alignbit(d[1], d[0], sh);
    const uint32_t sg = __builtin_amdgcn_alignbit(d[3], d[2], sh);
    const float dd = half_bits_to_f32(d[6]) * 0.25f;
    const h2 bias = {static_cast<_Float16>(-1024.0f), static_cast<_Float16>(-1024.0f)};
#pragma unroll
    for (int l2 = 0; l2 < 4; ++l2) {
      const uint32_t idx = __builtin_amdgcn_ubfe(ix, 8 * l2, 8) | (__builtin_amdgcn_ubfe(d[4], 2 * l2, 2) << 8);
      const unsigned long long e = kIq2sGrid[idx];  // 8 magnitude bytes
      const uint32_t e0 = static_cast<uint32_t>(e), e1 = static_cast<uint32_t>(e >> 32);
      const uint32_t sgn = __builtin_amdgcn_ubfe(sg, 8 * l2, 8);
      const float dl = dd * (0.5f + static_cast<float>(__builtin_amdgcn_ubfe(d[5], 4 * (l2 >> 1), 4)));
      const h2 dh = {static_cast<_Float16>(dl), static_cast<_Float16>(dl)};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        // bytes -> fp16 1024 + b, minus 1024 (exact), times the scale; sign bits 2k, 2k+1 of the
        // sign byte -> bits 15, 31
        const uint32_t src = k < 2 ? e0 : e1;
        const h2 p = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, src, k & 1 ? 0x04030402u : 0x04010400u));
        const uint32_t m = ((sgn >> (2 * k)) & 1u) << 15 | ((sgn >> (2 * k + 1)) & 1u) << 31;
        out[4 * l2 + k] = __builtin_bit_cast(uint32_t, (p + bias) * dh) ^ m;
      }
    }
  }
}

// 8 bf16 -> 8 fp16 (as they are: |x| < 65504)
__device__ __forceinline__ u4 bf16x8_to_f16(const u4 &v) {
  u4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) o[j] = pack_h2(__uint_as_float(v[j] << 16), __uint_as_float(v[j] & 0xffff0000u));
  return o;
}

// One unit u (split, m-tile, weight tile) of the 128-row tiling; every thread of the workgroup
// calls it. XB: X is bf16, converted to fp16 as it is staged into LDS (vybdq_gemm without a
// workspace; |x| < 65504).
template <int FMT, bool XB = false>
__device__ __forceinline__ void kq2_tile(const Kq2Args &a, int u, _Float16 *As, _Float16 *Bs) {
  const int mn_tiles = a.m_tiles * a.n_tiles;
  const int split = u / mn_tiles;
  const int mn = u - split * mn_tiles;
  // weight tiles fastest: the workgroups of one XCD share one 128-row X tile (K/splits x 256 B,
  // held in the XCD's L2) and stream the weight tiles; X is read 4 x as many bytes per step as
  // the weights
  const int nt = mn % a.n_tiles, mt = mn / a.n_tiles;
  const int s0 = split * a.sps;
  const int s1 = s0 + a.sps < a.S2 ? s0 + a.sps : a.S2;
  const int row0 = mt * kK2BM;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave >> 1, wc = wave & 1;

  // decode task: run `run` of the step for weight row `brow`: the four runs of a row sit in four
  // adjacent lanes, so a weight load instruction touches 16 rows (one wave per run, 64 rows per
  // instruction, measured 13-25% slower: the address unit is busy for the whole kernel and
  // serves a load by the cache lines it touches)
  const int brow = tid >> 2, run = tid & 3;
  const uint8_t *wtile = a.W + static_cast<int64_t>(nt) * kK2BN * a.rowbytes;
  const uint32_t wlane = static_cast<uint32_t>(brow) * a.rowbytes;
  constexpr int SB = KqSb<FMT>::BYTES;
  _Float16 *bdst = Bs + brow * kK2Lda + (FMT == FMT_Q6_K ? 64 * (run & 1) + 32 * (run >> 1) : 32 * run);
  // X task: chunk c = tid + 256 i: tile row c >> 4, k offset 8 (c & 15) (a wave loads 4 rows x
  // 256 contiguous bytes per instruction; fragment-ordered loads of 16 rows x 64 B measured 28%
  // slower); rows past M read row M - 1 (they feed only outputs that are never stored); byte
  // offsets from the tile's first row (128 K fp16 < 2^32 bytes for K < 2^24)
  uint32_t xoff[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = tid + 256 * i;
    int m = row0 + (c >> 4);
    m = m < a.M ? m : a.M - 1;
    xoff[i] = 2u * (static_cast<uint32_t>(m - row0) * static_cast<uint32_t>(a.K) + 8u * static_cast<uint32_t>(c & 15));
  }
  const uint8_t *xb = reinterpret_cast<const uint8_t *>(a.X + static_cast<int64_t>(row0) * a.K);

  f4 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  // one register stage of loads, refilled right after its step's LDS stores (a second stage, two
  // workgroups per CU, measured 5-15% slower)
  u4 xr[8];
  auto load_x = [&](int s) {
    const uint8_t *xs = xb + static_cast<int64_t>(s) * (2 * kK2BK);
#pragma unroll
    for (int i = 0; i < 8; ++i) xr[i] = *reinterpret_cast<const u4 *>(xs + xoff[i]);
  };
  auto bar = [] {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS accesses are done
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
  };
  auto mfma_step = [&] {
    bar();
#pragma unroll
    for (int kk = 0; kk < kK2BK / 32; ++kk) {
      kh8 bf[2];
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bf[j] = *reinterpret_cast<const kh8 *>(Bs + (32 * wc + 16 * j + (lane & 15)) * kK2Lda + 32 * kk + 8 * (lane >> 4));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const kh8 af =
            *reinterpret_cast<const kh8 *>(As + (64 * wr + 16 * i + (lane & 15)) * kK2Lda + 32 * kk + 8 * (lane >> 4));
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[i][j], 0, 0, 0);
      }
    }
    bar();
  };

  if constexpr (FMT == FMT_Q6_K) {
    // The four lanes of a weight row load the row's super-block once per two steps: lane r takes
    // ql[32 r ..] (8 dwords and the next), qh[16 r ..] (4 dwords and the next), and its run's
    // scale pairs of both halves; each step gathers the run's ql / qh windows from the quad by
    // DPP lane moves. Half the load instructions of one run-window set per step.
    uint32_t rq[9], rh[5], rd = 0, rsc[2], sh = 0;
    const uint32_t part = static_cast<uint32_t>(run) >> 1, nh = static_cast<uint32_t>(run) & 1u;
    auto load_sb = [&](int sbi) {
      const uint32_t o = wlane + static_cast<uint32_t>(sbi) * SB;  // this lane's super-block
      const uint32_t of = o & ~3u;
      const uint32_t qo = of + 32 * static_cast<uint32_t>(run), ho = of + 128 + 16 * static_cast<uint32_t>(run);
      const u4a4 a0 = *reinterpret_cast<const u4a4 *>(wtile + qo), a1 = *reinterpret_cast<const u4a4 *>(wtile + qo + 16);
      const u4a4 b0 = *reinterpret_cast<const u4a4 *>(wtile + ho);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rq[i] = a0[i];
        rq[4 + i] = a1[i];
        rh[i] = b0[i];
      }
      rq[8] = ld_u32(wtile, qo + 32);
      rh[4] = ld_u32(wtile, ho + 16);
      rsc[0] = ld_u16(wtile + 192, o + 4 * nh + 2 * part);
      rsc[1] = ld_u16(wtile + 200, o + 4 * nh + 2 * part);
      rd = ld_u16(wtile + 208, o);
      sh = (o & 2) ? 16u : 0u;
    };
    // half HF: the run's ql window is lane 2 HF + part's, its qh window lanes 2 HF and 2 HF + 1's;
    // the window dwords are fetched from the quad as the decode reaches them
    auto stage_q6 = [&](auto hf_c) {
      constexpr int HF = decltype(hf_c)::value;
      constexpr int QL = (2 * HF) | (2 * HF) << 2 | (2 * HF + 1) << 4 | (2 * HF + 1) << 6;
      constexpr int H0 = 0x55 * (2 * HF), H1 = 0x55 * (2 * HF + 1);
      auto qlw = [&](int t) { return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(rq[t]), QL, 0xf, 0xf, false)); };
      auto qhw = [&](int t) {
        return t < 4 ? static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(rh[t]), H0, 0xf, 0xf, false))
                     : static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(rh[t - 4]), H1, 0xf, 0xf, false));
      };
      const uint32_t qls = 4 * nh, qhs = 2 * part + 4 * nh;  // nibble of ql, bit pair of qh
      const float dd = half_bits_to_f32(rd);
      const uint32_t sc = rsc[HF];
      const h2 ds0 = {static_cast<_Float16>(dd * static_cast<float>(static_cast<int8_t>(sc & 0xffu))),
                      static_cast<_Float16>(dd * static_cast<float>(static_cast<int8_t>(sc & 0xffu)))};
      const h2 ds1 = {static_cast<_Float16>(dd * static_cast<float>(static_cast<int8_t>(sc >> 8))),
                      static_cast<_Float16>(dd * static_cast<float>(static_cast<int8_t>(sc >> 8)))};
      const h2 bias = {static_cast<_Float16>(-1056.0f), static_cast<_Float16>(-1056.0f)};
      uint32_t w[16];
      uint32_t l0 = qlw(0), h0 = qhw(0);
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t l1 = qlw(t + 1);
        const uint32_t h1 = t + 1 < 8 ? qhw(t + 1)
                                      : static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(rh[4]), H1, 0xf, 0xf, false));
        const uint32_t ql = __builtin_amdgcn_alignbit(l1, l0, sh) >> qls;
        const uint32_t qh = (__builtin_amdgcn_alignbit(h1, h0, sh) >> qhs) & 0x03030303u;
        const uint32_t v = (ql & 0x0F0F0F0Fu) | (qh << 4);
        const h2 p0 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u));
        const h2 p1 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u));
        const h2 ds = t < 4 ? ds0 : ds1;
        w[2 * t] = __builtin_bit_cast(uint32_t, (p0 + bias) * ds);
        w[2 * t + 1] = __builtin_bit_cast(uint32_t, (p1 + bias) * ds);
        l0 = l1;
        h0 = h1;
      }
      store_run32(bdst, w);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int c = tid + 256 * i;
        *reinterpret_cast<u4 *>(As + (c >> 4) * kK2Lda + 8 * (c & 15)) = XB ? bf16x8_to_f16(xr[i]) : xr[i];
      }
    };
    if (s0 < s1) {
      load_sb(s0 >> 1);
      load_x(s0);
    }
    for (int s = s0; s < s1; ++s) {
      if (s & 1) stage_q6(std::integral_constant<int, 1>{});
      else stage_q6(std::integral_constant<int, 0>{});
      if (s + 1 < s1) {  // these loads run under this step's MFMAs
        if (s & 1) load_sb((s + 1) >> 1);
        load_x(s + 1);
      }
      mfma_step();
    }
  } else {
    constexpr int DW = K2Run<FMT>::DW;
    // the step's decoded run and X chunks -> LDS
    auto stage = [&](const uint32_t (&d)[DW], uint32_t sh, int rr) {
      {
        uint32_t w[16];
        k2_decode_run<FMT>(d, sh, rr, w);
        store_run32(bdst, w);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int c = tid + 256 * i;
        *reinterpret_cast<u4 *>(As + (c >> 4) * kK2Lda + 8 * (c & 15)) = XB ? bf16x8_to_f16(xr[i]) : xr[i];
      }
    };
    uint32_t dw[DW], sh = 0;
    auto load_step = [&](int s) {
      const uint32_t o = wlane + static_cast<uint32_t>(s >> 1) * SB;  // this lane's super-block
      k2_load_run<FMT>(wtile, o, s & 1, run, dw);
      sh = (o & 2) ? 0u : 16u;
      load_x(s);
    };
    if (s0 < s1) load_step(s0);
    for (int s = s0; s < s1; ++s) {
      // Q4_K / Q5_K decode by sub-block index 4 hf + run
      stage(dw, sh, FMT == FMT_IQ2_S ? run : run + 4 * (s & 1));
      if (s + 1 < s1) load_step(s + 1);  // these loads run under this step's MFMAs
      mfma_step();
    }
  }

  // acc[i][j][q] = C[row0 + 64 wr + 16 i + 4 (lane >> 4) + q][64 nt + 32 wc + 16 j + (lane & 15)]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int m = row0 + 64 * wr + 16 * i + 4 * (lane >> 4) + q;
      if (m >= a.M) continue;
      const float xs = a.xscale ? a.xscale[m] : 1.0f;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t n = static_cast<int64_t>(nt) * kK2BN + 32 * wc + 16 * j + (lane & 15);
        if (a.splits > 1) {
          a.part[(static_cast<int64_t>(split) * a.M + m) * a.N + n] = acc[i][j][q];
          continue;
        }
        const int64_t idx = static_cast<int64_t>(m) * a.ldy + n;
        const float v = acc[i][j][q] * xs;
        switch (a.ydt) {
          case VYBDQ_F32: store_elem<VYBDQ_F32>(a.Y, a.RS, idx, v); break;
          case VYBDQ_F16: store_elem<VYBDQ_F16>(a.Y, a.RS, idx, v); break;
          case VYBDQ_BF16: store_elem<VYBDQ_BF16>(a.Y, a.RS, idx, v); break;
          default: store_elem<VYBDQ_F64>(a.Y, a.RS, idx, v); break;
        }
      }
    }
}

template <int FMT, bool XB>
__global__ void __launch_bounds__(256, 3) k_kq_mm(Kq2Args a) {
  __shared__ __attribute__((aligned(16))) _Float16 As[kK2BM * kK2Lda];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[kK2BN * kK2Lda];
  const int units = a.m_tiles * a.n_tiles * a.splits;
  int u = static_cast<int>(blockIdx.x);
  if (a.xcd) u = (u & 7) * (units >> 3) + (u >> 3);  // workgroups are dealt to the 8 XCDs in turn
  kq2_tile<FMT, XB>(a, u, As, Bs);
}

// The reference's set_gemm block with fp16 X (the GEMM_XH kind; see k_kq_gemm_pb for the words)
// on the 128-row tiles: a persistent grid of three workgroups per CU walks the tiles, one split.
template <int FMT>
__global__ void __launch_bounds__(256, 3) k_kq_mm_pb(const int64_t *__restrict__ pb, uint32_t *__restrict__ status) {
  __shared__ __attribute__((aligned(16))) _Float16 As[kK2BM * kK2Lda];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[kK2BN * kK2Lda];
  const int64_t W = pb[0], X = pb[1], Y = pb[2], M = pb[3], N = pb[4], K = pb[5], LDY = pb[6], RS = pb[7];
  const int64_t ldy = LDY < 0 ? -LDY : LDY;
  const bool ok = W && X && Y && M >= 1 && M < (1 << 24) && N >= 64 && N % 64 == 0 && N < (1 << 24) && K >= 256 &&
                  K % 256 == 0 && K < (1 << 24) && ldy >= N && (W & 3) == 0 && (X & 15) == 0;
  if (!ok) {
    if (blockIdx.x == 0 && threadIdx.x == 0) __hip_atomic_fetch_or(status, 4u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  Kq2Args a{};
  a.W = gptr<const uint8_t>(W);
  a.rowbytes = static_cast<uint32_t>(K / 256 * KqSb<FMT>::BYTES);
  a.X = gptr<const _Float16>(X);
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.K = static_cast<int>(K);
  a.S2 = static_cast<int>(K / 128);
  a.m_tiles = static_cast<int>((M + kK2BM - 1) / kK2BM);
  a.n_tiles = static_cast<int>(N / kK2BN);
  a.splits = 1;
  a.sps = a.S2;
  a.Y = gptr<void>(Y);
  a.ydt = LDY < 0 ? VYBDQ_F32 : VYBDQ_F64;
  a.ldy = ldy;
  a.RS = LDY < 0 ? nullptr : gptr<const void>(RS);
  const int units = a.m_tiles * a.n_tiles;
  for (int u = blockIdx.x; u < units; u += gridDim.x) {
    kq2_tile<FMT>(a, u, As, Bs);
    __builtin_amdgcn_s_barrier();  // the next tile's first LDS stores wait for this tile's last reads
  }
}

// Sum of the split partials in split order, times the X row scale, then the epilogue; four
// consecutive columns per thread (N % 64 == 0).
template <int YDT>
__global__ void __launch_bounds__(256) k_kq_reduce(const float *__restrict__ part, int splits, int M, int N,
                                                  const float *__restrict__ xscale, void *Y, int64_t ldy,
                                                  const void *RS) {
  const int64_t mn = static_cast<int64_t>(M) * N;
  const int64_t n4 = mn / 4;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; e < n4;
       e += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t i0 = 4 * e;
    f4 v = *reinterpret_cast<const f4 *>(part + i0);
    for (int sp = 1; sp < splits; ++sp) {
      const f4 w = *reinterpret_cast<const f4 *>(part + sp * mn + i0);
      v = v + w;
    }
    const int64_t m = i0 / N, n = i0 - m * N;
    const float xs = xscale ? xscale[m] : 1.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) store_elem<YDT>(Y, RS, m * ldy + n + q, v[q] * xs);
  }
}

struct Kq2Plan {
  int m_tiles, n_tiles, splits, sps;
  int64_t part_bytes;
};

// K split minimising the busiest CU's time plus the partial traffic (written once, read back
// once). Three workgroups fit a CU; a CU with c workgroups runs them three at a time, and a step
// costs (MI355X, Q6_K at the prefill shapes, in µs per step of the group) 2.98 with three
// resident, 2.19 with two, ~1.7 with one.
static Kq2Plan kq2_plan(int M, int N, int S2, bool allow_split) {
  const int cus = device_cu_count();
  const int m_tiles = (M + kK2BM - 1) / kK2BM, n_tiles = N / kK2BN;
  Kq2Plan best{m_tiles, n_tiles, 1, S2, 0};
  double best_t = -1;
  for (int splits = 1; splits <= (allow_split ? 8 : 1) && splits <= S2; ++splits) {
    const int sps = (S2 + splits - 1) / splits;
    if ((splits - 1) * sps >= S2) continue;
    const int64_t units = static_cast<int64_t>(m_tiles) * n_tiles * splits;
    const int64_t c = (units + cus - 1) / cus;
    const double rem = c % 3 == 0 ? 0.0 : (c % 3 == 2 ? 2.19 : 1.7);
    double t = sps * (static_cast<double>(c / 3) * 2.98 + rem);
    if (splits > 1) t += static_cast<double>(M) * N * 4 * (splits + 1) / 5.0e6 + 3.0;
    if (best_t < 0 || t < best_t - 1e-9) {
      best_t = t;
      best.splits = splits;
      best.sps = sps;
    }
  }
  // tuning / test override: VYBDQ_KQ2_SPLITS=n (ignored when it does not fit the shape)
  if (const char *ov = tuning_env("VYBDQ_KQ2_SPLITS")) {
    const int splits = atoi(ov);
    if (splits >= 1 && splits <= 8 && splits <= S2 && (splits == 1 || allow_split)) {
      const int sps = (S2 + splits - 1) / splits;
      if ((splits - 1) * sps < S2) {
        best.splits = splits;
        best.sps = sps;
      }
    }
  }
  best.part_bytes = best.splits > 1 ? static_cast<int64_t>(best.splits) * M * N * 4 : 0;
  return best;
}

static int64_t kq_align256(int64_t b) { return (b + 255) / 256 * 256; }

// 32-bit byte offsets: X (M K fp16), a weight tile (64 rows)
bool kq2_supported(int wtype, int64_t M, int64_t N, int64_t K) {
  return (wtype == 12 || wtype == 13 || wtype == 14 || wtype == 22) && M >= 96 && M * N < (int64_t(1) << 31) &&
         N % 64 == 0 && K % 256 == 0 && K < (int64_t(1) << 24);
}

// workspace: [split partials][fp16 copy of X][X row scales]
int64_t kq2_workspace_size(int wtype, int64_t M, int64_t N, int64_t K) {
  if (!kq2_supported(wtype, M, N, K)) return 0;
  const Kq2Plan p = kq2_plan(static_cast<int>(M), static_cast<int>(N), static_cast<int>(K / 128), true);
  return kq_align256(p.part_bytes) + kq_align256(M * K * 2) + kq_align256(M * 4);
}

int x_rows_to_f16(const void *X, int xdt, int64_t M, int64_t K, void *xh, float *xscale, hipStream_t s);

template <int FMT>
static int kq2_launch(const Kq2Args &a, bool xb, hipStream_t s) {
  const unsigned grid = static_cast<unsigned>(a.m_tiles) * a.n_tiles * a.splits;
  if (xb) hipLaunchKernelGGL((k_kq_mm<FMT, true>), dim3(grid), dim3(256), 0, s, a);
  else hipLaunchKernelGGL((k_kq_mm<FMT, false>), dim3(grid), dim3(256), 0, s, a);
  return check_launch("super-block gemm (128-row tiles)");
}

// Q6_K / IQ2_S with fp16 or bf16 X, or f32 X with a workspace of kq2_workspace_size bytes. Returns
// 1 when the call does not fit this path (the caller takes the 64-row tiles).
int kq2_gemm(int wtype, const void *W, const void *X, int xdt, void *Y, int ydt, int64_t M, int64_t N, int64_t K,
             int64_t ldy, const void *RS, void *ws, int64_t ws_bytes, hipStream_t s) {
  if (!kq2_supported(wtype, M, N, K)) return 1;
  const int S2 = static_cast<int>(K / 128);
  int64_t need_x = xdt == VYBDQ_F16 ? 0 : kq_align256(M * K * 2) + kq_align256(M * 4);
  // bf16 X without room for its scaled fp16 copy: converted in the tile as it is (|x| < 65504)
  const bool xb = xdt == VYBDQ_BF16 && (!ws || ws_bytes < need_x);
  if (xb) need_x = 0;
  if (need_x && (!ws || ws_bytes < need_x)) return 1;
  Kq2Plan p = kq2_plan(static_cast<int>(M), static_cast<int>(N), S2, ws != nullptr);
  if (p.splits > 1 && ws_bytes < kq_align256(p.part_bytes) + need_x)
    p = kq2_plan(static_cast<int>(M), static_cast<int>(N), S2, false);
  const int64_t xh_off = p.splits > 1 ? kq_align256(p.part_bytes) : 0;
  const float *xscale = nullptr;
  if (need_x) {
    char *base = static_cast<char *>(ws) + xh_off;
    float *sc = reinterpret_cast<float *>(base + kq_align256(M * K * 2));
    const int rc = x_rows_to_f16(X, xdt, M, K, base, sc, s);
    if (rc) return rc;
    X = base;
    xscale = sc;
  }
  Kq2Args a{};
  a.W = static_cast<const uint8_t *>(W);
  a.rowbytes = static_cast<uint32_t>(K / 256 * (wtype == 12   ? KqSb<FMT_Q4_K>::BYTES
                                                  : wtype == 13 ? KqSb<FMT_Q5_K>::BYTES
                                                  : wtype == 14 ? KqSb<FMT_Q6_K>::BYTES
                                                                : KqSb<FMT_IQ2_S>::BYTES));
  a.X = static_cast<const _Float16 *>(X);  // fp16, or bf16 bits when xb
  a.xscale = xscale;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.K = static_cast<int>(K);
  a.S2 = S2;
  a.m_tiles = p.m_tiles;
  a.n_tiles = p.n_tiles;
  a.splits = p.splits;
  a.sps = p.sps;
  a.xcd = (static_cast<int64_t>(p.m_tiles) * p.n_tiles * p.splits) % 8 == 0 ? 1 : 0;
  a.Y = Y;
  a.ydt = ydt;
  a.ldy = ldy;
  a.RS = RS;
  a.part = p.splits > 1 ? static_cast<float *>(ws) : nullptr;
  int rc;
  switch (wtype) {
    case 12: rc = kq2_launch<FMT_Q4_K>(a, xb, s); break;
    case 13: rc = kq2_launch<FMT_Q5_K>(a, xb, s); break;
    case 14: rc = kq2_launch<FMT_Q6_K>(a, xb, s); break;
    default: rc = kq2_launch<FMT_IQ2_S>(a, xb, s); break;
  }
  if (rc || p.splits == 1) return rc;
  const int64_t n4 = M * N / 4;
  const unsigned grid = static_cast<unsigned>(n4 / 256 < 4096 ? (n4 + 255) / 256 : 4096);
  switch (ydt) {
    case VYBDQ_F32: hipLaunchKernelGGL(k_kq_reduce<VYBDQ_F32>, dim3(grid), dim3(256), 0, s, a.part, p.splits, a.M, a.N, xscale, Y, ldy, RS); break;
    case VYBDQ_F16: hipLaunchKernelGGL(k_kq_reduce<VYBDQ_F16>, dim3(grid), dim3(256), 0, s, a.part, p.splits, a.M, a.N, xscale, Y, ldy, RS); break;
    case VYBDQ_BF16: hipLaunchKernelGGL(k_kq_reduce<VYBDQ_BF16>, dim3(grid), dim3(256), 0, s, a.part, p.splits, a.M, a.N, xscale, Y, ldy, RS); break;
    default: hipLaunchKernelGGL(k_kq_reduce<VYBDQ_F64>, dim3(grid), dim3(256), 0, s, a.part, p.splits, a.M, a.N, xscale, Y, ldy, RS); break;
  }
  return check_launch("super-block gemm split reduce");
}

// The GEMM kind of vybdq_launch_pblock for wtype 12, 13, 14, 22 (pblock.hip); xdt F32 or F16.
// Q6_K / IQ2_S with fp16 X run the 128-row tiles.
int kq_gemm_pblock(int wtype, int xdt, const int64_t *pb, uint32_t *status, hipStream_t s) {
  if ((wtype == 14 || wtype == 22) && xdt == VYBDQ_F16) {
    const unsigned grid = static_cast<unsigned>(3 * device_cu_count());
    if (wtype == 14) hipLaunchKernelGGL((k_kq_mm_pb<FMT_Q6_K>), dim3(grid), dim3(256), 0, s, pb, status);
    else hipLaunchKernelGGL((k_kq_mm_pb<FMT_IQ2_S>), dim3(grid), dim3(256), 0, s, pb, status);
    return check_launch("p-block super-block gemm (128-row tiles)");
  }
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
