// Decode GEMV on xq8 activations for IQ2_S, Q4_K and Q5_K rows, gfx950.
//
// Y[n] = RS[n] + sum_b dx[b] * (integer dot of block b's quants with xq[32b .. 32b+31]) * scales
//
// x arrives as the q8 copy the RMSNorm / SwiGLU producers write (xq8: int8 xq[K] and one float32
// scale dx per 32 values), and every 32-weight sub-block product is an exact integer dot product
// (v_dot4_i32_i8, four int8 products per instruction) scaled once in float32, as the reference's
// default decode path does (q8_1 activations + dp4a, native/kernels/rgemv7.vyb:3-96 for IQ2_S,
// native/kernels/rq4kq.vyb:7-89 for Q4_K, native/kernels/rq5kq.vyb:8-80 for Q5_K). The result is
// the GEMV of the dequantized x' = dx * xq, not of x: lossy against the exact entry points, and
// exact up to float32 scaling against the float64 GEMV of x'.
//   Q4_K / Q5_K sub-block j: d sc_j dx sum(q xq) - dmin m_j dx sum(xq) with q the 4-bit (5-bit)
//     quants (0..15 / 0..31: exact as signed int8 operands) and sum(xq) the block sum of x, formed
//     once per launch while x is staged;
//   IQ2_S sub-block: per 8-weight group the grid magnitudes (8, 25 or 43) negated per the group's
//     sign byte, d (0.5 + s) / 4 per 16 weights with the 4-bit scales s.
//
// Work split and loads as the exact pair GEMV (gemv_pair.h): G lanes per row walk its 64-weight
// units with stride G, U unit windows in flight per lane (load_unit_kq), the first batch issued
// before x is staged, partial sums combined by the DPP tree. LDS holds, per unit p, the 64 xq
// bytes at 80 p (16 bytes of padding put the G lanes reading consecutive units on distinct banks:
// a lane reads its unit's x with four conflict-free ds_read_b128) and float4 {dx, sum(xq)} x 2 of
// its two blocks; IQ2_S adds the grid as bytes (1024 x 8 B) and the 256 sign patterns as byte
// masks (0x00 / 0xFF per sign bit).
#include "gemv_pair.h"

namespace vybdq {

constexpr int kXq8UnitBytes = 80;  // LDS bytes per unit of xq (64 + 16 padding)
constexpr int kXq8UnitMeta = 16;   // {dx, sum} of the unit's two blocks
constexpr int kXq8Iq2sBytes = 1024 * 8 + 256 * 8;

__host__ __device__ constexpr size_t xq8_lds_bytes(int64_t P, bool iq2s) {
  return static_cast<size_t>(P) * (kXq8UnitBytes + kXq8UnitMeta) + (iq2s ? kXq8Iq2sBytes : 0);
}

// bytes 0x00 / 0x01 from the four bits of n (bit j -> byte j): the four shifted copies of n occupy
// disjoint bit ranges, so the product is their OR
__device__ __forceinline__ uint32_t spread4(uint32_t n) { return (n * 0x00204081u) & 0x01010101u; }

template <int FMT>
__device__ __forceinline__ float unit_dot_xq8(const uint32_t (&dw)[Fmt<FMT>::PAIR_DWORDS], const char *lq,
                                              const float4 *lmeta, const uint2 *lgrid, const uint2 *lsign, int p) {
  const u4 *xv = reinterpret_cast<const u4 *>(lq + static_cast<size_t>(p) * kXq8UnitBytes);
  const u4 x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
  const uint32_t xd[2][8] = {{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]},
                             {x2[0], x2[1], x2[2], x2[3], x3[0], x3[1], x3[2], x3[3]}};
  const float4 meta = lmeta[p];  // dx and sum(xq) of blocks 2p, 2p + 1
  const float dxb[2] = {meta.x, meta.z}, sxb[2] = {meta.y, meta.w};
  const int g = p & 3;
  if constexpr (FMT == FMT_Q4_K || FMT == FMT_Q5_K) {
    constexpr int QS = FMT == FMT_Q4_K ? 4 : 12;  // first qs dword of the window
    const float d = half_bits_to_f32(dw[0] & 0xffffu);
    const float dmin = half_bits_to_f32(dw[0] >> 16);
    float r = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float sc, mn;
      scale_min_k4(dw[1], dw[2], dw[3], 2 * g + h, sc, mn);
      int dot = 0;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        uint32_t v = h == 0 ? (dw[QS + t] & 0x0F0F0F0Fu) : ((dw[QS + t] >> 4) & 0x0F0F0F0Fu);
        if constexpr (FMT == FMT_Q5_K) v |= ((dw[4 + t] >> (2 * g + h)) & 0x01010101u) << 4;
        dot = __builtin_amdgcn_sdot4(static_cast<int>(v), static_cast<int>(xd[h][t]), dot, false);
      }
      r = fmaf(dxb[h], d * sc * static_cast<float>(dot) - dmin * mn * sxb[h], r);
    }
    return r;
  } else {
    static_assert(FMT == FMT_IQ2_S, "xq8 GEMV formats");
    const uint32_t sh = dw[9];
    const uint32_t ix[2] = {__builtin_amdgcn_alignbit(dw[1], dw[0], sh), __builtin_amdgcn_alignbit(dw[2], dw[1], sh)};
    const uint32_t sg[2] = {__builtin_amdgcn_alignbit(dw[4], dw[3], sh), __builtin_amdgcn_alignbit(dw[5], dw[4], sh)};
    const float d = half_bits_to_f32(dw[8]) * 0.25f;
    float r = 0.f;
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {  // sub-block 2g + ib of the super-block = x block 2p + ib
      int si[2] = {0, 0};             // groups 0, 1 (first 16 weights) and 2, 3
#pragma unroll
      for (int l2 = 0; l2 < 4; ++l2) {
        const uint32_t idx = __builtin_amdgcn_ubfe(ix[ib], 8 * l2, 8) |
                             (__builtin_amdgcn_ubfe(dw[6], 8 * ib + 2 * l2, 2) << 8);
        const uint2 gv = lgrid[idx];
        const uint2 m = lsign[__builtin_amdgcn_ubfe(sg[ib], 8 * l2, 8)];
        // negated magnitude bytes: (g ^ 0xFF) + 1 = 256 - g, with no carry out of a byte (g >= 8)
        const uint32_t s0 = (gv.x ^ m.x) + (m.x & 0x01010101u);
        const uint32_t s1 = (gv.y ^ m.y) + (m.y & 0x01010101u);
        int &acc = si[l2 >> 1];
        acc = __builtin_amdgcn_sdot4(static_cast<int>(s0), static_cast<int>(xd[ib][2 * l2]), acc, false);
        acc = __builtin_amdgcn_sdot4(static_cast<int>(s1), static_cast<int>(xd[ib][2 * l2 + 1]), acc, false);
      }
      const uint32_t sc = __builtin_amdgcn_ubfe(dw[7], 8 * ib, 8);
      const float dlo = d * (static_cast<float>(sc & 15u) + 0.5f);
      const float dhi = d * (static_cast<float>(sc >> 4) + 0.5f);
      r = fmaf(dxb[ib], dlo * static_cast<float>(si[0]) + dhi * static_cast<float>(si[1]), r);
    }
    return r;
  }
}

template <int FMT, int G, int U>
__global__ void __launch_bounds__(256) k_gemv_xq8(const int8_t *__restrict__ Xq, const float *__restrict__ Xs,
                                                  int64_t K, Segs segs) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int PD = Fmt<FMT>::PAIR_DWORDS;
  constexpr bool IQ = FMT == FMT_IQ2_S;
  const int P = static_cast<int>(K >> 6);
  char *lq = smem;
  float4 *lmeta = reinterpret_cast<float4 *>(smem + static_cast<size_t>(P) * kXq8UnitBytes);
  uint2 *lgrid = reinterpret_cast<uint2 *>(lmeta + P);
  uint2 *lsign = lgrid + 1024;

  const int T = blockDim.x;
  const int lane = threadIdx.x & 63;
  const int ks = lane % G;
  const int rs = lane / G;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x / G) + (threadIdx.x >> 6) * (64 / G) + rs;
  const bool active = row < segs.end[2];
  int sg = 0;
  if (row >= segs.end[0]) sg = (row >= segs.end[1]) ? 2 : 1;
  if (!active) sg = 0;
  const int64_t seg_lo = sg == 0 ? 0 : (sg == 1 ? segs.end[0] : segs.end[1]);
  const int64_t lrow = active ? row - seg_lo : 0;
  const uint8_t *wrow = pick3_ptr(segs.W, sg) + lrow * unit_row_bytes<FMT>(P);
  const int nunits = active && ks < P ? (P - ks + G - 1) / G : 0;
  // a lane past its last unit re-reads one of its own row (inactive lanes: row 0 of segment 0)
  auto unit_idx = [&](int i) {
    const int p = ks + G * i;
    return p < P ? p : (ks < P ? ks : 0);
  };

  // 1. the first batch of weight windows
  uint32_t dw[U][PD];
#pragma unroll
  for (int u = 0; u < U; ++u) load_unit_kq<FMT>(wrow, unit_idx(u), dw[u]);

  // 2. x -> LDS under those loads: 16-byte chunks of xq (chunk c = bytes 16c .. 16c+15, block c / 2,
  // unit c / 4) with the block sums by one DPP swap between the chunk pair's two threads (K / 16 is
  // even and T is a multiple of 64, so both threads of a pair run the same iterations)
  for (int c = threadIdx.x; c < P * 4; c += T) {
    const u4 v = *reinterpret_cast<const u4 *>(Xq + 16 * static_cast<int64_t>(c));
    *reinterpret_cast<u4 *>(lq + (c >> 2) * kXq8UnitBytes + (c & 3) * 16) = v;
    int s = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) s = __builtin_amdgcn_sdot4(static_cast<int>(v[j]), 0x01010101, s, false);
    const float bs = dpp_add<DPP_QUAD_XOR1>(static_cast<float>(s));  // exact: |sum| <= 4096
    if ((c & 1) == 0) reinterpret_cast<float *>(lmeta)[(c >> 1) * 2 + 1] = bs;
  }
  for (int b = threadIdx.x; b < P * 2; b += T) reinterpret_cast<float *>(lmeta)[2 * b] = Xs[b];
  if constexpr (IQ) {
    // the table is 8-byte aligned: 8-byte loads, four per thread in flight
    const uint2 *grid = reinterpret_cast<const uint2 *>(kIq2sGrid);
    for (int i0 = threadIdx.x; i0 < 1024; i0 += 4 * T) {
      uint2 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (i0 + u * T < 1024) v[u] = grid[i0 + u * T];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (i0 + u * T < 1024) lgrid[i0 + u * T] = v[u];
    }
    for (int e = threadIdx.x; e < 256; e += T)
      lsign[e] = uint2{spread4(e & 15u) * 0xFFu, spread4(static_cast<uint32_t>(e) >> 4) * 0xFFu};
  }
  __syncthreads();

  float acc = 0.f;
  for (int i0 = 0; i0 < nunits; i0 += U) {
    if (i0 > 0) {
#pragma unroll
      for (int u = 0; u < U; ++u) load_unit_kq<FMT>(wrow, unit_idx(i0 + u), dw[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i0 + u < nunits) acc += unit_dot_xq8<FMT>(dw[u], lq, lmeta, lgrid, lsign, ks + G * (i0 + u));
  }
  acc = group_sum<G>(acc);
  if (active && ks == G - 1) {
    void *Y = pick3_ptr(segs.Y, sg);
    const void *RS = pick3_ptr(segs.RS, sg);
    switch (pick3(segs.ydt, sg)) {
      case VYBDQ_F32: store_elem<VYBDQ_F32>(Y, RS, lrow, acc); break;
      case VYBDQ_F16: store_elem<VYBDQ_F16>(Y, RS, lrow, acc); break;
      case VYBDQ_BF16: store_elem<VYBDQ_BF16>(Y, RS, lrow, acc); break;
      default: store_elem<VYBDQ_F64>(Y, RS, lrow, acc); break;
    }
  }
}

template <int FMT, int G, int U>
static int xq8_launch_gu(const int8_t *Xq, const float *Xs, int64_t K, const Segs &segs, int threads, hipStream_t s) {
  const int64_t P = K / 64;
  const size_t lds = xq8_lds_bytes(P, FMT == FMT_IQ2_S);
  if (lds > static_cast<size_t>(kMaxLds)) return set_error(VYBDQ_ERR_SHAPE, "gemv_xq8: K too large for the LDS x stage");
  if (lds > 64 * 1024) {
    static std::atomic<uint64_t> raised{0};
    const int rc = ensure_lds_limit(reinterpret_cast<const void *>(&k_gemv_xq8<FMT, G, U>), kMaxLds, raised, "gemv_xq8");
    if (rc) return rc;
  }
  const int rows_per_wg = threads / G;
  const unsigned grid = static_cast<unsigned>((segs.end[2] + rows_per_wg - 1) / rows_per_wg);
  hipLaunchKernelGGL((k_gemv_xq8<FMT, G, U>), dim3(grid), dim3(threads), lds, s, Xq, Xs, K, segs);
  return check_launch("gemv_xq8");
}

template <int FMT, int G>
static int xq8_launch_g(const int8_t *Xq, const float *Xs, int64_t K, const Segs &segs, const PairPlan &pl,
                        hipStream_t s) {
  constexpr int UM = kUmax<FMT>();
  switch (pl.U) {
    case 1: return xq8_launch_gu<FMT, G, 1>(Xq, Xs, K, segs, pl.T, s);
    case 2: return xq8_launch_gu<FMT, G, 2>(Xq, Xs, K, segs, pl.T, s);
    case 3: return xq8_launch_gu<FMT, G, (UM < 3 ? UM : 3)>(Xq, Xs, K, segs, pl.T, s);
    default: return xq8_launch_gu<FMT, G, UM>(Xq, Xs, K, segs, pl.T, s);
  }
}

template <int FMT>
static int xq8_launch(const int8_t *Xq, const float *Xs, int64_t K, const Segs &segs, hipStream_t s) {
  const PairPlan pl = pair_plan(FMT, segs.end[2], static_cast<int>(K / 64), 1);
  switch (pl.G) {
    case 8: return xq8_launch_g<FMT, 8>(Xq, Xs, K, segs, pl, s);
    case 16: return xq8_launch_g<FMT, 16>(Xq, Xs, K, segs, pl, s);
    case 32: return xq8_launch_g<FMT, 32>(Xq, Xs, K, segs, pl, s);
    default: return xq8_launch_g<FMT, 64>(Xq, Xs, K, segs, pl, s);
  }
}

static int gemv_xq8_common(int wtype, uint64_t Xq, uint64_t Xs, int64_t K, Segs &segs, uint64_t stream) {
  VYBDQ_REQUIRE(wtype == 12 || wtype == 13 || wtype == 22, VYBDQ_ERR_ARG,
                "wtype must be 12 (Q4_K), 13 (Q5_K) or 22 (IQ2_S)");
  VYBDQ_REQUIRE(Xq && Xs, VYBDQ_ERR_ARG, "null Xq or Xs");
  VYBDQ_REQUIRE((Xq & 15) == 0, VYBDQ_ERR_ALIGN, "Xq must be 16-byte aligned");
  VYBDQ_REQUIRE((Xs & 3) == 0, VYBDQ_ERR_ALIGN, "Xs must be 4-byte aligned");
  VYBDQ_REQUIRE(K > 0 && K % 256 == 0, VYBDQ_ERR_SHAPE, "K must be a positive multiple of 256");
  VYBDQ_REQUIRE(K <= 65536, VYBDQ_ERR_SHAPE, "K must be at most 65536");
  int64_t acc = 0;
  for (int i = 0; i < 3; ++i) {
    const int64_t n = segs.end[i];
    VYBDQ_REQUIRE(n >= 0, VYBDQ_ERR_SHAPE, "N < 0");
    if (n > 0) {
      VYBDQ_REQUIRE(segs.W[i] && segs.Y[i], VYBDQ_ERR_ARG, "null W or Y");
      VYBDQ_REQUIRE((reinterpret_cast<uintptr_t>(segs.W[i]) & 3) == 0, VYBDQ_ERR_ALIGN, "W must be 4-byte aligned");
      VYBDQ_REQUIRE(dt_valid_out(segs.ydt[i]), VYBDQ_ERR_ARG, "y_dt must be F32, F16, BF16 or F64");
    }
    acc += n;
    segs.end[i] = acc;
  }
  VYBDQ_REQUIRE(acc > 0, VYBDQ_ERR_SHAPE, "N must be > 0");
  VYBDQ_REQUIRE(acc < (int64_t(1) << 31), VYBDQ_ERR_SHAPE, "too many rows");
  const int8_t *xq = reinterpret_cast<const int8_t *>(Xq);
  const float *xs = reinterpret_cast<const float *>(Xs);
  hipStream_t s = as_stream(stream);
  if (wtype == 12) return xq8_launch<FMT_Q4_K>(xq, xs, K, segs, s);
  if (wtype == 13) return xq8_launch<FMT_Q5_K>(xq, xs, K, segs, s);
  return xq8_launch<FMT_IQ2_S>(xq, xs, K, segs, s);
}

}  // namespace vybdq

using namespace vybdq;

extern "C" int vybdq_gemv_xq8(int wtype, uint64_t W, uint64_t Xq, uint64_t Xs, uint64_t Y, int64_t N, int64_t K,
                              int y_dt, uint64_t RS, uint64_t stream) {
  Segs s{};
  s.W[0] = reinterpret_cast<const uint8_t *>(W);
  s.Y[0] = reinterpret_cast<void *>(Y);
  s.RS[0] = reinterpret_cast<const void *>(RS);
  s.ydt[0] = s.ydt[1] = s.ydt[2] = y_dt;
  s.end[0] = N;
  return gemv_xq8_common(wtype, Xq, Xs, K, s, stream);
}

extern "C" int vybdq_gemv_xq8_seg3(int wtype, uint64_t Xq, uint64_t Xs, int64_t K,
                                   uint64_t W, uint64_t Y, int64_t N, int y_dt, uint64_t RS,
                                   uint64_t W2, uint64_t Y2, int64_t N2, int y_dt2, uint64_t RS2,
                                   uint64_t W3, uint64_t Y3, int64_t N3, int y_dt3, uint64_t RS3, uint64_t stream) {
  Segs s{};
  const uint64_t w[3] = {W, W2, W3}, y[3] = {Y, Y2, Y3}, rs[3] = {RS, RS2, RS3};
  const int64_t n[3] = {N, N2, N3};
  const int dt[3] = {y_dt, y_dt2, y_dt3};
  for (int i = 0; i < 3; ++i) {
    s.W[i] = reinterpret_cast<const uint8_t *>(w[i]);
    s.Y[i] = reinterpret_cast<void *>(y[i]);
    s.RS[i] = reinterpret_cast<const void *>(rs[i]);
    s.ydt[i] = n[i] > 0 ? dt[i] : VYBDQ_F32;
    s.end[i] = n[i];
  }
  return gemv_xq8_common(wtype, Xq, Xs, K, s, stream);
}
