// The pair GEMV kernel and its launch plan, shared by the q4_0 / Q8_0 (gemv.hip) and K-quant
// (gemv_kq.hip) translation units.
//
// Y[m, n] = RS[m, n] + sum_k X[m, k] * W[n, k]
//
// Work split. A "pair" is two consecutive 32-weight blocks of one row: 36 B for q4_0,
// 68 B for Q8_0. Rows are 4-byte aligned when K % 64 == 0, so a lane fetches its pair with
// dword-aligned vector loads and re-aligns the 2-byte-offset half with v_alignbit. The G
// lanes of a row-slot walk the row's pairs with stride G (consecutive lanes read consecutive
// pairs), each lane keeps one float32 accumulator per X row, and the G partials are combined
// by a fixed DPP tree on the VALU (group_sum; no LDS round trips in the tail). G (8..64) is
// picked per launch so that the grid holds enough waves to cover HBM latency while each lane's
// pairs fit one batch of registers.
//
// Latency. Every lane issues the loads of its first batch of pairs before anything else;
// the x stage (coalesced 16-B loads -> LDS, block sums by 4-lane DPP swaps, one barrier)
// runs under those loads.
//
// Arithmetic. x is staged as fp16 in natural order. A quant byte becomes an fp16 with
//   fp16 bits 0x6400 | v == 1024 + v   (v < 1024)
// built by v_perm_b32 from the masked quant dword and a 0x64 byte constant, two consecutive
// weights per register, and v_dot2_f32_f16 multiplies-and-accumulates two weights per op in
// float32. Per block, sum_k x_k (q_k - OFF) = dot - (1024 + OFF) * sum_k x_k with the block
// sum of the same fp16 x from the stage, then y += d * partial. OFF = 8 for q4_0 nibbles;
// Q8_0 bytes are biased to unsigned (q ^ 0x80 = q + 128), OFF = 128. Float32 and bf16 x are
// staged as fp16 per 32-element block after a power-of-two block scale (gemv_dev.h block_scale:
// no overflow, no subnormals), which multiplies into d; the fp16 rounding of float32 x
// (~1e-4 relative) is well inside the 2e-3 gate.
#pragma once
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include "gemv_dev.h"

namespace vybdq {

template <int FMT, int G, int ORDER, int M, int XW, int U>
__global__ void __launch_bounds__(256) k_gemv_pair(const void *__restrict__ X, int xdt, int64_t K, Segs segs) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int PD = Fmt<FMT>::PAIR_DWORDS;
  constexpr int XC = 5;  // x chunks per thread prefetched ahead of the weight loads
  const int P = static_cast<int>(K >> 6);
  char *lds = smem;
  float *sx = reinterpret_cast<float *>(smem + static_cast<size_t>(M) * P * XPAIR_STRIDE);

  const int T = blockDim.x;  // 64, 128 or 256
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
  const int64_t rowbytes = unit_row_bytes<FMT>(P);
  const uint8_t *wrow = pick3_ptr(segs.W, sg) + lrow * rowbytes;
  const int npairs = active && ks < P ? (P - ks + G - 1) / G : 0;
  // loads are unconditional (no divergent branches, no register shuffling): a lane past its
  // last pair re-reads a pair of its own row (inactive lanes: row 0 of segment 0)
  auto pair_idx = [&](int i) {
    const int p = ks + G * i;
    return p < P ? p : (ks < P ? ks : 0);
  };

  // 1. x chunks (L2-resident, short latency) first, so waiting on them never waits on weights
  const int nchunk = M * 8 * P;
  uint32_t xr[XC][XW];
#pragma unroll
  for (int j = 0; j < XC; ++j) {
    const int c = threadIdx.x + T * j;
    if (c < nchunk) load_x_chunk<XW>(X, 8 * static_cast<int64_t>(c), xr[j]);
  }
  // 2. the first batch of weight pairs
  uint32_t dw[U][PD];
#pragma unroll
  for (int u = 0; u < U; ++u) load_unit<FMT>(wrow, pair_idx(u), dw[u]);
  // 3. x -> LDS while the weights stream in
#pragma unroll
  for (int j = 0; j < XC; ++j) {
    const int c = threadIdx.x + T * j;
    if (c < nchunk) stage_chunk<XW>(xr[j], xdt, c, lds, sx);
  }
  for (int c = threadIdx.x + T * XC; c < nchunk; c += T) {
    uint32_t r[XW];
    load_x_chunk<XW>(X, 8 * static_cast<int64_t>(c), r);
    stage_chunk<XW>(r, xdt, c, lds, sx);
  }
  if constexpr (FMT == FMT_IQ2_S) {
    // after the x stage: the IQ2_S grid as fp16 (16 KB: entry i = its 8 magnitudes, exact) and
    // the 256 sign patterns as fp16 sign-bit masks (4 KB: bit j of s -> bit 15 of half j),
    // copied from the table the generator precomputed (converting them here cost ~150 VALU
    // instructions per wave, a fifth of a 9728 x 2560 GEMV's)
    u4 *gridh = iq2s_lds_grid(sx, M, P);
    for (int i0 = threadIdx.x; i0 < 1024 + 256; i0 += 5 * T) {  // five 16-B loads in flight per thread
      u4 v[5];
    #pragma unroll
      for (int u = 0; u < 5; ++u)
        if (i0 + u * T < 1024 + 256) v[u] = reinterpret_cast<const u4 *>(kIq2sLdsTab)[i0 + u * T];
    #pragma unroll
      for (int u = 0; u < 5; ++u)
        if (i0 + u * T < 1024 + 256) gridh[i0 + u * T] = v[u];
    }
  }
  __syncthreads();

  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.f;

  for (int i0 = 0; i0 < npairs; i0 += U) {
    if (i0 > 0) {
#pragma unroll
      for (int u = 0; u < U; ++u) load_unit<FMT>(wrow, pair_idx(i0 + u), dw[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i0 + u < npairs) unit_dot<FMT, ORDER, M>(dw[u], lds, sx, P, ks + G * (i0 + u), acc);
  }
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = group_sum<G>(acc[m]);
  if (active && ks == G - 1) {
    const int64_t N = pick3(segs.end, sg) - seg_lo;
    void *Y = pick3_ptr(segs.Y, sg);
    const void *RS = pick3_ptr(segs.RS, sg);
    const int ydt = pick3(segs.ydt, sg);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int64_t i = m * N + lrow;
      switch (ydt) {
        case VYBDQ_F32: store_elem<VYBDQ_F32>(Y, RS, i, acc[m]); break;
        case VYBDQ_F16: store_elem<VYBDQ_F16>(Y, RS, i, acc[m]); break;
        case VYBDQ_BF16: store_elem<VYBDQ_BF16>(Y, RS, i, acc[m]); break;
        default: store_elem<VYBDQ_F64>(Y, RS, i, acc[m]); break;
      }
    }
  }
}

// ---- host launch --------------------------------------------------------------------------

static constexpr int kMaxLds = 160 * 1024;

// Launch shape of the pair kernel: G lanes per row, U pairs per lane and load batch, T threads
// per workgroup (T / G rows).
struct PairPlan {
  int G, U, T;
};

// Largest load batch per format (VGPRs: U unit windows of PAIR_DWORDS dwords in flight per lane).
template <int FMT> constexpr int kUmax() {
  return FMT == FMT_Q4_0 ? 5 : FMT == FMT_Q8_0 ? 3 : (FMT == FMT_Q4_K || FMT == FMT_IQ2_S) ? 4 : 2;
}
static int pair_umax(int fmt) {
  switch (fmt) {
    case FMT_Q4_0: return kUmax<FMT_Q4_0>();
    case FMT_Q8_0: return kUmax<FMT_Q8_0>();
    case FMT_Q4_K: return kUmax<FMT_Q4_K>();
    case FMT_Q5_K: return kUmax<FMT_Q5_K>();
    case FMT_IQ2_S: return kUmax<FMT_IQ2_S>();
    default: return kUmax<FMT_Q6_K>();
  }
}

// For one X row (decode): the widest G that still gives each lane at least two pairs (two pair
// windows in flight per lane; one-pair lanes were measured slower at every decode shape), widened
// further while the grid would hold fewer rows than 64 / G per CU x 4 waves, a batch of exactly
// ceil(P / G) pairs (up to the format's largest), narrowed while the grid would not be resident in
// one round; 256 threads (one workgroup of 16 waves per CU was measured 16% slower on the decode
// stack). For batches (M > 1) the smallest G with ~4 waves per CU whose row fits one widest batch.
// VYBDQ_GEMV_PLAN="G,U,T" overrides the plan (read only with VYBDQ_TUNING set, common.h).
static PairPlan pair_plan(int fmt, int64_t rows, int P, int64_t M) {
  const int umax = pair_umax(fmt);
  PairPlan pl{64, umax, 256};
  if (M > 1) {
    int G = 8;
    while (G < 64 && (rows * G / 64 < 1024 || (P + G - 1) / G > umax)) G *= 2;
    pl.G = G;
  } else {
    int G = 8;
    while (G < 64 && (P + 2 * G - 1) / (2 * G) >= 2) G *= 2;  // ceil(P / 2G) >= 2
    while (G < 64 && rows * G / 256 < device_cu_count()) G *= 2;
    // more waves than fit at once (8 per SIMD) would start a second round one HBM latency late:
    // narrow G (more pairs per lane) until the grid is resident in one round
    const int64_t resident = 32LL * device_cu_count();
    while (G > 16 && rows * G / 64 > resident) G /= 2;
    // q4_0 rows of exactly 64 pairs (K = 4096): one pair per lane over a whole wave (no idle lane,
    // one DPP step more) beats two pairs over half a wave (the decode stack's 2560 x 4096 launch,
    // full-stack graph: 843.0 -> 832.7 us per token)
    if (fmt == FMT_Q4_0 && P == 64 && rows <= resident) G = 64;
    const int U = (P + G - 1) / G;
    pl.G = G;
    pl.U = U < umax ? U : umax;
  }
  if (const char *e = tuning_env("VYBDQ_GEMV_PLAN")) {
    int g = 0, u = 0, t = 0;
    if (sscanf(e, "%d,%d,%d", &g, &u, &t) == 3 && (g == 8 || g == 16 || g == 32 || g == 64) && u >= 1 &&
        u <= umax && (t == 64 || t == 128 || t == 256) && t >= g) {
      pl.G = g; pl.U = u; pl.T = t;
    }
  }
  return pl;
}

template <int FMT, int G, int ORDER, int M, int XW, int U>
static int launch_gu(const void *X, int xdt, int64_t K, const Segs &segs, int threads, hipStream_t s) {
  const int64_t rows = segs.end[2];
  const int P = static_cast<int>(K / 64);
  const size_t lds = static_cast<size_t>(M) * P * XSTAGE_PAIR_BYTES + (FMT == FMT_IQ2_S ? kIq2sLdsBytes : 0);
  if (lds > static_cast<size_t>(kMaxLds)) return set_error(VYBDQ_ERR_SHAPE, "gemv: K too large for the LDS x stage at this M");
  const int rows_per_wg = threads / G;
  const unsigned grid = static_cast<unsigned>((rows + rows_per_wg - 1) / rows_per_wg);
  if (lds > 64 * 1024) {
    static std::atomic<uint64_t> raised{0};  // one attribute call per instantiation and device
    const int rc = ensure_lds_limit(reinterpret_cast<const void *>(&k_gemv_pair<FMT, G, ORDER, M, XW, U>), kMaxLds,
                                    raised, "gemv");
    if (rc) return rc;
  }
  hipLaunchKernelGGL((k_gemv_pair<FMT, G, ORDER, M, XW, U>), dim3(grid), dim3(threads), lds, s, X, xdt, K, segs);
  return check_launch("gemv");
}

template <int FMT, int G, int ORDER, int M, int XW>
static int launch_g(const void *X, int xdt, int64_t K, const Segs &segs, const PairPlan &pl, hipStream_t s) {
  constexpr int UM = kUmax<FMT>();
  if constexpr (M > 1) {
    return launch_gu<FMT, G, ORDER, M, XW, UM>(X, xdt, K, segs, pl.T, s);
  } else {
    switch (pl.U) {
      case 1: return launch_gu<FMT, G, ORDER, M, XW, 1>(X, xdt, K, segs, pl.T, s);
      case 2: return launch_gu<FMT, G, ORDER, M, XW, 2>(X, xdt, K, segs, pl.T, s);
      case 3: return launch_gu<FMT, G, ORDER, M, XW, (UM < 3 ? UM : 3)>(X, xdt, K, segs, pl.T, s);
      case 4: return launch_gu<FMT, G, ORDER, M, XW, (UM < 4 ? UM : 4)>(X, xdt, K, segs, pl.T, s);
      default: return launch_gu<FMT, G, ORDER, M, XW, UM>(X, xdt, K, segs, pl.T, s);
    }
  }
}

template <int FMT, int ORDER, int M, int XW>
static int launch_mx(const void *X, int xdt, int64_t K, const Segs &segs, hipStream_t s) {
  const PairPlan pl = pair_plan(FMT, segs.end[2], static_cast<int>(K / 64), M);
  switch (pl.G) {
    case 8: return launch_g<FMT, 8, ORDER, M, XW>(X, xdt, K, segs, pl, s);
    case 16: return launch_g<FMT, 16, ORDER, M, XW>(X, xdt, K, segs, pl, s);
    case 32: return launch_g<FMT, 32, ORDER, M, XW>(X, xdt, K, segs, pl, s);
    default: return launch_g<FMT, 64, ORDER, M, XW>(X, xdt, K, segs, pl, s);
  }
}

template <int FMT, int ORDER, int M>
static int launch_m(const void *X, int xdt, int64_t K, const Segs &segs, hipStream_t s) {
  if (xdt == VYBDQ_F32) return launch_mx<FMT, ORDER, M, 8>(X, xdt, K, segs, s);
  return launch_mx<FMT, ORDER, M, 4>(X, xdt, K, segs, s);
}

template <int FMT, int ORDER>
static int launch_pair(const void *X, int xdt, int64_t M, int64_t K, const Segs &segs, hipStream_t s) {
  switch (M) {
    case 1: return launch_m<FMT, ORDER, 1>(X, xdt, K, segs, s);
    case 2: return launch_m<FMT, ORDER, 2>(X, xdt, K, segs, s);
    case 3: return launch_m<FMT, ORDER, 3>(X, xdt, K, segs, s);
    default: return launch_m<FMT, ORDER, 4>(X, xdt, K, segs, s);
  }
}

// X rows in chunks of at most 4 (each chunk re-streams W), K % 64 == 0.
template <int FMT, int ORDER>
static int launch_pair_chunks(const void *X, int64_t M, int64_t K, int x_dt, const Segs &segs, hipStream_t s) {
  const int xs = dt_size(x_dt);
  for (int64_t m0 = 0; m0 < M; m0 += 4) {
    const int64_t mc = (M - m0) < 4 ? (M - m0) : 4;
    Segs sc = segs;
    for (int i = 0; i < 3; ++i) {
      const int64_t n = segs.end[i] - (i == 0 ? 0 : segs.end[i - 1]);
      if (sc.Y[i]) sc.Y[i] = static_cast<char *>(sc.Y[i]) + m0 * n * dt_size(segs.ydt[i]);
      if (sc.RS[i]) sc.RS[i] = static_cast<const char *>(sc.RS[i]) + m0 * n * dt_size(segs.ydt[i]);
    }
    const void *Xc = static_cast<const char *>(X) + m0 * K * xs;
    const int rc = launch_pair<FMT, ORDER>(Xc, x_dt, mc, K, sc, s);
    if (rc) return rc;
  }
  return VYBDQ_OK;
}

// K-quant GEMV (gemv_kq.hip): fmt FMT_Q4_K / FMT_Q5_K / FMT_Q6_K, K % 256 == 0.
int gemv_kq_dispatch(int fmt, const void *X, int64_t M, int64_t K, int x_dt, const Segs &segs, hipStream_t s);

}  // namespace vybdq
