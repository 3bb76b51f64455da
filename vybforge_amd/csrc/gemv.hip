// Fused dequant GEMV on packed GGUF rows (q4_0 and Q8_0), gfx950.
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
// Q8_0 bytes are biased to unsigned (q ^ 0x80 = q + 128), OFF = 128. Float32 x is rounded to
// fp16 at staging; the resulting error (~1e-4 relative) is well inside the 2e-3 gate.
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
  const int64_t rowbytes = static_cast<int64_t>(P) * Fmt<FMT>::PAIR_BYTES;
  const uint8_t *wrow = pick3_ptr(segs.W, sg) + lrow * rowbytes;
  const int npairs = active && ks < P ? (P - ks + G - 1) / G : 0;
  // loads are unconditional (no divergent branches, no register shuffling): a lane past its
  // last pair re-reads a pair of its own row (inactive lanes: row 0 of segment 0)
  auto pair_ptr = [&](int i) {
    int p = ks + G * i;
    p = p < P ? p : (ks < P ? ks : 0);
    return wrow + static_cast<int64_t>(p) * Fmt<FMT>::PAIR_BYTES;
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
  for (int u = 0; u < U; ++u) load_pair<FMT>(pair_ptr(u), dw[u]);
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
  __syncthreads();

  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.f;

  for (int i0 = 0; i0 < npairs; i0 += U) {
    if (i0 > 0) {
#pragma unroll
      for (int u = 0; u < U; ++u) load_pair<FMT>(pair_ptr(i0 + u), dw[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i0 + u < npairs) pair_dot<FMT, ORDER, M>(dw[u], lds, sx, P, ks + G * (i0 + u), acc);
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

// Reference-order fallback for K % 64 == 32 (odd block count per row): one wave per row,
// lane = block, byte loads, exact float32 products.
template <int FMT, int ORDER, int XDT>
__global__ void __launch_bounds__(64) k_gemv_generic(const void *__restrict__ X, int64_t M, int64_t K, Segs segs) {
  const int64_t row = blockIdx.x;
  int sg = 0;
  if (row >= segs.end[0]) sg = (row >= segs.end[1]) ? 2 : 1;
  const int64_t lrow = row - (sg == 0 ? 0 : segs.end[sg - 1]);
  const int64_t nb = K / 32;
  constexpr int BB = FMT == FMT_Q4_0 ? 18 : 34;
  const uint8_t *wrow = segs.W[sg] + lrow * nb * BB;
  const int64_t N = segs.end[sg] - (sg == 0 ? 0 : segs.end[sg - 1]);
  for (int64_t m = 0; m < M; ++m) {
    float acc = 0.f;
    for (int64_t b = threadIdx.x; b < nb; b += 64) {
      const uint8_t *blk = wrow + b * BB;
      const float d = half_bits_to_f32(blk[0] | (static_cast<uint32_t>(blk[1]) << 8));
      float ps = 0.f;
      for (int e = 0; e < 32; ++e) {
        int qv;
        if constexpr (FMT == FMT_Q8_0) qv = static_cast<int8_t>(blk[2 + e]);
        else if constexpr (ORDER == VYBDQ_Q4_GGML) qv = ((blk[2 + (e & 15)] >> (4 * (e >> 4))) & 15) - 8;
        else qv = ((blk[2 + (e >> 1)] >> (4 * (e & 1))) & 15) - 8;
        ps = fmaf(load_elem<XDT>(X, m * K + b * 32 + e), static_cast<float>(qv), ps);
      }
      acc = fmaf(d, ps, acc);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (threadIdx.x == 0) {
      const int64_t i = m * N + lrow;
      switch (segs.ydt[sg]) {
        case VYBDQ_F32: store_elem<VYBDQ_F32>(segs.Y[sg], segs.RS[sg], i, acc); break;
        case VYBDQ_F16: store_elem<VYBDQ_F16>(segs.Y[sg], segs.RS[sg], i, acc); break;
        case VYBDQ_BF16: store_elem<VYBDQ_BF16>(segs.Y[sg], segs.RS[sg], i, acc); break;
        default: store_elem<VYBDQ_F64>(segs.Y[sg], segs.RS[sg], i, acc); break;
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

// Largest load batch per format (VGPRs: U pair windows of 9 or 17 dwords in flight per lane).
static int pair_umax(int fmt) { return fmt == FMT_Q8_0 ? 3 : 5; }

// For one X row (decode): the widest G that still gives each lane at least two pairs (two pair
// windows in flight per lane; one-pair lanes were measured slower at every decode shape), widened
// further while the grid has fewer workgroups than CUs, 256 threads, and a batch of exactly
// ceil(P / G) pairs (up to the format's largest). For batches (M > 1) the smallest G with ~4 waves
// per CU whose row fits one widest batch. VYBDQ_GEMV_PLAN="G,U,T" overrides the plan.
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
    const int U = (P + G - 1) / G;
    pl.G = G;
    pl.U = U < umax ? U : umax;
  }
  if (const char *e = getenv("VYBDQ_GEMV_PLAN")) {
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
  const size_t lds = static_cast<size_t>(M) * P * (XPAIR_STRIDE + 2 * 4);
  if (lds > static_cast<size_t>(kMaxLds)) return set_error(VYBDQ_ERR_SHAPE, "gemv: K too large for the LDS x stage at this M");
  const int rows_per_wg = threads / G;
  const unsigned grid = static_cast<unsigned>((rows + rows_per_wg - 1) / rows_per_wg);
  if (lds > 64 * 1024) {
    static bool raised = false;  // one attribute call per instantiation
    if (!raised) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemv_pair<FMT, G, ORDER, M, XW, U>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
      if (e != hipSuccess) return set_error(VYBDQ_ERR_HIP, std::string("gemv: LDS attribute: ") + hipGetErrorString(e));
      raised = true;
    }
  }
  hipLaunchKernelGGL((k_gemv_pair<FMT, G, ORDER, M, XW, U>), dim3(grid), dim3(threads), lds, s, X, xdt, K, segs);
  return check_launch("gemv");
}

template <int FMT, int G, int ORDER, int M, int XW>
static int launch_g(const void *X, int xdt, int64_t K, const Segs &segs, const PairPlan &pl, hipStream_t s) {
  constexpr int UM = FMT == FMT_Q8_0 ? 3 : 5;
  if constexpr (M > 1) {
    return launch_gu<FMT, G, ORDER, M, XW, UM>(X, xdt, K, segs, pl.T, s);
  } else {
    switch (pl.U) {
      case 1: return launch_gu<FMT, G, ORDER, M, XW, 1>(X, xdt, K, segs, pl.T, s);
      case 2: return launch_gu<FMT, G, ORDER, M, XW, 2>(X, xdt, K, segs, pl.T, s);
      case 3: return launch_gu<FMT, G, ORDER, M, XW, 3>(X, xdt, K, segs, pl.T, s);
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

template <int FMT, int ORDER>
static int gemv_dispatch(const void *X, int64_t M, int64_t K, int x_dt, Segs segs, hipStream_t s) {
  const int xs = dt_size(x_dt);
  if (K % 64 != 0) {
    const unsigned grid = static_cast<unsigned>(segs.end[2]);
    VYBDQ_DISPATCH_IN(x_dt, XDT,
        hipLaunchKernelGGL((k_gemv_generic<FMT, ORDER, XDT>), dim3(grid), dim3(64), 0, s, X, M, K, segs));
    return check_launch("gemv(generic)");
  }
  // M > 4: split X rows into chunks of at most 4 (each chunk re-streams W)
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

static int gemv_common(int fmt, int order, uint64_t X, int64_t M, int64_t K, int x_dt, Segs &segs,
                       uint64_t stream) {
  VYBDQ_REQUIRE(X, VYBDQ_ERR_ARG, "null X");
  VYBDQ_REQUIRE((X & 15) == 0, VYBDQ_ERR_ALIGN, "X must be 16-byte aligned");
  VYBDQ_REQUIRE(dt_valid_in(x_dt), VYBDQ_ERR_ARG, "x_dt must be F32, F16 or BF16");
  VYBDQ_REQUIRE(M >= 1 && M <= 8, VYBDQ_ERR_SHAPE, "M must be in [1, 8]");
  VYBDQ_REQUIRE(K > 0 && K % 32 == 0, VYBDQ_ERR_SHAPE, "K must be a positive multiple of 32");
  VYBDQ_REQUIRE(K <= (1 << 20), VYBDQ_ERR_SHAPE, "K too large");
  VYBDQ_REQUIRE(order == VYBDQ_Q4_GGML || order == VYBDQ_Q4_INTERLEAVED, VYBDQ_ERR_ARG, "unknown q4_0 order");
  int64_t acc = 0;
  for (int i = 0; i < 3; ++i) {
    const int64_t n = segs.end[i];
    VYBDQ_REQUIRE(n >= 0, VYBDQ_ERR_SHAPE, "N < 0");
    if (n > 0) {
      VYBDQ_REQUIRE(segs.W[i] && segs.Y[i], VYBDQ_ERR_ARG, "null W or Y");
      VYBDQ_REQUIRE(dt_valid_out(segs.ydt[i]), VYBDQ_ERR_ARG, "y_dt must be F32, F16, BF16 or F64");
      if (K % 64 == 0)
        VYBDQ_REQUIRE((reinterpret_cast<uintptr_t>(segs.W[i]) & 3) == 0, VYBDQ_ERR_ALIGN, "W must be 4-byte aligned");
    }
    acc += n;
    segs.end[i] = acc;
  }
  VYBDQ_REQUIRE(acc > 0, VYBDQ_ERR_SHAPE, "N must be > 0");
  VYBDQ_REQUIRE(acc < (int64_t(1) << 31), VYBDQ_ERR_SHAPE, "too many rows");
  const void *x = reinterpret_cast<const void *>(X);
  hipStream_t s = as_stream(stream);
  if (fmt == FMT_Q8_0) return gemv_dispatch<FMT_Q8_0, VYBDQ_Q4_GGML>(x, M, K, x_dt, segs, s);
  if (order == VYBDQ_Q4_GGML) return gemv_dispatch<FMT_Q4_0, VYBDQ_Q4_GGML>(x, M, K, x_dt, segs, s);
  return gemv_dispatch<FMT_Q4_0, VYBDQ_Q4_INTERLEAVED>(x, M, K, x_dt, segs, s);
}

static Segs one_seg(uint64_t W, uint64_t Y, uint64_t RS, int64_t N, int y_dt) {
  Segs s{};
  s.W[0] = reinterpret_cast<const uint8_t *>(W);
  s.Y[0] = reinterpret_cast<void *>(Y);
  s.RS[0] = reinterpret_cast<const void *>(RS);
  s.ydt[0] = y_dt;
  s.ydt[1] = s.ydt[2] = y_dt;
  s.end[0] = N;
  s.end[1] = s.end[2] = 0;
  return s;
}

}  // namespace vybdq

using namespace vybdq;

extern "C" int vybdq_gemv_q4_0(uint64_t W, uint64_t X, uint64_t Y, int64_t M, int64_t N, int64_t K,
                               int x_dt, int y_dt, uint64_t RS, int order, uint64_t stream) {
  Segs s = one_seg(W, Y, RS, N, y_dt);
  return gemv_common(FMT_Q4_0, order, X, M, K, x_dt, s, stream);
}

extern "C" int vybdq_gemv_q8_0(uint64_t W, uint64_t X, uint64_t Y, int64_t M, int64_t N, int64_t K,
                               int x_dt, int y_dt, uint64_t RS, uint64_t stream) {
  Segs s = one_seg(W, Y, RS, N, y_dt);
  return gemv_common(FMT_Q8_0, VYBDQ_Q4_GGML, X, M, K, x_dt, s, stream);
}

extern "C" int vybdq_gemv_q4_0_seg3(uint64_t X, int64_t K, int x_dt, int order,
                                    uint64_t W, uint64_t Y, int64_t N, int y_dt,
                                    uint64_t W2, uint64_t Y2, int64_t N2, int y_dt2,
                                    uint64_t W3, uint64_t Y3, int64_t N3, int y_dt3, uint64_t stream) {
  Segs s{};
  s.W[0] = reinterpret_cast<const uint8_t *>(W);
  s.W[1] = reinterpret_cast<const uint8_t *>(W2);
  s.W[2] = reinterpret_cast<const uint8_t *>(W3);
  s.Y[0] = reinterpret_cast<void *>(Y);
  s.Y[1] = reinterpret_cast<void *>(Y2);
  s.Y[2] = reinterpret_cast<void *>(Y3);
  s.ydt[0] = y_dt;
  s.ydt[1] = y_dt2;
  s.ydt[2] = y_dt3;
  s.end[0] = N;
  s.end[1] = N2;
  s.end[2] = N3;
  return gemv_common(FMT_Q4_0, order, X, 1, K, x_dt, s, stream);
}
