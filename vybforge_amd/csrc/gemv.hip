// Fused dequant GEMV on packed GGUF rows (q4_0 and Q8_0), gfx950.
//
// Y[m, n] = RS[m, n] + sum_k X[m, k] * W[n, k]
//
// Work split. A "pair" is two consecutive 32-weight blocks of one row: 36 B for q4_0,
// 68 B for Q8_0. Rows are 4-byte aligned when K % 64 == 0, so a lane fetches its pair with
// dword-aligned vector loads and re-aligns the 2-byte-offset half with v_alignbit. The G
// lanes of a row-slot walk the row's pairs with stride G (consecutive lanes read consecutive
// pairs: a row-slot's loads cover one contiguous span), each lane keeps one float32
// accumulator per X row, and the G partials are combined by a fixed xor-shuffle tree.
//
// Arithmetic. X is staged once per workgroup in LDS as fp16 pairs, permuted so that pair s
// of a quant dword lines up with the two quants that one v_and_or_b32 extracts:
//   fp16 bits 0x6400 | v == 1024 + v   (v < 1024)
// so each quant dword turns into fp16 pairs (1024+q0, 1024+q1) with one op per pair, and
// v_dot2_f32_f16 multiplies-and-accumulates two weights per op in float32. Per block,
//   sum_k x_k (q_k - OFF) = dot - (1024 + OFF) * sum_k x_k,
// with sum_k x_k of the same fp16-rounded x precomputed at staging, then y += d * partial.
// OFF = 8 for q4_0 nibbles; Q8_0 bytes are biased to unsigned (q ^ 0x80 = q + 128), OFF = 128.
// Float32 X is rounded to fp16 at staging; the float32 accumulation error budget is far
// inside the 2e-3 gate (documented with the measurements).
#include "common.h"

namespace vybdq {

enum { FMT_Q4_0 = 0, FMT_Q8_0 = 1 };

template <int FMT> struct Fmt;
template <> struct Fmt<FMT_Q4_0> {
  static constexpr int PAIR_BYTES = 36;
  static constexpr int PAIR_DWORDS = 9;
  static constexpr int QDW = 4;                 // quant dwords per block
  static constexpr float CORR = 1032.0f;        // 1024 + 8
};
template <> struct Fmt<FMT_Q8_0> {
  static constexpr int PAIR_BYTES = 68;
  static constexpr int PAIR_DWORDS = 17;
  static constexpr int QDW = 8;
  static constexpr float CORR = 1152.0f;        // 1024 + 128
};

// Element index (within a 32-weight block) of the two quants that land in half s of the
// fp16 pair extracted from quant dword t.
//   q4_0: dword t holds qs bytes 4t..4t+3; s = 0..3 selects (w >> 4s) & 0x000F000F,
//         i.e. bytes (0,2) low, (0,2) high, (1,3) low, (1,3) high.
//   Q8_0: dword t holds q[4t..4t+3]; s = 0 -> bytes (0,2), s = 1 -> bytes (1,3).
template <int FMT, int ORDER>
__device__ __forceinline__ void pair_elems(int t, int s, int &e0, int &e1) {
  if constexpr (FMT == FMT_Q8_0) {
    e0 = 4 * t + s;
    e1 = 4 * t + s + 2;
  } else {
    const int byte_a = 4 * t + (s >> 1);      // byte 0 or 1 of the dword
    const int byte_b = byte_a + 2;            // byte 2 or 3
    const int hi = s & 1;                     // high nibble?
    if constexpr (ORDER == VYBDQ_Q4_GGML) {
      e0 = byte_a + 16 * hi;
      e1 = byte_b + 16 * hi;
    } else {
      e0 = 2 * byte_a + hi;
      e1 = 2 * byte_b + hi;
    }
  }
}

// LDS layout per X row m: chunk c (16 B = 4 fp16 pairs) of pair p at xs[m][c * P + p], so the
// G lanes of a row-slot, which read consecutive pairs, read consecutive 16-B LDS words
// (conflict-free); block sums at sx[m][2p + h].
struct Segs {
  const uint8_t *W[3];
  void *Y[3];
  const void *RS[3];
  int ydt[3];
  int64_t end[3];  // cumulative row ends
};

template <int FMT, int ORDER, int XDT, int M>
__device__ __forceinline__ void stage_x(const void *__restrict__ X, int64_t K, int P, u4 *xs,
                                        float *sx) {
  constexpr int CH_PER_BLOCK = 4;                       // 16-B chunks per block
  const int nchunks = P * 2 * CH_PER_BLOCK;
  for (int m = 0; m < M; ++m) {
    const void *xm = nullptr;
    if constexpr (XDT == VYBDQ_F32) xm = static_cast<const float *>(X) + m * K;
    else xm = static_cast<const uint16_t *>(X) + m * K;
    for (int c = threadIdx.x; c < nchunks; c += blockDim.x) {
      const int j = c / P;          // chunk within pair 0..7
      const int p = c - j * P;      // pair
      const int h = j >> 2;         // block within pair
      const int64_t kb = (2 * static_cast<int64_t>(p) + h) * 32;
      u4 out;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // chunk j%4 holds 4 consecutive fp16 pairs (t, s) of this block
        const int idx = (j & 3) * 4 + q;
        int t, s;
        if constexpr (FMT == FMT_Q4_0) { t = idx >> 2; s = idx & 3; }
        else { t = idx >> 1; s = idx & 1; }
        int e0, e1;
        pair_elems<FMT, ORDER>(t, s, e0, e1);
        const _Float16 a = static_cast<_Float16>(load_elem<XDT>(xm, kb + e0));
        const _Float16 b = static_cast<_Float16>(load_elem<XDT>(xm, kb + e1));
        h2 v = {a, b};
        out[q] = __builtin_bit_cast(uint32_t, v);
      }
      xs[m * nchunks + j * P + p] = out;
    }
    for (int b = threadIdx.x; b < 2 * P; b += blockDim.x) {
      float s = 0.f;
      for (int e = 0; e < 32; ++e)
        s += static_cast<float>(static_cast<_Float16>(load_elem<XDT>(xm, static_cast<int64_t>(b) * 32 + e)));
      sx[m * 2 * P + b] = s;
    }
  }
}

typedef uint32_t u4a4 __attribute__((ext_vector_type(4), aligned(4)));

template <int FMT>
__device__ __forceinline__ void load_pair(const uint8_t *p, uint32_t (&dw)[Fmt<FMT>::PAIR_DWORDS]) {
  const u4a4 *v = reinterpret_cast<const u4a4 *>(p);
#pragma unroll
  for (int i = 0; i < Fmt<FMT>::PAIR_DWORDS / 4; ++i) {
    const u4a4 t = __builtin_nontemporal_load(v + i);
    dw[4 * i + 0] = t[0];
    dw[4 * i + 1] = t[1];
    dw[4 * i + 2] = t[2];
    dw[4 * i + 3] = t[3];
  }
  dw[Fmt<FMT>::PAIR_DWORDS - 1] =
      __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p) + Fmt<FMT>::PAIR_DWORDS - 1);
}

// Dot products of one pair (two blocks) of one row with the M staged x rows.
template <int FMT, int M>
__device__ __forceinline__ void pair_dot(const uint32_t (&dw)[Fmt<FMT>::PAIR_DWORDS], const u4 *xs,
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
    // fp16 pairs (1024 + v0, 1024 + v1)
    h2 wv[16];
#pragma unroll
    for (int t = 0; t < QDW; ++t) {
      if constexpr (FMT == FMT_Q4_0) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
          wv[4 * t + s] = __builtin_bit_cast(h2, ((q[t] >> (4 * s)) & 0x000F000Fu) | 0x64006400u);
      } else {
        const uint32_t u = q[t] ^ 0x80808080u;
        wv[2 * t + 0] = __builtin_bit_cast(h2, (u & 0x00FF00FFu) | 0x64006400u);
        wv[2 * t + 1] = __builtin_bit_cast(h2, ((u >> 8) & 0x00FF00FFu) | 0x64006400u);
      }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const u4 *xc = xs + m * P * 8 + (4 * h) * P + p;
      float ps = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u4 xv = xc[c * P];
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) {
          // copy the element to a scalar first: bit-casting a vector element expression
          // directly reads element 0 with this compiler
          const uint32_t xw = xv[q2];
          ps = __builtin_amdgcn_fdot2(wv[4 * c + q2], __builtin_bit_cast(h2, xw), ps, false);
        }
      }
      const float part = fmaf(-Fmt<FMT>::CORR, sx[m * 2 * P + 2 * p + h], ps);
      acc[m] = fmaf(d, part, acc[m]);
    }
  }
}

template <int FMT, int G, int ORDER, int XDT, int M>
__global__ void __launch_bounds__(256) k_gemv_pair(const void *__restrict__ X, int64_t K, Segs segs) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int P = static_cast<int>(K >> 6);
  u4 *xs = reinterpret_cast<u4 *>(smem);
  float *sx = reinterpret_cast<float *>(smem + static_cast<size_t>(M) * P * 8 * 16);
  stage_x<FMT, ORDER, XDT, M>(X, K, P, xs, sx);
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int ks = lane % G;
  const int rs = lane / G;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x / G) + (threadIdx.x >> 6) * (64 / G) + rs;
  const int64_t total = segs.end[2];
  const bool active = row < total;
  int sg = 0;
  if (row >= segs.end[0]) sg = (row >= segs.end[1]) ? 2 : 1;
  const int64_t lrow = row - (sg == 0 ? 0 : segs.end[sg - 1]);
  const int64_t rowbytes = static_cast<int64_t>(P) * Fmt<FMT>::PAIR_BYTES;
  const uint8_t *wrow = segs.W[sg] + lrow * rowbytes;

  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.f;

  if (active) {
    // U pairs in flight per lane: all loads of a batch are issued before any use.
    constexpr int U = FMT == FMT_Q4_0 ? 4 : 2;
    for (int p0 = ks; p0 < P; p0 += G * U) {
      uint32_t dw[U][Fmt<FMT>::PAIR_DWORDS];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int p = p0 + u * G;
        if (p < P) load_pair<FMT>(wrow + static_cast<int64_t>(p) * Fmt<FMT>::PAIR_BYTES, dw[u]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int p = p0 + u * G;
        if (p < P) pair_dot<FMT, M>(dw[u], xs, sx, P, p, acc);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) acc[m] += __shfl_xor(acc[m], off, 64);
  }
  if (active && ks == 0) {
    const int64_t N = segs.end[sg] - (sg == 0 ? 0 : segs.end[sg - 1]);
    void *Y = segs.Y[sg];
    const void *RS = segs.RS[sg];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int64_t i = m * N + lrow;
      switch (segs.ydt[sg]) {
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

template <int FMT, int ORDER, int XDT, int M>
static int launch_pair_m(const void *X, int64_t K, const Segs &segs, hipStream_t s) {
  const int64_t rows = segs.end[2];
  const int P = static_cast<int>(K / 64);
  const size_t lds = static_cast<size_t>(M) * P * (8 * 16 + 2 * 4);
  if (lds > static_cast<size_t>(kMaxLds)) return set_error(VYBDQ_ERR_SHAPE, "gemv: K too large for the LDS x stage at this M");
  // lanes per row: 8 keeps every BASELINE K (2560, 4096, 9728, 6144, 2048) a whole number of
  // pair sweeps; small row counts use 16 lanes to put more waves on the chip.
  constexpr int G = 8;
  int threads = 256;
  if (rows <= 4096) threads = 128;
  if (rows <= 1024) threads = 64;
  const int rows_per_wg = threads / G;
  const unsigned grid = static_cast<unsigned>((rows + rows_per_wg - 1) / rows_per_wg);
  if (lds > 64 * 1024) {
    static bool raised = false;  // one attribute call per instantiation
    if (!raised) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemv_pair<FMT, G, ORDER, XDT, M>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
      if (e != hipSuccess) return set_error(VYBDQ_ERR_HIP, std::string("gemv: LDS attribute: ") + hipGetErrorString(e));
      raised = true;
    }
  }
  hipLaunchKernelGGL((k_gemv_pair<FMT, G, ORDER, XDT, M>), dim3(grid), dim3(threads), lds, s, X, K, segs);
  return check_launch("gemv");
}

template <int FMT, int ORDER, int XDT>
static int launch_pair(const void *X, int64_t M, int64_t K, const Segs &segs, hipStream_t s) {
  switch (M) {
    case 1: return launch_pair_m<FMT, ORDER, XDT, 1>(X, K, segs, s);
    case 2: return launch_pair_m<FMT, ORDER, XDT, 2>(X, K, segs, s);
    case 3: return launch_pair_m<FMT, ORDER, XDT, 3>(X, K, segs, s);
    default: return launch_pair_m<FMT, ORDER, XDT, 4>(X, K, segs, s);
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
    int rc;
    VYBDQ_DISPATCH_IN(x_dt, XDT, rc = launch_pair<FMT, ORDER, XDT>(Xc, mc, K, sc, s));
    if (rc) return rc;
  }
  return VYBDQ_OK;
}

static int gemv_common(int fmt, int order, uint64_t X, int64_t M, int64_t K, int x_dt, Segs &segs,
                       uint64_t stream) {
  VYBDQ_REQUIRE(X, VYBDQ_ERR_ARG, "null X");
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
