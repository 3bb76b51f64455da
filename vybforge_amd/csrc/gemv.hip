// GEMV entry points on packed GGUF rows, gfx950: q4_0 / Q8_0 (the pair kernel of gemv_pair.h,
// and a reference-order fallback for K % 64 == 32), and the type-id dispatch vybdq_gemv that also
// reaches the K-quants (gemv_kq.hip).
#include "gemv_pair.h"

namespace vybdq {

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

template <int FMT, int ORDER>
static int gemv_dispatch(const void *X, int64_t M, int64_t K, int x_dt, Segs segs, hipStream_t s) {
  if (K % 64 != 0) {
    const unsigned grid = static_cast<unsigned>(segs.end[2]);
    VYBDQ_DISPATCH_IN(x_dt, XDT,
        hipLaunchKernelGGL((k_gemv_generic<FMT, ORDER, XDT>), dim3(grid), dim3(64), 0, s, X, M, K, segs));
    return check_launch("gemv(generic)");
  }
  return launch_pair_chunks<FMT, ORDER>(X, M, K, x_dt, segs, s);
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
      if (K % 64 == 0 || fmt >= FMT_Q4_K)
        VYBDQ_REQUIRE((reinterpret_cast<uintptr_t>(segs.W[i]) & 3) == 0, VYBDQ_ERR_ALIGN, "W must be 4-byte aligned");
    }
    acc += n;
    segs.end[i] = acc;
  }
  VYBDQ_REQUIRE(acc > 0, VYBDQ_ERR_SHAPE, "N must be > 0");
  VYBDQ_REQUIRE(acc < (int64_t(1) << 31), VYBDQ_ERR_SHAPE, "too many rows");
  const void *x = reinterpret_cast<const void *>(X);
  hipStream_t s = as_stream(stream);
  if (fmt == FMT_Q4_K || fmt == FMT_Q5_K || fmt == FMT_Q6_K || fmt == FMT_IQ2_S) {
    VYBDQ_REQUIRE(K % 256 == 0, VYBDQ_ERR_SHAPE, "K-quant rows need K % 256 == 0");
    return gemv_kq_dispatch(fmt, x, M, K, x_dt, segs, s);
  }
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

// GGML type id -> pair-kernel format, or -1
static int wtype_fmt(int wtype) {
  switch (wtype) {
    case 2: return FMT_Q4_0;
    case 8: return FMT_Q8_0;
    case 12: return FMT_Q4_K;
    case 13: return FMT_Q5_K;
    case 14: return FMT_Q6_K;
    case 22: return FMT_IQ2_S;
    default: return -1;
  }
}

extern "C" int vybdq_gemv(int wtype, uint64_t W, uint64_t X, uint64_t Y, int64_t M, int64_t N, int64_t K,
                          int x_dt, int y_dt, uint64_t RS, uint64_t stream) {
  const int fmt = wtype_fmt(wtype);
  if (fmt < 0)
    return set_error(VYBDQ_ERR_ARG, "vybdq_gemv: wtype must be 2 (q4_0), 8 (Q8_0), 12 (Q4_K), 13 (Q5_K), 14 (Q6_K) or 22 (IQ2_S)");
  Segs s = one_seg(W, Y, RS, N, y_dt);
  return gemv_common(fmt, VYBDQ_Q4_GGML, X, M, K, x_dt, s, stream);
}

extern "C" int vybdq_gemv_seg3(int wtype, uint64_t X, int64_t M, int64_t K, int x_dt,
                               uint64_t W, uint64_t Y, int64_t N, int y_dt, uint64_t RS,
                               uint64_t W2, uint64_t Y2, int64_t N2, int y_dt2, uint64_t RS2,
                               uint64_t W3, uint64_t Y3, int64_t N3, int y_dt3, uint64_t RS3, uint64_t stream) {
  const int fmt = wtype_fmt(wtype);
  if (fmt < 0)
    return set_error(VYBDQ_ERR_ARG, "vybdq_gemv_seg3: wtype must be 2 (q4_0), 8 (Q8_0), 12 (Q4_K), 13 (Q5_K), 14 (Q6_K) or 22 (IQ2_S)");
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
  return gemv_common(fmt, VYBDQ_Q4_GGML, X, M, K, x_dt, s, stream);
}
