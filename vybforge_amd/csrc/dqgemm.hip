// Dequant GEMM on packed GGUF rows with fp16 MFMA, gfx950: prefill projections and the grouped
// (per-expert) MoE GEMMs.
//
// Y[r, n] = epilogue( sum_k X[map(r), k] * W_g[n, k] ) for the rows r of group g.
//
// A group is one weight matrix (an expert; one group for a plain GEMM) and a contiguous range
// of output rows. Groups, their row ranges and their tile counts live in device memory (the
// MoE bucketing kernel writes them), so a whole MoE layer is launched without host syncs.
// The grid is sized for the worst case; workgroups whose tile index falls past the last group's
// tiles exit at once.
//
// Per K step (KP block pairs of 64 k, KP chosen so that the BN weight rows give every thread one
// 32-weight block): each thread dequantizes its block to fp16 (d * (q - OFF) computed exactly in
// fp16 then rounded once by the scale multiply) into LDS, X rows are gathered, converted to fp16
// and staged into LDS, and every wave issues v_mfma_f32_16x16x32_f16 over its 16x16 sub-tiles.
// Each thread keeps D steps of weight loads in flight (a register ring) and prefetches the next
// step's X before the MFMAs, so HBM latency is overlapped across steps. A last step with fewer
// than KP pairs is zero-filled. X is converted to fp16: activations must stay below 65504 in
// magnitude.
//
// Epilogues: STORE (f32/f16/bf16/f64, optional residual of the output type) and SWIGLU: the
// workgroup's weight rows are BN/2 rows of the gate matrix and the same BN/2 rows of the up
// matrix, and y = silu(min(g, L)) * clamp(u, -L, L) (native/glm53/moe_ref.py:81-84).
#include "gemv_dev.h"

#include <type_traits>

namespace vybdq {

typedef _Float16 hf8 __attribute__((ext_vector_type(8)));

enum { EPI_STORE = 0, EPI_SWIGLU = 1 };

// the MFMA GEMM with weights in operand registers (mmq_host.hip)
bool mmq_supported(int64_t M, int64_t N, int64_t K);
int64_t mmq_workspace_size(int wtype, int64_t M, int64_t N, int64_t K);
int mmq_gemm(int wtype, const void *W, const void *X, int xdt, void *Y, int ydt, int64_t M, int64_t N, int64_t K,
             int64_t ldy, const void *RS, void *ws, int64_t ws_bytes, hipStream_t s);
int64_t mmq_i8_workspace_size(int64_t M, int64_t N, int64_t K);
// the super-block (Q4_K, Q5_K, Q6_K, IQ2_S) GEMM (kqgemm.hip)
int64_t kq2_workspace_size(int wtype, int64_t M, int64_t N, int64_t K);
int kq2_gemm(int wtype, const void *W, const void *X, int xdt, void *Y, int ydt, int64_t M, int64_t N, int64_t K,
             int64_t ldy, const void *RS, void *ws, int64_t ws_bytes, hipStream_t s);
int kq_gemm(int wtype, const void *W, const void *X, int xdt, void *Y, int ydt, int64_t M, int64_t N, int64_t K,
            int64_t ldy, const void *RS, hipStream_t s);
int mmq_i8_gemm(const void *W, const int8_t *Xq, const float *Xs, void *Y, int ydt, int64_t M, int64_t N, int64_t K,
                int64_t ldy, const void *RS, void *ws, int64_t ws_bytes, hipStream_t s);

struct GemmArgs {
  const uint8_t *W;       // group g's matrix at W + g * w_stride (gate matrix for SWIGLU)
  const uint8_t *W2;      // SWIGLU: up matrix, same layout
  int64_t w_stride;       // bytes between consecutive groups' matrices
  const void *X;
  int xdt;
  int64_t ldx;            // elements between X rows
  const int *row_map;     // output row -> X row (null: identity)
  const int *grp_rows;    // [G+1] output row ranges (null: one group of M rows)
  const int *grp_tiles;   // [G+1] cumulative m-tile counts (null: one group)
  const int *grp_ids;     // [G] matrix index of group g (null: g)
  int G;
  int M;                  // rows when grp_rows is null
  int N;                  // output columns (weight rows per matrix; SWIGLU: rows of gate = of up)
  int64_t K;
  void *Y;
  int ydt;
  int64_t ldy;
  const void *RS;
  float limit;            // SWIGLU clamp
};

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }

// dequantize one 32-weight block (qs dwords q[0..QDW-1], scale bits d16) to 32 fp16 in k order
template <int FMT, int ORDER>
__device__ __forceinline__ void dequant_block_f16(const uint32_t (&q)[Fmt<FMT>::QDW], uint32_t d16, h2 (&out)[16]) {
  h2 wv[16];
  unpack_block<FMT, ORDER>(q, wv);  // (OFF' + v) pairs in element order
  const _Float16 d = __builtin_bit_cast(_Float16, static_cast<uint16_t>(d16));
  const h2 dd = {d, d};
  constexpr float corr = FMT == FMT_Q4_0 ? 1032.0f : 1152.0f;
  const h2 off = {static_cast<_Float16>(-corr), static_cast<_Float16>(-corr)};
#pragma unroll
  for (int i = 0; i < 16; ++i) out[i] = (wv[i] + off) * dd;  // exact (q - OFF), one rounding
}

// X chunk (8 consecutive k of one row at element offset off) -> 8 fp16 in a u4
template <int XDT>
__device__ __forceinline__ u4 load_x8_f16(const void *X, int64_t off) {
  u4 hv;
  if constexpr (XDT == VYBDQ_F16) {
    hv = *reinterpret_cast<const u4 *>(static_cast<const _Float16 *>(X) + off);
  } else if constexpr (XDT == VYBDQ_BF16) {
    const u4 v = *reinterpret_cast<const u4 *>(static_cast<const uint16_t *>(X) + off);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = v[j];
      hv[j] = __builtin_bit_cast(uint32_t, h2{static_cast<_Float16>(__uint_as_float(w << 16)),
                                              static_cast<_Float16>(__uint_as_float(w & 0xffff0000u))});
    }
  } else {
    const f4 *src = reinterpret_cast<const f4 *>(static_cast<const float *>(X) + off);
    const f4 x0 = src[0], x1 = src[1];
    hv[0] = __builtin_bit_cast(uint32_t, h2{static_cast<_Float16>(x0[0]), static_cast<_Float16>(x0[1])});
    hv[1] = __builtin_bit_cast(uint32_t, h2{static_cast<_Float16>(x0[2]), static_cast<_Float16>(x0[3])});
    hv[2] = __builtin_bit_cast(uint32_t, h2{static_cast<_Float16>(x1[0]), static_cast<_Float16>(x1[1])});
    hv[3] = __builtin_bit_cast(uint32_t, h2{static_cast<_Float16>(x1[2]), static_cast<_Float16>(x1[3])});
  }
  return hv;
}

template <int FMT, int ORDER, int XDT, int BM, int BN, int EPI>
__global__ void __launch_bounds__(256) k_dq_gemm(GemmArgs a) {
  // KP weight pairs (64 k each) per step so that BN rows x 2 blocks x KP = 256 block tasks
  constexpr int KP = BN * 2 >= 256 ? 1 : 256 / (BN * 2);
  constexpr int BK = 64 * KP;
  static_assert(BN * 2 * KP == 256, "one 32-weight block per thread per step");
  constexpr int LDA = BK + 8;  // fp16 row stride in LDS (pad: 16 B)
  constexpr int PD = Fmt<FMT>::PAIR_DWORDS;
  constexpr int QDW = Fmt<FMT>::QDW;
  constexpr int NT = BN / 64;  // 16-column MFMA tiles per wave (4 waves split BN)
  constexpr int MT = BM / 16;
  constexpr int D = FMT == FMT_Q4_0 ? 4 : 2;  // weight steps in flight per thread
  constexpr int XC = (BM * BK / 8 + 255) / 256;  // X chunks (8 k) per thread per step
  __shared__ __attribute__((aligned(16))) _Float16 As[BM * LDA];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[BN * LDA];

  // ---- locate (group, m-tile, n-tile)
  const int n_tiles = (EPI == EPI_SWIGLU ? a.N * 2 : a.N) / BN;
  const int ntile = blockIdx.x % n_tiles;
  const int mt_global = blockIdx.x / n_tiles;
  int g = 0, row0 = 0, rows = a.M;
  if (a.grp_tiles) {
    const int total = a.grp_tiles[a.G];
    if (mt_global >= total) return;
    int lo = 0, hi = a.G - 1;  // last group with grp_tiles[g] <= mt_global (skips empty groups)
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (a.grp_tiles[mid] <= mt_global) lo = mid; else hi = mid - 1;
    }
    g = lo;
    row0 = a.grp_rows[g] + (mt_global - a.grp_tiles[g]) * BM;
    rows = a.grp_rows[g + 1] - row0;
  } else {
    row0 = mt_global * BM;
    rows = a.M - row0;
    if (rows <= 0) return;
  }
  if (rows > BM) rows = BM;
  const int mat = a.grp_ids ? a.grp_ids[g] : g;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int P = static_cast<int>(a.K >> 6);
  const int S = (P + KP - 1) / KP;  // K steps; the last one may hold fewer than KP pairs
  const int64_t rowbytes = static_cast<int64_t>(P) * Fmt<FMT>::PAIR_BYTES;

  // ---- dequant task: weight row br, pair kp of the step, block bh of the pair
  const int br = tid / (2 * KP);
  const int kp = (tid / 2) % KP;
  const int bh = tid & 1;
  const uint8_t *wrow;
  {
    int n = ntile * BN + br;
    const uint8_t *base = a.W;
    if constexpr (EPI == EPI_SWIGLU) {
      // rows [0, BN/2) of the tile: gate rows; [BN/2, BN): the same rows of up
      const int half = BN / 2;
      n = ntile * half + (br % half);
      if (br >= half) base = a.W2;
    }
    wrow = base + static_cast<int64_t>(mat) * a.w_stride + static_cast<int64_t>(n) * rowbytes;
  }
  auto wptr = [&](int step) {
    int pi = step * KP + kp;
    pi = pi < P ? pi : P - 1;  // loads past the end re-read the last pair
    return wrow + static_cast<int64_t>(pi) * Fmt<FMT>::PAIR_BYTES;
  };
  // ---- X task: chunks c = tid + 256 i of the BM x BK tile. Row offsets (through row_map) are
  // resolved once here: a dependent index load inside the K loop would make the wait for it
  // drain every weight load in flight. Loads are unconditional: tile rows past `rows` read row
  // row0 (they only feed output rows that are never stored) and k past K (a last step with
  // fewer than KP pairs) re-reads k - 64, which meets zero weights.
  int64_t xbase[XC];
  int xk[XC];
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = tid + 256 * i;
    const int m = c / (BK / 8), kc = c % (BK / 8);
    const int r = row0 + (c < BM * BK / 8 && m < rows ? m : 0);
    const int64_t xr = a.row_map ? a.row_map[r] : r;
    xbase[i] = xr * a.ldx;
    xk[i] = 8 * kc;
  }
  auto x_off = [&](int i, int step) {
    int64_t k = static_cast<int64_t>(step) * BK + xk[i];
    k = k < a.K ? k : k - 64;
    return xbase[i] + k;
  };

  f4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  // ring of D steps: X and weights of step s + D are issued, in that order, when step s is consumed
  // (loads complete in issue order, so X fetched one step ahead would make every wait for it also
  // wait for the weight loads issued before it); the prologue issues in the same order
  uint32_t dw[D][PD];
  u4 xr[D][XC];
#pragma unroll
  for (int d = 0; d < D; ++d) {
#pragma unroll
    for (int i = 0; i < XC; ++i) xr[d][i] = load_x8_f16<XDT>(a.X, x_off(i, d < S ? d : S - 1));
    load_pair<FMT>(wptr(d), dw[d]);
    // keep the issue order (the scheduler would otherwise interleave the stages, and the loop's
    // first wait would then have to drain them all)
    __builtin_amdgcn_sched_barrier(0);
  }

  // one K step from ring slot DC; REFILL: issue the loads of step + D into the slot
  auto k_step = [&](auto dc, auto refill, int step) {
    constexpr int d = decltype(dc)::value;
    // weights of this step -> LDS (block bh of the pair, branch-free: bh differs between lanes)
    {
      uint32_t q[QDW];
#pragma unroll
      for (int t = 0; t < QDW; ++t)
        q[t] = bh ? dw[d][QDW + 1 + t] : __builtin_amdgcn_alignbit(dw[d][t + 1], dw[d][t], 16);
      uint32_t d16 = bh ? dw[d][QDW] >> 16 : dw[d][0] & 0xffffu;
      if (KP > 1) d16 = step * KP + kp < P ? d16 : 0u;  // pair past the end: zero scale, zero weights
      h2 w16[16];
      dequant_block_f16<FMT, ORDER>(q, d16, w16);
      u4 *dst = reinterpret_cast<u4 *>(Bs + br * LDA + 64 * kp + 32 * bh);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        dst[i] = u4{__builtin_bit_cast(uint32_t, w16[4 * i]), __builtin_bit_cast(uint32_t, w16[4 * i + 1]),
                    __builtin_bit_cast(uint32_t, w16[4 * i + 2]), __builtin_bit_cast(uint32_t, w16[4 * i + 3])};
    }
    // X of this step -> LDS
#pragma unroll
    for (int i = 0; i < XC; ++i) {
      const int c = tid + 256 * i;
      if (c < BM * BK / 8) *reinterpret_cast<u4 *>(As + (c / (BK / 8)) * LDA + 8 * (c % (BK / 8))) = xr[d][i];
    }
    if constexpr (decltype(refill)::value) {
      const int nx = step + D < S ? step + D : S - 1;  // past the end: re-read the last step (cache hits)
#pragma unroll
      for (int i = 0; i < XC; ++i) xr[d][i] = load_x8_f16<XDT>(a.X, x_off(i, nx));
      load_pair<FMT>(wptr(step + D), dw[d]);
    }
    __syncthreads();
    // MFMA: wave owns weight rows [wave*BN/4, (wave+1)*BN/4)
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
      hf8 bf[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int n = wave * (BN / 4) + 16 * j + (lane & 15);
        bf[j] = *reinterpret_cast<const hf8 *>(Bs + n * LDA + 32 * kk + 8 * (lane >> 4));
      }
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int m = 16 * i + (lane & 15);
        const hf8 af = *reinterpret_cast<const hf8 *>(As + m * LDA + 32 * kk + 8 * (lane >> 4));
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[i][j], 0, 0, 0);
      }
    }
    __syncthreads();
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  using Yes = std::true_type;
  using No = std::false_type;
  static_assert(D == 2 || D == 4, "ring depth");
  // steady state: whole groups of D steps, every path through the body issues the same loads in
  // the same order, so the waits at the top stay partial; the tail has no back edge
  int s0 = 0;
  for (; s0 + D <= S; s0 += D) {
    k_step(I0{}, Yes{}, s0);
    k_step(I1{}, Yes{}, s0 + 1);
    if constexpr (D == 4) {
      k_step(I2{}, Yes{}, s0 + 2);
      k_step(I3{}, Yes{}, s0 + 3);
    }
  }
  if (s0 < S) k_step(I0{}, No{}, s0);
  if (s0 + 1 < S) k_step(I1{}, No{}, s0 + 1);
  if constexpr (D == 4) {
    if (s0 + 2 < S) k_step(I2{}, No{}, s0 + 2);
  }

  // ---- epilogue: acc[i][j][r] = C[m = 16i + 4(lane>>4) + r][n = wave*BN/4 + 16j + (lane&15)]
  if constexpr (EPI == EPI_STORE) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 16 * i + 4 * (lane >> 4) + r;
          if (m >= rows) continue;
          const int64_t n = static_cast<int64_t>(ntile) * BN + wave * (BN / 4) + 16 * j + (lane & 15);
          const int64_t idx = static_cast<int64_t>(row0 + m) * a.ldy + n;
          switch (a.ydt) {
            case VYBDQ_F32: store_elem<VYBDQ_F32>(a.Y, a.RS, idx, acc[i][j][r]); break;
            case VYBDQ_F16: store_elem<VYBDQ_F16>(a.Y, a.RS, idx, acc[i][j][r]); break;
            case VYBDQ_BF16: store_elem<VYBDQ_BF16>(a.Y, a.RS, idx, acc[i][j][r]); break;
            default: store_elem<VYBDQ_F64>(a.Y, a.RS, idx, acc[i][j][r]); break;
          }
        }
  } else {
    // gate rows live in waves 0,1 and the matching up rows in waves 2,3 (BN/4 rows each):
    // exchange the up half through LDS, then waves 0,1 apply the clamped SwiGLU
    float *ex = reinterpret_cast<float *>(As);  // reuse: needs BM * BN/2 floats
    static_assert(BM * (BN / 2) * 4 <= BM * LDA * 2, "exchange buffer too small");
    if (wave >= 2) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = 16 * i + 4 * (lane >> 4) + r;
            const int c = (wave - 2) * (BN / 4) + 16 * j + (lane & 15);
            ex[m * (BN / 2) + c] = acc[i][j][r];
          }
    }
    __syncthreads();
    if (wave < 2) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = 16 * i + 4 * (lane >> 4) + r;
            if (m >= rows) continue;
            const int c = wave * (BN / 4) + 16 * j + (lane & 15);
            float gv = acc[i][j][r];
            float uv = ex[m * (BN / 2) + c];
            gv = fminf(gv, a.limit);
            uv = fminf(fmaxf(uv, -a.limit), a.limit);
            const float y = silu_f(gv) * uv;
            const int64_t n = static_cast<int64_t>(ntile) * (BN / 2) + c;
            const int64_t idx = static_cast<int64_t>(row0 + m) * a.ldy + n;
            switch (a.ydt) {
              case VYBDQ_F32: store_elem<VYBDQ_F32>(a.Y, nullptr, idx, y); break;
              case VYBDQ_F16: store_elem<VYBDQ_F16>(a.Y, nullptr, idx, y); break;
              default: store_elem<VYBDQ_BF16>(a.Y, nullptr, idx, y); break;
            }
          }
    }
  }
}

template <int FMT, int ORDER, int XDT, int BM, int BN, int EPI>
static int launch_dq(const GemmArgs &a, int max_mtiles, hipStream_t s) {
  const int n_tiles = (EPI == EPI_SWIGLU ? a.N * 2 : a.N) / BN;
  const int64_t grid = static_cast<int64_t>(max_mtiles) * n_tiles;
  if (grid <= 0) return VYBDQ_OK;
  if (grid >= (int64_t(1) << 31)) return set_error(VYBDQ_ERR_SHAPE, "dq gemm: grid too large");
  hipLaunchKernelGGL((k_dq_gemm<FMT, ORDER, XDT, BM, BN, EPI>), dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, a);
  return check_launch("dq gemm");
}

template <int FMT, int BM, int BN, int EPI>
static int launch_x(const GemmArgs &a, int max_mtiles, hipStream_t s) {
  switch (a.xdt) {
    case VYBDQ_F16: return launch_dq<FMT, VYBDQ_Q4_GGML, VYBDQ_F16, BM, BN, EPI>(a, max_mtiles, s);
    case VYBDQ_BF16: return launch_dq<FMT, VYBDQ_Q4_GGML, VYBDQ_BF16, BM, BN, EPI>(a, max_mtiles, s);
    default: return launch_dq<FMT, VYBDQ_Q4_GGML, VYBDQ_F32, BM, BN, EPI>(a, max_mtiles, s);
  }
}

// Plain GEMM: Y [M, N] = X [M, K] W^T (+ RS). BM chosen by M.
template <int FMT>
static int gemm_plain(GemmArgs a, hipStream_t s) {
  if (a.M >= 128) return launch_x<FMT, 128, 128, EPI_STORE>(a, (a.M + 127) / 128, s);
  if (a.M >= 64) return launch_x<FMT, 64, 128, EPI_STORE>(a, (a.M + 63) / 64, s);
  return launch_x<FMT, 16, 64, EPI_STORE>(a, (a.M + 15) / 16, s);
}

// Grouped entry used by the MoE pipeline: BM = 16 token rows per tile, BN = 64 weight rows.
int dq_gemm_bm() { return 16; }

int dq_gemm_grouped(int wtype, bool swiglu, const uint8_t *W, const uint8_t *W2, int64_t w_stride, const void *X,
                    int xdt, int64_t ldx, const int *row_map, const int *grp_rows, const int *grp_tiles, int G,
                    int M, int N, int64_t K, void *Y, int ydt, int64_t ldy, float limit, int max_mtiles,
                    hipStream_t s) {
  GemmArgs a{};
  a.W = W;
  a.W2 = W2;
  a.w_stride = w_stride;
  a.X = X;
  a.xdt = xdt;
  a.ldx = ldx;
  a.row_map = row_map;
  a.grp_rows = grp_rows;
  a.grp_tiles = grp_tiles;
  a.G = G;
  a.M = M;
  a.N = N;
  a.K = K;
  a.Y = Y;
  a.ydt = ydt;
  a.ldy = ldy;
  a.limit = limit;
  if (swiglu) {
    if (wtype == 2) return launch_x<FMT_Q4_0, 16, 64, EPI_SWIGLU>(a, max_mtiles, s);
    return launch_x<FMT_Q8_0, 16, 64, EPI_SWIGLU>(a, max_mtiles, s);
  }
  if (wtype == 2) return launch_x<FMT_Q4_0, 16, 64, EPI_STORE>(a, max_mtiles, s);
  return launch_x<FMT_Q8_0, 16, 64, EPI_STORE>(a, max_mtiles, s);
}

}  // namespace vybdq

using namespace vybdq;

static int gemm_check(int wtype, uint64_t W, uint64_t X, uint64_t Y, int64_t M, int64_t N, int64_t K, int x_dt,
                      int y_dt, int64_t ldy) {
  VYBDQ_REQUIRE(W && X && Y, VYBDQ_ERR_ARG, "null W, X or Y");
  VYBDQ_REQUIRE(wtype == 2 || wtype == 8 || wtype == 12 || wtype == 13 || wtype == 14 || wtype == 22, VYBDQ_ERR_ARG,
                "wtype must be 2 (q4_0), 8 (Q8_0), 12 (Q4_K), 13 (Q5_K), 14 (Q6_K) or 22 (IQ2_S)");
  VYBDQ_REQUIRE(dt_valid_in(x_dt), VYBDQ_ERR_ARG, "x_dt must be F32, F16 or BF16");
  VYBDQ_REQUIRE(dt_valid_out(y_dt), VYBDQ_ERR_ARG, "y_dt must be F32, F16, BF16 or F64");
  VYBDQ_REQUIRE(M >= 1 && M < (1 << 24), VYBDQ_ERR_SHAPE, "M out of range");
  if (wtype >= 12) {  // super-block types: K % 256 == 0, tiles of 64 weight rows
    VYBDQ_REQUIRE(K >= 256 && K % 256 == 0 && K < (1 << 24), VYBDQ_ERR_SHAPE,
                  "super-block types need K a positive multiple of 256");
    VYBDQ_REQUIRE(N >= 64 && N % 64 == 0 && N < (1 << 24), VYBDQ_ERR_SHAPE,
                  "super-block types need N a positive multiple of 64");
    VYBDQ_REQUIRE(M * K < (int64_t(1) << 40), VYBDQ_ERR_SHAPE, "M * K too large");
    VYBDQ_REQUIRE(ldy == 0 || ldy >= N, VYBDQ_ERR_SHAPE, "ldy must be 0 (= N) or >= N");
    VYBDQ_REQUIRE((W & 3) == 0 && (X & 15) == 0, VYBDQ_ERR_ALIGN, "W must be 4-byte and X 16-byte aligned");
    return VYBDQ_OK;
  }
  VYBDQ_REQUIRE(K >= 64 && K % 64 == 0, VYBDQ_ERR_SHAPE, "K must be a positive multiple of 64");
  VYBDQ_REQUIRE(N >= 16 && N % 16 == 0 && N < (1 << 24), VYBDQ_ERR_SHAPE, "N must be a positive multiple of 16");
  VYBDQ_REQUIRE(N % 64 == 0 || (M >= 64 && mmq_supported(M, N, K)), VYBDQ_ERR_SHAPE,
                "N must be a multiple of 64 unless M >= 64 and K % 256 == 0");
  VYBDQ_REQUIRE(ldy == 0 || ldy >= N, VYBDQ_ERR_SHAPE, "ldy must be 0 (= N) or >= N");
  VYBDQ_REQUIRE((W & 3) == 0 && (X & 15) == 0, VYBDQ_ERR_ALIGN, "W must be 4-byte and X 16-byte aligned");
  return VYBDQ_OK;
}

extern "C" int64_t vybdq_gemm_workspace_size(int wtype, int64_t M, int64_t N, int64_t K) {
  if (wtype == 14 || wtype == 22) return M >= 1 && N >= 64 && K >= 256 ? kq2_workspace_size(wtype, M, N, K) : 0;
  if ((wtype != 2 && wtype != 8 && wtype != 12 && wtype != 13) || M < 64 || !mmq_supported(M, N, K)) return 0;
  return mmq_workspace_size(wtype, M, N, K);
}

extern "C" int vybdq_gemm_ws(int wtype, uint64_t W, uint64_t X, uint64_t Y, int64_t M, int64_t N, int64_t K,
                             int x_dt, int y_dt, int64_t ldy, uint64_t RS, uint64_t ws, int64_t ws_bytes,
                             uint64_t stream) {
  const int rc = gemm_check(wtype, W, X, Y, M, N, K, x_dt, y_dt, ldy);
  if (rc) return rc;
  VYBDQ_REQUIRE(ws == 0 || (ws & 255) == 0, VYBDQ_ERR_ALIGN, "workspace must be 256-byte aligned");
  VYBDQ_REQUIRE(ws_bytes >= 0, VYBDQ_ERR_WORKSPACE, "negative workspace size");
  // Q4_K / Q5_K: the register-operand body streams fp16 X, so bf16 / f32 X needs room for its
  // conversion
  const bool q4k_ok = (wtype == 12 || wtype == 13) && M >= 64 && K < (int64_t(1) << 22) && mmq_supported(M, N, K) &&
                      (x_dt == VYBDQ_F16 || (ws && ws_bytes >= mmq_workspace_size(wtype, M, N, K)));
  if (wtype == 14 || wtype == 22) {  // 128-row tiles over the workspace's fp16 copy of X
    const int r = kq2_gemm(wtype, reinterpret_cast<const void *>(W), reinterpret_cast<const void *>(X), x_dt,
                           reinterpret_cast<void *>(Y), y_dt, M, N, K, ldy ? ldy : N,
                           reinterpret_cast<const void *>(RS), ws ? reinterpret_cast<void *>(ws) : nullptr,
                           ws ? ws_bytes : 0, as_stream(stream));
    if (r != 1) return r;
  }
  if ((wtype <= 8 && M >= 64 && mmq_supported(M, N, K)) || q4k_ok)
    return mmq_gemm(wtype, reinterpret_cast<const void *>(W), reinterpret_cast<const void *>(X), x_dt,
                    reinterpret_cast<void *>(Y), y_dt, M, N, K, ldy ? ldy : N, reinterpret_cast<const void *>(RS),
                    ws ? reinterpret_cast<void *>(ws) : nullptr, ws ? ws_bytes : 0, as_stream(stream));
  return vybdq_gemm(wtype, W, X, Y, M, N, K, x_dt, y_dt, ldy, RS, stream);
}

extern "C" int vybdq_gemm(int wtype, uint64_t W, uint64_t X, uint64_t Y, int64_t M, int64_t N, int64_t K,
                          int x_dt, int y_dt, int64_t ldy, uint64_t RS, uint64_t stream) {
  const int rc = gemm_check(wtype, W, X, Y, M, N, K, x_dt, y_dt, ldy);
  if (rc) return rc;
  GemmArgs a{};
  a.W = reinterpret_cast<const uint8_t *>(W);
  a.X = reinterpret_cast<const void *>(X);
  a.xdt = x_dt;
  a.ldx = K;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.K = K;
  a.Y = reinterpret_cast<void *>(Y);
  a.ydt = y_dt;
  a.ldy = ldy ? ldy : N;
  a.RS = reinterpret_cast<const void *>(RS);
  a.G = 1;
  hipStream_t s = as_stream(stream);
  // Q4_K / Q5_K from 64 rows with fp16 X: the register-operand tile body (with a workspace any X
  // type, vybdq_gemm_ws); the other super-block types and the other calls decode tiles into LDS
  if ((wtype == 12 || wtype == 13) && x_dt == VYBDQ_F16 && M >= 64 && K < (int64_t(1) << 22) &&
      mmq_supported(M, N, K))
    return mmq_gemm(wtype, a.W, a.X, x_dt, a.Y, y_dt, M, N, K, a.ldy, a.RS, nullptr, 0, s);
  // fp16 / bf16 X from 96 rows (Q4_K / Q5_K: bf16, fp16 took the register body above): 128-row tiles
  if ((wtype == 14 || wtype == 22) ? x_dt != VYBDQ_F32 : (wtype >= 12 && x_dt == VYBDQ_BF16)) {
    const int r = kq2_gemm(wtype, a.W, a.X, x_dt, a.Y, y_dt, M, N, K, a.ldy, a.RS, nullptr, 0, s);
    if (r != 1) return r;
  }
  if (wtype >= 12) return kq_gemm(wtype, a.W, a.X, x_dt, a.Y, y_dt, M, N, K, a.ldy, a.RS, s);
  if (M >= 64 && mmq_supported(M, N, K))
    return mmq_gemm(wtype, a.W, a.X, x_dt, a.Y, y_dt, M, N, K, a.ldy, a.RS, nullptr, 0, s);
  if (N % 128 != 0 || M < 64) {
    if (wtype == 2) return launch_x<FMT_Q4_0, 16, 64, EPI_STORE>(a, static_cast<int>((M + 15) / 16), s);
    return launch_x<FMT_Q8_0, 16, 64, EPI_STORE>(a, static_cast<int>((M + 15) / 16), s);
  }
  if (wtype == 2) return gemm_plain<FMT_Q4_0>(a, s);
  return gemm_plain<FMT_Q8_0>(a, s);
}

extern "C" int64_t vybdq_gemm_q8_0_i8_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || !mmq_supported(M, N, K)) return 0;
  return mmq_i8_workspace_size(M, N, K);
}

extern "C" int vybdq_gemm_q8_0_i8(uint64_t W, uint64_t Xq, uint64_t Xs, uint64_t Y, int64_t M, int64_t N, int64_t K,
                                  int y_dt, int64_t ldy, uint64_t RS, uint64_t ws, int64_t ws_bytes, uint64_t stream) {
  VYBDQ_REQUIRE(W && Xq && Xs && Y, VYBDQ_ERR_ARG, "null W, Xq, Xs or Y");
  VYBDQ_REQUIRE(dt_valid_out(y_dt), VYBDQ_ERR_ARG, "y_dt must be F32, F16, BF16 or F64");
  VYBDQ_REQUIRE(M >= 1 && M < (1 << 24), VYBDQ_ERR_SHAPE, "M out of range");
  VYBDQ_REQUIRE(K >= 256 && K % 256 == 0, VYBDQ_ERR_SHAPE, "K must be a positive multiple of 256");
  VYBDQ_REQUIRE(N >= 16 && N % 16 == 0 && N < (1 << 24), VYBDQ_ERR_SHAPE, "N must be a positive multiple of 16");
  VYBDQ_REQUIRE(M * K < (int64_t(1) << 31), VYBDQ_ERR_SHAPE, "M * K too large");
  VYBDQ_REQUIRE(ldy == 0 || ldy >= N, VYBDQ_ERR_SHAPE, "ldy must be 0 (= N) or >= N");
  VYBDQ_REQUIRE((W & 15) == 0 && (Xq & 15) == 0 && (Xs & 15) == 0, VYBDQ_ERR_ALIGN,
                "W, Xq and Xs must be 16-byte aligned");
  VYBDQ_REQUIRE(ws == 0 || (ws & 255) == 0, VYBDQ_ERR_ALIGN, "workspace must be 256-byte aligned");
  return mmq_i8_gemm(reinterpret_cast<const void *>(W), reinterpret_cast<const int8_t *>(Xq),
                     reinterpret_cast<const float *>(Xs), reinterpret_cast<void *>(Y), y_dt, M, N, K, ldy ? ldy : N,
                     reinterpret_cast<const void *>(RS), ws ? reinterpret_cast<void *>(ws) : nullptr, ws ? ws_bytes : 0,
                     as_stream(stream));
}

