// Grouped multi-token dequant GEMV for the MoE experts when each expert receives few tokens
// (decode-sized batches), gfx950.
//
// Work unit: (group a, block of output columns). A group is an expert that received tokens (or
// the shared expert) with its rows [r0, r1) of the bucketed row order; row_map gives each row's
// token. The workgroup stages the x rows of its (at most MC) tokens into LDS (fp16 + block sums,
// the layout pair_dot reads) and then walks its weight rows in passes of T/G rows, G lanes per row
// reading consecutive pairs (one contiguous run of the row per load instruction), with the next
// passes' pair windows in flight while the current pass computes (a register ring). The bucketing splits experts with
// more rows into groups of MC rows over the same weights (the kernel would otherwise repeat the
// walk per chunk of MC tokens).
//
// SwiGLU (gate|up): each wave holds gate rows in its first 32 lanes and the up rows of the same
// output columns in its last 32, so after the DPP row reduction the pair (g, u) is one lane
// exchange apart; the epilogue writes silu(min(g, L)) * clamp(u, -L, L) as fp16
// (native/glm53/moe_ref.py:81-84). Otherwise the row sums are stored as f32.
#pragma once
#include "gemv_dev.h"

namespace vybdq {

struct MoeGvArgs {
  const uint8_t *W, *W2;   // expert 0's matrix (SWI: gate, up); expert e at + e * w_stride
  int64_t w_stride;
  const uint8_t *Ws, *W2s; // the shared expert's matrices
  int64_t rowbytes;
  int P;                   // pairs per row (K = 64 P)
  const void *X;
  int xdt;
  int64_t ldx;             // elements between X rows
  const int *row_map;      // row -> X row (null: the row itself)
  const int4 *groups;      // {expert (-1 shared), r0, r1, -}
  const int *ngroups;
  int N;                   // output columns
  int cols_per_wg;         // output columns per workgroup
  void *Y;
  int ydt;                 // F16 or F32
  int64_t ldy;
  float limit;
  int mc;                  // tokens per group (x stage), 1..kMoeGvMC
};

constexpr int kMoeGvMC = 4;  // largest x stage
constexpr int kMoeGvD = 3;   // passes of pair windows in flight per lane (a register ring)

__device__ __forceinline__ float moe_silu(float g) { return g / (1.0f + __expf(-g)); }

// One chunk of MC tokens (rows r0c .. r0c + MC - 1) over the workgroup's columns.
template <int FMT, int G, int U, int MC, bool SWI, int XW>
__device__ __forceinline__ void moe_gv_chunk(const MoeGvArgs &a, const uint8_t *Wg, const uint8_t *Wu, int r0c,
                                             int n0, int ncols, char *lds, float *sx) {
  constexpr int PD = Fmt<FMT>::PAIR_DWORDS;
  constexpr int T = 256;
  const int P = a.P;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int ks = lane % G;
  const int rs = lane / G;  // row slot within the wave
  constexpr int RPW = 64 / G;                 // rows per wave per pass
  constexpr int CPW = SWI ? RPW / 2 : RPW;    // output columns per wave per pass
  static_assert(!SWI || RPW >= 2, "SwiGLU needs a gate and an up row per wave");
  constexpr int CPP = 4 * CPW;                // columns per pass
  // this lane's column offset within the pass and its matrix
  const bool up = SWI && rs >= RPW / 2;
  const int cslot = w * CPW + (up ? rs - RPW / 2 : rs);
  const uint8_t *Wm = up ? Wu : Wg;

  // x rows of the chunk -> LDS (fp16 pairs + block sums)
  __syncthreads();  // the previous chunk's readers are done
  const int nchunk = MC * 8 * P;
  for (int c = threadIdx.x; c < nchunk; c += T) {
    const int m = c / (8 * P);
    const int xr = a.row_map ? a.row_map[r0c + m] : r0c + m;
    uint32_t r[XW];
    load_x_chunk<XW>(a.X, static_cast<int64_t>(xr) * a.ldx + 8 * static_cast<int64_t>(c - m * 8 * P), r);
    stage_chunk<XW>(r, a.xdt, c, lds, sx);
  }
  __syncthreads();

  const int npairs = ks < P ? (P - ks + G - 1) / G : 0;
  auto pair_ptr = [&](int col, int i) {
    int p = ks + G * i;
    p = p < P ? p : (ks < P ? ks : 0);
    return Wm + static_cast<int64_t>(col) * a.rowbytes + static_cast<int64_t>(p) * Fmt<FMT>::PAIR_BYTES;
  };
  const int npass = (ncols + CPP - 1) / CPP;
  auto pass_col = [&](int ps) {
    const int col = n0 + ps * CPP + cslot;
    return col < n0 + ncols ? col : n0 + ncols - 1;
  };
  auto load_pass = [&](int ps, uint32_t (&d)[U][PD]) {
    const int col = pass_col(ps);
#pragma unroll
    for (int u = 0; u < U; ++u) load_pair<FMT>(pair_ptr(col, u), d[u]);
  };
  // pass ps from buffer cur; first pass ps + kMoeGvD - 1 is issued into nxt (the buffer of pass
  // ps - 1, already consumed), so kMoeGvD - 1 passes stay in flight while a pass computes
  auto pass = [&](int ps, uint32_t (&cur)[U][PD], uint32_t (&nxt)[U][PD]) {
    if (ps + kMoeGvD - 1 < npass) load_pass(ps + kMoeGvD - 1, nxt);
    float acc[MC];
#pragma unroll
    for (int m = 0; m < MC; ++m) acc[m] = 0.f;
    for (int i0 = 0; i0 < npairs; i0 += U) {
      if (i0 > 0) {  // rows with more than U pairs per lane (long K): the next batch, unprefetched
        const int col = pass_col(ps);
#pragma unroll
        for (int u = 0; u < U; ++u) load_pair<FMT>(pair_ptr(col, i0 + u), cur[u]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (i0 + u < npairs) pair_dot<FMT, VYBDQ_Q4_GGML, MC>(cur[u], lds, sx, P, ks + G * (i0 + u), acc);
    }
#pragma unroll
    for (int m = 0; m < MC; ++m) acc[m] = group_sum<G>(acc[m]);
    const int col = n0 + ps * CPP + cslot;
    if constexpr (SWI) {
#pragma unroll
      for (int m = 0; m < MC; ++m) {
        const float o = __shfl_xor(acc[m], 32, 64);  // gate lane <- up lane of the same column
        if (!up && ks == G - 1 && col < n0 + ncols) {
          const float gt = fminf(acc[m], a.limit);
          const float uv = fminf(fmaxf(o, -a.limit), a.limit);
          store_elem<VYBDQ_F16>(a.Y, nullptr, static_cast<int64_t>(r0c + m) * a.ldy + col, moe_silu(gt) * uv);
        }
      }
    } else {
      if (ks == G - 1 && col < n0 + ncols) {
#pragma unroll
        for (int m = 0; m < MC; ++m)
          store_elem<VYBDQ_F32>(a.Y, nullptr, static_cast<int64_t>(r0c + m) * a.ldy + col, acc[m]);
      }
    }
  };
  uint32_t ring[kMoeGvD][U][PD];
#pragma unroll
  for (int j = 0; j < kMoeGvD - 1; ++j)
    if (j < npass) load_pass(j, ring[j]);
  for (int ps = 0; ps < npass; ps += kMoeGvD) {
#pragma unroll
    for (int k = 0; k < kMoeGvD; ++k)
      if (ps + k < npass) pass(ps + k, ring[k], ring[(k + kMoeGvD - 1) % kMoeGvD]);
  }
}

template <int FMT, int G, int U, bool SWI, int XW>
__global__ void __launch_bounds__(256) k_moe_gemv(MoeGvArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int nblk = (a.N + a.cols_per_wg - 1) / a.cols_per_wg;
  const int g = blockIdx.x / nblk;
  const int blk = blockIdx.x - g * nblk;
  if (g >= *a.ngroups) return;
  const int4 d = a.groups[g];
  const uint8_t *Wg, *Wu = nullptr;
  if (d.x < 0) {
    Wg = a.Ws;
    Wu = a.W2s;
  } else {
    Wg = a.W + static_cast<int64_t>(d.x) * a.w_stride;
    if constexpr (SWI) Wu = a.W2 + static_cast<int64_t>(d.x) * a.w_stride;
  }
  const int n0 = blk * a.cols_per_wg;
  const int ncols = a.N - n0 < a.cols_per_wg ? a.N - n0 : a.cols_per_wg;
  char *lds = smem;
  float *sx = reinterpret_cast<float *>(smem + static_cast<size_t>(a.mc) * a.P * XPAIR_STRIDE);
  for (int r = d.y; r < d.z; r += a.mc) {
    switch (d.z - r < a.mc ? d.z - r : a.mc) {
      case 1: moe_gv_chunk<FMT, G, U, 1, SWI, XW>(a, Wg, Wu, r, n0, ncols, lds, sx); break;
      case 2: moe_gv_chunk<FMT, G, U, 2, SWI, XW>(a, Wg, Wu, r, n0, ncols, lds, sx); break;
      case 3: moe_gv_chunk<FMT, G, U, 3, SWI, XW>(a, Wg, Wu, r, n0, ncols, lds, sx); break;
      default: moe_gv_chunk<FMT, G, U, 4, SWI, XW>(a, Wg, Wu, r, n0, ncols, lds, sx); break;
    }
  }
}

template <int FMT, int G, int U, bool SWI, int XW>
int moe_gemv_launch1(const MoeGvArgs &a, int max_groups, hipStream_t s) {
  const size_t lds = static_cast<size_t>(a.mc) * a.P * (XPAIR_STRIDE + 2 * 4);
  if (lds > 64 * 1024) {
    static bool raised = false;  // one attribute call per instantiation
    if (!raised) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_moe_gemv<FMT, G, U, SWI, XW>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
      if (e != hipSuccess) return set_error(VYBDQ_ERR_HIP, std::string("moe gemv: LDS attribute: ") + hipGetErrorString(e));
      raised = true;
    }
  }
  const int nblk = (a.N + a.cols_per_wg - 1) / a.cols_per_wg;
  hipLaunchKernelGGL((k_moe_gemv<FMT, G, U, SWI, XW>), dim3(static_cast<unsigned>(max_groups * nblk)), dim3(256), lds, s, a);
  return check_launch("moe grouped gemv");
}

// gate|up (swi): 32 lanes per row; down: 16. The pair batch covers a row's pairs per lane (at
// most 4 pairs in flight per lane; longer rows take extra unprefetched batches).
template <int FMT>
int moe_gemv_launch(bool swi, const MoeGvArgs &a, int max_groups, hipStream_t s) {
  const int G = swi ? 32 : 16;
  int U = (a.P + G - 1) / G;
  U = U < 1 ? 1 : (U > 4 ? 4 : U);
  if (swi) {
    if (a.xdt == VYBDQ_F32) {
      switch (U) {
        case 1: return moe_gemv_launch1<FMT, 32, 1, true, 8>(a, max_groups, s);
        case 2: return moe_gemv_launch1<FMT, 32, 2, true, 8>(a, max_groups, s);
        case 3: return moe_gemv_launch1<FMT, 32, 3, true, 8>(a, max_groups, s);
        default: return moe_gemv_launch1<FMT, 32, 4, true, 8>(a, max_groups, s);
      }
    }
    switch (U) {
      case 1: return moe_gemv_launch1<FMT, 32, 1, true, 4>(a, max_groups, s);
      case 2: return moe_gemv_launch1<FMT, 32, 2, true, 4>(a, max_groups, s);
      case 3: return moe_gemv_launch1<FMT, 32, 3, true, 4>(a, max_groups, s);
      default: return moe_gemv_launch1<FMT, 32, 4, true, 4>(a, max_groups, s);
    }
  }
  switch (U) {  // down: X is the fp16 activations
    case 1: return moe_gemv_launch1<FMT, 16, 1, false, 4>(a, max_groups, s);
    case 2: return moe_gemv_launch1<FMT, 16, 2, false, 4>(a, max_groups, s);
    case 3: return moe_gemv_launch1<FMT, 16, 3, false, 4>(a, max_groups, s);
    default: return moe_gemv_launch1<FMT, 16, 4, false, 4>(a, max_groups, s);
  }
}

// moe_gemv_q4.hip / moe_gemv_q8.hip
int moe_gemv_q4(bool swi, const MoeGvArgs &a, int max_groups, hipStream_t s);
int moe_gemv_q8(bool swi, const MoeGvArgs &a, int max_groups, hipStream_t s);

}  // namespace vybdq
