// Grouped expert GEMM of the MoE layer on the register-operand MFMA body (mmq.h), gfx950.
//
// A unit of work is (m-tile j, n-tile). The bucketing kernel lists the m-tiles in device memory:
// tile j = {expert e (-1: the shared expert), first row r0, end row r1, m-tile index within the
// group}, rows being positions in the bucketed row order (row_map gives each row's token). Only
// experts that received tokens have tiles, so the grid (sized for the worst case on the host)
// has no work for idle experts: units past the listed tiles exit at once.
//
// gate|up (SWI): each wave owns two 16-column fragments of the gate matrix and the same two of
// the up matrix, and the epilogue writes silu(min(g, L)) * clamp(u, -L, L) as fp16
// (native/glm53/moe_ref.py:81-84). down: the routed rows' f32 outputs, combined afterwards.
#pragma once
#include "mmq.h"

namespace vybdq {

struct MoeMmArgs {
  MmArgs m;                 // W (W2): expert 0's gate (up) rows; X, ldx, row_map, N, S, F, n_tiles, Y, ldy, limit
  int64_t w_stride;         // bytes between consecutive experts' matrices
  const uint8_t *Ws, *W2s;  // the shared expert's matrices
  const int4 *tiles;        // m-tile list {expert, r0, r1, m-tile}
  const int *ntiles;        // number of listed m-tiles
};

constexpr int kMoeNF = 2;          // fragments (pairs for SWI) per wave
constexpr int kMoeF = 4 * kMoeNF;  // 16-column fragments per n-tile (128 columns)

template <int FMT, int XDT, int MT, bool SWI>
__global__ void __launch_bounds__(256, 2) k_moe_mm(MoeMmArgs g) {
  constexpr int NA = MmFmt<FMT>::D;
  __shared__ __attribute__((aligned(16))) uint8_t a0[MT * 4096];
  __shared__ __attribute__((aligned(16))) uint8_t a1[MT * 4096];
  __shared__ __attribute__((aligned(16))) uint8_t a2[NA > 2 ? MT * 4096 : 16];
  __shared__ __attribute__((aligned(16))) uint8_t a3[NA > 3 ? MT * 4096 : 16];
  const MmLds<MT> sm{{a0, a1, a2, a3}, nullptr};
  const int nt = blockIdx.x % g.m.n_tiles;
  const int j = blockIdx.x / g.m.n_tiles;
  if (j >= *g.ntiles) return;
  const int4 d = g.tiles[j];
  MmArgs a = g.m;
  if (d.x < 0) {
    a.W = g.Ws;
    a.W2 = g.W2s;
  } else {
    a.W = g.m.W + static_cast<int64_t>(d.x) * g.w_stride;
    if constexpr (SWI) a.W2 = g.m.W2 + static_cast<int64_t>(d.x) * g.w_stride;
  }
  a.M = d.z;  // rows at or past r1 are clamped on load and skipped on store
  const int row0 = d.y + d.w * 16 * MT;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int fb = nt * kMoeF + w * kMoeNF;
  mm_body<FMT, XDT, MT, kMoeNF, kMoeNF, SWI>(a, sm, 0, 0, row0, fb, 0, a.S);
}

// Launch over max_tiles x n_tiles units (m-tiles past *ntiles exit).
template <int FMT, int XDT, int MT, bool SWI>
int moe_mm_launch(const MoeMmArgs &g, int max_tiles, hipStream_t s) {
  const int64_t units = static_cast<int64_t>(max_tiles) * g.m.n_tiles;
  hipLaunchKernelGGL((k_moe_mm<FMT, XDT, MT, SWI>), dim3(static_cast<unsigned>(units)), dim3(256), 0, s, g);
  return check_launch("moe grouped gemm");
}

// moe_mm_q4.hip / moe_mm_q8.hip: xdt = X's type (gate|up: x; down: the fp16 activations),
// mt = 16-row fragments per m-tile (1 or 2).
int moe_mm_q4(int xdt, int mt, bool swi, const MoeMmArgs &g, int max_tiles, hipStream_t s);
int moe_mm_q8(int xdt, int mt, bool swi, const MoeMmArgs &g, int max_tiles, hipStream_t s);

}  // namespace vybdq
