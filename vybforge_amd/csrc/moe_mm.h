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
  int tile_rows;            // 4: the list holds 4-row tiles (LDS-staged body only); 0: 16 MT rows
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

namespace vybdq {

// ---- q4_0 grouped GEMM with the weights staged through LDS (fp16 X) ----------------------------
//
// At a few rows per expert the register-operand body above is bound by its loads, not by HBM or
// the matrix cores: a wave's weight load covers 16 rows x 72 B and touches ~57 cache lines, and
// the texture address unit stays busy ~70% of the kernel. Here a workgroup owns 256 weight rows
// (R = 128: gate|up 64 gate + the same 64 up columns, down 128 columns; R = 256 twice that) and
// streams them into LDS with direct-to-LDS loads of whole row runs: a stage is two super-steps
// (8 blocks, 144 B per row, 16-byte aligned), lane q of the workgroup's stage copy takes chunk
// q % 9 of row q / 9, so one load instruction covers ~7 consecutive 144-B runs (~15 lines). Three
// stages are in flight (with R = 128 and one m-fragment, two workgroups per CU). Each
// lane then reads its block's 20-byte window from LDS and dequantizes it into the MFMA B operand
// exactly as the body above does (same k-slot assignment, same X fragments).
constexpr int kMlRun = 8 * 18;  // bytes per row per stage (q4_0, two super-steps)

// R weight rows per workgroup (256: 1 workgroup per CU; 128: 2), MT 16-row m-fragments, XR token
// rows staged per tile: 16 (MT m-fragments of 16 rows, three stages in flight) or 4 (one m-fragment
// whose A operand repeats the tile's 4 rows: the X part of a stage shrinks from 8 KB to 2 KB, so four
// stages fit the same LDS and three stay in flight while one computes)
template <int R, int MT, int XR = 16> struct MlShape {
  static_assert(XR == 16 || (XR == 4 && MT == 1), "4-row tiles: one m-fragment");
  static constexpr int STAGE_W = R * kMlRun;
  static constexpr int XB = XR == 16 ? MT * 4096 : 1024;  // X bytes per super-step
  static constexpr int STAGE = STAGE_W + 2 * XB;         // + the X chunks of the two super-steps
  static constexpr int J = STAGE_W / 1024;             // direct-to-LDS weight loads per stage
  static constexpr int NB = R / 64;                    // B fragments per wave per super-step
  static constexpr int NS = XR == 4 ? 4 : 3;           // stage buffers
  static constexpr int PER_CU = NS * STAGE <= 80 * 1024 ? 2 : 1;
};

template <int R, int MT, bool SWI, int XR = 16>
__global__ void __launch_bounds__(256, (MlShape<R, MT, XR>::PER_CU)) k_moe_mm_lds(MoeMmArgs g) {
  using Sh = MlShape<R, MT, XR>;
  constexpr int STAGE = Sh::STAGE, STAGE_W = Sh::STAGE_W, J = Sh::J, NB = Sh::NB, XB = Sh::XB, NS = Sh::NS;
  // one array per stage: the weight rows, then the X chunks of its two super-steps
  __shared__ __attribute__((aligned(16))) uint8_t s0[STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t s1[STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t s2[STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t s3[NS > 3 ? STAGE : 16];
  constexpr int COLS = SWI ? R / 2 : R;  // output columns per workgroup
  constexpr int NF = SWI ? NB / 2 : NB;  // fragments per wave per matrix
  const int n_tiles = g.m.N / COLS;
  const int nt = blockIdx.x % n_tiles;
  const int j = blockIdx.x / n_tiles;
  if (j >= *g.ntiles) return;
  const int4 d = g.tiles[j];
  MmArgs a = g.m;
  const uint8_t *Wa, *Wb;
  if (d.x < 0) {
    Wa = g.Ws;
    Wb = SWI ? g.W2s : g.Ws;
  } else {
    Wa = g.m.W + static_cast<int64_t>(d.x) * g.w_stride;
    Wb = SWI ? g.m.W2 + static_cast<int64_t>(d.x) * g.w_stride : Wa;
  }
  const int row0 = d.y + d.w * (XR == 4 ? 4 : 16 * MT);
  // rows at or past r1 (and, with 4-row tiles, past the tile's 4 rows) are clamped on load and
  // skipped on store
  a.M = XR == 4 && row0 + 4 < d.z ? row0 + 4 : d.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gq = lane >> 4, nl = lane & 15;
  const int n0 = nt * COLS;
  const int S2 = a.S >> 1;

  // weight copy: load jj of wave w is stage load j = w + 4 jj (J / 4 or J / 4 + 1 per wave); lane
  // q = 64 j + lane takes chunk q % 9 of workgroup row q / 9 (SwiGLU: rows R / 2.. are the up rows)
  constexpr int JW = (J + 3) / 4;
  const int nj = J / 4 + (w < J % 4 ? 1 : 0);
  const uint8_t *wsrc[JW];
  uint32_t woff[JW];
#pragma unroll
  for (int jj = 0; jj < JW; ++jj) {
    const int jx = w + 4 * jj;
    const int q = (jx < J ? jx : J - 1) * 64 + lane;
    const int r = q / 9, c = q - 9 * (q / 9);
    const bool up = SWI && r >= COLS;
    const int col = n0 + (up ? r - COLS : r);
    wsrc[jj] = up ? Wb : Wa;
    woff[jj] = static_cast<uint32_t>(static_cast<int64_t>(col) * a.rowbytes) + 16u * c;
  }
  // X chunks. XR = 16: thread (w, lane) stages chunk (i, t = w): row row0 + 16 i + nl, k = 128 s +
  // 32 gq + 8 w. XR = 4: waves 2 and 3 stage super-steps 0 and 1 of a stage (at R = 128 waves 0 and 1
  // issue one weight load more, so every wave issues five per stage); lane L takes row L / 16 and
  // 16-byte chunk (L % 16) ^ (L / 16) of the super-step, so chunk c of row r sits at 16-byte slot
  // 16 r + (c ^ r): the A reads of one step (rows r < 4, chunks 4 gq + t) fall on 16 distinct slots.
  uint32_t xoff[XR == 4 ? 1 : MT];
  if constexpr (XR == 4) {
    const int rr = lane >> 4;
    int r = row0 + rr;
    r = r < a.M ? r : a.M - 1;
    const int xr = a.row_map ? a.row_map[r] : r;
    xoff[0] = static_cast<uint32_t>(static_cast<int64_t>(xr) * a.ldx) + 8 * ((lane & 15) ^ rr);
  } else {
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      int r = row0 + 16 * i + nl;
      r = r < a.M ? r : a.M - 1;
      const int xr = a.row_map ? a.row_map[r] : r;
      xoff[i] = static_cast<uint32_t>(static_cast<int64_t>(xr) * a.ldx) + 32 * gq + 8 * w;
    }
  }
  // stage buffer B, chosen at compile time
  auto sb = [&](auto bi) -> uint8_t * {
    constexpr int B = decltype(bi)::value;
    if constexpr (B == 0) return s0;
    else if constexpr (B == 1) return s1;
    else if constexpr (B == 2) return s2;
    else return s3;
  };
  // Direct-to-LDS loads issued from asm (M0 = the wave-uniform LDS base): the compiler does not
  // track them, so it adds no waits of its own before the LDS reads (it merges its direct-to-LDS
  // bookkeeping conservatively at the loop head and would drain every load there); the waits
  // below are explicit. Loads the compiler does track only get longer waits from these.
  auto dma = [](const void *src, const void *dst) {
    const uint32_t l = __builtin_amdgcn_readfirstlane(
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void *)dst)));
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(l) : "memory", "m0");
  };
  auto issue = [&](auto bi, int st) {
    const int64_t kb = static_cast<int64_t>(st) * kMlRun;
#pragma unroll
    for (int jj = 0; jj < JW; ++jj)
      if (jj < nj) dma(wsrc[jj] + kb + woff[jj], sb(bi) + (w + 4 * jj) * 1024);
    if constexpr (XR == 4) {
      if (w >= 2)
        dma(static_cast<const uint16_t *>(a.X) + xoff[0] + static_cast<uint32_t>(2 * st + w - 2) * 128u,
            sb(bi) + STAGE_W + (w - 2) * XB);
    } else {
#pragma unroll
      for (int ss = 0; ss < 2; ++ss) {
        const uint32_t k = static_cast<uint32_t>(2 * st + ss) * 128u;
#pragma unroll
        for (int i = 0; i < MT; ++i)
          dma(static_cast<const uint16_t *>(a.X) + xoff[i] + k, sb(bi) + STAGE_W + ss * XB + (i * 4 + w) * 1024);
      }
    }
  };
  // vmcnt wait leaving the loads of `later` stages in flight (a wave issues nj + 2 MT loads per
  // stage; with 4-row tiles nj, plus one on waves 2 and 3)
  auto wait_stages = [&](auto later) {
    constexpr int K = decltype(later)::value;
    auto wait_vm = [](auto n) {
      constexpr int N = decltype(n)::value;
      static_assert(N >= 0 && N < 64, "vmcnt range");
      __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
    };
    if constexpr (XR == 4) {
      const int per = nj + (w >= 2 ? 1 : 0);  // JW - 1, JW or JW + 1
      if (per == JW + 1) wait_vm(std::integral_constant<int, K * (JW + 1)>{});
      else if (per == JW) wait_vm(std::integral_constant<int, K * JW>{});
      else wait_vm(std::integral_constant<int, K * (JW - 1)>{});
    } else {
      if (nj == JW) wait_vm(std::integral_constant<int, K * (JW + 2 * MT)>{});
      else wait_vm(std::integral_constant<int, K * (JW - 1 + 2 * MT)>{});
    }
  };
  auto bar = [] {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
  };

  f4 acc[MT][NB];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int f = 0; f < NB; ++f) acc[i][f] = f4{0.f, 0.f, 0.f, 0.f};
  // this lane's LDS row of fragment f (SwiGLU: f < NF gate, f >= NF up)
  int lrow[NB];
#pragma unroll
  for (int f = 0; f < NB; ++f) {
    const int ff = f < NF ? f : f - NF;
    lrow[f] = (w * NF + ff) * 16 + nl + (SWI && f >= NF ? COLS : 0);
  }
  const uint32_t sel = (gq & 1) ? 0x07060504u : 0x05040302u;
  const uint32_t shd = (gq & 1) ? 16u : 0u;

  // two super-steps from stage buffer B
  auto compute = [&](auto bi) {
#pragma unroll
    for (int ss = 0; ss < 2; ++ss) {
      const int blk = 4 * ss + gq;
      const int wo = 18 * blk - 2 * (blk & 1);
      uint32_t win[NB][5];
#pragma unroll
      for (int f = 0; f < NB; ++f) {
        const uint32_t *p = reinterpret_cast<const uint32_t *>(sb(bi) + lrow[f] * kMlRun + wo);
#pragma unroll
        for (int k = 0; k < 5; ++k) win[f][k] = p[k];
      }
      const uint8_t *abase = sb(bi) + STAGE_W + ss * XB;
      // A fragment (m-fragment i, step t): XR = 16 in fragment order; XR = 4 the tile's row nl % 4
      const int xr4 = nl & 3;
      auto aoff = [&](int i, int t) {
        if constexpr (XR == 4) return 256 * xr4 + 16 * ((4 * gq + t) ^ xr4);
        else return ((i * 4 + t) * 64 + lane) * 16;
      };
      hf8 af[2][MT];
#pragma unroll
      for (int i = 0; i < MT; ++i) af[0][i] = *reinterpret_cast<const hf8 *>(abase + aoff(i, 0));
      hf8 bcur = dequant_step<FMT_Q4_0>(win[0], 0, sel, shd);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (t < 3) {
#pragma unroll
          for (int i = 0; i < MT; ++i)
            af[(t + 1) & 1][i] = *reinterpret_cast<const hf8 *>(abase + aoff(i, t + 1));
        }
#pragma unroll
        for (int f = 0; f < NB; ++f) {
          const bool last = t == 3 && f == NB - 1;
          const int fn = f + 1 < NB ? f + 1 : 0;
          const int tn = f + 1 < NB ? t : t + 1;
          hf8 bnext = bcur;
          if (!last) bnext = dequant_step<FMT_Q4_0>(win[fn], tn, sel, shd);
#pragma unroll
          for (int i = 0; i < MT; ++i)
            acc[i][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t & 1][i], bcur, acc[i][f], 0, 0, 0);
          bcur = bnext;
        }
      }
    }
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  // stage i is in buffer i % NS. One barrier per stage: it follows every wave's wait for stage i
  // and every wave's reads of stage i - 1, so right after it stage i + NS - 1 is issued into the
  // buffer of stage i - 1
  issue(I0{}, 0);
  if (S2 > 1) issue(I1{}, 1);
  if (NS > 3 && S2 > 2) issue(I2{}, 2);
  auto iter = [&](auto bi, int i) {
    constexpr int B = decltype(bi)::value;
    if (NS > 3 && i + 2 < S2) wait_stages(I2{});
    else if (i + 1 < S2) wait_stages(I1{});
    else wait_stages(I0{});
    bar();
    if (i + NS - 1 < S2) issue(std::integral_constant<int, (B + NS - 1) % NS>{}, i + NS - 1);
    compute(bi);
  };
  int i = 0;
  if constexpr (NS == 4) {
    for (; i + 4 <= S2; i += 4) {
      iter(I0{}, i);
      iter(I1{}, i + 1);
      iter(I2{}, i + 2);
      iter(I3{}, i + 3);
    }
    if (i < S2) iter(I0{}, i);
    if (i + 1 < S2) iter(I1{}, i + 1);
    if (i + 2 < S2) iter(I2{}, i + 2);
  } else {
    for (; i + 3 <= S2; i += 3) {
      iter(I0{}, i);
      iter(I1{}, i + 1);
      iter(I2{}, i + 2);
    }
    if (i < S2) iter(I0{}, i);
    if (i + 1 < S2) iter(I1{}, i + 1);
  }

  const int fb = (n0 >> 4) + w * NF;
  mm_finish<MT, NF, NF, 4, SWI>(a, nullptr, 0, 0, row0, fb, acc);
}

template <int R, int MT, bool SWI, int XR = 16>
int moe_mm_lds_launch(const MoeMmArgs &g, int max_tiles, hipStream_t s) {
  constexpr int COLS = SWI ? R / 2 : R;
  const int64_t units = static_cast<int64_t>(max_tiles) * (g.m.N / COLS);
  hipLaunchKernelGGL((k_moe_mm_lds<R, MT, SWI, XR>), dim3(static_cast<unsigned>(units)), dim3(256), 0, s, g);
  return check_launch("moe grouped gemm (LDS weights)");
}

// the LDS-staged body (R = 128, one m-fragment: two workgroups per CU) applies: q4_0, fp16 X, an
// even number of super-steps, whole column tiles (gate|up 64 columns, down 128). Measured on the
// GLM-5 layer (H = 6144, I = 2048, 256 experts, top-8): T = 256 1.52 ms against 1.92 ms for the
// register-operand body with 32-row tiles; R = 256 (one workgroup per CU) 1.87 ms, and 32-row
// tiles at R = 128 (one workgroup per CU) 2.14 ms.
inline bool moe_mm_lds_ok(int fmt, int xdt, bool swi, const MoeMmArgs &g) {
  return fmt == FMT_Q4_0 && xdt == VYBDQ_F16 && g.m.S % 2 == 0 && g.m.N % (swi ? 64 : 128) == 0;
}

}  // namespace vybdq
