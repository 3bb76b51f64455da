// Host side of the MFMA dequant GEMM: tiling plan (fragments per tile, split-K) and dispatch.
// The kernels are instantiated one format x activation type per translation unit (mmq_k_*.hip).
#include "mmq.h"
#include "mmq_i8.h"

#include <cstdio>
#include <cstdlib>

namespace vybdq {

extern template int mmq_launch<FMT_Q4_0, VYBDQ_F16>(MmArgs &, hipStream_t);
extern template int mmq_launch<FMT_Q4_0, VYBDQ_BF16>(MmArgs &, hipStream_t);
extern template int mmq_launch<FMT_Q4_0, VYBDQ_F32>(MmArgs &, hipStream_t);
extern template int mmq_launch<FMT_Q8_0, VYBDQ_F16>(MmArgs &, hipStream_t);
extern template int mmq_launch<FMT_Q8_0, VYBDQ_BF16>(MmArgs &, hipStream_t);
extern template int mmq_launch<FMT_Q8_0, VYBDQ_F32>(MmArgs &, hipStream_t);
extern template int mmq_launch<FMT_Q4_K, VYBDQ_F16>(MmArgs &, hipStream_t);
extern template int mmq_launch<FMT_Q5_K, VYBDQ_F16>(MmArgs &, hipStream_t);

// ---- host --------------------------------------------------------------------------------


struct MmPlan {
  int m_tiles, n_tiles, F, splits, sps;
  int64_t ws_bytes;  // partials + counters (0 without split-K)
};

static int64_t mm_part_bytes(int64_t tiles, int splits) {
  return tiles * splits * static_cast<int64_t>(kMmPartFrags) * kMmMT * 64 * 4 * 4;
}

// Tiling: pick fragments per tile F and the K split that minimise an estimate of the run time:
//   rounds(units / CUs) x super-steps per unit x cycles per super-step
// where a super-step costs the larger of its MFMA time (64 MT cycles per fragment a wave owns, at
// ~80% issue efficiency) and its LDS time (the X tile: 4 waves read it, one writes it, ~156 MT
// cycles at 128 B/cycle), plus the HBM traffic of split partials (written, then read back).
// nfx: most fragments one wave can own; a super-step costs fixed_cycles (X tile traffic, barrier)
// plus frag_cycles per fragment the busiest wave owns (measured on MI355X at the prefill shapes,
// in 2.4 GHz cycles).
static MmPlan mm_plan(int M, int N, int S, bool allow_split, int nfx = kMmNFX, double frag_cycles = 1584.0,
                      double fixed_cycles = 1440.0) {
  const int cus = device_cu_count();
  const int m_tiles = (M + 16 * kMmMT - 1) / (16 * kMmMT);
  const int Ftot = N / 16;
  MmPlan best{};
  double best_t = -1;
  for (int F = 1; F <= 4 * nfx && F <= Ftot; ++F) {
    const int n_tiles = (Ftot + F - 1) / F;
    if ((n_tiles - 1) * F >= Ftot) continue;
    const int nfw = (F + 3) / 4;
    const double step_us = (fixed_cycles + frag_cycles * nfw) / 2.4e3;
    for (int splits = 1; splits <= (allow_split ? 8 : 1) && splits <= S; ++splits) {
      const int sps = (S + splits - 1) / splits;
      if ((splits - 1) * sps >= S) continue;
      const int64_t units = static_cast<int64_t>(m_tiles) * n_tiles * splits;
      const int64_t rounds = (units + cus - 1) / cus;
      double t = static_cast<double>(rounds) * sps * step_us;
      if (splits > 1) {
        const double bytes = static_cast<double>(units) * 16 * kMmMT * F * 16 * 4 * (2.0 - 1.0 / splits);
        t += bytes / 2.5e6;  // written, then read back by the reducing workgroups
      }
      if (best_t < 0 || t < best_t - 1e-9) {
        best_t = t;
        best.m_tiles = m_tiles;
        best.n_tiles = n_tiles;
        best.F = F;
        best.splits = splits;
        best.sps = sps;
      }
    }
  }
  // tuning / test override: VYBDQ_MMQ_PLAN="F,splits" (ignored when it does not fit the shape)
  if (const char *ov = tuning_env("VYBDQ_MMQ_PLAN")) {
    int F = 0, splits = 1;
    if (sscanf(ov, "%d,%d", &F, &splits) >= 1 && F >= 1 && F <= 4 * nfx && F <= Ftot && splits >= 1 &&
        splits <= 8 && splits <= S && (splits == 1 || allow_split)) {
      const int sps = (S + splits - 1) / splits;
      if ((splits - 1) * sps < S) {
        best.F = F;
        best.n_tiles = (Ftot + F - 1) / F;
        best.splits = splits;
        best.sps = sps;
      }
    }
  }
  const int64_t tiles = static_cast<int64_t>(best.m_tiles) * best.n_tiles;
  best.ws_bytes = best.splits > 1 ? mm_part_bytes(tiles, best.splits) : 0;
  return best;
}

// K < 2^24: the 8-wave body addresses a wave's weight rows by 32-bit offsets
bool mmq_supported(int64_t M, int64_t N, int64_t K) {
  return M >= 1 && K % 256 == 0 && K < (int64_t(1) << 24) && N % 16 == 0 && N >= 16 && M * K < (int64_t(1) << 31);
}

// X -> fp16 copy, one workgroup per row: the row's largest |x| is brought into [2^14, 2^15) by a
// power of two 2^-e (exact; all-zero rows and rows whose e would leave [-100, 113] are clamped),
// the scaled row is rounded to fp16 (bf16 values exactly, f32 to nearest even) and 2^e goes to
// xscale[row], which the GEMM epilogue multiplies back: activations of any magnitude neither
// overflow nor flush to zero. The GEMM then streams the fp16 copy straight into LDS.
template <int XDT, int CH>
__global__ void __launch_bounds__(256) k_x_to_f16(const void *__restrict__ X, u4 *__restrict__ Xh,
                                                  float *__restrict__ xscale, int64_t K) {
  __shared__ float wmax[4];
  x_row_to_f16<XDT, CH>(X, Xh, xscale, K, blockIdx.x, wmax);
}

template <int XDT>
static void x_to_f16_launch(const void *X, u4 *o, float *xscale, int64_t M, int64_t K, hipStream_t s) {
  const unsigned grid = static_cast<unsigned>(M);
  const int per = x_row_chunks(K);
  if (per <= 2) hipLaunchKernelGGL((k_x_to_f16<XDT, 2>), dim3(grid), dim3(256), 0, s, X, o, xscale, K);
  else if (per <= 4) hipLaunchKernelGGL((k_x_to_f16<XDT, 4>), dim3(grid), dim3(256), 0, s, X, o, xscale, K);
  else if (per <= 8) hipLaunchKernelGGL((k_x_to_f16<XDT, 8>), dim3(grid), dim3(256), 0, s, X, o, xscale, K);
  else if (per <= 12) hipLaunchKernelGGL((k_x_to_f16<XDT, 12>), dim3(grid), dim3(256), 0, s, X, o, xscale, K);
  else hipLaunchKernelGGL((k_x_to_f16<XDT, 0>), dim3(grid), dim3(256), 0, s, X, o, xscale, K);
}

int x_rows_to_f16(const void *X, int xdt, int64_t M, int64_t K, void *xh, float *xscale, hipStream_t s) {
  u4 *o = static_cast<u4 *>(xh);
  if (xdt == VYBDQ_BF16) x_to_f16_launch<VYBDQ_BF16>(X, o, xscale, M, K, s);
  else x_to_f16_launch<VYBDQ_F32>(X, o, xscale, M, K, s);
  return check_launch("x -> f16 rows");
}

static int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

// workspace: [split partials][fp16 copy of X][X row scales]
// Q4_K / Q5_K tiles: at most 16 fragments (two per wave: its nibble windows, the scale words and
// 96 accumulators fill the 256 registers of a wave at three)
static int mm_nfx(int wtype) { return wtype == 12 || wtype == 13 ? 4 : kMmNFX; }

int64_t mmq_workspace_size(int wtype, int64_t M, int64_t N, int64_t K) {
  if (!mmq_supported(M, N, K)) return 0;
  return align256(mm_plan(static_cast<int>(M), static_cast<int>(N), static_cast<int>(K / 128), true, mm_nfx(wtype)).ws_bytes) +
         align256(M * K * 2) + align256(M * 4);
}

int mmq_gemm(int wtype, const void *W, const void *X, int xdt, void *Y, int ydt, int64_t M, int64_t N, int64_t K,
             int64_t ldy, const void *RS, void *ws, int64_t ws_bytes, hipStream_t s) {
  const int S = static_cast<int>(K / 128);
  MmPlan p = mm_plan(static_cast<int>(M), static_cast<int>(N), S, ws != nullptr, mm_nfx(wtype));
  if (p.splits > 1 && ws_bytes < p.ws_bytes) p = mm_plan(static_cast<int>(M), static_cast<int>(N), S, false, mm_nfx(wtype));
  // with room for it, a non-fp16 X is converted once up front (instead of once per N tile)
  const int64_t xh_off = align256(p.ws_bytes);
  const int64_t sc_off = xh_off + align256(M * K * 2);
  const float *xscale = nullptr;
  if (ws && xdt != VYBDQ_F16 && ws_bytes >= sc_off + M * 4) {
    u4 *xh = reinterpret_cast<u4 *>(static_cast<char *>(ws) + xh_off);
    float *sc = reinterpret_cast<float *>(static_cast<char *>(ws) + sc_off);
    const int rc = x_rows_to_f16(X, xdt, M, K, xh, sc, s);
    if (rc) return rc;
    X = xh;
    xdt = VYBDQ_F16;
    xscale = sc;
  }
  MmArgs a{};
  a.W = static_cast<const uint8_t *>(W);
  a.rowbytes = wtype == 12   ? K / 256 * MmFmt<FMT_Q4_K>::SB
               : wtype == 13 ? K / 256 * MmFmt<FMT_Q5_K>::SB
                             : K / 32 * (wtype == 2 ? 18 : 34);
  a.X = X;
  a.ldx = K;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.S = S;
  a.F = p.F;
  a.m_tiles = p.m_tiles;
  a.n_tiles = p.n_tiles;
  a.splits = p.splits;
  a.sps = p.sps;
  a.Y = Y;
  a.ydt = ydt;
  a.ldy = ldy;
  a.RS = RS;
  a.xscale = xscale;
  if (p.splits > 1) {
    a.part = static_cast<float *>(ws);
  }
  if (wtype == 12 || wtype == 13) {
    // the super-block body streams fp16 X: bf16 / f32 X needs the workspace for its conversion
    if (xdt != VYBDQ_F16)
      return set_error(VYBDQ_ERR_WORKSPACE, "mmq gemm: Q4_K / Q5_K with bf16/f32 X needs the workspace");
    return wtype == 12 ? mmq_launch<FMT_Q4_K, VYBDQ_F16>(a, s) : mmq_launch<FMT_Q5_K, VYBDQ_F16>(a, s);
  }
  if (wtype == 2) {
    switch (xdt) {
      case VYBDQ_F16: return mmq_launch<FMT_Q4_0, VYBDQ_F16>(a, s);
      case VYBDQ_BF16: return mmq_launch<FMT_Q4_0, VYBDQ_BF16>(a, s);
      default: return mmq_launch<FMT_Q4_0, VYBDQ_F32>(a, s);
    }
  }
  switch (xdt) {
    case VYBDQ_F16: return mmq_launch<FMT_Q8_0, VYBDQ_F16>(a, s);
    case VYBDQ_BF16: return mmq_launch<FMT_Q8_0, VYBDQ_BF16>(a, s);
    default: return mmq_launch<FMT_Q8_0, VYBDQ_F32>(a, s);
  }
}

// ---- int8 path -------------------------------------------------------------------------------

static MmPlan i8_plan(int M, int N, int S, bool allow_split) {
  return mm_plan(M, N, S, allow_split, kI8NFX, 2200.0, 2500.0);
}

int64_t mmq_i8_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (!mmq_supported(M, N, K)) return 0;
  return align256(i8_plan(static_cast<int>(M), static_cast<int>(N), static_cast<int>(K / 128), true).ws_bytes);
}

int mmq_i8_gemm(const void *W, const int8_t *Xq, const float *Xs, void *Y, int ydt, int64_t M, int64_t N, int64_t K,
                int64_t ldy, const void *RS, void *ws, int64_t ws_bytes, hipStream_t s) {
  const int S = static_cast<int>(K / 128);
  MmPlan p = i8_plan(static_cast<int>(M), static_cast<int>(N), S, ws != nullptr);
  if (p.splits > 1 && ws_bytes < p.ws_bytes) p = i8_plan(static_cast<int>(M), static_cast<int>(N), S, false);
  I8Args ia{};
  MmArgs &a = ia.m;
  a.W = static_cast<const uint8_t *>(W);
  a.rowbytes = K / 32 * 34;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.S = S;
  a.F = p.F;
  a.m_tiles = p.m_tiles;
  a.n_tiles = p.n_tiles;
  a.splits = p.splits;
  a.sps = p.sps;
  a.Y = Y;
  a.ydt = ydt;
  a.ldy = ldy;
  a.RS = RS;
  if (p.splits > 1) {
    a.part = static_cast<float *>(ws);
  }
  ia.Xq = Xq;
  ia.Xs = Xs;
  ia.ldq = K;
  ia.lds = K / 32;
  const int64_t units = static_cast<int64_t>(a.m_tiles) * a.n_tiles * a.splits;
  a.xcd = units % 8 == 0 ? 1 : 0;
  hipLaunchKernelGGL(k_mmq_i8, dim3(static_cast<unsigned>(units)), dim3(kI8Threads), 0, s, ia);
  const int rc = check_launch("mmq int8 gemm");
  if (rc) return rc;
  return mm_reduce_launch<8, kI8MT / 2, kI8NFX, 2>(a, s);
}

}  // namespace vybdq

