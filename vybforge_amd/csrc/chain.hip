// GEMV stages over the reference's GEMV parameter blocks, gfx950: the persistent multi-stage chain
// (vybdq_gemv_chain, k_gemv_chain2) and the one-stage kernel of the parameter-block GEMV kind
// (k_gemv_chain with nstages = 1, pblock.hip).
//
// Stage descriptors are the reference's GEMV parameter blocks, read from device memory
// (native/host/ridge_decode.vyb:264-270, native/kernels/qwen3.vyb:410-440), one per stage at
// P + s * pstride, little-endian int64 words:
//   W@0 X@8 Y@16 M@24 N@32 K@40 YE@48 W2@56 NS2@64 Y2@72 YE2@80 W3@88 NS3@96 Y3@104 YE3@112
//   RS@120 GRID@128, and two words the reference does not have: XE@136 (x element type) and
//   ORDER@144 (q4_0 nibble order). YE: 4 = f32, 2 = f16, 258 = bf16, anything else = f64 (the
//   reference's f64 mode, with the f64 residual RS). XE: 2 = f16, 258 = bf16, else f32. M must be 1.
//
// A decode step is a sequence of GEMVs where stage s may consume stage s-1's output. As separate
// launches each stage pays the dependent-launch floor (~1.7 us per graph node) plus an HBM round
// trip before its first weight byte arrives; the chain runs every stage in one persistent grid
// and streams the next stage's weights during the handover. Measured on the 36-layer decode
// stack it is nevertheless slower than the graph of launches (1.5 against 0.84 ms per step): the
// handover itself (device-scope arrival, a poll round trip, the next x read) takes ~3-5 us, more
// than a dependent graph node, and a stage's dequant-dot work can only start after its x arrives,
// where a launch overlaps it with its weight stream.
#include "gemv_dev.h"

#include <atomic>

namespace vybdq {

constexpr int kChainThreads = 256;

// units (64 weights) per lane per load batch
template <int FMT> constexpr int chain_batch() {
  return FMT == FMT_Q4_0 ? 4 : (FMT == FMT_Q4_K || FMT == FMT_IQ2_S) ? 4 : 2;
}

struct StageDesc {
  const uint8_t *W[3];
  void *Y[3];
  int ydt[3];
  int64_t end[3];
  const void *X;
  const void *RS;
  int64_t K;
  int xdt;
  int order;
};

__device__ __forceinline__ int ye_to_dt(int64_t ye) {
  if (ye == 4) return VYBDQ_F32;
  if (ye == 2) return VYBDQ_F16;
  if (ye == 258) return VYBDQ_BF16;
  return VYBDQ_F64;
}

// ref_layout: the reference's 136-byte block (x is f32, q4_0 in GGUF order; no XE / ORDER words)
__device__ __forceinline__ StageDesc read_stage(const int64_t *pb, bool ref_layout) {
  StageDesc d;
  d.W[0] = gptr<const uint8_t>(pb[0]);
  d.X = gptr<const void>(pb[1]);
  d.Y[0] = gptr<void>(pb[2]);
  const int64_t n1 = pb[4];
  d.K = pb[5];
  d.ydt[0] = ye_to_dt(pb[6]);
  d.W[1] = gptr<const uint8_t>(pb[7]);
  const int64_t n2 = pb[8];
  d.Y[1] = gptr<void>(pb[9]);
  d.ydt[1] = ye_to_dt(pb[10]);
  d.W[2] = gptr<const uint8_t>(pb[11]);
  const int64_t n3 = pb[12];
  d.Y[2] = gptr<void>(pb[13]);
  d.ydt[2] = ye_to_dt(pb[14]);
  d.RS = gptr<const void>(pb[15]);
  if (ref_layout) {
    d.xdt = VYBDQ_F32;
    d.order = VYBDQ_Q4_GGML;
  } else {
    d.xdt = pb[17] == 2 ? VYBDQ_F16 : pb[17] == 258 ? VYBDQ_BF16 : VYBDQ_F32;
    d.order = static_cast<int>(pb[18]);
  }
  // the reference adds RS only in its f64 output mode (native/kernels/rgemv.vyb:13-15)
  if (ref_layout && d.ydt[0] != VYBDQ_F64) d.RS = nullptr;
  d.end[0] = n1;
  d.end[1] = n1 + n2;
  d.end[2] = n1 + n2 + n3;
  return d;
}

// Lanes per row for a stage (log2: 4, 5 or 6): minimise (tiles per wave) x (pairs per lane), ties ->
// smaller G. 32-bit unsigned arithmetic (rows < 2^30): this runs at the start of every launch, before
// the first weight load can be issued.
__device__ __forceinline__ int chain_pick_lg(uint32_t rows, uint32_t P, uint32_t nwaves) {
  int best = 4;
  uint32_t best_cost = 0xffffffffu;
#pragma unroll
  for (int lg = 4; lg <= 6; ++lg) {
    const uint32_t tiles = (rows + (64u >> lg) - 1) >> (6 - lg);
    const uint32_t cost = ((tiles + nwaves - 1) / nwaves) * ((P + (1u << lg) - 1) >> lg);
    if (cost < best_cost) { best = lg; best_cost = cost; }
  }
  return best;
}

// One GEMV stage in the reference's own block layout (the GEMV kind of vybdq_launch_pblock): the
// first batch of weight loads goes out before x is staged; an invalid block computes nothing and
// sets bit 2 of the status word.
template <int FMT, int NT = kChainThreads>
__global__ void __launch_bounds__(NT) k_pb_gemv(const int64_t *__restrict__ pb, int64_t maxK,
                                                uint32_t *__restrict__ status) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int U = chain_batch<FMT>();
  constexpr int PD = Fmt<FMT>::PAIR_DWORDS;
  constexpr int KALIGN = is_kquant<FMT>() ? 256 : 64;
  const int maxP = static_cast<int>(maxK >> 6);
  char *lds = smem;
  float *sx = reinterpret_cast<float *>(smem + static_cast<size_t>(maxP) * XPAIR_STRIDE);
  const int nwg = gridDim.x;
  const int nwaves = nwg * (NT / 64);
  const int gw = blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  {
    const StageDesc st = read_stage(pb, true);
    const int P = static_cast<int>(st.K >> 6);
    // every word that addresses memory is checked before use: null or misaligned pointers, negative
    // segment sizes, M != 1 or a K the LDS stage does not hold leave the stage uncomputed (error bit)
    bool segs_ok = st.end[0] >= 0 && st.end[1] >= st.end[0] && st.end[2] >= st.end[1];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const bool used = st.end[i] > (i == 0 ? 0 : st.end[i - 1]);
      segs_ok = segs_ok && (!used || (st.W[i] && st.Y[i] && (reinterpret_cast<uintptr_t>(st.W[i]) & 3) == 0));
    }
    const bool valid = segs_ok && st.K > 0 && st.K % KALIGN == 0 && st.K <= maxK && st.end[2] > 0 &&
                       st.end[2] < (int64_t(1) << 30) && st.X && (reinterpret_cast<uintptr_t>(st.X) & 15) == 0 &&
                       pb[3] == 1;
    const int64_t rows = valid ? st.end[2] : 0;
    const int lg = valid ? chain_pick_lg(static_cast<uint32_t>(rows), static_cast<uint32_t>(P),
                                         static_cast<uint32_t>(nwaves)) : 6;
    const int G = 1 << lg;
    const int rpt = 64 >> lg;  // rows per wave tile
    const int64_t tiles = (rows + rpt - 1) >> (6 - lg);
    const int ks = lane & (G - 1);
    const int npl = ks < P ? (P - ks + G - 1) >> lg : 0;  // pairs per lane per row

    // tile -> (segment, local row, row pointer); lanes past the end read row 0 of segment 0
    auto tile_row = [&](int64_t t, int &sg, int64_t &lrow, const uint8_t *&wrow, bool &act) {
      const int64_t row = t * rpt + (lane >> lg);
      act = row < rows;
      sg = 0;
      if (row >= st.end[0]) sg = (row >= st.end[1]) ? 2 : 1;
      if (!act) sg = 0;
      lrow = act ? row - (sg == 0 ? 0 : (sg == 1 ? st.end[0] : st.end[1])) : 0;
      wrow = pick3_ptr(st.W, sg) + lrow * unit_row_bytes<FMT>(P);
    };
    auto pair_idx = [&](int i) {
      const int p = ks + G * i;
      return p < P ? p : (ks < P ? ks : 0);
    };

    // a workgroup without a tile (the grid is sized for the largest stage) is done: it stages no x
    if (valid && static_cast<int64_t>(blockIdx.x) * (NT / 64) >= tiles) return;

    // 1. the first x chunks (the block's x is f32: 8 dwords per 8 elements), five per thread,
    // before any weight load: loads return in order, so the x stage below waits for x alone
    constexpr int XC = 5;
    const int nchunk = valid ? 8 * P : 0;
    uint32_t xr[XC][8];
#pragma unroll
    for (int j = 0; j < XC; ++j) {
      const int c = threadIdx.x + NT * j;
      if (c < nchunk) load_x_chunk<8>(st.X, 8 * static_cast<int64_t>(c), xr[j]);
    }

    // 2. the first batch of this wave's first tile
    int64_t t = gw;
    uint32_t dw[U][PD];
    {
      int sg; int64_t lrow; const uint8_t *wrow; bool act;
      tile_row(t < tiles ? t : 0, sg, lrow, wrow, act);
      if (valid) {
#pragma unroll
        for (int u = 0; u < U; ++u) load_unit<FMT>(wrow, pair_idx(u), dw[u]);
      }
    }

    // 3. stage x into LDS (the rest of its chunks loaded as they are staged); IQ2_S: then its grid
    // tables behind the block sums, where the unit dot of this stage's P reads them
    if (valid) {
#pragma unroll
      for (int j = 0; j < XC; ++j) {
        const int c = threadIdx.x + NT * j;
        if (c < nchunk) stage_chunk<8>(xr[j], VYBDQ_F32, c, lds, sx);
      }
      if constexpr (FMT == FMT_IQ2_S) {
        u4 *gridh = iq2s_lds_grid(sx, 1, P);
        for (int i0 = threadIdx.x; i0 < 1024 + 256; i0 += 5 * NT) {  // five 16-B loads in flight per thread
          u4 v[5];
        #pragma unroll
          for (int u = 0; u < 5; ++u)
            if (i0 + u * NT < 1024 + 256) v[u] = reinterpret_cast<const u4 *>(kIq2sLdsTab)[i0 + u * NT];
        #pragma unroll
          for (int u = 0; u < 5; ++u)
            if (i0 + u * NT < 1024 + 256) gridh[i0 + u * NT] = v[u];
        }
      }
      for (int c = threadIdx.x + NT * XC; c < nchunk; c += NT) {
        uint32_t r[8];
        load_x_chunk<8>(st.X, 8 * static_cast<int64_t>(c), r);
        stage_chunk<8>(r, VYBDQ_F32, c, lds, sx);
      }
    }
    __syncthreads();

    // 4. tiles of this wave
    if (valid) {
      bool first = true;
      for (; t < tiles; t += nwaves) {
        int sg; int64_t lrow; const uint8_t *wrow; bool act;
        tile_row(t, sg, lrow, wrow, act);
        float acc[1] = {0.f};
        for (int i0 = 0; i0 < npl; i0 += U) {
          if (!first || i0 > 0) {
#pragma unroll
            for (int u = 0; u < U; ++u) load_unit<FMT>(wrow, pair_idx(i0 + u), dw[u]);
          }
          if (act) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
              if (i0 + u < npl) {
                if (FMT != FMT_Q4_0 || st.order == VYBDQ_Q4_GGML)
                  unit_dot<FMT, VYBDQ_Q4_GGML, 1>(dw[u], lds, sx, P, ks + G * (i0 + u), acc);
                else
                  unit_dot<FMT, VYBDQ_Q4_INTERLEAVED, 1>(dw[u], lds, sx, P, ks + G * (i0 + u), acc);
              }
            }
          }
        }
        first = false;
        acc[0] = G == 16 ? group_sum<16>(acc[0]) : (G == 32 ? group_sum<32>(acc[0]) : group_sum<64>(acc[0]));
        if (act && ks == G - 1) {
          const void *RS = sg == 0 ? st.RS : nullptr;
          void *Y = pick3_ptr(st.Y, sg);
          switch (pick3(st.ydt, sg)) {
            case VYBDQ_F32: store_elem<VYBDQ_F32>(Y, RS, lrow, acc[0]); break;
            case VYBDQ_F16: store_elem<VYBDQ_F16>(Y, RS, lrow, acc[0]); break;
            case VYBDQ_BF16: store_elem<VYBDQ_BF16>(Y, RS, lrow, acc[0]); break;
            default: store_elem<VYBDQ_F64>(Y, RS, lrow, acc[0]); break;
          }
        }
      }
    } else if (threadIdx.x == 0) {
      __hip_atomic_fetch_or(status, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---- the multi-stage chain: stage weights in registers before the handover -------------------
//
// One workgroup of kC2Waves waves per CU. Wave 0 runs the handover and stages x; waves 1..7 own
// rows. Per stage every row-owning wave takes at most one tile (64 / G rows, G lanes per row; the
// largest G in {64, .., 4} whose tiles fit the row-owning waves of the grid) and holds the first
// first units of each of its lanes in registers; those loads for stage s + 1 are issued as soon as
// the workgroup has announced its stage-s rows, so the weights stream during the handover instead
// of after it. Handover, with no L2 writeback or invalidation:
//  - results go out with device-coherent stores (written through the XCD's L2), and each wave
//    waits for them (vmcnt 0) before the workgroup barrier;
//  - wave 0 then adds 1 to one arrival counter (monotonic over the call: stage s is complete at
//    workgroups * (s + 1)), polls it with device-coherent loads (bounded: a timeout sets an error
//    bit and the wait is abandoned, so every wave always reaches the end), reads the next stage's
//    x with device-coherent loads into LDS, and the workgroup converts it to the staged fp16 form;
//  - the last arrival of the last stage resets the counter: the workspace is zero between calls.
constexpr int kC2Waves = 8;
constexpr int kC2Threads = 64 * kC2Waves;
// polls of one wait: ~1 s; after a timeout a workgroup waits no more in that call, so a call with
// missing workgroups still ends within about a second
constexpr uint32_t kC2SpinLimit = 1u << 22;
constexpr int kC2Polls = 4;       // polls in flight
constexpr int kC2PollSleep = 4;   // s_sleep units (64 clocks each) between polls
// units held per lane: about 90 registers of weights
template <int FMT> constexpr int c2_maxu() {
  return 90 / Fmt<FMT>::PAIR_DWORDS > 2 ? 90 / Fmt<FMT>::PAIR_DWORDS : 2;
}

// store of one result row, device-coherent (written through the L2), with the residual of the
// reference's f64 mode read the same way
template <int DT>
__device__ __forceinline__ void store_coherent(void *p, const void *rs, int64_t i, float v) {
  if constexpr (DT == VYBDQ_F64) {
    double d = static_cast<double>(v);
    if (rs)
      d += __builtin_bit_cast(double, __hip_atomic_load(static_cast<const uint64_t *>(rs) + i, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT));
    __hip_atomic_store(static_cast<uint64_t *>(p) + i, __builtin_bit_cast(uint64_t, d), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  } else if constexpr (DT == VYBDQ_F32) {
    if (rs)
      v += __uint_as_float(__hip_atomic_load(static_cast<const uint32_t *>(rs) + i, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT));
    __hip_atomic_store(static_cast<uint32_t *>(p) + i, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    const uint16_t r16 = rs ? __hip_atomic_load(static_cast<const uint16_t *>(rs) + i, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT) : 0;
    uint16_t o;
    if constexpr (DT == VYBDQ_F16) {
      if (rs) v += half_bits_to_f32(r16);
      o = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
    } else {
      if (rs) v += bf16_to_f32(r16);
      o = f32_to_bf16(v);
    }
    __hip_atomic_store(static_cast<uint16_t *>(p) + i, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Direct global -> LDS load of 16 bytes per lane, device-coherent (sc1: past the XCD's L2, which
// may hold an older copy of the line): lane L's bytes at src go to LDS dst + 16 L (dst wave-uniform).
// Issued from asm: the caller waits for it with an explicit vmcnt.
__device__ __forceinline__ void lds_dma16_coherent(const void *src, const void *dst) {
  const uint32_t l = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void *)dst)));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off sc1" ::"v"(src), "s"(l)
               : "memory", "m0");
}

// lanes per row for a stage: the largest of 64 .. 4 whose tiles fit the row-owning waves (4 when
// none does: several rounds of tiles)
__device__ __forceinline__ int c2_pick_lg(uint32_t rows, uint32_t ncw) {
#pragma unroll
  for (int lg = 6; lg > 2; --lg)
    if (((rows + (64u >> lg) - 1) >> (6 - lg)) <= ncw) return lg;
  return 2;
}

template <int FMT>
__global__ void __launch_bounds__(kC2Threads) k_gemv_chain2(const int64_t *__restrict__ pblocks, int nstages,
                                                            int64_t pstride_words, int64_t maxK,
                                                            uint32_t *__restrict__ ws) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int PD = Fmt<FMT>::PAIR_DWORDS;
  constexpr int MAXU = c2_maxu<FMT>();
  constexpr int KALIGN = is_kquant<FMT>() ? 256 : 64;
  uint32_t *err = ws;
  uint32_t *cnt = ws + 1;
  const int maxP = static_cast<int>(maxK >> 6);
  char *lds = smem;
  float *sx = reinterpret_cast<float *>(smem + static_cast<size_t>(maxP) * XPAIR_STRIDE);
  char *raw = smem + static_cast<size_t>(maxP) * XSTAGE_PAIR_BYTES + (FMT == FMT_IQ2_S ? kIq2sLdsBytes : 0);
  const int nwg = gridDim.x;
  const int ncw = nwg * (kC2Waves - 1);  // row-owning waves of the grid
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int gcw = wave > 0 ? static_cast<int>(blockIdx.x) + nwg * (wave - 1) : 0;  // this wave's first tile

  // a stage's descriptor and work split, the same in every wave
  struct Plan {
    StageDesc st;
    bool valid;
    int P, lg, G, npl, ks;
    int64_t rows, tiles;
  };
  auto plan = [&](int s) __attribute__((always_inline)) {
    Plan q;
    const int64_t *pb = pblocks + s * pstride_words;
    q.st = read_stage(pb, false);
    q.P = static_cast<int>(q.st.K >> 6);
    bool segs_ok = q.st.end[0] >= 0 && q.st.end[1] >= q.st.end[0] && q.st.end[2] >= q.st.end[1];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const bool used = q.st.end[i] > (i == 0 ? 0 : q.st.end[i - 1]);
      segs_ok = segs_ok && (!used || (q.st.W[i] && q.st.Y[i] && (reinterpret_cast<uintptr_t>(q.st.W[i]) & 3) == 0));
    }
    q.valid = segs_ok && q.st.K > 0 && q.st.K % KALIGN == 0 && q.st.K <= maxK && q.st.end[2] > 0 &&
              q.st.end[2] < (int64_t(1) << 30) && q.st.X && (reinterpret_cast<uintptr_t>(q.st.X) & 15) == 0 &&
              pb[3] == 1;
    q.rows = q.valid ? q.st.end[2] : 0;
    q.lg = c2_pick_lg(static_cast<uint32_t>(q.rows), static_cast<uint32_t>(ncw));
    q.G = 1 << q.lg;
    q.tiles = (q.rows + (64 >> q.lg) - 1) >> (6 - q.lg);
    q.ks = lane & (q.G - 1);
    q.npl = q.ks < q.P ? (q.P - q.ks + q.G - 1) >> q.lg : 0;
    return q;
  };
  // tile -> (segment, local row, weight row); lanes past the end read row 0 of segment 0
  auto tile_row = [&](const Plan &q, int64_t t, int &sg, int64_t &lrow, const uint8_t *&wrow, bool &act)
      __attribute__((always_inline)) {
    const int64_t row = t * (64 >> q.lg) + (lane >> q.lg);
    act = row < q.rows;
    sg = 0;
    if (row >= q.st.end[0]) sg = (row >= q.st.end[1]) ? 2 : 1;
    if (!act) sg = 0;
    lrow = act ? row - (sg == 0 ? 0 : (sg == 1 ? q.st.end[0] : q.st.end[1])) : 0;
    wrow = pick3_ptr(q.st.W, sg) + lrow * unit_row_bytes<FMT>(q.P);
  };
  uint32_t dw[MAXU][PD];
  // the held units of this wave's first tile of a stage (issued before the stage's wait)
  auto prefetch = [&](const Plan &q) __attribute__((always_inline)) {
    if (!q.valid || gcw >= q.tiles) return;
    int sg; int64_t lrow; const uint8_t *wrow; bool act;
    tile_row(q, gcw, sg, lrow, wrow, act);
#pragma unroll
    for (int u = 0; u < MAXU; ++u)
      if (u < q.npl) load_unit<FMT>(wrow, q.ks + q.G * u, dw[u]);
  };
  // the rows of a stage (ORDER: its q4_0 nibble order, fixed per stage): the held units of the
  // wave's first tile, then (a stage too large for the held registers) the remaining units one at
  // a time and further tiles
  auto rows_pass = [&](const Plan &q, auto order_c) __attribute__((always_inline)) {
    constexpr int ORDER = decltype(order_c)::value;
    // one tile; HELD: the wave's first tile, whose first MAXU units per lane are in dw
    auto tile = [&](int64_t t, auto held_c) __attribute__((always_inline)) {
      constexpr bool HELD = decltype(held_c)::value;
      int sg; int64_t lrow; const uint8_t *wrow; bool act;
      tile_row(q, t, sg, lrow, wrow, act);
      float acc[1] = {0.f};
      int i0 = 0;
      if constexpr (HELD) {
        // one unit at a time: interleaved by the scheduler, every unit's unpacked weights would be
        // live at once
#pragma unroll
        for (int u = 0; u < MAXU; ++u) {
          if (u < q.npl && act) unit_dot<FMT, ORDER, 1>(dw[u], lds, sx, q.P, q.ks + q.G * u, acc);
          __builtin_amdgcn_sched_barrier(0);
        }
        i0 = MAXU;
      }
      for (; i0 < q.npl; ++i0) {
        uint32_t dl[PD];
        load_unit<FMT>(wrow, q.ks + q.G * i0, dl);
        if (act) unit_dot<FMT, ORDER, 1>(dl, lds, sx, q.P, q.ks + q.G * i0, acc);
      }
      switch (q.lg) {
        case 2: acc[0] = group_sum<4>(acc[0]); break;
        case 3: acc[0] = group_sum<8>(acc[0]); break;
        case 4: acc[0] = group_sum<16>(acc[0]); break;
        case 5: acc[0] = group_sum<32>(acc[0]); break;
        default: acc[0] = group_sum<64>(acc[0]); break;
      }
      if (act && q.ks == q.G - 1) {
        const void *RS = sg == 0 ? q.st.RS : nullptr;
        void *Y = pick3_ptr(q.st.Y, sg);
        switch (pick3(q.st.ydt, sg)) {
          case VYBDQ_F32: store_coherent<VYBDQ_F32>(Y, RS, lrow, acc[0]); break;
          case VYBDQ_F16: store_coherent<VYBDQ_F16>(Y, RS, lrow, acc[0]); break;
          case VYBDQ_BF16: store_coherent<VYBDQ_BF16>(Y, RS, lrow, acc[0]); break;
          default: store_coherent<VYBDQ_F64>(Y, RS, lrow, acc[0]); break;
        }
      }
    };
    // the rows of a stage: the held first tile, then (more tiles than row-owning waves) the rest
    if (gcw < q.tiles) tile(gcw, std::true_type{});
    for (int64_t t = gcw + ncw; t < q.tiles; t += ncw) tile(t, std::false_type{});
  };
  // one plan is live at a time: a stage's is read at the top of its iteration (the block is in
  // the L2 by then), the next one's only for the addresses of its held units
  if (wave > 0) prefetch(plan(0));
  bool gave_up = false;  // wave 0: a wait timed out
  for (int s = 0; s < nstages; ++s) {
    const Plan cur = plan(s);
    // 1. wave 0: wait until every workgroup has completed stage s - 1, then x_s -> LDS (raw)
    if (wave == 0) {
      if (s > 0 && !gave_up) {
        // kC2Polls device-coherent polls in flight, a new one as each returns below the target:
        // the wait ends about one round trip after the last arrival
        const uint32_t target = static_cast<uint32_t>(nwg) * static_cast<uint32_t>(s);
        auto poll = [&]() { return __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
        uint32_t q[kC2Polls];
#pragma unroll
        for (int u = 0; u < kC2Polls; ++u) {
          q[u] = poll();
          __builtin_amdgcn_s_sleep(kC2PollSleep);
        }
        bool done = false;
        for (uint32_t spins = 0; !done; spins += kC2Polls) {
#pragma unroll
          for (int u = 0; u < kC2Polls; ++u) {
            if (!done && q[u] >= target) done = true;
            if (!done) {
              q[u] = poll();
              __builtin_amdgcn_s_sleep(kC2PollSleep);
            }
          }
          if (!done && spins > kC2SpinLimit) {
            if (lane == 0) __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            gave_up = true;
            done = true;
          }
        }
      }
      if (cur.valid) {
        // x_s straight into LDS in one round trip: 1 KB per load instruction, device-coherent (the x
        // of a stage may have been written in an earlier stage by another XCD's workgroups)
        const int nbytes = static_cast<int>(cur.st.K * (cur.st.xdt == VYBDQ_F32 ? 4 : 2));
        const char *src = static_cast<const char *>(cur.st.X);
        for (int off = 0; off < nbytes; off += 1024)
          if (off + 16 * lane < nbytes) lds_dma16_coherent(src + off + 16 * lane, raw + off);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
    }
    __syncthreads();
    // 2. the workgroup stages x_s: fp16 pairs and block sums (IQ2_S: then its grid tables)
    if (cur.valid) {
      if constexpr (FMT == FMT_IQ2_S) {
        u4 *gridh = iq2s_lds_grid(sx, 1, cur.P);
        for (int i0 = threadIdx.x; i0 < 1024 + 256; i0 += 5 * kC2Threads) {
          u4 v[5];
#pragma unroll
          for (int u = 0; u < 5; ++u)
            if (i0 + u * kC2Threads < 1024 + 256) v[u] = reinterpret_cast<const u4 *>(kIq2sLdsTab)[i0 + u * kC2Threads];
#pragma unroll
          for (int u = 0; u < 5; ++u)
            if (i0 + u * kC2Threads < 1024 + 256) gridh[i0 + u * kC2Threads] = v[u];
        }
      }
      const int nchunk = 8 * cur.P;
      for (int c = threadIdx.x; c < nchunk; c += kC2Threads) {
        if (cur.st.xdt == VYBDQ_F32) {
          uint32_t r[8];
          const u4 *q = reinterpret_cast<const u4 *>(raw + 32 * static_cast<size_t>(c));
          const u4 a = q[0], b = q[1];
          r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3]; r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
          stage_chunk<8>(r, cur.st.xdt, c, lds, sx);
        } else {
          uint32_t r[4];
          const u4 a = *reinterpret_cast<const u4 *>(raw + 16 * static_cast<size_t>(c));
          r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
          stage_chunk<4>(r, cur.st.xdt, c, lds, sx);
        }
      }
    }
    __syncthreads();
    const bool last = s + 1 == nstages;
    // 3. rows
    if (wave > 0 && cur.valid) {
      if (FMT == FMT_Q4_0 && cur.st.order == VYBDQ_Q4_INTERLEAVED)
        rows_pass(cur, std::integral_constant<int, VYBDQ_Q4_INTERLEAVED>{});
      else
        rows_pass(cur, std::integral_constant<int, VYBDQ_Q4_GGML>{});
    } else if (wave > 0 && threadIdx.x == 64) {
      __hip_atomic_fetch_or(err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // 4. this wave's results are performed
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // 5. arrival, not waited for (the last one of the last stage resets the counter for the next
    // call); only then the next stage's held units: issued first, their loads delayed the arrival
    // and queued the waits behind them (per-stage timestamps: 1.78 against 1.51 ms per decode step)
    if (threadIdx.x == 0) {
      if (!last) {
        __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == static_cast<uint32_t>(nwg) * static_cast<uint32_t>(nstages) - 1u)
          __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (wave > 0 && !last) prefetch(plan(s + 1));
  }
}

template <int FMT>
static int chain2_launch(uint64_t P, int nstages, int64_t pstride, int64_t maxK, uint64_t ws, hipStream_t s) {
  const int maxP = static_cast<int>(maxK / 64);
  const size_t lds = static_cast<size_t>(maxP) * XSTAGE_PAIR_BYTES + (FMT == FMT_IQ2_S ? kIq2sLdsBytes : 0) +
                     static_cast<size_t>(maxK) * 4;
  if (lds > 160 * 1024) return set_error(VYBDQ_ERR_SHAPE, "gemv chain: max_K too large for the LDS x stage");
  const void *fn = reinterpret_cast<const void *>(&k_gemv_chain2<FMT>);
  if (lds > 64 * 1024) {
    static std::atomic<uint64_t> raised{0};
    const int rc = ensure_lds_limit(fn, 160 * 1024, raised, "gemv chain");
    if (rc) return rc;
  }
  static std::atomic<int64_t> occ[64];
  int per_cu = 0;
  const int orc = resident_per_cu(fn, kC2Threads, lds, occ, per_cu, "gemv chain");
  if (orc) return orc;
  if (per_cu < 1) return set_error(VYBDQ_ERR_SHAPE, "gemv chain: a workgroup does not fit on a CU");
  hipLaunchKernelGGL((k_gemv_chain2<FMT>), dim3(static_cast<unsigned>(device_cu_count())), dim3(kC2Threads), lds, s,
                     reinterpret_cast<const int64_t *>(P), nstages, pstride / 8, maxK, reinterpret_cast<uint32_t *>(ws));
  return check_launch("gemv chain");
}

static int chain2_dispatch(int wtype, uint64_t P, int nstages, int64_t pstride, int64_t maxK, uint64_t ws,
                           hipStream_t s) {
  switch (wtype) {
    case 2: return chain2_launch<FMT_Q4_0>(P, nstages, pstride, maxK, ws, s);
    case 8: return chain2_launch<FMT_Q8_0>(P, nstages, pstride, maxK, ws, s);
    case 12: return chain2_launch<FMT_Q4_K>(P, nstages, pstride, maxK, ws, s);
    case 13: return chain2_launch<FMT_Q5_K>(P, nstages, pstride, maxK, ws, s);
    case 14: return chain2_launch<FMT_Q6_K>(P, nstages, pstride, maxK, ws, s);
    default: return chain2_launch<FMT_IQ2_S>(P, nstages, pstride, maxK, ws, s);
  }
}

// The GEMV kind of vybdq_launch_pblock: 256-thread workgroups, as many as fit per CU, so that a
// wave's rows are covered in one round (512-thread workgroups hold fewer waves per CU at these
// register counts: measured slower).
template <int FMT>
static int pb_gemv_launch(uint64_t P, int64_t maxK, uint32_t *status, hipStream_t s) {
  const int maxP = static_cast<int>(maxK / 64);
  const size_t lds = static_cast<size_t>(maxP) * XSTAGE_PAIR_BYTES + (FMT == FMT_IQ2_S ? kIq2sLdsBytes : 0);
  if (lds > 160 * 1024) return set_error(VYBDQ_ERR_SHAPE, "p-block gemv: max K too large for the LDS x stage");
  const void *fn = reinterpret_cast<const void *>(&k_pb_gemv<FMT>);
  // resident workgroups per CU for this LDS size: queried once per device and size (the LDS
  // attribute and the occupancy query stay out of later launches, which may be under capture)
  if (lds > 64 * 1024) {
    static std::atomic<uint64_t> raised{0};
    const int rc = ensure_lds_limit(fn, 160 * 1024, raised, "p-block gemv");
    if (rc) return rc;
  }
  static std::atomic<int64_t> occ[64];
  int per_cu = 0;
  const int orc = resident_per_cu(fn, kChainThreads, lds, occ, per_cu, "p-block gemv");
  if (orc) return orc;
  hipLaunchKernelGGL((k_pb_gemv<FMT>), dim3(device_cu_count() * (per_cu < 8 ? per_cu : 8)), dim3(kChainThreads), lds,
                     s, reinterpret_cast<const int64_t *>(P), maxK, status);
  return check_launch("p-block gemv");
}

// GGML type id -> the one-stage launch of that format
int pb_gemv_dispatch(int wtype, uint64_t P, int64_t maxK, uint32_t *status, hipStream_t s) {
  switch (wtype) {
    case 2: return pb_gemv_launch<FMT_Q4_0>(P, maxK, status, s);
    case 8: return pb_gemv_launch<FMT_Q8_0>(P, maxK, status, s);
    case 12: return pb_gemv_launch<FMT_Q4_K>(P, maxK, status, s);
    case 13: return pb_gemv_launch<FMT_Q5_K>(P, maxK, status, s);
    case 14: return pb_gemv_launch<FMT_Q6_K>(P, maxK, status, s);
    default: return pb_gemv_launch<FMT_IQ2_S>(P, maxK, status, s);
  }
}

}  // namespace vybdq

using namespace vybdq;

extern "C" int64_t vybdq_chain_workspace_size(int nstages) {
  if (nstages < 1) return 0;
  return 4 * (1 + static_cast<int64_t>(nstages));
}

extern "C" int vybdq_gemv_chain(int wtype, uint64_t P, int nstages, int64_t pstride, int64_t max_K, uint64_t ws,
                                uint64_t stream) {
  VYBDQ_REQUIRE(P && ws, VYBDQ_ERR_ARG, "null P or workspace");
  VYBDQ_REQUIRE(wtype == 2 || wtype == 8 || wtype == 12 || wtype == 13 || wtype == 14 || wtype == 22, VYBDQ_ERR_ARG,
                "wtype must be 2 (q4_0), 8 (Q8_0), 12 (Q4_K), 13 (Q5_K), 14 (Q6_K) or 22 (IQ2_S)");
  VYBDQ_REQUIRE(nstages >= 1 && nstages <= (1 << 20), VYBDQ_ERR_SHAPE, "nstages out of range");
  VYBDQ_REQUIRE(pstride >= 152 && pstride % 8 == 0, VYBDQ_ERR_SHAPE, "pstride must be >= 152 and a multiple of 8");
  VYBDQ_REQUIRE(max_K >= 64 && max_K % 64 == 0, VYBDQ_ERR_SHAPE, "max_K must be a positive multiple of 64");
  VYBDQ_REQUIRE((P & 7) == 0 && (ws & 3) == 0, VYBDQ_ERR_ALIGN, "P must be 8-byte and ws 4-byte aligned");
  VYBDQ_REQUIRE(wtype <= 8 || max_K % 256 == 0, VYBDQ_ERR_SHAPE, "super-block types need max_K % 256 == 0");
  return chain2_dispatch(wtype, P, nstages, pstride, max_K, ws, as_stream(stream));
}

extern "C" int vybdq_chain_status(uint64_t ws) {
  VYBDQ_REQUIRE(ws, VYBDQ_ERR_ARG, "null workspace");
  uint32_t v = 0;
  hipError_t e = hipMemcpy(&v, reinterpret_cast<const void *>(ws), 4, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return set_error(VYBDQ_ERR_HIP, std::string("vybdq_chain_status: ") + hipGetErrorString(e));
  if (v & 1u) return set_error(VYBDQ_ERR_HIP, "gemv chain: a stage wait timed out (workgroups not co-resident?)");
  if (v & 2u) return set_error(VYBDQ_ERR_SHAPE, "gemv chain: a stage descriptor was invalid (K, N or max_K)");
  return VYBDQ_OK;
}
