// Persistent chain of dependent GEMV stages (any GGUF type of the pair GEMV) in one launch, gfx950.
//
// A decode step is a sequence of GEMVs where stage s may consume stage s-1's output. As
// separate launches each stage pays the dependent-launch floor (~1.7 us per graph node) plus
// a full HBM round trip before its first weight byte arrives. Here one persistent grid runs
// every stage: a workgroup issues the weight loads of its first tile of stage s (weights never
// depend on activations), THEN waits until every workgroup has finished stage s-1 (an acquire
// spin on a per-stage counter), stages x_s into LDS and computes. HBM keeps streaming across
// stage boundaries.
//
// Stage descriptors are the reference's GEMV parameter blocks, read from device memory
// (native/host/ridge_decode.vyb:264-270, native/kernels/qwen3.vyb:410-440), one per stage at
// P + s * pstride, little-endian int64 words:
//   W@0 X@8 Y@16 M@24 N@32 K@40 YE@48 W2@56 NS2@64 Y2@72 YE2@80 W3@88 NS3@96 Y3@104 YE3@112
//   RS@120 GRID@128, and two words the reference does not have: XE@136 (x element type) and
//   ORDER@144 (q4_0 nibble order). YE: 4 = f32, 2 = f16, 258 = bf16, anything else = f64 (the
//   reference's f64 mode, with the f64 residual RS). XE: 2 = f16, 258 = bf16, else f32. M must be 1.
//
// Synchronisation: after its last tile of stage s the workgroup barriers and one thread adds 1
// to counter[s] with agent-scope release semantics; a waiting workgroup polls the counter with
// relaxed loads, then one thread issues an agent-scope acquire fence before the barrier. Waits are
// bounded (spin limit -> an error word in the workspace, and the wait is abandoned) so every
// wave always reaches the end of the kernel. The grid is sized from the occupancy API so all
// workgroups are resident together. The workgroup that completes the last stage last resets
// the counters, leaving the workspace zero-filled for the next call.
#include "gemv_dev.h"

#include <atomic>

namespace vybdq {

constexpr int kChainThreads = 256;
constexpr uint32_t kSpinLimit = 1u << 22;  // ~0.5 s of s_sleep polling before giving up

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

template <int FMT, int NT = kChainThreads>
__global__ void __launch_bounds__(NT) k_gemv_chain(const int64_t *__restrict__ pblocks, int nstages,
                                                              int64_t pstride_words, int64_t maxK,
                                                              uint32_t *__restrict__ ws, int ref_layout) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int U = chain_batch<FMT>();
  constexpr int PD = Fmt<FMT>::PAIR_DWORDS;
  constexpr int KALIGN = is_kquant<FMT>() ? 256 : 64;
  uint32_t *err = ws;
  uint32_t *cnt = ws + 1;
  const int maxP = static_cast<int>(maxK >> 6);
  char *lds = smem;
  float *sx = reinterpret_cast<float *>(smem + static_cast<size_t>(maxP) * XPAIR_STRIDE);
  const int nwg = gridDim.x;
  const int nwaves = nwg * (NT / 64);
  const int gw = blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  for (int s = 0; s < nstages; ++s) {
    const StageDesc st = read_stage(pblocks + s * pstride_words, ref_layout != 0);
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
                       pblocks[s * pstride_words + 3] == 1;
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

    // 1. prefetch the first batch of this wave's first tile (independent of stage s-1)
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

    // 2. wait until every workgroup finished stage s-1
    if (s > 0) {
      if (threadIdx.x == 0) {
        uint32_t spins = 0;
        // relaxed polls (an acquire per poll would invalidate the caches of the whole chip
        // 512 times per stage); one acquire fence follows the successful poll
        while (__hip_atomic_load(cnt + (s - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) <
               static_cast<uint32_t>(nwg)) {
          __builtin_amdgcn_s_sleep(2);
          if (++spins > kSpinLimit) {
            __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
        }
        // one acquire per workgroup: invalidates this CU's L1 and the stale L2 lines; the
        // barrier below orders every other thread's loads after it
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      }
      __syncthreads();
    }

    // 3. stage x_s into LDS (it may be stage s-1's output); IQ2_S: then its grid tables behind the
    // block sums, where the unit dot of this stage's P reads them
    if (valid) {
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
      const int nchunk = 8 * P;
      for (int c = threadIdx.x; c < nchunk; c += NT) {
        if (st.xdt == VYBDQ_F32) {
          uint32_t r[8];
          load_x_chunk<8>(st.X, 8 * static_cast<int64_t>(c), r);
          stage_chunk<8>(r, st.xdt, c, lds, sx);
        } else {
          uint32_t r[4];
          load_x_chunk<4>(st.X, 8 * static_cast<int64_t>(c), r);
          stage_chunk<4>(r, st.xdt, c, lds, sx);
        }
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
      __hip_atomic_fetch_or(err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // 5. publish: the barrier drains every thread's stores into this XCD's L2; one thread's
    // agent-scope release (an L2 writeback, then the increment) makes them visible chip-wide.
    // A fence per thread would write back the whole L2 256 times per workgroup per stage.
    // __syncthreads() does not wait for outstanding global stores, so wait for them first.
    // A single stage has no waiter: the end of the kernel publishes its stores.
    if (nstages == 1) break;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t old = __hip_atomic_fetch_add(cnt + s, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
      if (s == nstages - 1 && old == static_cast<uint32_t>(nwg - 1)) {
        // every workgroup has passed every wait: leave the counters zeroed for the next call
        for (int i = 0; i < nstages; ++i)
          __hip_atomic_store(cnt + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

template <int FMT, int NT>
static int chain_launch_nt(uint64_t P, int nstages, int64_t pstride, int64_t maxK, uint64_t ws, int ref_layout,
                        int max_per_cu, hipStream_t s) {
  const int maxP = static_cast<int>(maxK / 64);
  const size_t lds = static_cast<size_t>(maxP) * XSTAGE_PAIR_BYTES + (FMT == FMT_IQ2_S ? kIq2sLdsBytes : 0);
  if (lds > 160 * 1024) return set_error(VYBDQ_ERR_SHAPE, "gemv chain: max_K too large for the LDS x stage");
  const int cus = device_cu_count();
  const void *fn = reinterpret_cast<const void *>(&k_gemv_chain<FMT, NT>);
  // resident workgroups per CU for this LDS size: queried once per device and size (the LDS
  // attribute and the occupancy query stay out of later launches, which may be under capture)
  if (lds > 64 * 1024) {
    static std::atomic<uint64_t> raised{0};
    const int rc = ensure_lds_limit(fn, 160 * 1024, raised, "gemv chain");
    if (rc) return rc;
  }
  static std::atomic<int64_t> occ[64];
  int per_cu = 0;
  const int orc = resident_per_cu(fn, NT, lds, occ, per_cu, "gemv chain");
  if (orc) return orc;
  // a chain: two workgroups per CU keep the waits short while every workgroup stays resident; one
  // stage (no waits): as many as fit
  const int grid = cus * (per_cu < max_per_cu ? per_cu : max_per_cu);
  hipLaunchKernelGGL((k_gemv_chain<FMT, NT>), dim3(grid), dim3(NT), lds, s,
                     reinterpret_cast<const int64_t *>(P), nstages, pstride / 8, maxK,
                     reinterpret_cast<uint32_t *>(ws), ref_layout);
  return check_launch("gemv chain");
}

// 256-thread workgroups: a chain runs two per CU (short waits), a single stage (no waits, the GEMV
// kind of vybdq_launch_pblock) as many as fit, so that a wave's rows are covered in one round
// (512-thread workgroups hold fewer waves per CU at these register counts: measured slower).
template <int FMT>
static int chain_launch(uint64_t P, int nstages, int64_t pstride, int64_t maxK, uint64_t ws, int ref_layout,
                        int max_per_cu, hipStream_t s) {
  return chain_launch_nt<FMT, kChainThreads>(P, nstages, pstride, maxK, ws, ref_layout, max_per_cu, s);
}

// GGML type id -> the chain launch of that format (also the GEMV kind of vybdq_launch_pblock:
// one stage in the reference's own block layout, pblock.hip)
int chain_dispatch(int wtype, uint64_t P, int nstages, int64_t pstride, int64_t maxK, uint64_t ws, int ref_layout,
                   int max_per_cu, hipStream_t s) {
  switch (wtype) {
    case 2: return chain_launch<FMT_Q4_0>(P, nstages, pstride, maxK, ws, ref_layout, max_per_cu, s);
    case 8: return chain_launch<FMT_Q8_0>(P, nstages, pstride, maxK, ws, ref_layout, max_per_cu, s);
    case 12: return chain_launch<FMT_Q4_K>(P, nstages, pstride, maxK, ws, ref_layout, max_per_cu, s);
    case 13: return chain_launch<FMT_Q5_K>(P, nstages, pstride, maxK, ws, ref_layout, max_per_cu, s);
    case 14: return chain_launch<FMT_Q6_K>(P, nstages, pstride, maxK, ws, ref_layout, max_per_cu, s);
    default: return chain_launch<FMT_IQ2_S>(P, nstages, pstride, maxK, ws, ref_layout, max_per_cu, s);
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
  return chain_dispatch(wtype, P, nstages, pstride, max_K, ws, 0, 2, as_stream(stream));
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
