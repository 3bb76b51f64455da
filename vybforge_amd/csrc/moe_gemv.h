// Grouped multi-token dequant GEMV for the MoE experts when each expert receives few tokens
// (decode-sized batches), gfx950.
//
// A group is an expert that received tokens (or the shared expert) with its rows [r0, r1) of the
// bucketed row order; row_map gives each row's token. The bucketing splits experts with more rows
// into groups of at most MC rows over the same weights, so that no workgroup repeats a walk over
// the weights per chunk of MC tokens. The work is (group, slice of CPP output columns) units in
// group-major order, cut in one of two ways:
//  - single tokens (every group one row, so every unit costs the same): equal contiguous ranges,
//    one per workgroup of a grid sized to the workgroups the device holds at once, so every
//    workgroup streams the same number of weight rows (a range can span the end of one group
//    and the start of the next) and none waits for a second round of the grid;
//  - several tokens (units cost more in groups with more rows): one block of columns of one
//    group per workgroup, many more workgroups than the device holds, so the dispatcher evens
//    out the cost.
// For each group in its range the workgroup stages the x
// rows of the group's tokens into LDS (fp16 + block sums, the layout pair_dot reads) and walks
// its weight rows in passes of 256/G rows, G lanes per row reading consecutive pairs (one
// contiguous run of the row per load instruction), with the next passes' pair windows in flight
// while the current pass computes (a register ring).
//
// SwiGLU (gate|up): each wave holds gate rows in its first 32 lanes and the up rows of the same
// output columns in its last 32, so after the DPP row reduction the pair (g, u) is one lane
// exchange apart; the epilogue writes silu(min(g, L)) * clamp(u, -L, L) as fp16
// (native/glm53/moe_ref.py:81-84). Otherwise the row sums are stored as f32.
#pragma once
#include "gemv_dev.h"
#include "moe_route.h"

namespace vybdq {

// One token routed inside the gate|up launch (E > 0; see moe_gv_route).
struct MoeGvRoute {
  const void *logits;
  int ldt;                 // F64, F32, F16 or BF16
  const float *bias;       // selection bias or null
  int E, topk, shared;     // shared: 1 with a shared expert
  double scale;
  int *idx_out;            // [topk] expert ids (workgroup 0 writes them)
  float *w_out;            // [topk] routing weights
  int *pos;                // [topk] row of each slot: the slot itself
  int4 *groups_out;        // the groups below, for the down launch
  int *ngroups_out;
};

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
  int cols_per_wg;         // > 0: one (group, block of this many columns) per workgroup
  int wg_per_cu;           // cols_per_wg = 0: grid = wg_per_cu x CUs (0: what a CU holds at
                           // once, -k: k times that)
  void *Y;
  int ydt;                 // F16 or F32
  int64_t ldy;
  float limit;
  int mc;                  // tokens per group (x stage), 1..kMoeGvMC
  MoeGvRoute rt;           // rt.E > 0: route the token here (one token, gate|up, mc = 1)
};

constexpr int kMoeGvMC = 4;  // largest x stage
constexpr int kMoeGvD = 3;   // passes of pair windows in flight per lane (a register ring)

// output columns per pass: 4 waves x (64 / G rows, SwiGLU: half of them gate, half up)
constexpr int moe_gv_cpp(int G, bool swi) { return 4 * (swi ? 32 / G : 64 / G); }

__device__ __forceinline__ float moe_silu(float g) { return g / (1.0f + __expf(-g)); }

// One chunk of MC tokens (rows r0c .. r0c + MC - 1) over the workgroup's columns. LONG: rows of more
// than U G pairs, whose lanes take further batches beyond the prefetched U pairs; without it every
// lane's pairs are the prefetched ones and the pass has no loop (a loop whose batches reload the
// ring slot made the compiler wait for every load in flight, the next passes' included, before
// each pass).
template <int FMT, int G, int U, int MC, bool SWI, int XW, bool LONG>
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
  constexpr int CPP = moe_gv_cpp(G, SWI);     // columns per pass (4 CPW)
  // this lane's column offset within the pass and its matrix
  const bool up = SWI && rs >= RPW / 2;
  const int cslot = w * CPW + (up ? rs - RPW / 2 : rs);
  const uint8_t *Wm = up ? Wu : Wg;

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
  // Order of the loads: the chunk's token rows, the first NB x chunks of every thread, then the
  // first passes' weights (which do not depend on x), so the weights are in flight while x is
  // staged; longer x stages (several tokens, long rows) load the rest afterwards.
  int xr[MC];
#pragma unroll
  for (int m = 0; m < MC; ++m) xr[m] = a.row_map ? a.row_map[r0c + m] : r0c + m;
  const int cpr = 8 * P;  // 16-byte chunks per x row
  const int nchunk = MC * cpr;
  constexpr int NB = 4;
  auto load_x = [&](int c, uint32_t (&r)[XW]) {
    const int m = c / cpr;
    int row = xr[0];
#pragma unroll
    for (int mm = 1; mm < MC; ++mm) row = m == mm ? xr[mm] : row;
    load_x_chunk<XW>(a.X, static_cast<int64_t>(row) * a.ldx + 8 * static_cast<int64_t>(c - m * cpr), r);
  };
  // (no branches around these loads: out-of-range chunks and passes re-read the last one)
  uint32_t r0[NB][XW];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int c = threadIdx.x + b * T;
    load_x(c < nchunk ? c : nchunk - 1, r0[b]);
  }
  uint32_t ring[kMoeGvD][U][PD];
#pragma unroll
  for (int j = 0; j < kMoeGvD - 1; ++j) load_pass(j < npass ? j : npass - 1, ring[j]);

  // x rows of the chunk -> LDS (fp16 pairs + block sums)
  __syncthreads();  // the previous chunk's readers are done
#pragma unroll
  for (int b = 0; b < NB; ++b)
    if (threadIdx.x + b * T < nchunk) stage_chunk<XW>(r0[b], a.xdt, threadIdx.x + b * T, lds, sx);
  for (int c0 = threadIdx.x + NB * T; c0 < nchunk; c0 += NB * T) {
    uint32_t r[NB][XW];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int c = c0 + b * T;
      load_x(c < nchunk ? c : nchunk - 1, r[b]);
    }
#pragma unroll
    for (int b = 0; b < NB; ++b)
      if (c0 + b * T < nchunk) stage_chunk<XW>(r[b], a.xdt, c0 + b * T, lds, sx);
  }
  __syncthreads();

  // pass ps from buffer cur; first pass ps + kMoeGvD - 1 is issued into nxt (the buffer of pass
  // ps - 1, already consumed), so kMoeGvD - 1 passes stay in flight while a pass computes
  auto pass = [&](int ps, uint32_t (&cur)[U][PD], uint32_t (&nxt)[U][PD]) {
    // issued on every pass (the last ones re-read the chunk's last pass): the same loads on every
    // path, so the waits below leave the next passes in flight
    load_pass(ps + kMoeGvD - 1 < npass ? ps + kMoeGvD - 1 : npass - 1, nxt);
    float acc[MC];
#pragma unroll
    for (int m = 0; m < MC; ++m) acc[m] = 0.f;
    if constexpr (LONG) {
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
    } else {
      // branch-free: a lane with fewer than U pairs (K not a multiple of 64 G) drops the products
      // of its clamped re-reads
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float t[MC];
#pragma unroll
        for (int m = 0; m < MC; ++m) t[m] = 0.f;
        pair_dot<FMT, VYBDQ_Q4_GGML, MC>(cur[u], lds, sx, P, u < npairs ? ks + G * u : (ks < P ? ks : 0), t);
#pragma unroll
        for (int m = 0; m < MC; ++m) acc[m] += u < npairs ? t[m] : 0.f;
      }
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
  // LONG: passes past the chunk are skipped. Otherwise every round runs its kMoeGvD passes (those
  // past the chunk re-read its last pass and store nothing), so every path issues the same loads
  // and the compiler's waits keep the next passes in flight.
  for (int ps = 0; ps < npass; ps += kMoeGvD) {
#pragma unroll
    for (int k = 0; k < kMoeGvD; ++k)
      if (!LONG || ps + k < npass) pass(ps + k, ring[k], ring[(k + kMoeGvD - 1) % kMoeGvD]);
  }
}

// LDS bytes of the x stage, and of the routing area after it (RENT experts per router lane):
// groups (80 x 16 B), slot ids and weights (64 + 64 words), keys and scores (64 RENT x 8 B each)
__host__ __device__ inline size_t moe_gv_xstage_bytes(int mc, int P) { return (static_cast<size_t>(mc) * P * XSTAGE_PAIR_BYTES + 15) & ~size_t(15); }
constexpr size_t moe_gv_route_bytes(int RENT) { return RENT ? 1280 + 512 + 2 * 64 * 8 * static_cast<size_t>(RENT) : 0; }

// One token's routing by the workgroup (the router of k_moe_route_bucket_w: route_wg), into the
// groups of the grouped GEMV in LDS: slot s -> group {idx[s], s, s + 1} (row s), the shared expert
// -> {-1, topk, topk + 1}. Every workgroup routes the token (the same keys, the same selection);
// workgroup 0 also writes the ids, weights, rows and groups that the down launch and the combine
// read. Returns the number of groups.
template <int RENT>
__device__ __forceinline__ int moe_gv_route(const MoeGvRoute &r, char *buf) {
  int4 *grp = reinterpret_cast<int4 *>(buf);
  int *idl = reinterpret_cast<int *>(buf + 1280);
  float *wl = reinterpret_cast<float *>(buf + 1536);
  uint64_t *key = reinterpret_cast<uint64_t *>(buf + 1792);
  double *score = reinterpret_cast<double *>(key + 64 * RENT);
  if (threadIdx.x < 64) idl[threadIdx.x] = 0;  // every slot names an expert (topk <= E selects only real ones)
  switch (r.ldt) {
    case VYBDQ_F64: route_wg_keys<VYBDQ_F64>(r.logits, r.bias, 0, r.E, key, score); break;
    case VYBDQ_F16: route_wg_keys<VYBDQ_F16>(r.logits, r.bias, 0, r.E, key, score); break;
    case VYBDQ_BF16: route_wg_keys<VYBDQ_BF16>(r.logits, r.bias, 0, r.E, key, score); break;
    default: route_wg_keys<VYBDQ_F32>(r.logits, r.bias, 0, r.E, key, score); break;
  }
  __syncthreads();
  if (threadIdx.x < 64) route_wg_select<RENT>(0, r.E, r.topk, r.scale, idl, wl, nullptr, key, score);
  __syncthreads();
  const int tid = threadIdx.x, k = r.topk;
  if (tid <= k) {
    const int4 d = tid < k ? make_int4(idl[tid], tid, tid + 1, 0) : make_int4(-1, k, k + 1, 0);
    if (tid < k || r.shared) {
      grp[tid] = d;
      if (blockIdx.x == 0) r.groups_out[tid] = d;
    }
    if (blockIdx.x == 0 && tid < k) {
      r.idx_out[tid] = idl[tid];
      r.w_out[tid] = wl[tid];
      r.pos[tid] = tid;
    }
    if (blockIdx.x == 0 && tid == 0) *r.ngroups_out = k + r.shared;
  }
  __syncthreads();
  return k + r.shared;
}

// MCMAX: the largest group (1 when every group holds one row: a single token). RENT > 0: the
// token is routed here first (moe_gv_route; one token, mc = 1, no column blocks).
template <int FMT, int G, int U, bool SWI, int XW, int MCMAX, bool LONG, int RENT = 0>
__global__ void __launch_bounds__(256) k_moe_gemv(MoeGvArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int CPP = moe_gv_cpp(G, SWI);
  const int spg = (a.N + CPP - 1) / CPP;  // column slices per group
  const int4 *groups = a.groups;
  int ngroups;
  if constexpr (RENT > 0) {
    char *rbuf = smem + moe_gv_xstage_bytes(a.mc, a.P);
    ngroups = moe_gv_route<RENT>(a.rt, rbuf);
    groups = reinterpret_cast<const int4 *>(rbuf);
  } else {
    ngroups = *a.ngroups;
  }
  int64_t beg, end;
  if (a.cols_per_wg > 0) {
    const int bs = a.cols_per_wg / CPP;  // slices per block
    const int nblk = (spg + bs - 1) / bs;
    const int g = blockIdx.x / nblk;
    if (g >= ngroups) return;
    beg = static_cast<int64_t>(g) * spg + static_cast<int64_t>(blockIdx.x - g * nblk) * bs;
    end = beg + bs < static_cast<int64_t>(g + 1) * spg ? beg + bs : static_cast<int64_t>(g + 1) * spg;
  } else {
    const int64_t tot = static_cast<int64_t>(ngroups) * spg;
    beg = tot * blockIdx.x / gridDim.x;
    end = tot * (blockIdx.x + 1) / gridDim.x;
  }
  char *lds = smem;
  float *sx = reinterpret_cast<float *>(smem + static_cast<size_t>(a.mc) * a.P * XPAIR_STRIDE);
  for (int64_t u = beg; u < end;) {
    const int g = static_cast<int>(u / spg);
    const int64_t gb = static_cast<int64_t>(g) * spg;
    const int n0 = static_cast<int>(u - gb) * CPP;
    const int s1 = static_cast<int>(end - gb < spg ? end - gb : spg);
    const int ncols = (s1 * CPP < a.N ? s1 * CPP : a.N) - n0;
    const int4 d = groups[g];
    const uint8_t *Wg, *Wu = nullptr;
    if (d.x < 0) {
      Wg = a.Ws;
      Wu = a.W2s;
    } else {
      Wg = a.W + static_cast<int64_t>(d.x) * a.w_stride;
      if constexpr (SWI) Wu = a.W2 + static_cast<int64_t>(d.x) * a.w_stride;
    }
    for (int r = d.y; r < d.z; r += a.mc) {
      if constexpr (MCMAX == 1) {
        moe_gv_chunk<FMT, G, U, 1, SWI, XW, LONG>(a, Wg, Wu, r, n0, ncols, lds, sx);
      } else {
        switch (d.z - r < a.mc ? d.z - r : a.mc) {
          case 1: moe_gv_chunk<FMT, G, U, 1, SWI, XW, LONG>(a, Wg, Wu, r, n0, ncols, lds, sx); break;
          case 2: moe_gv_chunk<FMT, G, U, 2, SWI, XW, LONG>(a, Wg, Wu, r, n0, ncols, lds, sx); break;
          case 3: moe_gv_chunk<FMT, G, U, 3, SWI, XW, LONG>(a, Wg, Wu, r, n0, ncols, lds, sx); break;
          default: moe_gv_chunk<FMT, G, U, 4, SWI, XW, LONG>(a, Wg, Wu, r, n0, ncols, lds, sx); break;
        }
      }
    }
    u = gb + spg;
  }
}

template <int FMT, int G, int U, bool SWI, int XW, int MCMAX, bool LONG, int RENT = 0>
int moe_gemv_launch2(const MoeGvArgs &a, int max_groups, hipStream_t s) {
  const void *fn = reinterpret_cast<const void *>(&k_moe_gemv<FMT, G, U, SWI, XW, MCMAX, LONG, RENT>);
  const size_t lds = RENT ? moe_gv_xstage_bytes(a.mc, a.P) + moe_gv_route_bytes(RENT)
                          : static_cast<size_t>(a.mc) * a.P * XSTAGE_PAIR_BYTES;
  if (lds > 64 * 1024) {
    static std::atomic<uint64_t> raised{0};
    const int rc = ensure_lds_limit(fn, 160 * 1024, raised, "moe gemv");
    if (rc) return rc;
  }
  constexpr int CPP = moe_gv_cpp(G, SWI);
  const int spg = (a.N + CPP - 1) / CPP;
  if (a.cols_per_wg > 0) {
    if (a.cols_per_wg % CPP) return set_error(VYBDQ_ERR_SHAPE, "moe gemv: columns per workgroup not a multiple of the pass");
    const int bs = a.cols_per_wg / CPP;
    const int64_t grid = static_cast<int64_t>(max_groups) * ((spg + bs - 1) / bs);
    hipLaunchKernelGGL((k_moe_gemv<FMT, G, U, SWI, XW, MCMAX, LONG, RENT>), dim3(static_cast<unsigned>(grid)), dim3(256), lds, s, a);
    return check_launch("moe grouped gemv");
  }
  int per_cu = a.wg_per_cu;
  if (per_cu <= 0) {
    const int mult = per_cu < 0 ? -per_cu : 1;
    // resident workgroups per CU for this LDS size (per device; the last size queried is kept)
    static std::atomic<int64_t> occ[64];
    int nb = 1;
    const int rc = resident_per_cu(fn, 256, lds, occ, nb, "moe gemv");
    if (rc) return rc;
    per_cu = nb * mult;
  }
  const int64_t units = static_cast<int64_t>(max_groups) * spg;
  int64_t grid = static_cast<int64_t>(per_cu) * device_cu_count();
  grid = grid < units ? grid : units;
  hipLaunchKernelGGL((k_moe_gemv<FMT, G, U, SWI, XW, MCMAX, LONG, RENT>), dim3(static_cast<unsigned>(grid)), dim3(256), lds, s, a);
  return check_launch("moe grouped gemv");
}

template <int FMT, int G, int U, bool SWI, int XW, bool LONG = false>
int moe_gemv_launch1(const MoeGvArgs &a, int max_groups, hipStream_t s) {
  if constexpr (SWI) {
    if (a.rt.E > 0) {
      if (a.mc != 1 || a.cols_per_wg > 0 || a.rt.E > 256 || a.rt.topk < 1 || a.rt.topk > a.rt.E)
        return set_error(VYBDQ_ERR_ARG, "moe gemv: routing in the gate|up launch needs one token, E <= 256, no column blocks");
      return moe_gemv_launch2<FMT, G, U, SWI, XW, 1, LONG, 4>(a, max_groups, s);
    }
  }
  return a.mc == 1 ? moe_gemv_launch2<FMT, G, U, SWI, XW, 1, LONG>(a, max_groups, s)
                   : moe_gemv_launch2<FMT, G, U, SWI, XW, kMoeGvMC, LONG>(a, max_groups, s);
}

// gate|up (swi): 32 lanes per row; down: 16. The pair batch covers a row's pairs per lane (at
// most 4 pairs in flight per lane; longer rows take extra unprefetched batches: U = 5 below).
template <int FMT>
int moe_gemv_launch(bool swi, const MoeGvArgs &a, int max_groups, hipStream_t s) {
  const int G = swi ? 32 : 16;
  int U = (a.P + G - 1) / G;
  U = U < 1 ? 1 : (U > 4 ? 5 : U);
  if (swi) {
    if (a.xdt == VYBDQ_F32) {
      switch (U) {
        case 1: return moe_gemv_launch1<FMT, 32, 1, true, 8>(a, max_groups, s);
        case 2: return moe_gemv_launch1<FMT, 32, 2, true, 8>(a, max_groups, s);
        case 3: return moe_gemv_launch1<FMT, 32, 3, true, 8>(a, max_groups, s);
        case 4: return moe_gemv_launch1<FMT, 32, 4, true, 8>(a, max_groups, s);
        default: return moe_gemv_launch1<FMT, 32, 4, true, 8, true>(a, max_groups, s);
      }
    }
    switch (U) {
      case 1: return moe_gemv_launch1<FMT, 32, 1, true, 4>(a, max_groups, s);
      case 2: return moe_gemv_launch1<FMT, 32, 2, true, 4>(a, max_groups, s);
      case 3: return moe_gemv_launch1<FMT, 32, 3, true, 4>(a, max_groups, s);
      case 4: return moe_gemv_launch1<FMT, 32, 4, true, 4>(a, max_groups, s);
      default: return moe_gemv_launch1<FMT, 32, 4, true, 4, true>(a, max_groups, s);
    }
  }
  switch (U) {  // down: X is the fp16 activations
    case 1: return moe_gemv_launch1<FMT, 16, 1, false, 4>(a, max_groups, s);
    case 2: return moe_gemv_launch1<FMT, 16, 2, false, 4>(a, max_groups, s);
    case 3: return moe_gemv_launch1<FMT, 16, 3, false, 4>(a, max_groups, s);
    case 4: return moe_gemv_launch1<FMT, 16, 4, false, 4>(a, max_groups, s);
    default: return moe_gemv_launch1<FMT, 16, 4, false, 4, true>(a, max_groups, s);
  }
}

// moe_gemv_q4.hip / moe_gemv_q8.hip
int moe_gemv_q4(bool swi, const MoeGvArgs &a, int max_groups, hipStream_t s);
int moe_gemv_q8(bool swi, const MoeGvArgs &a, int max_groups, hipStream_t s);

}  // namespace vybdq
