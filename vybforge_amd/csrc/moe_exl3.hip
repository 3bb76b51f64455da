// GLM-5.3 MoE layer with EXL3 4-bpw routed experts and a bf16 shared expert in one call, gfx950.
//
// The reference's production layer (native/glm53/glm_engine.vyb:2728-2990): sigmoid scores of the
// router logits, top-k over score + e_score_correction_bias (the bias only selects), weights
// score / sum * 2.5; then per used expert e a host loop resolves gate/up/down_proj.{trellis,suh,svh},
// dequantizes each matrix with exl3_deq32 to W [in, out] = diag(suh) Hs What Hs diag(svh) per
// 128 x 128 block (Hs = H128 / sqrt(128)), and computes a = silu(min(x Wg, L)) * clamp(x Wu, -L, L),
// y = a Wd, out[t] += w * y; the shared expert's bf16 mlp.shared_experts.{gate,up,down}_proj.weight
// ([out][in]) runs the same FFN on every token with weight 1 (:2955-2990).
//
// Here on the stream, with no host loop, no host synchronisation and no dequantized copy of any
// weight (x W = svh * FWHT(FWHT(x * suh)/sqrt(128) What)/sqrt(128) per 128 chunk):
//  1. route + bucket (moe.hip): rows = (token, slot) pairs grouped by expert; groups of <= BP rows.
//  2. k_mx_xprep: x'[p][row] = FWHT(x[token] * suh_{e,p}) / sqrt(128), p = gate, up, stored as fp16
//     after a power-of-two scale per row that brings its largest |x'| into [2^14, 2^15) (exact;
//     multiplied back after the product, which is linear in x'): no overflow, no fp16 subnormals.
//  3. k_mx_gemm: z[split][row][p I + n] = sum over the split's k of x'[p][row][k] What_{e,p}[k][n];
//     the trellis is decoded in registers with the mcg hash exactly as in the fused GEMM
//     (exl3_dev.h): row groups of one or two rows dot the two fp16 halves of each value with
//     (x', x') pairs; larger groups write the decoded values to a per-wave LDS tile and multiply
//     on the matrix cores, with the x' rows read straight from the workspace as the A operand.
//  4. k_mx_mid: g, u = FWHT(sum_split z)/sqrt(128) * svh; a = silu(min(g, L)) * clamp(u, -L, L);
//     a' = FWHT(a * suh_down)/sqrt(128) per row, stored as fp16 with its own power-of-two row scale
//     (a' is small: activations times suh, and subnormal in fp16 without it).
//  5. k_mx_gemm (down): zd[split][row][n] from a' and the down trellis.
//  6. shared expert, carried by the launches of 3 / 4 / 5 as extra workgroups (its bf16 weights
//     stream from HBM while the routed workgroups decode trellis): gate | up over every token on
//     the bf16 matrix cores into per-split partials (activations that are not bf16 enter as two
//     bf16 terms hi + lo, 16 significant bits), the SwiGLU with the mid launch, the down projection
//     into per-split partials.
//  7. k_mx_combine: out[t] = sum_s w[t,s] svh_down * FWHT(scale_row sum_split zd[row(t,s)])/sqrt(128)
//     + sum_split shared[t], slots in order (deterministic).
//
// Routed experts come as a device table of 9 addresses per expert (uint64 [E][9]: gate trellis,
// suh, svh, up trellis, suh, svh, down trellis, suh, svh), so each expert's tensors stay wherever
// the loader put them (the reference resolves them per expert from the checkpoint shards,
// glm_engine.vyb:2845-2862). Trellis int16 [in/16][out/16][64], 16-byte aligned; suh fp16 [in],
// svh fp16 [out]; codebook mcg (the only one the reference has).
#include "exl3_dev.h"

namespace vybdq {

// moe.hip
int moe_route_bucket(const void *logits, int logits_dt, const float *bias, int64_t T, int64_t E, int64_t topk,
                     double scale, int BMr, int *idx, float *w, int *pos, int *row_map, int4 *tiles, int *ntiles,
                     int4 *tiles2, int *ntiles2, hipStream_t s);
int64_t moe_tiles_bound(int64_t T, int64_t E, int64_t k, int64_t rows);

constexpr int kMxTab = 9;  // table words per expert
// table word of projection p (0 gate, 1 up, 2 down) and field f (0 trellis, 1 suh, 2 svh)
__host__ __device__ constexpr int mx_word(int p, int f) { return 3 * p + f; }

template <class T>
__device__ __forceinline__ const T *mx_ptr(const uint64_t *tab, int e, int p, int f) {
  return gptr<const T>(static_cast<int64_t>(tab[kMxTab * e + mx_word(p, f)]));
}

__device__ __forceinline__ float mx_silu(float g) { return g / (1.0f + __expf(-g)); }

// mx_sum_splits of two pairs (a and b, the same splits), their loads in the same groups
__device__ __forceinline__ void mx_sum_splits2(const float *a, const float *b, int64_t stride, int S, f2 &sa, f2 &sb) {
  sa = sb = f2{0.f, 0.f};
  for (int s0 = 0; s0 < S; s0 += 8) {
    f2 va[8], vb[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t o = static_cast<int64_t>(s0 + u) * stride;
      va[u] = s0 + u < S ? *reinterpret_cast<const f2 *>(a + o) : f2{0.f, 0.f};
      vb[u] = s0 + u < S ? *reinterpret_cast<const f2 *>(b + o) : f2{0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (s0 + u < S) {
        sa[0] += va[u][0];
        sa[1] += va[u][1];
        sb[0] += vb[u][0];
        sb[1] += vb[u][1];
      }
  }
}

// sum over s < S of the float pair at base + s * stride, added in split order: loads in groups of 8
// independent 8-byte loads (one round trip per group; a loop that adds each load as it arrives
// waits S round trips)
__device__ __forceinline__ f2 mx_sum_splits(const float *base, int64_t stride, int S) {
  f2 acc = f2{0.f, 0.f};
  for (int s0 = 0; s0 < S; s0 += 8) {
    f2 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      v[u] = s0 + u < S ? *reinterpret_cast<const f2 *>(base + static_cast<int64_t>(s0 + u) * stride) : f2{0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (s0 + u < S) {
        acc[0] += v[u][0];
        acc[1] += v[u][1];
      }
  }
  return acc;
}

// ---- 2. x' rows -------------------------------------------------------------------------------
// One workgroup of kMxRowWaves waves per ((token, slot), projection); wave w rotates the 128-chunks
// w, w + kMxRowWaves, ... (at most CPW each), then the row's largest |x'| sets its scale.
constexpr int kMxRowWaves = 8;

// the workgroup's largest value of v (every wave's lanes hold theirs)
__device__ __forceinline__ float mx_row_max(float v, float *wm) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = v;
  __syncthreads();
  float m = wm[0];
#pragma unroll
  for (int w = 1; w < kMxRowWaves; ++w) m = fmaxf(m, wm[w]);
  return m;
}

template <int XDT, int CPW>
__global__ void __launch_bounds__(64 * kMxRowWaves) k_mx_xprep(const void *__restrict__ X,
                                                              const uint64_t *__restrict__ tab,
                                                              const int *__restrict__ idx, const int *__restrict__ pos,
                                                              int topk, int64_t H, int rows, _Float16 *__restrict__ xp,
                                                              float *__restrict__ xscale) {
  __shared__ float wm[kMxRowWaves];
  const int i = blockIdx.x, p = blockIdx.y, lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t t = i / topk;
  const int e = idx[i], r = pos[i];
  const _Float16 *suh = mx_ptr<_Float16>(tab, e, p, 1);
  const int nch = static_cast<int>(H / 128);
  float a[CPW][2];
  float amax = 0.f;
#pragma unroll
  for (int q = 0; q < CPW; ++q) {
    const int c = wave + kMxRowWaves * q;
    a[q][0] = a[q][1] = 0.f;
    if (c < nch) {
      const int64_t k0 = 128 * static_cast<int64_t>(c) + 2 * lane;
      a[q][0] = load_elem<XDT>(X, t * H + k0) * static_cast<float>(suh[k0]);
      a[q][1] = load_elem<XDT>(X, t * H + k0 + 1) * static_cast<float>(suh[k0 + 1]);
      fwht128_wave(a[q][0], a[q][1]);
      amax = fmaxf(amax, fmaxf(fabsf(a[q][0]), fabsf(a[q][1])));
    }
  }
  float inv;
  const float sc = block_scale(mx_row_max(amax, wm) * kRScale, inv);
  const float f = kRScale * inv;
#pragma unroll
  for (int q = 0; q < CPW; ++q) {
    const int c = wave + kMxRowWaves * q;
    if (c < nch)
      *reinterpret_cast<h2 *>(xp + (static_cast<int64_t>(p) * rows + r) * H + 128 * static_cast<int64_t>(c) + 2 * lane) =
          h2{static_cast<_Float16>(a[q][0] * f), static_cast<_Float16>(a[q][1] * f)};
  }
  if (threadIdx.x == 0) xscale[p * rows + r] = sc;
}

// ---- 6. shared expert: bf16 weights on the matrix cores, carried by the routed launches ----------

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));

struct Bf16MmArgs {
  const uint16_t *W, *W2;     // bf16 [N][K] row-major (W2: the up matrix of gate | up, else null)
  const uint16_t *X, *Xlo;    // bf16 [T][K]; Xlo: the low terms (X + Xlo = the activations) or null
  int T, N;
  int64_t K;
  int kps;                    // 32-wide k-steps per split
  float *part;                // [S][T][nout] (nout = N, or 2 N for gate | up: gate then up)
};

// f32 -> two bf16 terms: hi = bf16(v) (nearest even), lo = bf16(v - hi) (v - hi is exact)
__device__ __forceinline__ void bf16_split(float v, uint16_t &hi, uint16_t &lo) {
  hi = f32_to_bf16(v);
  lo = f32_to_bf16(v - bf16_to_f32(hi));
}

// tile (column group bx of N / 64, split s, token tile bz of ceil(T / 16)), 4 waves: wave w owns
// columns 64 bx + 16 w .. + 16 (PAIR: of both gate and up) for 16 tokens over the split's k-range.
// Lane l reads row (l & 15) of the A and B operands at k offset 8 (l >> 4): 16 contiguous bytes
// of one weight row per lane, so each load instruction covers 64 bytes of 16 rows and two
// consecutive k-steps a whole 128-byte line of each row. kD k-steps of loads in flight.
template <bool PAIR, bool LO>
__device__ __forceinline__ void bf16_mm_tile(const Bf16MmArgs &a, int bx, int s, int bz) {
  constexpr int kD = 4;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)), lane = threadIdx.x & 63;
  const int n0 = 64 * bx + 16 * wave;
  const int m0 = 16 * bz;
  const int64_t K = a.K;
  const int nks = static_cast<int>(K / 32);
  const int ks0 = s * a.kps;
  const int ks1 = min(ks0 + a.kps, nks);
  const int am = m0 + (lane & 15);
  const bool arow_ok = am < a.T;
  const int64_t koff = 8 * (lane >> 4);
  const uint16_t *ap = a.X + static_cast<int64_t>(arow_ok ? am : 0) * K + koff;
  const uint16_t *alp = LO ? a.Xlo + static_cast<int64_t>(arow_ok ? am : 0) * K + koff : nullptr;
  const uint16_t *bp = a.W + static_cast<int64_t>(n0 + (lane & 15)) * K + koff;
  const uint16_t *bp2 = PAIR ? a.W2 + static_cast<int64_t>(n0 + (lane & 15)) * K + koff : nullptr;
  struct Step { bf8 x, xl, w, w2; };
  auto load = [&](int ks) {
    Step st;
    const int kc = ks < ks1 ? ks : ks0;  // in range
    const int64_t o = 32 * static_cast<int64_t>(kc);
    st.w = *reinterpret_cast<const bf8 *>(bp + o);
    if constexpr (PAIR) st.w2 = *reinterpret_cast<const bf8 *>(bp2 + o);
    st.x = arow_ok ? *reinterpret_cast<const bf8 *>(ap + o) : bf8{};
    if constexpr (LO) st.xl = arow_ok ? *reinterpret_cast<const bf8 *>(alp + o) : bf8{};
    return st;
  };
  f4 acc = f4{0.f, 0.f, 0.f, 0.f}, acc2 = f4{0.f, 0.f, 0.f, 0.f};
  auto mma = [&](const Step &st) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(st.x, st.w, acc, 0, 0, 0);
    if constexpr (LO) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(st.xl, st.w, acc, 0, 0, 0);
    if constexpr (PAIR) {
      acc2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(st.x, st.w2, acc2, 0, 0, 0);
      if constexpr (LO) acc2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(st.xl, st.w2, acc2, 0, 0, 0);
    }
  };
  Step ring[kD];
#pragma unroll
  for (int d = 0; d < kD; ++d) ring[d] = load(ks0 + d);
  int k = ks0;
  for (; k + kD <= ks1; k += kD) {
#pragma unroll
    for (int d = 0; d < kD; ++d) {
      mma(ring[d]);
      ring[d] = load(k + d + kD);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int d = 0; d < kD - 1; ++d)
    if (k + d < ks1) mma(ring[d]);
  // acc[r] = C[token m0 + 4 (lane >> 4) + r][column n0 + (lane & 15)]
  const int n = n0 + (lane & 15);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = m0 + 4 * (lane >> 4) + r;
    if (m >= a.T) continue;
    const int nout = PAIR ? 2 * a.N : a.N;
    float *o = a.part + (static_cast<int64_t>(s) * a.T + m) * nout;
    o[n] = acc[r];
    if constexpr (PAIR) o[a.N + n] = acc2[r];
  }
}

// The shared expert's tiles carried by a routed launch: tile i = (column group i mod ngx, split,
// token tile), ngx = N / 64; `tiles` of them in all.
struct MxShared {
  Bf16MmArgs mm;
  int ngx, S, tiles;
};

// gate | up partials [S][T][2 N] -> act hi + lo bf16 [T][N], splits summed in order; element i
__device__ __forceinline__ void bf16_swiglu_elem(const float *__restrict__ part, int S, int T, int N, float limit,
                                                 uint16_t *__restrict__ act, uint16_t *__restrict__ act_lo, int64_t i) {
  if (i >= static_cast<int64_t>(T) * N) return;
  const int64_t m = i / N, n = i % N;
  const float *o = part + m * (2 * N) + n;
  const int64_t stride = static_cast<int64_t>(T) * (2 * N);
  float g = 0.f, u = 0.f;
  for (int s0 = 0; s0 < S; s0 += 8) {  // groups of 8 independent loads, added in split order
    float gv[8], uv[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      gv[q] = s0 + q < S ? o[static_cast<int64_t>(s0 + q) * stride] : 0.f;
      uv[q] = s0 + q < S ? o[static_cast<int64_t>(s0 + q) * stride + N] : 0.f;
    }
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (s0 + q < S) {
        g += gv[q];
        u += uv[q];
      }
  }
  g = fminf(g, limit);
  u = fminf(fmaxf(u, -limit), limit);
  uint16_t hi, lo;
  bf16_split(mx_silu(g) * u, hi, lo);
  act[i] = hi;
  act_lo[i] = lo;
}

// activations that are not bf16 -> hi + lo bf16 terms
template <int XDT>
__global__ void __launch_bounds__(256) k_bf16_terms(const void *__restrict__ X, int64_t n, uint16_t *__restrict__ hi,
                                                    uint16_t *__restrict__ lo) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  bf16_split(load_elem<XDT>(X, i), hi[i], lo[i]);
}

// ---- 3. / 5. grouped EXL3 products -------------------------------------------------------------

struct MxGemmArgs {
  const uint64_t *tab;
  int proj0;           // table projection of the first output block: 0 (gate | up) or 2 (down)
  const int4 *groups;  // {expert, r0, r1, 0}: rows [r0, r1) of one expert, at most BP
  const int *ngroups;
  const _Float16 *xp;  // [nproj][rows][K] rotated inputs
  int rows;            // rows of the bucketing (T topk)
  float *zpart;        // [S][rows][ncat]
  int64_t K;           // input features (multiple of 128)
  int Np;              // output features per projection (multiple of 128)
  int ncat;            // nproj Np
  int kbs;             // 16-row k-blocks per split (a multiple of 8)
  int gy;              // grid y of the routed column blocks; shared-expert workgroups follow
};

constexpr int kMxRedStride = 132;  // floats per row of the per-wave partials (16-column groups on distinct banks)

__host__ __device__ constexpr size_t mx_lds_bytes(int BP, int kbs) {
  // BP <= 2: the split's (x', x') pairs; larger: one decoded-value tile per wave; both reused for
  // the per-wave partials [4][BP][kMxRedStride] after the loop
  return (BP <= 2 ? static_cast<size_t>(BP) * 16 * kbs * 4 : static_cast<size_t>(4) * kExl3WtBytes) >
                 static_cast<size_t>(4) * BP * kMxRedStride * 4
             ? (BP <= 2 ? static_cast<size_t>(BP) * 16 * kbs * 4 : static_cast<size_t>(4) * kExl3WtBytes)
             : static_cast<size_t>(4) * BP * kMxRedStride * 4;
}

// grid (groups bound rounded to 8, nproj Np / 128 column blocks, S splits), 4 waves: each wave a
// quarter of the split's k-blocks on the block's 128 columns, the waves' partials summed in LDS in
// a fixed order. The group index is the fastest grid dimension and the bound is a multiple of 8,
// so every column block of one group runs on the same XCD (its L2 holds the group's x' rows).
// SH: the launch also carries the shared expert's tiles (0 none; 1 gate | up, bf16 activations;
// 2 gate | up, activations as bf16 hi + lo terms; 3 down, hi + lo), as workgroups with blockIdx.x
// past the routed groups' bound: its bf16 weights stream from HBM while the routed workgroups
// decode trellis on the VALU.
template <int BP, int SH>
__global__ void __launch_bounds__(256) k_mx_gemm(const MxGemmArgs a, const MxShared sh) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int jt = blockIdx.x;
  if constexpr (SH != 0) {
    if (static_cast<int>(blockIdx.y) >= a.gy) {  // rows of y past the routed column blocks
      const int i = ((static_cast<int>(blockIdx.y) - a.gy) * static_cast<int>(gridDim.z) + static_cast<int>(blockIdx.z)) *
                        static_cast<int>(gridDim.x) + jt;
      if (i >= sh.tiles) return;
      const int bx = i % sh.ngx, rest = i / sh.ngx;
      bf16_mm_tile<SH != 3, SH != 1>(sh.mm, bx, rest % sh.S, rest / sh.S);
      return;
    }
  }
  if (jt >= *a.ngroups) return;
  const int4 grp = a.groups[jt];
  const int e = grp.x, r0 = grp.y, B = grp.z - grp.y;  // 1 <= B <= BP
  const int nbp = a.Np / 128;
  const int p = static_cast<int>(blockIdx.y) / nbp, g = static_cast<int>(blockIdx.y) - p * nbp;
  const int s = blockIdx.z;
  const uint16_t *__restrict__ trellis = mx_ptr<uint16_t>(a.tab, e, a.proj0 + p, 0);
  const int NB = a.Np / 16;
  const int64_t K = a.K;
  const int KB = static_cast<int>(K / 16);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)), lane = threadIdx.x & 63;
  const int t = lane >> 3, j = lane & 7;
  const int kb_begin = s * a.kbs;
  const int kb_end = min(kb_begin + a.kbs, KB);
  const int nkb = kb_end - kb_begin;  // a multiple of 8 (K % 128 == 0)
  constexpr bool HALVES = BP <= 2;
  constexpr int kD = 4;  // trellis chunks in flight per lane
  const int per_wave = (nkb + 3) / 4;  // even: wave ranges start at even k-blocks
  const int w_begin = wave * per_wave;
  const int w_end = min(w_begin + per_wave, nkb);
  const int64_t nb = 8 * static_cast<int64_t>(g) + t;
  auto load_chunk = [&](int kk) {
    const int kc = kk < w_end ? kk : (w_end > w_begin ? w_end - 1 : 0);  // in range: re-read the last
    const int64_t tile = static_cast<int64_t>(kb_begin + kc) * NB + nb;
    return *reinterpret_cast<const u4 *>(trellis + tile * 64 + 8 * j);
  };
  // this group's x' rows from the split's first k
  const _Float16 *xsrc = a.xp + (static_cast<int64_t>(p) * a.rows + r0) * K + 16 * static_cast<int64_t>(kb_begin);
  const int krows = 16 * nkb;

  // BP <= 2: the rows' (x', x') pairs of the split in LDS; rows past the group read as zero. All
  // of a thread's 16-byte reads (at most 8: the stage holds at most 64 KB, nc <= 2048) go out
  // before the trellis ring (loads return in order), and none after it: x loads issued after the
  // ring (a staging loop) made the compiler wait for the whole ring at the top of every k-loop
  // iteration.
  const int per_row = krows / 8;
  const int nc = HALVES ? BP * per_row : 0;
  auto x_chunk = [&](int i) {
    const int b = i / per_row, c = i - b * per_row;
    u4 v = u4{0u, 0u, 0u, 0u};
    if (b < B) v = *reinterpret_cast<const u4 *>(xsrc + b * K + 8 * c);
    return v;
  };
  auto x_store = [&](int i, const u4 v) {
    const int b = i / per_row, c = i - b * per_row;
    u4 *d = reinterpret_cast<u4 *>(reinterpret_cast<uint32_t *>(smem) + b * krows + 8 * c);
    auto dup = [](uint32_t h) { return (h & 0xffffu) | (h << 16); };
    d[0] = u4{dup(v[0]), dup(v[0] >> 16), dup(v[1]), dup(v[1] >> 16)};
    d[1] = u4{dup(v[2]), dup(v[2] >> 16), dup(v[3]), dup(v[3] >> 16)};
  };
  constexpr int XV = HALVES ? 8 : 1;
  u4 xv[XV];
  if constexpr (HALVES) {
#pragma unroll
    for (int u = 0; u < XV; ++u) {
      const int i = threadIdx.x + 256 * u;
      if (i < nc) xv[u] = x_chunk(i);
    }
  }
  // larger groups: the matrix-core A values of k-block kk: x' row lane & 15 (zero past the group),
  // k offset 4 (lane >> 4), four fp16 read from the workspace (L2) one group of kD k-blocks ahead,
  // beside the trellis ring (each is used twice in the A fragment, see step)
  const int am = lane & 15;
  const _Float16 *arow = xsrc + static_cast<int64_t>(am < B ? am : 0) * K + 4 * (lane >> 4);
  auto load_a = [&](int kk) {
    u2 v = u2{0u, 0u};
    const int kc = kk < w_end ? kk : w_begin;
    if (am < B) v = *reinterpret_cast<const u2 *>(arow + 16 * kc);
    return v;
  };
  __builtin_amdgcn_sched_barrier(0);
  u4 ring[kD];
  u2 aring[HALVES ? 1 : kD];
  if constexpr (HALVES) aring[0] = u2{0u, 0u};
#pragma unroll
  for (int d = 0; d < kD; ++d) {
    ring[d] = load_chunk(w_begin + d);
    if constexpr (!HALVES) aring[d] = load_a(w_begin + d);
  }
  if constexpr (HALVES) {
#pragma unroll
    for (int u = 0; u < XV; ++u)
      if (threadIdx.x + 256 * u < nc) x_store(threadIdx.x + 256 * u, xv[u]);
    __syncthreads();
  }

  float acc[BP][2];
#pragma unroll
  for (int b = 0; b < BP; ++b) acc[b][0] = acc[b][1] = 0.f;
  f4 accm[HALVES ? 1 : 8];
#pragma unroll
  for (int f = 0; f < (HALVES ? 1 : 8); ++f) accm[f] = f4{0.f, 0.f, 0.f, 0.f};
  char *wt = smem + static_cast<size_t>(wave) * kExl3WtBytes;
  auto step = [&](int kk, const u4 c, const u2 av) {
    uint32_t w[6];
    chunk_window(c, w);
    if constexpr (HALVES) {
      uint32_t xq[BP][16];
#pragma unroll
      for (int b = 0; b < BP; ++b) {
        const u4 *src = reinterpret_cast<const u4 *>(reinterpret_cast<const uint32_t *>(smem) + b * krows + 16 * kk);
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
          const u4 v4 = src[c4];
          xq[b][4 * c4 + 0] = v4[0];
          xq[b][4 * c4 + 1] = v4[1];
          xq[b][4 * c4 + 2] = v4[2];
          xq[b][4 * c4 + 3] = v4[3];
        }
      }
#pragma unroll
      for (int q = 0; q < 32; ++q) {
        const h2 y = __builtin_bit_cast(h2, slot_halves(w, q));
#pragma unroll
        for (int b = 0; b < BP; ++b)
          acc[b][q >> 4] = __builtin_amdgcn_fdot2(y, __builtin_bit_cast(h2, xq[b][q & 15]), acc[b][q >> 4], false);
      }
    } else {
      // the 32 slot words as they are (two fp16 halves per value, whose sum is the value): column
      // c's 16 words in k order are the tile row [c][k' = 2 k + h], and the MFMA with each x'
      // value twice in A adds x lo + x hi in float32 (as the k_exl3_gemm matrix-core path)
      const int c0 = 16 * t + j;
      uint32_t hw[32];
#pragma unroll
      for (int q = 0; q < 32; ++q) hw[q] = slot_halves(w, q);
      u4 *d0 = reinterpret_cast<u4 *>(wt + c0 * kExl3WtStride);
      u4 *d1 = reinterpret_cast<u4 *>(wt + (c0 + 8) * kExl3WtStride);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        d0[i] = u4{hw[4 * i], hw[4 * i + 1], hw[4 * i + 2], hw[4 * i + 3]};
        d1[i] = u4{hw[16 + 4 * i], hw[16 + 4 * i + 1], hw[16 + 4 * i + 2], hw[16 + 4 * i + 3]};
      }
      const h8 a = __builtin_bit_cast(h8, u4{__builtin_amdgcn_perm(av[0], av[0], 0x01000100u),
                                             __builtin_amdgcn_perm(av[0], av[0], 0x03020302u),
                                             __builtin_amdgcn_perm(av[1], av[1], 0x01000100u),
                                             __builtin_amdgcn_perm(av[1], av[1], 0x03020302u)});
      const int gk = lane >> 4;
#pragma unroll
      for (int f = 0; f < 8; ++f) {
        const h8 bw = *reinterpret_cast<const h8 *>(wt + (16 * f + am) * kExl3WtStride + 16 * gk);
        accm[f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bw, accm[f], 0, 0, 0);
      }
    }
  };
  // Whole groups of kD k-blocks, each ring slot (trellis chunk and A values) refilled right after the
  // step that consumed it; the last blocks are in the ring.
  int k0 = w_begin;
  for (; k0 + kD <= w_end; k0 += kD) {
#pragma unroll
    for (int d = 0; d < kD; ++d) {
      step(k0 + d, ring[d], aring[HALVES ? 0 : d]);
      ring[d] = load_chunk(k0 + d + kD);
      if constexpr (!HALVES) aring[d] = load_a(k0 + d + kD);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int d = 0; d < kD - 1; ++d)
    if (k0 + d < w_end) step(k0 + d, ring[d], aring[HALVES ? 0 : d]);

  // reduce the 4 waves (same columns, different k) in a fixed order, then this split's partial
  __syncthreads();
  float *red = reinterpret_cast<float *>(smem);  // [4][BP][kMxRedStride]
  if constexpr (!HALVES) {
    // accm[f][r] = z[row 4 (lane >> 4) + r][column 16 f + (lane & 15)]
#pragma unroll
    for (int f = 0; f < 8; ++f)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int b = 4 * (lane >> 4) + r;
        if (b < BP) red[(wave * BP + b) * kMxRedStride + 16 * f + (lane & 15)] = accm[f][r];
      }
  } else {
    const int c0 = 16 * t + j;  // this lane's columns: c0 and c0 + 8
#pragma unroll
    for (int b = 0; b < BP; ++b) {
      red[(wave * BP + b) * kMxRedStride + c0] = acc[b][0];
      red[(wave * BP + b) * kMxRedStride + c0 + 8] = acc[b][1];
    }
  }
  __syncthreads();
  float *zo = a.zpart + (static_cast<int64_t>(s) * a.rows + r0) * a.ncat + static_cast<int64_t>(p) * a.Np + 128 * g;
  for (int i = threadIdx.x; i < B * 128; i += 256) {
    const int b = i >> 7, c = i & 127;
    zo[static_cast<int64_t>(b) * a.ncat + c] =
        ((red[(0 * BP + b) * kMxRedStride + c] + red[(1 * BP + b) * kMxRedStride + c]) +
         red[(2 * BP + b) * kMxRedStride + c]) + red[(3 * BP + b) * kMxRedStride + c];
  }
}

// the shared expert's SwiGLU carried by the mid launch (workgroups past the routed rows)
struct MxSwiglu {
  const float *part;  // [S][T][2 N] gate | up partials
  int S, T, N;
  uint16_t *act, *act_lo;
};

// ---- 4. output rotation of gate | up, SwiGLU, input rotation of down ----------------------------
// One workgroup per (token, slot) row, wave w on the 128-chunks w, w + kMxRowWaves, ...; the
// splits' partials are summed in split order and multiplied by the row's x' scale. Workgroups past
// the rows apply the shared expert's SwiGLU.
template <int CPW>
__global__ void __launch_bounds__(64 * kMxRowWaves) k_mx_mid(const uint64_t *__restrict__ tab,
                                                            const int *__restrict__ idx, const int *__restrict__ pos,
                                                            const float *__restrict__ zpart,
                                                            const float *__restrict__ xscale, int S, int rows,
                                                            int64_t I, float limit, _Float16 *__restrict__ act,
                                                            float *__restrict__ ascale, const MxSwiglu sh) {
  __shared__ float wm[kMxRowWaves];
  const int i = blockIdx.x, lane = threadIdx.x & 63;
  if (i >= rows) {  // the shared expert's SwiGLU, 64 kMxRowWaves elements per workgroup
    bf16_swiglu_elem(sh.part, sh.S, sh.T, sh.N, limit, sh.act, sh.act_lo,
                     static_cast<int64_t>(i - rows) * (64 * kMxRowWaves) + threadIdx.x);
    return;
  }
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int e = idx[i], r = pos[i];
  const int nch = static_cast<int>(I / 128);
  const float sg = xscale[r], su = xscale[rows + r];
  const _Float16 *svg = mx_ptr<_Float16>(tab, e, 0, 2), *svu = mx_ptr<_Float16>(tab, e, 1, 2);
  const _Float16 *suhd = mx_ptr<_Float16>(tab, e, 2, 1);
  float a[CPW][2];
  float amax = 0.f;
#pragma unroll
  for (int q = 0; q < CPW; ++q) {
    const int c = wave + kMxRowWaves * q;
    a[q][0] = a[q][1] = 0.f;
    if (c < nch) {
      const int64_t n0 = 128 * static_cast<int64_t>(c) + 2 * lane;
      const float *zr = zpart + static_cast<int64_t>(r) * (2 * I) + n0;
      f2 gs, us;
      mx_sum_splits2(zr, zr + I, static_cast<int64_t>(rows) * (2 * I), S, gs, us);
      float g0 = gs[0], g1 = gs[1], u0 = us[0], u1 = us[1];
      g0 *= sg;
      g1 *= sg;
      u0 *= su;
      u1 *= su;
      fwht128_wave(g0, g1);
      fwht128_wave(u0, u1);
      g0 = fminf(g0 * kRScale * static_cast<float>(svg[n0]), limit);
      g1 = fminf(g1 * kRScale * static_cast<float>(svg[n0 + 1]), limit);
      u0 = fminf(fmaxf(u0 * kRScale * static_cast<float>(svu[n0]), -limit), limit);
      u1 = fminf(fmaxf(u1 * kRScale * static_cast<float>(svu[n0 + 1]), -limit), limit);
      a[q][0] = mx_silu(g0) * u0 * static_cast<float>(suhd[n0]);
      a[q][1] = mx_silu(g1) * u1 * static_cast<float>(suhd[n0 + 1]);
      fwht128_wave(a[q][0], a[q][1]);
      amax = fmaxf(amax, fmaxf(fabsf(a[q][0]), fabsf(a[q][1])));
    }
  }
  float inv;
  const float sc = block_scale(mx_row_max(amax, wm) * kRScale, inv);
  const float f = kRScale * inv;
#pragma unroll
  for (int q = 0; q < CPW; ++q) {
    const int c = wave + kMxRowWaves * q;
    if (c < nch)
      *reinterpret_cast<h2 *>(act + static_cast<int64_t>(r) * I + 128 * static_cast<int64_t>(c) + 2 * lane) =
          h2{static_cast<_Float16>(a[q][0] * f), static_cast<_Float16>(a[q][1] * f)};
  }
  if (threadIdx.x == 0) ascale[r] = sc;
}

// ---- 7. combine -----------------------------------------------------------------------------------
// grid (T, H / (128 CH)), kMxRowWaves waves, CH 128-column chunks per workgroup. The slots go in
// groups of kMxRowWaves: wave j finishes slot g + j of the group on every chunk (splits summed, their
// loads for all chunks issued together; output rotation, svh) into LDS, then wave q < CH adds that
// group's slots of chunk q with their routing weights in slot order; the shared expert's partials
// follow in split order. CH = 4 where the grid has workgroups to spare, 1 where it is small
template <int ODT, int CH>
__global__ void __launch_bounds__(64 * kMxRowWaves) k_mx_combine(const uint64_t *__restrict__ tab,
                                                                const int *__restrict__ idx,
                                                                const int *__restrict__ pos,
                                                                const float *__restrict__ w, int topk,
                                                                const float *__restrict__ zd,
                                                                const float *__restrict__ ascale, int S, int rows,
                                                                int64_t H, const float *__restrict__ sh, int Ssh,
                                                                int T, void *__restrict__ out) {
  __shared__ f2 zs[kMxRowWaves][CH][64];
  const int t = blockIdx.x, lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int nch = static_cast<int>(H / 128);
  const int c0 = blockIdx.y * CH;
  const bool adder = wave < CH && c0 + wave < nch;
  const int64_t n0 = 128 * static_cast<int64_t>(adder ? c0 + wave : 0) + 2 * lane;
  float y0 = 0.f, y1 = 0.f;
  for (int g = 0; g < topk; g += kMxRowWaves) {
    const int sl = g + wave;
    if (sl < topk) {
      const int i = t * topk + sl;
      const int e = idx[i], r = pos[i];
      const _Float16 *svd = mx_ptr<_Float16>(tab, e, 2, 2);
      const float as = ascale[r];
      const float *zr = zd + static_cast<int64_t>(r) * H + 2 * lane;
      f2 z[CH];
#pragma unroll
      for (int q = 0; q < CH; ++q) z[q] = f2{0.f, 0.f};
      constexpr int U = 8 / CH;  // eight loads per round trip: U splits x every chunk
      for (int s0 = 0; s0 < S; s0 += U) {
        f2 v[U][CH];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int q = 0; q < CH; ++q) {
            const int c = c0 + q < nch ? c0 + q : nch - 1;
            v[u][q] = s0 + u < S ? *reinterpret_cast<const f2 *>(zr + static_cast<int64_t>(s0 + u) * rows * H + 128 * c)
                                 : f2{0.f, 0.f};
          }
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (s0 + u < S)
#pragma unroll
            for (int q = 0; q < CH; ++q) {
              z[q][0] += v[u][q][0];
              z[q][1] += v[u][q][1];
            }
      }
#pragma unroll
      for (int q = 0; q < CH; ++q) {
        const int c = c0 + q < nch ? c0 + q : nch - 1;
        const int64_t m = 128 * static_cast<int64_t>(c) + 2 * lane;
        float z0 = z[q][0] * as, z1 = z[q][1] * as;
        fwht128_wave(z0, z1);
        zs[wave][q][lane] = f2{z0 * kRScale * static_cast<float>(svd[m]), z1 * kRScale * static_cast<float>(svd[m + 1])};
      }
    }
    __syncthreads();
    if (adder) {
      const int ng = topk - g < kMxRowWaves ? topk - g : kMxRowWaves;
      for (int j = 0; j < ng; ++j) {
        const float wt = w[t * topk + g + j];
        y0 = fmaf(wt, zs[j][wave][lane][0], y0);
        y1 = fmaf(wt, zs[j][wave][lane][1], y1);
      }
    }
    __syncthreads();
  }
  if (!adder) return;
  if (sh) {
    const f2 v = mx_sum_splits(sh + static_cast<int64_t>(t) * H + n0, static_cast<int64_t>(T) * H, Ssh);
    y0 += v[0];
    y1 += v[1];
  }
  store_elem<ODT>(out, nullptr, static_cast<int64_t>(t) * H + n0, y0);
  store_elem<ODT>(out, nullptr, static_cast<int64_t>(t) * H + n0 + 1, y1);
}

// ---- host ---------------------------------------------------------------------------------------

// rows per group: one per expert at one token (every expert then holds one row), two while the
// experts hit average at most two rows, else 16-row groups on the matrix cores
static int mx_bp(int64_t T, int64_t E, int64_t k) {
  const int64_t n = T * k, hit = E < n ? E : n;
  if (T == 1) return 1;
  return n <= 2 * hit ? 2 : 16;
}

// K splits of a grouped product: ~2048 workgroups over the expected groups, whole 128 chunks
struct MxSplit {
  int S, kbs;
};
static MxSplit mx_splits(int64_t K, int64_t groups, int64_t col_blocks, int BP) {
  const int KB = static_cast<int>(K / 16);
  const int64_t units = groups * col_blocks;
  int64_t target = 2048;  // workgroups (VYBDQ_MX_WGS overrides)
  if (const char *e = tuning_env("VYBDQ_MX_WGS")) target = atoi(e) > 0 ? atoi(e) : target;
  int S = static_cast<int>((target + units - 1) / units);
  if (S > 16) S = 16;
  if (S > KB / 8) S = KB / 8;
  if (S < 1) S = 1;
  int kbs = (KB + S - 1) / S;
  kbs = (kbs + 7) / 8 * 8;
  // the (x', x') stage of a split in LDS (BP <= 2): at most 64 KB
  while (BP <= 2 && mx_lds_bytes(BP, kbs) > 64 * 1024) kbs -= 8;
  return {(KB + kbs - 1) / kbs, kbs};
}

// K splits of the shared expert's bf16 products: ~2048 waves
static int bf16_splits(int64_t K, int64_t N, int64_t T, int &kps) {
  const int nks = static_cast<int>(K / 32);
  const int64_t waves = (N / 16) * ((T + 15) / 16);
  int S = static_cast<int>((2048 + waves - 1) / waves);
  if (S > 32) S = 32;
  if (S > nks / 4) S = nks / 4 > 0 ? nks / 4 : 1;
  if (S < 1) S = 1;
  kps = (nks + S - 1) / S;
  return (nks + kps - 1) / kps;
}

struct MxPlan {
  int BP, max_groups;
  MxSplit gu, dn;
  int Ssg, kps_g, Ssd, kps_d;  // shared expert splits (gate | up, down)
};

static MxPlan mx_plan(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k) {
  MxPlan p{};
  p.BP = mx_bp(T, E, k);
  const int64_t n = T * k, hit = E < n ? E : n;
  const int64_t groups = p.BP == 16 ? hit + n / 16 : (p.BP == 2 ? (n + 1) / 2 : n);
  p.max_groups = static_cast<int>((moe_tiles_bound(T, E, k, p.BP) + 7) / 8 * 8);
  p.gu = mx_splits(H, groups, 2 * I / 128, p.BP);
  p.dn = mx_splits(I, groups, H / 128, p.BP);
  p.Ssg = bf16_splits(H, I, T, p.kps_g);
  p.Ssd = bf16_splits(I, H, T, p.kps_d);
  return p;
}

struct MxWs {
  int *idx, *pos, *row_map, *ntiles, *ngroups;
  float *w;
  int4 *tiles, *groups;
  _Float16 *xp, *act;
  float *xs, *as;  // row scales of x' [2][rows] and of a' [rows]
  float *zgu, *zd;
  uint16_t *xh, *xl, *ah, *al;
  float *sgu, *sd;
  int64_t bytes;
};

static MxWs mx_layout(char *base, const MxPlan &p, int64_t T, int64_t H, int64_t I, int64_t k) {
  MxWs m{};
  int64_t off = 0;
  auto take = [&](int64_t nb) {
    char *q = base ? base + off : nullptr;
    off += (nb + 255) / 256 * 256;
    return q;
  };
  const int64_t n = T * k;
  m.idx = reinterpret_cast<int *>(take(4 * n));
  m.w = reinterpret_cast<float *>(take(4 * n));
  m.pos = reinterpret_cast<int *>(take(4 * n));
  m.row_map = reinterpret_cast<int *>(take(4 * n));
  m.tiles = reinterpret_cast<int4 *>(take(16 * static_cast<int64_t>(p.max_groups)));
  m.ntiles = reinterpret_cast<int *>(take(4));
  m.groups = reinterpret_cast<int4 *>(take(16 * static_cast<int64_t>(p.max_groups)));
  m.ngroups = reinterpret_cast<int *>(take(4));
  m.xp = reinterpret_cast<_Float16 *>(take(2 * 2 * n * H));
  m.xs = reinterpret_cast<float *>(take(4 * 2 * n));
  m.as = reinterpret_cast<float *>(take(4 * n));
  m.zgu = reinterpret_cast<float *>(take(4 * static_cast<int64_t>(p.gu.S) * n * 2 * I));
  m.act = reinterpret_cast<_Float16 *>(take(2 * n * I));
  m.zd = reinterpret_cast<float *>(take(4 * static_cast<int64_t>(p.dn.S) * n * H));
  m.xh = reinterpret_cast<uint16_t *>(take(2 * T * H));
  m.xl = reinterpret_cast<uint16_t *>(take(2 * T * H));
  m.ah = reinterpret_cast<uint16_t *>(take(2 * T * I));
  m.al = reinterpret_cast<uint16_t *>(take(2 * T * I));
  m.sgu = reinterpret_cast<float *>(take(4 * static_cast<int64_t>(p.Ssg) * T * 2 * I));
  m.sd = reinterpret_cast<float *>(take(4 * static_cast<int64_t>(p.Ssd) * T * H));
  m.bytes = off;
  return m;
}

template <int BP, int SH>
static int mx_gemm_launch(const MxGemmArgs &a, const MxShared &sh, int nproj, int S, int max_groups, hipStream_t s) {
  const size_t lds = mx_lds_bytes(BP, a.kbs);
  const unsigned gx = static_cast<unsigned>(max_groups), gz = static_cast<unsigned>(S);
  const unsigned extra = SH ? static_cast<unsigned>((sh.tiles + gx * gz - 1) / (gx * gz)) : 0u;
  MxGemmArgs b = a;
  b.gy = nproj * a.Np / 128;
  hipLaunchKernelGGL((k_mx_gemm<BP, SH>), dim3(gx, static_cast<unsigned>(b.gy) + extra, gz), dim3(256), lds, s, b, sh);
  return check_launch("moe exl3 grouped product");
}

// the grouped product of the routed experts, carrying the shared expert's tiles of kind SH
template <int BP>
static int mx_gemm_bp(int SH, const MxGemmArgs &a, const MxShared &sh, int nproj, int S, int max_groups,
                      hipStream_t s) {
  switch (SH) {
    case 1: return mx_gemm_launch<BP, 1>(a, sh, nproj, S, max_groups, s);
    case 2: return mx_gemm_launch<BP, 2>(a, sh, nproj, S, max_groups, s);
    case 3: return mx_gemm_launch<BP, 3>(a, sh, nproj, S, max_groups, s);
    default: return mx_gemm_launch<BP, 0>(a, sh, nproj, S, max_groups, s);
  }
}

static int mx_gemm(int BP, int SH, const MxGemmArgs &a, const MxShared &sh, int nproj, int S, int max_groups,
                   hipStream_t s) {
  if (BP == 1) return mx_gemm_bp<1>(SH, a, sh, nproj, S, max_groups, s);
  if (BP == 2) return mx_gemm_bp<2>(SH, a, sh, nproj, S, max_groups, s);
  return mx_gemm_bp<16>(SH, a, sh, nproj, S, max_groups, s);
}

}  // namespace vybdq

using namespace vybdq;

static bool mx_shape_ok(int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk) {
  return T >= 1 && T < (1 << 19) && H >= 128 && I >= 128 && H % 128 == 0 && I % 128 == 0 &&
         H <= 128 * kMxRowWaves * 8 && I <= 128 * kMxRowWaves * 8 && E >= 1 && E <= 1024 && topk >= 1 && topk <= E && topk <= 64 && T * topk < (1 << 24) &&
         T * topk * (H > I ? H : I) * 2 < (int64_t(1) << 40);
}

extern "C" int64_t vybdq_moe_exl3_workspace_size(int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk) {
  if (!mx_shape_ok(T, H, I, E, topk)) return -1;
  return mx_layout(nullptr, mx_plan(T, H, I, E, topk), T, H, I, topk).bytes;
}

extern "C" int vybdq_moe_forward_exl3(uint64_t x, int x_dt, uint64_t logits, int logits_dt, uint64_t bias,
                                      uint64_t experts, uint64_t s_gate, uint64_t s_up, uint64_t s_down, uint64_t out,
                                      int out_dt, uint64_t idx_out, uint64_t w_out, int64_t T, int64_t H, int64_t I,
                                      int64_t E, int64_t topk, double scale, double limit, uint64_t ws,
                                      int64_t ws_bytes, uint64_t stream) {
  VYBDQ_REQUIRE(x && logits && experts && out, VYBDQ_ERR_ARG, "null x, logits, expert table or out");
  VYBDQ_REQUIRE((s_gate == 0) == (s_up == 0) && (s_up == 0) == (s_down == 0), VYBDQ_ERR_ARG,
                "shared expert: give all three matrices or none");
  VYBDQ_REQUIRE(dt_valid_in(x_dt), VYBDQ_ERR_ARG, "x_dt must be F32, F16 or BF16");
  VYBDQ_REQUIRE(dt_valid_out(logits_dt), VYBDQ_ERR_ARG, "logits_dt must be F32, F16, BF16 or F64");
  VYBDQ_REQUIRE(out_dt == VYBDQ_F32 || out_dt == VYBDQ_F16 || out_dt == VYBDQ_BF16, VYBDQ_ERR_ARG,
                "out_dt must be F32, F16 or BF16");
  VYBDQ_REQUIRE(mx_shape_ok(T, H, I, E, topk), VYBDQ_ERR_SHAPE,
                "need H, I multiples of 128 up to 8192, 1 <= topk <= E <= 1024, topk <= 64 and T topk < 2^24");
  const MxPlan p = mx_plan(T, H, I, E, topk);
  const int64_t need = mx_layout(nullptr, p, T, H, I, topk).bytes;
  VYBDQ_REQUIRE(ws && (ws & 255) == 0 && ws_bytes >= need, VYBDQ_ERR_WORKSPACE,
                "workspace must be 256-byte aligned and at least vybdq_moe_exl3_workspace_size bytes");
  VYBDQ_REQUIRE((x & 15) == 0 && (experts & 7) == 0, VYBDQ_ERR_ALIGN, "x must be 16-byte and the table 8-byte aligned");
  VYBDQ_REQUIRE(((s_gate | s_up | s_down) & 15) == 0, VYBDQ_ERR_ALIGN, "shared expert weights must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  MxWs m = mx_layout(reinterpret_cast<char *>(ws), p, T, H, I, topk);
  const uint64_t *tab = reinterpret_cast<const uint64_t *>(experts);
  int *idx = idx_out ? reinterpret_cast<int *>(idx_out) : m.idx;
  float *wts = w_out ? reinterpret_cast<float *>(w_out) : m.w;
  const int n = static_cast<int>(T * topk), k = static_cast<int>(topk);

  // 1. routing and row groups of at most BP rows
  int rc = moe_route_bucket(reinterpret_cast<const void *>(logits), logits_dt, reinterpret_cast<const float *>(bias),
                            T, E, topk, scale, p.BP, idx, wts, m.pos, m.row_map, m.tiles, m.ntiles, m.groups,
                            m.ngroups, s);
  if (rc) return rc;
  // 2. x' rows for gate and up
  const int cpw_h = static_cast<int>((H / 128 + kMxRowWaves - 1) / kMxRowWaves);
  const int cpw_i = static_cast<int>((I / 128 + kMxRowWaves - 1) / kMxRowWaves);
#define XP(XDT, CPW)                                                                                            \
  hipLaunchKernelGGL((k_mx_xprep<XDT, CPW>), dim3(static_cast<unsigned>(n), 2), dim3(64 * kMxRowWaves), 0, s,      \
                     reinterpret_cast<const void *>(x), tab, idx, m.pos, k, H, n, m.xp, m.xs)
  VYBDQ_DISPATCH_IN(x_dt, XDT, {
    if (cpw_h <= 1) XP(XDT, 1); else if (cpw_h <= 2) XP(XDT, 2); else if (cpw_h <= 4) XP(XDT, 4); else XP(XDT, 8);
  });
#undef XP
  rc = check_launch("moe exl3 x rotation");
  if (rc) return rc;
  // 3. gate | up products
  MxGemmArgs ga{};
  ga.tab = tab;
  ga.proj0 = 0;
  ga.groups = m.groups;
  ga.ngroups = m.ngroups;
  ga.xp = m.xp;
  ga.rows = n;
  ga.zpart = m.zgu;
  ga.K = H;
  ga.Np = static_cast<int>(I);
  ga.ncat = static_cast<int>(2 * I);
  ga.kbs = p.gu.kbs;
  // the shared expert's gate | up ride on this launch, its SwiGLU on the mid launch, its down
  // projection on the down launch (bf16 weights on the matrix cores: activations that are not
  // bf16 enter as two bf16 terms hi + lo, 16 significant bits)
  const bool shared = s_gate != 0;
  const bool lo = x_dt != VYBDQ_BF16;
  MxShared shg{}, shd{};
  if (shared) {
    const uint16_t *xh = reinterpret_cast<const uint16_t *>(x);
    if (lo) {
      const int64_t ne = T * H;
      VYBDQ_DISPATCH_IN(x_dt, XDT,
          hipLaunchKernelGGL((k_bf16_terms<XDT>), dim3(static_cast<unsigned>((ne + 255) / 256)), dim3(256), 0, s,
                             reinterpret_cast<const void *>(x), ne, m.xh, m.xl));
      rc = check_launch("moe shared expert activation terms");
      if (rc) return rc;
      xh = m.xh;
    }
    Bf16MmArgs &b = shg.mm;
    b.W = reinterpret_cast<const uint16_t *>(s_gate);
    b.W2 = reinterpret_cast<const uint16_t *>(s_up);
    b.X = xh;
    b.Xlo = lo ? m.xl : nullptr;
    b.T = static_cast<int>(T);
    b.N = static_cast<int>(I);
    b.K = H;
    b.kps = p.kps_g;
    b.part = m.sgu;
    shg.ngx = static_cast<int>(I / 64);
    shg.S = p.Ssg;
    shg.tiles = shg.ngx * p.Ssg * static_cast<int>((T + 15) / 16);
    Bf16MmArgs &d = shd.mm;
    d.W = reinterpret_cast<const uint16_t *>(s_down);
    d.X = m.ah;
    d.Xlo = m.al;
    d.T = static_cast<int>(T);
    d.N = static_cast<int>(H);
    d.K = I;
    d.kps = p.kps_d;
    d.part = m.sd;
    shd.ngx = static_cast<int>(H / 64);
    shd.S = p.Ssd;
    shd.tiles = shd.ngx * p.Ssd * static_cast<int>((T + 15) / 16);
  }
  rc = mx_gemm(p.BP, shared ? (lo ? 2 : 1) : 0, ga, shg, 2, p.gu.S, p.max_groups, s);
  if (rc) return rc;
  // 4. SwiGLU between the rotations
  MxSwiglu sw{m.sgu, p.Ssg, static_cast<int>(T), static_cast<int>(I), m.ah, m.al};
  const unsigned mid_sh = shared ? static_cast<unsigned>((T * I + 64 * kMxRowWaves - 1) / (64 * kMxRowWaves)) : 0u;
#define MID(CPW)                                                                                                \
  hipLaunchKernelGGL((k_mx_mid<CPW>), dim3(static_cast<unsigned>(n) + mid_sh), dim3(64 * kMxRowWaves), 0, s, tab, idx, \
                     m.pos, m.zgu, m.xs, p.gu.S, n, I, static_cast<float>(limit), m.act, m.as, sw)
  if (cpw_i <= 1) MID(1); else if (cpw_i <= 2) MID(2); else if (cpw_i <= 4) MID(4); else MID(8);
#undef MID
  rc = check_launch("moe exl3 swiglu");
  if (rc) return rc;
  // 5. down products
  MxGemmArgs da = ga;
  da.proj0 = 2;
  da.xp = m.act;
  da.zpart = m.zd;
  da.K = I;
  da.Np = static_cast<int>(H);
  da.ncat = static_cast<int>(H);
  da.kbs = p.dn.kbs;
  rc = mx_gemm(p.BP, shared ? 3 : 0, da, shd, 1, p.dn.S, p.max_groups, s);
  if (rc) return rc;
  // 7. combine
  // four chunks per workgroup once the grid holds 2048 workgroups with them, else one
  bool wide = T * (H / 512) >= 2048;
  if (const char *e = tuning_env("VYBDQ_MX_COMB")) wide = e[0] == '4';
  const int CHn = wide ? 4 : 1;
  VYBDQ_DISPATCH_IN(out_dt, ODT,
      hipLaunchKernelGGL((wide ? k_mx_combine<ODT, 4> : k_mx_combine<ODT, 1>),
                         dim3(static_cast<unsigned>(T), static_cast<unsigned>((H / 128 + CHn - 1) / CHn)),
                         dim3(64 * kMxRowWaves), 0, s, tab, idx, m.pos, wts, k, m.zd, m.as, p.dn.S, n, H, shared ? m.sd : nullptr, p.Ssd,
                         static_cast<int>(T), reinterpret_cast<void *>(out)));
  return check_launch("moe exl3 combine");
}
