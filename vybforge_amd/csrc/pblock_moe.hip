// VYBDQ_PB_MOE: the reference's GLM MoE block kernels (moe_route, moe_act, moe_down;
// native/kernels/moe.vyb:1-170) on their own parameter block, gfx950.
//
// The block (moe.vyb:15-19), little-endian int64 words, every one read on the device:
//   +0 y f32 [S][4096]   +8 G f32 [288][4096]   +16 bias f32 [288]   +24 LG f32 [S][288] (out)
//   +32 IX f32 [S][8] (out, expert ids as floats)   +40 WT f32 [S][8] (out)
//   +48 AC f32 [S][9][2048] (out)   +56/64/72 gate/up/down of the routed expert
//   +80/88/96 gate/up/down of the shared expert   +104 out f32 [S][4096]   +112 S
// Shapes are fixed (moe.vyb:5-8): H = 4096, I = 2048, 288 experts, top-8; gate/up are dense f32
// [in = 4096][out = 2048], down [in = 2048][out = 4096]. Every routed lane uses the same expert
// weights (+56..+72), lane 8 is the shared expert with weight 1.
// Semantics (f64 accumulation of f32 operands, results stored as f32):
//   LG = y G^T; choice = sigmoid(LG) + bias; IX = greedy top-8 of choice (strictly greater wins,
//   so ties go to the lower expert id; choices at or below -1e9 never win and an empty round
//   picks expert 0, moe.vyb:53-74); WT = sigmoid(LG[IX]) / (sum + 1e-20) * 2.5 (moe.vyb:76-89);
//   AC[s][l] = silu(min(g, 10)) * clamp(u, -10, 10), g, u = y W (moe.vyb:93-128);
//   out[s] = sum_l WT[s][l] (AC[s][l] Wd) + AC[s][8] Wsd (moe.vyb:131-170).
// S is read on the device, so the grids cover the largest S (256, the reference's one-workgroup
// route launch) and workgroups past S exit at once. Dot products are summed in a fixed tree
// order (not the reference's sequential one): the f64 results differ in the last bits and round
// to the same f32 in all but rare boundary cases. A block whose words are out of range is not
// computed: every kernel returns and the status word gets kPbBadMoe.
#include "common.h"

namespace vybdq {

int pb_status_address(uint64_t &ptr);

namespace {

constexpr uint32_t kPbBadMoe = 8u;
constexpr int kMH = 4096, kMI = 2048, kME = 288, kMK = 8, kMaxS = 256;
constexpr int kMTok = 16;  // tokens per workgroup tile
enum : int { PY = 0, PG, PBIAS, PLG, PIX, PWT, PAC, PWGE, PWUE, PWDE, PWGS, PWUS, PWDS, POUT, PS };

__device__ __forceinline__ bool moe_block_ok(const int64_t *pb, int64_t &S) {
  S = pb[PS];
  bool ok = S >= 1 && S <= kMaxS;
#pragma unroll
  for (int i = 0; i < PS; ++i) ok = ok && pb[i] != 0 && (pb[i] & 3) == 0;
  // y, G and AC are read 16 bytes at a time
  return ok && ((pb[PY] | pb[PG] | pb[PAC]) & 15) == 0;
}

__device__ __forceinline__ void flag_bad(uint32_t *status) {
  if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x == 0)
    __hip_atomic_fetch_or(status, kPbBadMoe, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ double sigm(double x) { return 1.0 / (1.0 + exp(0.0 - x)); }

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}

// LG[s][e] = y[s] . G[e]: workgroup = (4 experts, one per wave) x (16 tokens). Each lane first loads
// its 64 elements of the expert's row (h = 4 lane + 256 j + (0..3)), then y is staged in LDS 1024
// columns at a time (rows past S as zeros); the lane sums fold in a wave tree.
__global__ void __launch_bounds__(256) k_pbmoe_logits(const int64_t *__restrict__ pb, uint32_t *__restrict__ status) {
  constexpr int CH = 1024, JC = CH / 256;
  __shared__ __attribute__((aligned(16))) float ys[kMTok][CH];
  int64_t S;
  if (!moe_block_ok(pb, S)) {
    flag_bad(status);
    return;
  }
  const int s0 = blockIdx.y * kMTok;
  if (s0 >= S) return;
  const int ns = S - s0 < kMTok ? static_cast<int>(S - s0) : kMTok;
  const float *y = gptr<const float>(pb[PY]);
  const float *G = gptr<const float>(pb[PG]);
  float *LG = gptr<float>(pb[PLG]);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + w;
  float4 g[kMH / 256];
#pragma unroll
  for (int j = 0; j < kMH / 256; ++j)
    g[j] = *reinterpret_cast<const float4 *>(G + static_cast<int64_t>(e) * kMH + 4 * lane + 256 * j);
  double acc[kMTok];
#pragma unroll
  for (int i = 0; i < kMTok; ++i) acc[i] = 0.0;
#pragma unroll
  for (int ch = 0; ch < kMH / CH; ++ch) {
    __syncthreads();
    for (int q = threadIdx.x; q < kMTok * CH / 4; q += 256) {
      const int i = q / (CH / 4), c4 = q % (CH / 4);
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (i < ns) v = *reinterpret_cast<const float4 *>(y + static_cast<int64_t>(s0 + i) * kMH + ch * CH + 4 * c4);
      *reinterpret_cast<float4 *>(&ys[i][4 * c4]) = v;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < JC; ++j) {
      const float4 gv = g[ch * JC + j];
      const int hl = 4 * lane + 256 * j;
#pragma unroll
      for (int i = 0; i < kMTok; ++i) {
        const float4 v = *reinterpret_cast<const float4 *>(&ys[i][hl]);
        acc[i] = fma(static_cast<double>(v.x), static_cast<double>(gv.x), acc[i]);
        acc[i] = fma(static_cast<double>(v.y), static_cast<double>(gv.y), acc[i]);
        acc[i] = fma(static_cast<double>(v.z), static_cast<double>(gv.z), acc[i]);
        acc[i] = fma(static_cast<double>(v.w), static_cast<double>(gv.w), acc[i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kMTok; ++i) {
    const double t = wave_sum(acc[i]);
    if (lane == 0 && i < ns) LG[static_cast<int64_t>(s0 + i) * kME + e] = static_cast<float>(t);
  }
}

// Greedy top-8 of sigmoid(LG) + bias and the renormalised weights: one wave per token; lane l
// holds experts l + 64 q (q < 5).
__global__ void __launch_bounds__(256) k_pbmoe_topk(const int64_t *__restrict__ pb, uint32_t *__restrict__ status) {
  int64_t S;
  if (!moe_block_ok(pb, S)) {
    flag_bad(status);
    return;
  }
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int s = blockIdx.x * 4 + w;
  if (s >= S) return;
  const float *LG = gptr<const float>(pb[PLG]) + static_cast<int64_t>(s) * kME;
  const float *bias = gptr<const float>(pb[PBIAS]);
  float *IX = gptr<float>(pb[PIX]) + s * kMK;
  float *WT = gptr<float>(pb[PWT]) + s * kMK;
  constexpr int NQ = (kME + 63) / 64;
  double sc[NQ];
  bool used[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int e = lane + 64 * q;
    used[q] = false;
    sc[q] = e < kME ? sigm(static_cast<double>(LG[e])) + static_cast<double>(bias[e]) : -INFINITY;
  }
  int idx[kMK];
#pragma unroll
  for (int l = 0; l < kMK; ++l) {
    double bv = -1000000000.0;
    int bi = 0x7fffffff;
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      if (!used[q] && sc[q] > bv) {
        bv = sc[q];
        bi = lane + 64 * q;
      }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
      const double ov = __shfl_xor(bv, d, 64);
      const int oi = __shfl_xor(bi, d, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (bi == 0x7fffffff) bi = 0;  // no choice above -1e9: the reference keeps expert 0
    idx[l] = bi;
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      if (lane + 64 * q == bi) used[q] = true;
  }
  double tot = 0.0;
#pragma unroll
  for (int l = 0; l < kMK; ++l) tot = tot + sigm(static_cast<double>(LG[idx[l]]));
#pragma unroll
  for (int l = 0; l < kMK; ++l) {
    if (lane == l) {
      const double wv = sigm(static_cast<double>(LG[idx[l]])) / (tot + 0.00000000000000000001);
      IX[l] = static_cast<float>(idx[l]);
      WT[l] = static_cast<float>(wv * 2.5);
    }
  }
}

// The two dense products of a 16-column strip for NT tokens: acc0 += A0 B0, acc1 += A1 B1 over K
// rows (B row-major [K][ldb]; SAME_A: A1 is A0 and is staged once; A rows past ns are staged as
// zeros, so every fma runs unconditionally and those rows are never read back). 512 threads: lane
// (r = lane / 16, c = lane % 16) of wave w takes rows h = 32 j + 4 w + r of column col0 + c. Chunks
// of 256 rows: while a chunk's fmas run, the next chunk's B values and A rows are already loading
// (registers), then the A rows go to LDS between two barriers. The 32 per-thread partials fold by
// lane shuffles (r) and then over the waves in order through LDS.
constexpr int kStripCh = 256;
// LDS of a strip kernel (floats): the A stage of 16 tokens, or the fold of 8 waves x 2 x 16 x 16 doubles
constexpr int strip_lds_floats(int na) { return na * kMTok * kStripCh > 8 * 2 * kMTok * 16 * 2 ? na * kMTok * kStripCh
                                                                                           : 8 * 2 * kMTok * 16 * 2; }
template <int K, bool SAME_A, int NT>
__device__ __forceinline__ void ffn_strip(const float *A0, const float *A1, int64_t lda, const float *B0,
                                          const float *B1, int64_t ldb, int col0, int ns, float *lds,
                                          double (&out0)[NT], double (&out1)[NT]) {
  constexpr int CH = kStripCh, JN = CH / 32, NA = SAME_A ? 1 : 2;
  constexpr int AQ = NA * NT * CH / 4, AV = (AQ + 511) / 512;  // float4 of A rows per chunk, per thread
  auto as = reinterpret_cast<float (*)[NT][CH]>(lds);           // [NA][NT][CH]
  auto red = reinterpret_cast<double (*)[2][NT][16]>(lds);      // [8 waves][2][NT][16]
  const int t = threadIdx.x, w = t >> 6, lane = t & 63, r = lane >> 4, c = lane & 15;
  const int col = col0 + c;
  double a0[NT], a1[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) a0[i] = a1[i] = 0.0;
  float nb0[JN], nb1[JN];
  float4 na[AV];
  auto load_chunk = [&](int h0) {
#pragma unroll
    for (int j = 0; j < JN; ++j) {
      const int64_t h = h0 + 32 * j + 4 * w + r;
      nb0[j] = B0[h * ldb + col];
      nb1[j] = B1[h * ldb + col];
    }
#pragma unroll
    for (int v = 0; v < AV; ++v) {
      const int q = t + 512 * v;
      const int m = q / (NT * CH / 4), rest = q % (NT * CH / 4);
      const int i = rest / (CH / 4), c4 = rest % (CH / 4);
      const float *A = m ? A1 : A0;
      na[v] = q < AQ && i < ns ? *reinterpret_cast<const float4 *>(A + static_cast<int64_t>(i) * lda + h0 + 4 * c4)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  load_chunk(0);
  for (int h0 = 0; h0 < K; h0 += CH) {
    __syncthreads();  // the previous chunk's LDS reads are done
#pragma unroll
    for (int v = 0; v < AV; ++v) {
      const int q = t + 512 * v;
      const int m = q / (NT * CH / 4), rest = q % (NT * CH / 4);
      const int i = rest / (CH / 4), c4 = rest % (CH / 4);
      if (q < AQ) *reinterpret_cast<float4 *>(&as[m][i][4 * c4]) = na[v];
    }
    float b0[JN], b1[JN];
#pragma unroll
    for (int j = 0; j < JN; ++j) {
      b0[j] = nb0[j];
      b1[j] = nb1[j];
    }
    __syncthreads();
    if (h0 + CH < K) load_chunk(h0 + CH);
#pragma unroll 2
    for (int j = 0; j < JN; ++j) {
      const int hl = 32 * j + 4 * w + r;
      const double d0 = static_cast<double>(b0[j]), d1 = static_cast<double>(b1[j]);
#pragma unroll
      for (int i = 0; i < NT; ++i) {
        const double x0 = static_cast<double>(as[0][i][hl]);
        a0[i] = fma(x0, d0, a0[i]);
        a1[i] = fma(SAME_A ? x0 : static_cast<double>(as[NA - 1][i][hl]), d1, a1[i]);
      }
    }
  }
  // fold r (lanes c, c + 16, c + 32, c + 48), then the 8 waves in order
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    a0[i] += __shfl_xor(a0[i], 16, 64);
    a0[i] += __shfl_xor(a0[i], 32, 64);
    a1[i] += __shfl_xor(a1[i], 16, 64);
    a1[i] += __shfl_xor(a1[i], 32, 64);
  }
  __syncthreads();  // the A stage is free
  if (r == 0) {
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      red[w][0][i][c] = a0[i];
      red[w][1][i][c] = a1[i];
    }
  }
  __syncthreads();
  // every thread reads the sums of its column for all tokens (the epilogue picks what it needs)
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    double s0 = red[0][0][i][c], s1 = red[0][1][i][c];
#pragma unroll
    for (int ww = 1; ww < 8; ++ww) {
      s0 += red[ww][0][i][c];
      s1 += red[ww][1][i][c];
    }
    out0[i] = s0;
    out1[i] = s1;
  }
}

// Column strip of workgroup b: the 8 XCDs take contiguous ranges of strips (workgroups are dealt to
// XCDs round robin), so the two 16-column halves of a 128-byte line are read through one L2.
__device__ __forceinline__ int strip_of(int b, int nstrips) { return (b & 7) * (nstrips >> 3) + (b >> 3); }

// AC: grid (2048 / 16 column strips, 2: routed / shared, 16 token tiles); the routed pair's
// activation goes to lanes 0..7 of every token, the shared pair's to lane 8.
template <int NT>
__device__ __forceinline__ void act_tile(const int64_t *pb, int s0, int ns, bool shared, int col0, float *lds) {
  const float *y = gptr<const float>(pb[PY]) + static_cast<int64_t>(s0) * kMH;
  const float *Wg = gptr<const float>(pb[shared ? PWGS : PWGE]);
  const float *Wu = gptr<const float>(pb[shared ? PWUS : PWUE]);
  float *AC = gptr<float>(pb[PAC]);
  double g[NT], u[NT];
  ffn_strip<kMH, true, NT>(y, y, kMH, Wg, Wu, kMI, col0, ns, lds, g, u);
  const int t = threadIdx.x, i = t >> 4, c = t & 15;  // (token, column) outputs
  if (i < ns) {
    double gv = g[0], uv = u[0];
#pragma unroll
    for (int k = 1; k < NT; ++k)
      if (k == i) {
        gv = g[k];
        uv = u[k];
      }
    if (gv > 10.0) gv = 10.0;
    if (uv > 10.0) uv = 10.0;
    if (uv < -10.0) uv = -10.0;
    const float a = static_cast<float>((gv * sigm(gv)) * uv);
    float *row = AC + static_cast<int64_t>(s0 + i) * 9 * kMI + col0 + c;
    if (shared) {
      row[8 * kMI] = a;
    } else {
#pragma unroll
      for (int l = 0; l < kMK; ++l) row[l * kMI] = a;
    }
  }
}

__global__ void __launch_bounds__(512) k_pbmoe_act(const int64_t *__restrict__ pb, uint32_t *__restrict__ status) {
  __shared__ __attribute__((aligned(16))) float lds[strip_lds_floats(1)];
  int64_t S;
  if (!moe_block_ok(pb, S)) {
    flag_bad(status);
    return;
  }
  const int s0 = blockIdx.z * kMTok;
  if (s0 >= S) return;
  const int ns = S - s0 < kMTok ? static_cast<int>(S - s0) : kMTok;
  const bool shared = blockIdx.y == 1;
  const int col0 = strip_of(blockIdx.x, kMI / 16) * 16;
  if (ns <= 4) act_tile<4>(pb, s0, ns, shared, col0, lds);
  else if (ns <= 8) act_tile<8>(pb, s0, ns, shared, col0, lds);
  else act_tile<16>(pb, s0, ns, shared, col0, lds);
}

// out: grid (4096 / 16 column strips, 1, 16 token tiles). The routed lanes' activation rows are
// equal (one expert's weights on every lane), so AC lane 0 times Wd is each lane's product.
template <int NT>
__device__ __forceinline__ void down_tile(const int64_t *pb, int s0, int ns, int col0, float *lds) {
  const float *AC = gptr<const float>(pb[PAC]) + static_cast<int64_t>(s0) * 9 * kMI;
  const float *Wd = gptr<const float>(pb[PWDE]);
  const float *Wsd = gptr<const float>(pb[PWDS]);
  const float *WT = gptr<const float>(pb[PWT]);
  float *out = gptr<float>(pb[POUT]);
  double pe[NT], ps[NT];
  ffn_strip<kMI, false, NT>(AC, AC + 8 * kMI, 9 * kMI, Wd, Wsd, kMH, col0, ns, lds, pe, ps);
  const int t = threadIdx.x, i = t >> 4, c = t & 15;
  if (i < ns) {
    double e = pe[0], sh = ps[0];
#pragma unroll
    for (int k = 1; k < NT; ++k)
      if (k == i) {
        e = pe[k];
        sh = ps[k];
      }
    const int s = s0 + i;
    double acc = 0.0;
#pragma unroll
    for (int l = 0; l < kMK; ++l) acc = acc + static_cast<double>(WT[s * kMK + l]) * e;
    out[static_cast<int64_t>(s) * kMH + col0 + c] = static_cast<float>(acc + sh);
  }
}

__global__ void __launch_bounds__(512) k_pbmoe_down(const int64_t *__restrict__ pb, uint32_t *__restrict__ status) {
  __shared__ __attribute__((aligned(16))) float lds[strip_lds_floats(2)];
  int64_t S;
  if (!moe_block_ok(pb, S)) {
    flag_bad(status);
    return;
  }
  const int s0 = blockIdx.z * kMTok;
  if (s0 >= S) return;
  const int ns = S - s0 < kMTok ? static_cast<int>(S - s0) : kMTok;
  const int col0 = strip_of(blockIdx.x, kMH / 16) * 16;
  if (ns <= 4) down_tile<4>(pb, s0, ns, col0, lds);
  else if (ns <= 8) down_tile<8>(pb, s0, ns, col0, lds);
  else down_tile<16>(pb, s0, ns, col0, lds);
}

}  // namespace

int pb_moe_launch(const int64_t *pb, uint32_t *status, hipStream_t s) {
  constexpr unsigned tiles = kMaxS / kMTok;
  hipLaunchKernelGGL(k_pbmoe_logits, dim3(kME / 4, tiles), dim3(256), 0, s, pb, status);
  int rc = check_launch("p-block moe logits");
  if (rc) return rc;
  hipLaunchKernelGGL(k_pbmoe_topk, dim3(kMaxS / 4), dim3(256), 0, s, pb, status);
  rc = check_launch("p-block moe top-8");
  if (rc) return rc;
  hipLaunchKernelGGL(k_pbmoe_act, dim3(kMI / 16, 2, tiles), dim3(512), 0, s, pb, status);
  rc = check_launch("p-block moe act");
  if (rc) return rc;
  hipLaunchKernelGGL(k_pbmoe_down, dim3(kMH / 16, 1, tiles), dim3(512), 0, s, pb, status);
  return check_launch("p-block moe down");
}

}  // namespace vybdq
