// GLM-style MoE layer on one GPU: router, per-expert bucketing, grouped dequant GEMMs with a
// fused clamped-SwiGLU epilogue, and an atomics-free combine. gfx950.
//
// Semantics (native/glm53/moe_ref.py:25-112, native/kernels/moe.vyb:1-170):
//   scores = sigmoid(logits); choice = scores + bias (bias only selects); idx = top-k(choice)
//   (descending, ties to the lower expert id); w = scores[idx] / (sum + 1e-20) * scale
//   expert e: a = silu(min(x Wg_e, L)) * clamp(x Wu_e, -L, L); e_out = a Wd_e
//   out[t] = sum_s w[t, s] e_out[idx[t, s]](t) + shared(x[t])
// Without a bias the selection is by logit (sigmoid is monotone: exact order, no float32
// saturation ties); with a bias the choice is computed in double, as the reference does. One
// wave routes a token (route_wave).
//
// Pipeline (all on the stream, no host syncs), when H and I are multiples of 256: route ->
// bucket (one workgroup: per-expert counts, a parallel scan, the lists of row groups of the
// experts that received tokens, each (token, slot)'s row) -> grouped gate|up with the SwiGLU
// epilogue -> grouped down -> combine. The shared expert is one more group over all tokens. Up to
// 64 tokens the grouped kernels are multi-token GEMVs over groups of at most 4 rows (moe_gemv.h:
// each expert row is streamed as a contiguous run); above that, MFMA GEMMs over 16/32-row
// m-tiles (moe_mm.h). Other shapes run the routed and shared experts through the LDS-staged
// grouped GEMM of dqgemm.hip (one group per expert, 16-row tiles).
#include "gemv_dev.h"
#include "moe_gemv.h"
#include "moe_route.h"
#include "moe_mm.h"
#include <cstdio>
#include <mutex>
#include <string>
#include <type_traits>

namespace vybdq {

// defined in dqgemm.hip
int dq_gemm_grouped(int wtype, bool swiglu, const uint8_t *W, const uint8_t *W2, int64_t w_stride, const void *X,
                    int xdt, int64_t ldx, const int *row_map, const int *grp_rows, const int *grp_tiles, int G,
                    int M, int N, int64_t K, void *Y, int ydt, int64_t ldy, float limit, int max_mtiles,
                    hipStream_t s);
int dq_gemm_bm();

// one token per wave, four per workgroup
template <int LDT, int ENT>
__global__ void __launch_bounds__(256) k_moe_route(const void *__restrict__ logits, const float *__restrict__ bias,
                                                   int E, int topk, double scale, int *__restrict__ idx_out,
                                                   float *__restrict__ w_out, int T) {
  const int t = 4 * blockIdx.x + (threadIdx.x >> 6);
  if (t < T) route_wave<LDT, ENT>(logits, bias, t, E, topk, scale, idx_out, w_out, nullptr);
}

// One workgroup: per-expert counts, exclusive scans, and each (token, slot)'s bucket position
// in stable token order. grp_rows[E+1], grp_tiles[E+1] (ceil(count/BM) per expert), row_map[T*k]
// (bucket position -> token), pos[T*k] ((token, slot) -> bucket position).
__global__ void __launch_bounds__(256) k_moe_bucket(const int *__restrict__ idx, int T, int topk, int E, int BM,
                                                    int *__restrict__ grp_rows, int *__restrict__ grp_tiles,
                                                    int *__restrict__ row_map, int *__restrict__ pos) {
  extern __shared__ int sh[];
  int *cnt = sh;          // [E]
  int *scan_r = sh + E;   // [E + 1]
  int *scan_t = scan_r + E + 1;
  const int n = T * topk;
  for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) atomicAdd(&cnt[idx[i]], 1);  // counts are order-free
  __syncthreads();
  if (threadIdx.x == 0) {  // E <= 1024: a serial scan is a few microseconds at most
    int r = 0, tl = 0;
    for (int e = 0; e < E; ++e) {
      scan_r[e] = r;
      scan_t[e] = tl;
      r += cnt[e];
      tl += (cnt[e] + BM - 1) / BM;
    }
    scan_r[E] = r;
    scan_t[E] = tl;
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += blockDim.x) {
    grp_rows[e] = scan_r[e];
    grp_tiles[e] = scan_t[e];
  }
  // stable positions: the owner thread of expert e walks the tokens in order
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    if (cnt[e] == 0) continue;
    int p = scan_r[e];
    for (int t = 0; t < T; ++t)
      for (int s = 0; s < topk; ++s)
        if (idx[t * topk + s] == e) {
          row_map[p] = t;
          pos[t * topk + s] = p;
          ++p;
        }
  }
}

// One workgroup. Rows are grouped by expert: expert e's rows are [off_e, off_e + cnt_e) in
// expert order, the shared expert (when present) owns rows [n, n + T) (n = T * topk) in token
// order. Writes pos[t * topk + s] (the row of slot s of token t), row_map (row -> token), the
// m-tile list tiles[j] = {expert (-1 shared), r0, r1, m} (the shared expert's tiles first, then
// the routed experts' in expert order) and its length. A row's place inside its expert's range
// comes from an atomic cursor, so it may change from run to run; no result depends on it (each
// output row is computed from its own token row alone, and the combine reads through pos).
// Two tile lists of the same rows are written, of at most BMr and BMr2 rows per tile (one per
// grouped kernel of the layer); tiles2 may be null.
__device__ __forceinline__ void bucket_tiles(const int *idx, int T, int topk, int E, int BMr, int BMr2, int shared,
                                             int *__restrict__ pos, int *__restrict__ row_map,
                                             int4 *__restrict__ tiles, int *__restrict__ ntiles,
                                             int4 *__restrict__ tiles2, int *__restrict__ ntiles2, int *sh) {
  int *cnt = sh;       // [E]
  int *cur = sh + E;   // [E]
  __shared__ int scan_r[256], scan_t[256], scan_t2[256];
  const int tid = threadIdx.x;
  const int n = T * topk;
  for (int e = tid; e < E; e += 256) cnt[e] = 0;
  __syncthreads();
  for (int i = tid; i < n; i += 256) atomicAdd(&cnt[idx[i]], 1);
  __syncthreads();
  // thread tid owns experts [e0, e1): their row and m-tile totals, then a block scan of those
  const int per = (E + 255) / 256;
  const int e0 = tid * per < E ? tid * per : E;
  const int e1 = e0 + per < E ? e0 + per : E;
  int rs = 0, ts = 0, ts2 = 0;
  for (int e = e0; e < e1; ++e) {
    rs += cnt[e];
    ts += (cnt[e] + BMr - 1) / BMr;
    ts2 += (cnt[e] + BMr2 - 1) / BMr2;
  }
  scan_r[tid] = rs;
  scan_t[tid] = ts;
  scan_t2[tid] = ts2;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const int ar = tid >= off ? scan_r[tid - off] : 0;
    const int at = tid >= off ? scan_t[tid - off] : 0;
    const int at2 = tid >= off ? scan_t2[tid - off] : 0;
    __syncthreads();
    scan_r[tid] += ar;
    scan_t[tid] += at;
    scan_t2[tid] += at2;
    __syncthreads();
  }
  const int tsh = shared ? (T + BMr - 1) / BMr : 0;
  const int tsh2 = shared ? (T + BMr2 - 1) / BMr2 : 0;
  int r = scan_r[tid] - rs, t = tsh + scan_t[tid] - ts, t2 = tsh2 + scan_t2[tid] - ts2;
  for (int e = e0; e < e1; ++e) {
    const int c = cnt[e], mt = (c + BMr - 1) / BMr, mt2 = (c + BMr2 - 1) / BMr2;
    cur[e] = r;
    for (int m = 0; m < mt; ++m) tiles[t + m] = make_int4(e, r, r + c, m);
    if (tiles2)
      for (int m = 0; m < mt2; ++m) tiles2[t2 + m] = make_int4(e, r + m * BMr2, r + (c < (m + 1) * BMr2 ? c : (m + 1) * BMr2), 0);
    r += c;
    t += mt;
    t2 += mt2;
  }
  if (tid == 255) {
    *ntiles = tsh + scan_t[255];
    if (ntiles2) *ntiles2 = tsh2 + scan_t2[255];
  }
  for (int j = tid; j < tsh; j += 256) tiles[j] = make_int4(-1, n, n + T, j);
  if (tiles2)
    for (int j = tid; j < tsh2; j += 256)
      tiles2[j] = make_int4(-1, n + j * BMr2, n + (T < (j + 1) * BMr2 ? T : (j + 1) * BMr2), 0);
  if (shared)
    for (int i = tid; i < T; i += 256) row_map[n + i] = i;
  __syncthreads();
  for (int i = tid; i < n; i += 256) {
    const int p = atomicAdd(&cur[idx[i]], 1);
    pos[i] = p;
    row_map[p] = i / topk;
  }
}

__global__ void __launch_bounds__(256) k_moe_bucket_tiles(const int *__restrict__ idx, int T, int topk, int E, int BMr,
                                                          int BMr2, int shared, int *__restrict__ pos,
                                                          int *__restrict__ row_map, int4 *__restrict__ tiles,
                                                          int *__restrict__ ntiles, int4 *__restrict__ tiles2,
                                                          int *__restrict__ ntiles2) {
  extern __shared__ int sh[];
  bucket_tiles(idx, T, topk, E, BMr, BMr2, shared, pos, row_map, tiles, ntiles, tiles2, ntiles2, sh);
}

// The bucketing of k_moe_bucket_tiles in workgroup 0 and, in workgroups 1..T, the fp16 copy of
// the token rows for the grouped MFMA GEMM (x_row_to_f16): two independent jobs in one launch.
template <int XDT, int CH>
__global__ void __launch_bounds__(256) k_moe_bucket_xh(const int *__restrict__ idx, int T, int topk, int E, int BMr,
                                                       int BMr2, int shared, int *__restrict__ pos,
                                                       int *__restrict__ row_map, int4 *__restrict__ tiles,
                                                       int *__restrict__ ntiles, int4 *__restrict__ tiles2,
                                                       int *__restrict__ ntiles2, const void *__restrict__ X,
                                                       int64_t K, u4 *__restrict__ Xh, float *__restrict__ xscale) {
  extern __shared__ int sh[];
  if (blockIdx.x == 0) {
    bucket_tiles(idx, T, topk, E, BMr, BMr2, shared, pos, row_map, tiles, ntiles, tiles2, ntiles2, sh);
  } else {
    x_row_to_f16<XDT, CH>(X, Xh, xscale, K, blockIdx.x - 1, reinterpret_cast<float *>(sh));
  }
}

// Few tokens: routing (wave w takes tokens w, w + 4, ...) and bucketing in one workgroup; the
// routed ids also go to LDS, where the bucketing reads them.
template <int LDT, int ENT>
__global__ void __launch_bounds__(256) k_moe_route_bucket(const void *__restrict__ logits, const float *__restrict__ bias,
                                                          int E, int topk, double scale, int *__restrict__ idx_out,
                                                          float *__restrict__ w_out, int T, int BMr, int BMr2,
                                                          int shared, int *__restrict__ pos, int *__restrict__ row_map,
                                                          int4 *__restrict__ tiles, int *__restrict__ ntiles,
                                                          int4 *__restrict__ tiles2, int *__restrict__ ntiles2) {
  extern __shared__ int sh[];
  int *idx_lds = sh + 2 * E;  // [T * topk]
  for (int t = threadIdx.x >> 6; t < T; t += 4)
    route_wave<LDT, ENT>(logits, bias, t, E, topk, scale, idx_out, w_out, idx_lds);
  __syncthreads();
  bucket_tiles(idx_lds, T, topk, E, BMr, BMr2, shared, pos, row_map, tiles, ntiles, tiles2, ntiles2, sh);
}

// Few tokens and at most 64 rows: routing (wave w takes tokens w, w + 4, ...), then the one-wave
// bucketing above.
template <int LDT, int ENT>
__global__ void __launch_bounds__(256) k_moe_route_bucket_w(const void *__restrict__ logits, const float *__restrict__ bias,
                                                            int E, int topk, double scale, int *__restrict__ idx_out,
                                                            float *__restrict__ w_out, int T, int BMr, int BMr2,
                                                            int shared, int *__restrict__ pos, int *__restrict__ row_map,
                                                            int4 *__restrict__ tiles, int *__restrict__ ntiles,
                                                            int4 *__restrict__ tiles2, int *__restrict__ ntiles2) {
  __shared__ int idx_lds[64];
  __shared__ uint64_t key_lds[64 * ENT];
  __shared__ double score_lds[64 * ENT];
  if (T == 1 && bias) {  // one token with a bias: the sigmoids of every expert over the four waves
    route_wg<LDT, ENT>(logits, bias, 0, E, topk, scale, idx_out, w_out, idx_lds, key_lds, score_lds);
  } else {
    for (int t = threadIdx.x >> 6; t < T; t += 4)
      route_wave<LDT, ENT>(logits, bias, t, E, topk, scale, idx_out, w_out, idx_lds);
  }
  __syncthreads();
  if (threadIdx.x < 64) bucket_rows_wave(idx_lds, T, topk, BMr, BMr2, shared, pos, row_map, tiles, ntiles, tiles2, ntiles2);
}

// out[t][h] = sum_s w[t,s] * rows[pos[t,s]][h] (+ shared[t][h]); fixed slot order. Four columns per
// thread (16-byte row loads, H % 4 == 0), all the slots' loads issued before the sums.
template <int ODT>
__global__ void __launch_bounds__(256) k_moe_combine(const float *__restrict__ rows, const float *__restrict__ shared,
                                                     const int *__restrict__ pos, const float *__restrict__ w, int T,
                                                     int topk, int64_t H, void *__restrict__ out) {
  const int64_t i4 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i4 >= T * H / 4) return;
  const int64_t i = 4 * i4;
  const int t = static_cast<int>(i / H);
  const int64_t h = i % H;
  f4 acc = {0.f, 0.f, 0.f, 0.f};
  constexpr int SB = 8;  // slots loaded per round trip
  for (int s0 = 0; s0 < topk; s0 += SB) {
    f4 v[SB];
    float ws[SB];
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      if (s0 + u < topk) {
        v[u] = *reinterpret_cast<const f4 *>(rows + static_cast<int64_t>(pos[t * topk + s0 + u]) * H + h);
        ws[u] = w[t * topk + s0 + u];
      }
    }
#pragma unroll
    for (int u = 0; u < SB; ++u)
      if (s0 + u < topk)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = fmaf(ws[u], v[u][j], acc[j]);
  }
  if (shared) {
    const f4 sh = *reinterpret_cast<const f4 *>(shared + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] += sh[j];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) store_elem<ODT>(out, nullptr, i + j, acc[j]);
}

struct MoeWs {
  int *idx, *pos, *grp_rows, *grp_tiles, *row_map, *ntiles, *ntiles2;
  int4 *tiles, *tiles2;
  float *w, *rows, *shared;
  _Float16 *act, *act_s;
  int64_t bytes;
};

// Upper bound of the m-tile list for tiles of at least `rows` rows: ceil(T / rows) shared
// tiles, and per expert with rows at most one tile more than its rows / rows.
static int64_t moe_max_tiles(int64_t T, int64_t E, int64_t k, int64_t rows = 1) {
  const int64_t n = T * k;
  return (T + rows - 1) / rows + (E < n ? E : n) + n / rows + 1;
}

static MoeWs moe_layout(char *base, int64_t T, int64_t H, int64_t I, int64_t E, int64_t k) {
  MoeWs m{};
  int64_t off = 0;
  auto take = [&](int64_t n) {
    char *p = base ? base + off : nullptr;
    off += (n + 255) / 256 * 256;
    return p;
  };
  m.idx = reinterpret_cast<int *>(take(4 * T * k));
  m.w = reinterpret_cast<float *>(take(4 * T * k));
  m.pos = reinterpret_cast<int *>(take(4 * T * k));
  m.row_map = reinterpret_cast<int *>(take(4 * (T * k + T)));
  m.grp_rows = reinterpret_cast<int *>(take(4 * (E + 1)));
  m.grp_tiles = reinterpret_cast<int *>(take(4 * (E + 1)));
  m.tiles = reinterpret_cast<int4 *>(take(16 * moe_max_tiles(T, E, k)));
  m.ntiles = reinterpret_cast<int *>(take(4));
  m.tiles2 = reinterpret_cast<int4 *>(take(16 * moe_max_tiles(T, E, k)));
  m.ntiles2 = reinterpret_cast<int *>(take(4));
  m.act = reinterpret_cast<_Float16 *>(take(2 * (T * k + T) * I));
  m.rows = reinterpret_cast<float *>(take(4 * (T * k + T) * H));
  m.act_s = reinterpret_cast<_Float16 *>(take(2 * T * I));
  m.shared = reinterpret_cast<float *>(take(4 * T * H));
  m.bytes = off;
  return m;
}

}  // namespace vybdq

using namespace vybdq;

extern "C" int64_t vybdq_moe_workspace_size(int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk) {
  if (T < 1 || H < 64 || I < 64 || E < 1 || E > 1024 || topk < 1 || topk > E || topk > 64) return -1;
  return moe_layout(nullptr, T, H, I, E, topk).bytes;
}

// The router launch: without a selection bias and with 32-bit or narrower logits, the keyed
// kernel (selection by logit); otherwise the double-precision kernel (F64 logits select by
// their own value, with the same ties-to-the-lower-id rule).
static int launch_route(const void *lg, int logits_dt, const float *bias, int64_t T, int64_t E, int64_t topk,
                        double scale, int *idx, float *w, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((T + 3) / 4)), block(256);
  const int e = static_cast<int>(E), k = static_cast<int>(topk), tt = static_cast<int>(T);
  if (logits_dt == VYBDQ_F64) {
    VYBDQ_DISPATCH_ENT(E, ENT, hipLaunchKernelGGL((k_moe_route<VYBDQ_F64, ENT>), grid, block, 0, s, lg, bias, e, k,
                                                  scale, idx, w, tt));
  } else {
    VYBDQ_DISPATCH_IN(logits_dt, LDT, VYBDQ_DISPATCH_ENT(E, ENT, hipLaunchKernelGGL((k_moe_route<LDT, ENT>), grid, block,
                                                                                    0, s, lg, bias, e, k, scale, idx, w, tt)));
  }
  return check_launch("moe route");
}

namespace vybdq {

// Routing and bucketing for a grouped expert call without shared-expert rows (moe_exl3.hip):
// idx / w [T topk], pos ((token, slot) -> row), row_map (row -> token) and the row groups of at
// most BMr rows, both as m-tiles (tiles) and as explicit row ranges {expert, r0, r1, 0} (tiles2),
// in the caller's memory. Up to 8 tokens one launch (routing and bucketing in one workgroup),
// else the router and one bucketing workgroup.
int moe_route_bucket(const void *logits, int logits_dt, const float *bias, int64_t T, int64_t E, int64_t topk,
                     double scale, int BMr, int *idx, float *w, int *pos, int *row_map, int4 *tiles, int *ntiles,
                     int4 *tiles2, int *ntiles2, hipStream_t s) {
  const int e = static_cast<int>(E), k = static_cast<int>(topk), tt = static_cast<int>(T);
  if (T <= 8) {
    const bool wave_rows = T * topk <= 64;
    const size_t shb = static_cast<size_t>(2 * E + T * topk) * 4;
#define RB(LDT)                                                                                               \
  do {                                                                                                             \
    VYBDQ_DISPATCH_ENT(E, ENT,                                                                                     \
      if (wave_rows)                                                                                               \
        hipLaunchKernelGGL((k_moe_route_bucket_w<LDT, ENT>), dim3(1), dim3(256), 0, s, logits, bias, e, k, scale, \
                           idx, w, tt, BMr, BMr, 0, pos, row_map, tiles, ntiles, tiles2, ntiles2);                 \
      else                                                                                                         \
        hipLaunchKernelGGL((k_moe_route_bucket<LDT, ENT>), dim3(1), dim3(256), shb, s, logits, bias, e, k, scale, \
                           idx, w, tt, BMr, BMr, 0, pos, row_map, tiles, ntiles, tiles2, ntiles2));                \
  } while (0)
    if (logits_dt == VYBDQ_F64) RB(VYBDQ_F64);
    else { VYBDQ_DISPATCH_IN(logits_dt, LDT, RB(LDT)); }
#undef RB
    return check_launch("moe route + bucket");
  }
  const int rc = launch_route(logits, logits_dt, bias, T, E, topk, scale, idx, w, s);
  if (rc) return rc;
  hipLaunchKernelGGL(k_moe_bucket_tiles, dim3(1), dim3(256), static_cast<size_t>(2 * E) * 4, s, idx, tt, k, e, BMr,
                     BMr, 0, pos, row_map, tiles, ntiles, tiles2, ntiles2);
  return check_launch("moe bucket");
}

// Upper bound of the row-group list of moe_route_bucket for groups of at most `rows` rows.
int64_t moe_tiles_bound(int64_t T, int64_t E, int64_t k, int64_t rows) { return moe_max_tiles(T, E, k, rows); }

}  // namespace vybdq

extern "C" int vybdq_moe_route(uint64_t logits, int logits_dt, uint64_t bias, uint64_t idx_out, uint64_t w_out,
                               int64_t T, int64_t E, int64_t topk, double scale, uint64_t stream) {
  VYBDQ_REQUIRE(logits && idx_out && w_out, VYBDQ_ERR_ARG, "null logits, idx_out or w_out");
  VYBDQ_REQUIRE(dt_valid_out(logits_dt), VYBDQ_ERR_ARG, "logits_dt must be F32, F16, BF16 or F64");
  VYBDQ_REQUIRE(T >= 1 && T < (1 << 24) && E >= 1 && E <= 1024 && topk >= 1 && topk <= E && topk <= 64,
                VYBDQ_ERR_SHAPE, "need 1 <= topk <= E <= 1024 and topk <= 64");
  return launch_route(reinterpret_cast<const void *>(logits), logits_dt, reinterpret_cast<const float *>(bias), T, E,
                      topk, scale, reinterpret_cast<int *>(idx_out), reinterpret_cast<float *>(w_out),
                      as_stream(stream));
}

extern "C" int vybdq_moe_forward(int wtype, uint64_t x, int x_dt, uint64_t logits, int logits_dt, uint64_t bias,
                                 uint64_t w_gate, uint64_t w_up, uint64_t w_down, uint64_t s_gate, uint64_t s_up,
                                 uint64_t s_down, uint64_t out, int out_dt, uint64_t idx_out, uint64_t w_out,
                                 int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk, double scale,
                                 double limit, uint64_t ws, int64_t ws_bytes, uint64_t stream) {
  VYBDQ_REQUIRE(wtype == 2 || wtype == 8, VYBDQ_ERR_ARG, "wtype must be 2 (q4_0) or 8 (Q8_0)");
  VYBDQ_REQUIRE(x && logits && w_gate && w_up && w_down && out, VYBDQ_ERR_ARG, "null input or output");
  VYBDQ_REQUIRE((s_gate == 0) == (s_up == 0) && (s_up == 0) == (s_down == 0), VYBDQ_ERR_ARG,
                "shared expert: give all three matrices or none");
  VYBDQ_REQUIRE(dt_valid_in(x_dt), VYBDQ_ERR_ARG, "x_dt must be F32, F16 or BF16");
  VYBDQ_REQUIRE(dt_valid_out(logits_dt), VYBDQ_ERR_ARG, "logits_dt must be F32, F16, BF16 or F64");
  VYBDQ_REQUIRE(out_dt == VYBDQ_F32 || out_dt == VYBDQ_F16 || out_dt == VYBDQ_BF16, VYBDQ_ERR_ARG,
                "out_dt must be F32, F16 or BF16");
  const int64_t need = vybdq_moe_workspace_size(T, H, I, E, topk);
  VYBDQ_REQUIRE(need > 0, VYBDQ_ERR_SHAPE, "unsupported T, H, I, E or topk (E <= 1024, topk <= 64)");
  VYBDQ_REQUIRE(H % 64 == 0 && I % 64 == 0, VYBDQ_ERR_SHAPE, "H and I must be multiples of 64");
  VYBDQ_REQUIRE(T * topk < (1 << 24), VYBDQ_ERR_SHAPE, "too many tokens");
  VYBDQ_REQUIRE((T * topk + T) * (H > I ? H : I) < (int64_t(1) << 31), VYBDQ_ERR_SHAPE,
                "too many tokens for H and I (the routed and shared rows times max(H, I) must stay below 2^31)");
  VYBDQ_REQUIRE(ws && (ws & 255) == 0 && ws_bytes >= need, VYBDQ_ERR_WORKSPACE,
                "workspace must be 256-byte aligned and at least vybdq_moe_workspace_size bytes");
  VYBDQ_REQUIRE((x & 15) == 0 && (w_gate & 3) == 0 && (w_up & 3) == 0 && (w_down & 3) == 0, VYBDQ_ERR_ALIGN,
                "x must be 16-byte and weights 4-byte aligned");
  hipStream_t s = as_stream(stream);
  MoeWs m = moe_layout(reinterpret_cast<char *>(ws), T, H, I, E, topk);
  if (H % 256 == 0 && I % 256 == 0) {
    // 16-row fragments per m-tile (VYBDQ_MOE_MT overrides: 1 or 2). q4_0: 16-row tiles (the
    // LDS-staged body) while the experts average at most 20 rows, then 32-row tiles (measured on
    // H = 6144, I = 2048, 256 experts, top-8: 16-row tiles win up to T ~ 700). Q8_0: 32-row tiles
    // above 16 tokens.
    int MT = wtype == 2 ? (T * topk <= 20 * E ? 1 : 2) : (T > 16 ? 2 : 1);
    if (const char *e = tuning_env("VYBDQ_MOE_MT")) MT = atoi(e) == 1 ? 1 : 2;
    const int n = static_cast<int>(T * topk);
    // q4_0 with few rows per expert: 4-row tiles on the LDS-staged body (a smaller X stage, one more
    // weight stage in flight) while the experts hit average at most ROWS4 rows; the shared expert's
    // T rows then take ceil(T / 4) tiles over its weights. VYBDQ_MOE_ROWS4 overrides the bound
    // (0: never).
    const char *lds_env = tuning_env("VYBDQ_MOE_LDS");
    int rows4_max = 2;
    if (const char *e = tuning_env("VYBDQ_MOE_ROWS4")) rows4_max = atoi(e);
    const int64_t hit = E < T * topk ? E : T * topk;
    const bool rows4 = wtype == 2 && MT == 1 && !(lds_env && lds_env[0] == '0') && T * topk <= rows4_max * hit;
    const bool shared = s_gate != 0;
    int *idx = idx_out ? reinterpret_cast<int *>(idx_out) : m.idx;
    float *wts = w_out ? reinterpret_cast<float *>(w_out) : m.w;
    // up to 8 tokens: routing and bucketing in one launch (below)
    const bool fused_route = T <= 8;
    int rc = VYBDQ_OK;
    if (!fused_route) {
      rc = launch_route(reinterpret_cast<const void *>(logits), logits_dt, reinterpret_cast<const float *>(bias), T, E,
                        topk, scale, idx, wts, s);
      if (rc) return rc;
    }
    // few tokens per expert: grouped GEMV (one tile per expert); else the grouped MFMA GEMM.
    // Measured crossovers: q4_0 (LDS-staged MFMA body) the GEMV only at one token (T = 2: 2.8
    // against 2.5 TB/s, T = 16: 4.0 against 3.0); Q8_0 the GEMV up to 64 tokens.
    int gv_max = wtype == 2 ? 1 : 64;
    if (const char *e = tuning_env("VYBDQ_MOE_GEMV_MAX_T")) gv_max = atoi(e);
    const bool gv = T <= gv_max && H / 64 <= 256 * 4 && I / 64 <= 256 * 4;
    // GEMV groups hold at most one x stage of tokens: larger experts (and the shared expert)
    // become several groups over the same weights that run side by side
    int mc = kMoeGvMC;  // tokens per GEMV group (experts with more rows: several groups)
    if (const char *e = tuning_env("VYBDQ_MOE_GEMV_MC")) mc = atoi(e) < 1 ? 1 : (atoi(e) > kMoeGvMC ? kMoeGvMC : atoi(e));
    if (mc > T) mc = static_cast<int>(T);  // no group holds more rows than there are tokens
    // tiles: m-tiles of 16 MT (or 4) rows for the MFMA GEMM; tiles2: groups of at most mc rows for
    // the GEMV
    const int BMr = rows4 ? 4 : 16 * MT;
    // one token on the grouped GEMV (up to 256 experts): the gate|up launch routes the token itself
    // and writes the ids, weights, rows and groups for the down launch and the combine, so no
    // routing launch precedes it (VYBDQ_MOE_ROUTE_GV=0 keeps the routing launch)
    // many tokens on the grouped MFMA GEMM with bf16 / f32 x: the fp16 copy of x (into `rows`, which
    // only the down GEMM writes, after gate|up has read it) rides on the bucketing launch
    // (VYBDQ_MOE_XH_SEP=1: its own launch)
    const bool xh_with_bucket = !gv && !fused_route && x_dt != VYBDQ_F16 && !tuning_env("VYBDQ_MOE_XH_SEP");
    _Float16 *xh_copy = reinterpret_cast<_Float16 *>(m.rows);
    float *xh_scale = reinterpret_cast<float *>(xh_copy + T * H);
    bool route_in_gv = gv && T == 1 && E <= 256 && !tuning_env("VYBDQ_MOE_GEMV_COLS");
    if (const char *e = tuning_env("VYBDQ_MOE_ROUTE_GV")) route_in_gv = route_in_gv && e[0] != '0';
    if (route_in_gv) {
      // routed in the gate|up launch below
    } else if (fused_route) {
      const void *lg = reinterpret_cast<const void *>(logits);
      const float *bs = reinterpret_cast<const float *>(bias);
      const size_t shb = static_cast<size_t>(2 * E + T * topk) * 4;
      const int e = static_cast<int>(E), k = static_cast<int>(topk), tt = static_cast<int>(T);
      int4 *t2 = gv ? m.tiles2 : nullptr;
      int *n2 = gv ? m.ntiles2 : nullptr;
      // at most 64 rows: the one-wave bucketing (no LDS counts, scans or barriers)
      const bool wave_rows = T * topk <= 64;
#define RB(LDT)                                                                                               \
  do {                                                                                                             \
    VYBDQ_DISPATCH_ENT(E, ENT,                                                                                     \
      if (wave_rows)                                                                                               \
        hipLaunchKernelGGL((k_moe_route_bucket_w<LDT, ENT>), dim3(1), dim3(256), 0, s, lg, bs, e, k, scale, idx,  \
                           wts, tt, BMr, mc, shared ? 1 : 0, m.pos, m.row_map, m.tiles, m.ntiles, t2, n2);         \
      else                                                                                                         \
        hipLaunchKernelGGL((k_moe_route_bucket<LDT, ENT>), dim3(1), dim3(256), shb, s, lg, bs, e, k, scale, idx,  \
                           wts, tt, BMr, mc, shared ? 1 : 0, m.pos, m.row_map, m.tiles, m.ntiles, t2, n2));        \
  } while (0)
      if (logits_dt == VYBDQ_F64) RB(VYBDQ_F64);
      else { VYBDQ_DISPATCH_IN(logits_dt, LDT, RB(LDT)); }
#undef RB
      rc = check_launch("moe route + bucket");
    } else if (xh_with_bucket) {
      const int e = static_cast<int>(E), k = static_cast<int>(topk), tt = static_cast<int>(T);
      const size_t shb = static_cast<size_t>(2 * E) * 4 > 16 ? static_cast<size_t>(2 * E) * 4 : 16;
      u4 *xo = reinterpret_cast<u4 *>(xh_copy);
#define BX(XDT, CH)                                                                                                 \
  hipLaunchKernelGGL((k_moe_bucket_xh<XDT, CH>), dim3(static_cast<unsigned>(T + 1)), dim3(256), shb, s, idx, tt, k, e, \
                     BMr, mc, shared ? 1 : 0, m.pos, m.row_map, m.tiles, m.ntiles, nullptr, nullptr,                 \
                     reinterpret_cast<const void *>(x), H, xo, xh_scale)
#define BXC(XDT)                                                            \
  do {                                                                      \
    const int per = x_row_chunks(H);                                        \
    if (per <= 2) BX(XDT, 2);                                               \
    else if (per <= 4) BX(XDT, 4);                                          \
    else if (per <= 8) BX(XDT, 8);                                          \
    else if (per <= 12) BX(XDT, 12);                                        \
    else BX(XDT, 0);                                                        \
  } while (0)
      if (x_dt == VYBDQ_BF16) BXC(VYBDQ_BF16);
      else BXC(VYBDQ_F32);
#undef BXC
#undef BX
      rc = check_launch("moe bucket + x rows");
    } else {
      hipLaunchKernelGGL(k_moe_bucket_tiles, dim3(1), dim3(256), static_cast<size_t>(2 * E) * 4, s, idx,
                         static_cast<int>(T), static_cast<int>(topk), static_cast<int>(E), BMr, mc, shared ? 1 : 0,
                         m.pos, m.row_map, m.tiles, m.ntiles, gv ? m.tiles2 : nullptr, gv ? m.ntiles2 : nullptr);
      rc = check_launch("moe bucket");
    }
    if (rc) return rc;
    const int max_tiles = static_cast<int>(moe_max_tiles(T, E, topk, BMr));
    const int64_t rb_h = (H / 64) * (wtype == 2 ? 36 : 68);  // row bytes, K = H
    const int64_t rb_i = (I / 64) * (wtype == 2 ? 36 : 68);  // row bytes, K = I
    if (gv) {
      const int max_groups = static_cast<int>(moe_max_tiles(T, E, topk, mc));
      MoeGvArgs ga{};
      ga.W = reinterpret_cast<const uint8_t *>(w_gate);
      ga.W2 = reinterpret_cast<const uint8_t *>(w_up);
      ga.w_stride = I * rb_h;
      ga.Ws = reinterpret_cast<const uint8_t *>(s_gate);
      ga.W2s = reinterpret_cast<const uint8_t *>(s_up);
      ga.rowbytes = rb_h;
      ga.P = static_cast<int>(H / 64);
      ga.X = reinterpret_cast<const void *>(x);
      ga.xdt = x_dt;
      ga.ldx = H;
      ga.row_map = m.row_map;
      ga.groups = m.tiles2;
      ga.ngroups = m.ntiles2;
      // Up to 4 tokens (groups of one row, but for the shared expert's): equal ranges over a
      // grid of the workgroups the device holds at once (3-4 tokens: twice that, so that the
      // dispatcher evens out the shared expert's costlier units); VYBDQ_MOE_GEMV_GRID=
      // "gate_up,down" workgroups per CU overrides. More tokens: blocks of 128 columns, halved
      // while the grid would hold under two workgroups per CU (VYBDQ_MOE_GEMV_COLS="gate_up,down"
      // overrides; -1: equal ranges). Measured on H = 6144, I = 2048, 256 experts, top-8.
      const int grid_def = T <= 2 ? 0 : -2;
      // q4_0 at one token: the down GEMV at one workgroup per CU (two fit; one, with ranges twice as
      // long, measured 58.0-58.3 against 59.2-59.6 us per GLM-5 layer)
      int grid_env[2] = {grid_def, T == 1 && wtype == 2 ? 1 : grid_def}, cols_env[2] = {0, 0};
      if (const char *e = tuning_env("VYBDQ_MOE_GEMV_GRID")) sscanf(e, "%d,%d", &grid_env[0], &grid_env[1]);
      if (const char *e = tuning_env("VYBDQ_MOE_GEMV_COLS")) sscanf(e, "%d,%d", &cols_env[0], &cols_env[1]);
      const int cus = device_cu_count();
      auto cols_for = [&](int64_t N, int cpp, int forced) {
        if (forced < 0) return 0;
        if (forced > 0) return forced;
        if (T <= 4) return 0;
        int64_t c = 128;
        while (c > cpp && (N / c) * (1 + (E < n ? E : n)) < 2 * cus) c /= 2;
        return static_cast<int>(c);
      };
      ga.N = static_cast<int>(I);
      ga.cols_per_wg = cols_for(I, moe_gv_cpp(32, true), cols_env[0]);
      ga.wg_per_cu = grid_env[0];
      ga.Y = m.act;
      ga.ydt = VYBDQ_F16;
      ga.ldy = I;
      ga.limit = static_cast<float>(limit);
      ga.mc = mc;
      if (route_in_gv) {
        ga.rt = MoeGvRoute{reinterpret_cast<const void *>(logits), logits_dt, reinterpret_cast<const float *>(bias),
                           static_cast<int>(E), static_cast<int>(topk), shared ? 1 : 0, scale, idx, wts, m.pos,
                           m.tiles2, m.ntiles2};
        ga.row_map = nullptr;
        ga.ldx = 0;  // every row is token 0's
      }
      rc = wtype == 2 ? moe_gemv_q4(true, ga, max_groups, s) : moe_gemv_q8(true, ga, max_groups, s);
      if (rc) return rc;
      MoeGvArgs gd = ga;
      gd.W = reinterpret_cast<const uint8_t *>(w_down);
      gd.W2 = nullptr;
      gd.w_stride = H * rb_i;
      gd.Ws = reinterpret_cast<const uint8_t *>(s_down);
      gd.W2s = nullptr;
      gd.rowbytes = rb_i;
      gd.P = static_cast<int>(I / 64);
      gd.X = m.act;
      gd.xdt = VYBDQ_F16;
      gd.ldx = I;
      gd.row_map = nullptr;
      gd.rt = MoeGvRoute{};
      gd.N = static_cast<int>(H);
      gd.cols_per_wg = cols_for(H, moe_gv_cpp(16, false), cols_env[1]);
      gd.wg_per_cu = grid_env[1];
      gd.Y = m.rows;
      gd.ydt = VYBDQ_F32;
      gd.ldy = H;
      rc = wtype == 2 ? moe_gemv_q4(false, gd, max_groups, s) : moe_gemv_q8(false, gd, max_groups, s);
      if (rc) return rc;
    } else {
      auto run = [&](int xdt, bool swi, const MoeMmArgs &g) {
        return wtype == 2 ? moe_mm_q4(xdt, MT, swi, g, max_tiles, s) : moe_mm_q8(xdt, MT, swi, g, max_tiles, s);
      };
      // gate|up with SwiGLU -> act [n + T][I] fp16
      MoeMmArgs g{};
      g.m.W = reinterpret_cast<const uint8_t *>(w_gate);
      g.m.W2 = reinterpret_cast<const uint8_t *>(w_up);
      g.m.rowbytes = rb_h;
      g.m.X = reinterpret_cast<const void *>(x);
      g.m.ldx = H;
      g.m.row_map = m.row_map;
      g.m.N = static_cast<int>(I);
      g.m.S = static_cast<int>(H / 128);
      g.m.F = kMoeF;
      g.m.n_tiles = static_cast<int>(I / (16 * kMoeF));
      g.m.splits = 1;
      g.m.sps = g.m.S;
      g.m.Y = m.act;
      g.m.ydt = VYBDQ_F16;
      g.m.ldy = I;
      g.m.limit = static_cast<float>(limit);
      g.w_stride = I * rb_h;
      g.Ws = reinterpret_cast<const uint8_t *>(s_gate);
      g.W2s = reinterpret_cast<const uint8_t *>(s_up);
      g.tiles = m.tiles;
      g.ntiles = m.ntiles;
      g.tile_rows = rows4 ? 4 : 0;
      int gxdt = x_dt;
      if (x_dt != VYBDQ_F16) {
        // f32 / bf16 x: an fp16 copy with a power-of-two scale per token, so that the GEMM streams X
        // straight into LDS (its register path for other types waits on the X loads in issue
        // order, which drains the weight ring every step). The copy lives in `rows`, which only
        // the down GEMM writes, after gate|up has read it.
        if (!xh_with_bucket) {
          rc = x_rows_to_f16(reinterpret_cast<const void *>(x), x_dt, T, H, xh_copy, xh_scale, s);
          if (rc) return rc;
        }
        g.m.X = xh_copy;
        g.m.xscale = xh_scale;
        gxdt = VYBDQ_F16;
      }
      rc = run(gxdt, true, g);
      if (rc) return rc;
      // down -> rows [n + T][H] f32
      MoeMmArgs d = g;
      d.m.W = reinterpret_cast<const uint8_t *>(w_down);
      d.m.W2 = nullptr;
      d.m.rowbytes = rb_i;
      d.m.X = m.act;
      d.m.ldx = I;
      d.m.row_map = nullptr;
      d.m.xscale = nullptr;
      d.m.N = static_cast<int>(H);
      d.m.S = static_cast<int>(I / 128);
      d.m.n_tiles = static_cast<int>(H / (16 * kMoeF));
      d.m.sps = d.m.S;
      d.m.Y = m.rows;
      d.m.ydt = VYBDQ_F32;
      d.m.ldy = H;
      d.w_stride = H * rb_i;
      d.Ws = reinterpret_cast<const uint8_t *>(s_down);
      d.W2s = nullptr;
      rc = run(VYBDQ_F16, false, d);
      if (rc) return rc;
    }
    const float *shr = shared ? m.rows + static_cast<int64_t>(n) * H : nullptr;
    const int64_t tot = T * H / 4;  // four columns per thread
    const unsigned gc = static_cast<unsigned>((tot + 255) / 256);
    void *o = reinterpret_cast<void *>(out);
    switch (out_dt) {
      case VYBDQ_F32: hipLaunchKernelGGL((k_moe_combine<VYBDQ_F32>), dim3(gc), dim3(256), 0, s, m.rows, shr, m.pos, wts, static_cast<int>(T), static_cast<int>(topk), H, o); break;
      case VYBDQ_F16: hipLaunchKernelGGL((k_moe_combine<VYBDQ_F16>), dim3(gc), dim3(256), 0, s, m.rows, shr, m.pos, wts, static_cast<int>(T), static_cast<int>(topk), H, o); break;
      default: hipLaunchKernelGGL((k_moe_combine<VYBDQ_BF16>), dim3(gc), dim3(256), 0, s, m.rows, shr, m.pos, wts, static_cast<int>(T), static_cast<int>(topk), H, o); break;
    }
    return check_launch("moe combine");
  }
  const int BM = dq_gemm_bm();
  const int n = static_cast<int>(T * topk);
  int *idx = idx_out ? reinterpret_cast<int *>(idx_out) : m.idx;
  float *wts = w_out ? reinterpret_cast<float *>(w_out) : m.w;
  int rc = launch_route(reinterpret_cast<const void *>(logits), logits_dt, reinterpret_cast<const float *>(bias), T, E,
                        topk, scale, idx, wts, s);
  if (rc) return rc;
  const size_t sh = static_cast<size_t>(3 * E + 2) * 4;
  hipLaunchKernelGGL(k_moe_bucket, dim3(1), dim3(256), sh, s, idx, static_cast<int>(T), static_cast<int>(topk),
                     static_cast<int>(E), BM, m.grp_rows, m.grp_tiles, m.row_map, m.pos);
  rc = check_launch("moe bucket");
  if (rc) return rc;
  const int64_t rb_h = (H / 64) * (wtype == 2 ? 36 : 68);  // row bytes, K = H
  const int64_t rb_i = (I / 64) * (wtype == 2 ? 36 : 68);  // row bytes, K = I
  const int max_mt = static_cast<int>((n + BM - 1) / BM + (E < n ? E : n));
  // routed gate|up with SwiGLU -> act [n][I] (bucket order)
  rc = dq_gemm_grouped(wtype, true, reinterpret_cast<const uint8_t *>(w_gate), reinterpret_cast<const uint8_t *>(w_up),
                       I * rb_h, reinterpret_cast<const void *>(x), x_dt, H, m.row_map, m.grp_rows, m.grp_tiles,
                       static_cast<int>(E), n, static_cast<int>(I), H, m.act, VYBDQ_F16, I,
                       static_cast<float>(limit), max_mt, s);
  if (rc) return rc;
  // routed down -> rows [n][H]
  rc = dq_gemm_grouped(wtype, false, reinterpret_cast<const uint8_t *>(w_down), nullptr, H * rb_i, m.act, VYBDQ_F16,
                       I, nullptr, m.grp_rows, m.grp_tiles, static_cast<int>(E), n, static_cast<int>(H), I, m.rows,
                       VYBDQ_F32, H, 0.f, max_mt, s);
  if (rc) return rc;
  const float *shared = nullptr;
  if (s_gate) {
    const int mt = static_cast<int>((T + BM - 1) / BM);
    rc = dq_gemm_grouped(wtype, true, reinterpret_cast<const uint8_t *>(s_gate), reinterpret_cast<const uint8_t *>(s_up),
                         0, reinterpret_cast<const void *>(x), x_dt, H, nullptr, nullptr, nullptr, 1,
                         static_cast<int>(T), static_cast<int>(I), H, m.act_s, VYBDQ_F16, I, static_cast<float>(limit),
                         mt, s);
    if (rc) return rc;
    rc = dq_gemm_grouped(wtype, false, reinterpret_cast<const uint8_t *>(s_down), nullptr, 0, m.act_s, VYBDQ_F16, I,
                         nullptr, nullptr, nullptr, 1, static_cast<int>(T), static_cast<int>(H), I, m.shared,
                         VYBDQ_F32, H, 0.f, mt, s);
    if (rc) return rc;
    shared = m.shared;
  }
  const int64_t tot = T * H / 4;  // four columns per thread
  const unsigned gc = static_cast<unsigned>((tot + 255) / 256);
  void *o = reinterpret_cast<void *>(out);
  switch (out_dt) {
    case VYBDQ_F32: hipLaunchKernelGGL((k_moe_combine<VYBDQ_F32>), dim3(gc), dim3(256), 0, s, m.rows, shared, m.pos, wts, static_cast<int>(T), static_cast<int>(topk), H, o); break;
    case VYBDQ_F16: hipLaunchKernelGGL((k_moe_combine<VYBDQ_F16>), dim3(gc), dim3(256), 0, s, m.rows, shared, m.pos, wts, static_cast<int>(T), static_cast<int>(topk), H, o); break;
    default: hipLaunchKernelGGL((k_moe_combine<VYBDQ_BF16>), dim3(gc), dim3(256), 0, s, m.rows, shared, m.pos, wts, static_cast<int>(T), static_cast<int>(topk), H, o); break;
  }
  return check_launch("moe combine");
}

// ---- allocation-free variant --------------------------------------------------------------
//
// The workspace of vybdq_moe_forward_noalloc: one array per GPU (each device that loads this
// code object holds its own copy until the process ends). Host code never passes the array's
// name to a kernel: its device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) char scratch[VYBDQ_MOE_NOALLOC_MAX_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint64_t g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device (0: not yet set up)

// Device address of the current device's scratch array; set up on the first call per device.
int scratch_address(uint64_t &ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(VYBDQ_ERR_HIP, "vybdq_moe_forward_noalloc: no current HIP device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(VYBDQ_ERR_HIP, std::string("vybdq_moe_forward_noalloc: hipGetSymbolAddress failed: ") +
                                          hipGetErrorString(e));
    g_scratch_ptr[dev] = reinterpret_cast<uint64_t>(p);
  }
  ptr = g_scratch_ptr[dev];
  return VYBDQ_OK;
}
}  // namespace

extern "C" int vybdq_moe_forward_noalloc(int wtype, uint64_t x, int x_dt, uint64_t logits, int logits_dt,
                                         uint64_t bias, uint64_t w_gate, uint64_t w_up, uint64_t w_down,
                                         uint64_t s_gate, uint64_t s_up, uint64_t s_down, uint64_t out, int out_dt,
                                         uint64_t idx_out, uint64_t w_out, int64_t T, int64_t H, int64_t I,
                                         int64_t E, int64_t topk, double scale, double limit, uint64_t stream) {
  const int64_t need = vybdq_moe_workspace_size(T, H, I, E, topk);
  VYBDQ_REQUIRE(need > 0, VYBDQ_ERR_SHAPE, "unsupported T, H, I, E or topk (E <= 1024, topk <= 64)");
  VYBDQ_REQUIRE(need <= VYBDQ_MOE_NOALLOC_MAX_BYTES, VYBDQ_ERR_WORKSPACE,
                "the shape needs " + std::to_string(need) + " workspace bytes, more than the " +
                    std::to_string(static_cast<long long>(VYBDQ_MOE_NOALLOC_MAX_BYTES)) +
                    " of the library's scratch; use vybdq_moe_forward with a caller workspace");
  uint64_t ws = 0;
  const int rc = scratch_address(ws);
  if (rc) return rc;
  return vybdq_moe_forward(wtype, x, x_dt, logits, logits_dt, bias, w_gate, w_up, w_down, s_gate, s_up, s_down, out,
                           out_dt, idx_out, w_out, T, H, I, E, topk, scale, limit, ws, VYBDQ_MOE_NOALLOC_MAX_BYTES,
                           stream);
}
