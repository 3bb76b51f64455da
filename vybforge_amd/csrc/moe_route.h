// The MoE router of one token per wave and the one-wave bucketing of at most 64 rows, gfx950;
// shared by the q4_0 / Q8_0 layer (moe.hip) and the EXL3 layer (moe_exl3.hip).
//
// Semantics (native/glm53/moe_ref.py:25-60, native/kernels/moe.vyb:1-74): scores = sigmoid(logits);
// choice = scores + bias (the bias only selects); idx = top-k(choice), descending, ties to the lower
// expert id; w = scores[idx] / (sum + 1e-20) * scale.
#pragma once
#include "gemv_dev.h"

namespace vybdq {

// A router logit as float64 (F64 logits as stored; F32 / F16 / BF16 widened exactly).
template <int LDT>
__device__ __forceinline__ double load_logit(const void *p, int64_t i) {
  if constexpr (LDT == VYBDQ_F64) return static_cast<const double *>(p)[i];
  else return static_cast<double>(load_elem<LDT>(p, i));
}

// Smallest / largest 32-bit value over the wave, in every lane, on the VALU: DPP steps combine the
// lanes of each quad, half-row and row, then rows 1 and 3 take rows 0 and 2 (row_bcast 15) and row
// 3 takes rows 0-1 (row_bcast 31); lane 63 then holds the extreme, read back as a scalar.
template <bool MAX>
__device__ __forceinline__ uint32_t wave_ext_u32(uint32_t v) {
  auto step = [&](auto ctrl, auto rows) {
    constexpr int C = decltype(ctrl)::value, R = decltype(rows)::value;
    const uint32_t o = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
        static_cast<int>(MAX ? 0u : 0xffffffffu), static_cast<int>(v), C, R, 0xf, false));
    v = MAX ? (o > v ? o : v) : (o < v ? o : v);
  };
  step(std::integral_constant<int, DPP_QUAD_XOR1>{}, std::integral_constant<int, 0xf>{});
  step(std::integral_constant<int, DPP_QUAD_XOR2>{}, std::integral_constant<int, 0xf>{});
  step(std::integral_constant<int, DPP_HALF_MIRROR>{}, std::integral_constant<int, 0xf>{});
  step(std::integral_constant<int, DPP_ROW_MIRROR>{}, std::integral_constant<int, 0xf>{});
  step(std::integral_constant<int, DPP_BCAST15>{}, std::integral_constant<int, 0xa>{});
  step(std::integral_constant<int, DPP_BCAST31>{}, std::integral_constant<int, 0x8>{});
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// A double's order as an unsigned 64-bit key: larger double, larger key; -0 keys as +0 (they
// compare equal), and NaN keys below every number (a NaN never compares greater).
__device__ __forceinline__ uint64_t double_order_key(double d) {
  if (d != d) return 0;
  uint64_t b = __double_as_longlong(d);
  if (b == 0x8000000000000000ull) b = 0;
  return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}

constexpr uint32_t kRouteNone = 0x7fffffffu;  // no candidate (and above every expert id)

// The selection key of expert e: the order key of its double-precision sigmoid score + bias, or
// of the logit itself without a bias.
__device__ __forceinline__ uint64_t route_key(double l, const float *__restrict__ bias, int e) {
  return double_order_key(bias ? 1.0 / (1.0 + exp(-l)) + static_cast<double>(bias[e]) : l);
}

// The selection rounds of route_wave on this lane's entries; returns the expert of slot `lane`
// (lanes < topk), kRouteNone elsewhere.
template <int ENT>
__device__ __forceinline__ uint32_t route_select(uint64_t (&key)[ENT], uint32_t (&eid)[ENT], int topk) {
  constexpr uint32_t kNone = kRouteNone;
  const int lane = threadIdx.x & 63;
  uint32_t mine = kNone;  // lane s < topk: the expert of slot s
  for (int s = 0; s < topk; ++s) {
    uint64_t bk = 0;
    uint32_t be = kNone;
    // (an empty entry, key 0 and id kNone, never beats the start value: no test of it, no branch)
#pragma unroll
    for (int i = 0; i < ENT; ++i) {
      const bool take = (key[i] > bk) | ((key[i] == bk) & (eid[i] < be));
      bk = take ? key[i] : bk;
      be = take ? eid[i] : be;
    }
    const uint32_t khi = static_cast<uint32_t>(bk >> 32);
    const uint32_t mhi = wave_ext_u32<true>(khi);
    uint64_t own = __ballot(khi == mhi && be != kNone);
    if (__popcll(own) > 1) {
      const uint32_t klo = khi == mhi ? static_cast<uint32_t>(bk) : 0u;
      const uint32_t mlo = wave_ext_u32<true>(klo);
      const uint32_t e1 = wave_ext_u32<false>(khi == mhi && klo == mlo ? be : kNone);
      own = __ballot(be == e1 && e1 != kNone);
    }
    const int src = own ? static_cast<int>(__builtin_ctzll(own)) : 0;
    const uint32_t we = own ? static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(be), src)) : kNone;
    mine = lane == s ? we : mine;
#pragma unroll
    for (int i = 0; i < ENT; ++i) {
      const bool won = eid[i] == we;  // ids are unique: the winner's entry becomes empty
      eid[i] = won ? kNone : eid[i];
      key[i] = won ? 0 : key[i];
    }
  }
  return mine;
}

// The outputs of one routed token from the slot experts (lanes < topk) and their scores: the
// weights are the scores over their sum in slot order, times scale.
__device__ __forceinline__ void route_store(uint32_t mine, double sc, int t, int topk, double scale,
                                            int *__restrict__ idx_out, float *__restrict__ w_out,
                                            int *__restrict__ idx_copy) {
  const int lane = threadIdx.x & 63;
  const bool slot = lane < topk && mine != kRouteNone;
  if (!slot) sc = 0.0;
  const uint64_t sb = __double_as_longlong(sc);
  double tot = 0.0;  // the scores summed in slot order
  for (int q = 0; q < topk; ++q) {
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(sb), q);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(sb >> 32), q);
    tot += __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
  }
  if (slot) {
    idx_out[t * topk + lane] = static_cast<int>(mine);
    if (idx_copy) idx_copy[t * topk + lane] = static_cast<int>(mine);
  }
  if (lane < topk) w_out[t * topk + lane] = static_cast<float>(sc / (tot + 1e-20) * scale);
}

// Routing of one token by one wave: lane l holds experts l, l + 64, ..., l + 64 (ENT - 1) (E <= 64 ENT)
// with their order keys (of the double-precision sigmoid score + bias, or of the logit without a
// bias). A selection round takes each lane's best entry (branch-free), then the wave maximum (DPP, on
// the VALU) of the top 32 bits of those keys; only when several lanes share it, of the low 32 bits
// among those and then the lowest expert id (ties to the lower id); the winner is retired where it
// lives. After topk rounds lane s holds the expert of slot s and computes its score again (the same
// expression), and the weights are the scores over their sum in slot order, times scale. Keys, the
// tie rule and the weight arithmetic are one total order and one formula, so the result is that of
// a single pass over all E experts. (Four waves each selecting among a quarter of the experts, then
// merging their candidates through LDS, took 4.8 us per token against 3.3 (warm, E = 256, top-8);
// carrying each entry's score through the rounds instead of recomputing the winners' took 3.5.)
template <int LDT, int ENT>
__device__ __forceinline__ void route_wave(const void *__restrict__ logits, const float *__restrict__ bias, int t, int E,
                                           int topk, double scale, int *__restrict__ idx_out, float *__restrict__ w_out,
                                           int *__restrict__ idx_copy) {
  const int lane = threadIdx.x & 63;
  uint64_t key[ENT];
  uint32_t eid[ENT];
#pragma unroll
  for (int i = 0; i < ENT; ++i) {
    const int e = lane + 64 * i;
    key[i] = 0;
    eid[i] = kRouteNone;
    if (e < E) {
      key[i] = route_key(load_logit<LDT>(logits, static_cast<int64_t>(t) * E + e), bias, e);
      eid[i] = static_cast<uint32_t>(e);
    }
  }
  const uint32_t mine = route_select<ENT>(key, eid, topk);
  double sc = 0.0;
  if (lane < topk && mine != kRouteNone)
    sc = 1.0 / (1.0 + exp(-load_logit<LDT>(logits, static_cast<int64_t>(t) * E + mine)));
  route_store(mine, sc, t, topk, scale, idx_out, w_out, idx_copy);
}

// The same routing of token t by a whole workgroup (every thread calls it; it holds barriers):
// the keys and the double-precision scores of experts tid, tid + blockDim.x, ... are computed by
// every thread into LDS (keys: E words, scores: E doubles), so each thread evaluates the sigmoid
// about E / blockDim.x times instead of E / 64; wave 0 then runs the selection rounds on them and
// reads the winners' scores back. The keys, the selection and the score expression are those of
// route_wave, so the outputs are identical. route_wg_keys: the key and score part (no barrier).
template <int LDT>
__device__ __forceinline__ void route_wg_keys(const void *__restrict__ logits, const float *__restrict__ bias, int t,
                                              int E, uint64_t *key_lds, double *score_lds) {
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    const double l = load_logit<LDT>(logits, static_cast<int64_t>(t) * E + e);
    const double sc = 1.0 / (1.0 + exp(-l));
    score_lds[e] = sc;
    key_lds[e] = double_order_key(bias ? sc + static_cast<double>(bias[e]) : l);  // = route_key(l, bias, e)
  }
}

// The selection of route_wg on wave 0 (threads 0-63 call it, after a barrier behind route_wg_keys).
template <int ENT>
__device__ __forceinline__ void route_wg_select(int t, int E, int topk, double scale, int *__restrict__ idx_out,
                                                float *__restrict__ w_out, int *__restrict__ idx_copy,
                                                const uint64_t *key_lds, const double *score_lds) {
  const int lane = threadIdx.x & 63;
  uint64_t key[ENT];
  uint32_t eid[ENT];
#pragma unroll
  for (int i = 0; i < ENT; ++i) {
    const int e = lane + 64 * i;
    key[i] = e < E ? key_lds[e] : 0;
    eid[i] = e < E ? static_cast<uint32_t>(e) : kRouteNone;
  }
  const uint32_t mine = route_select<ENT>(key, eid, topk);
  const double sc = lane < topk && mine != kRouteNone ? score_lds[mine] : 0.0;
  route_store(mine, sc, t, topk, scale, idx_out, w_out, idx_copy);
}

template <int LDT, int ENT>
__device__ __forceinline__ void route_wg(const void *__restrict__ logits, const float *__restrict__ bias, int t, int E,
                                         int topk, double scale, int *__restrict__ idx_out, float *__restrict__ w_out,
                                         int *__restrict__ idx_copy, uint64_t *key_lds, double *score_lds) {
  route_wg_keys<LDT>(logits, bias, t, E, key_lds, score_lds);
  __syncthreads();
  if (threadIdx.x < 64) route_wg_select<ENT>(t, E, topk, scale, idx_out, w_out, idx_copy, key_lds, score_lds);
}

// experts per lane of the router for E experts: 4, 5, 8 or 16
inline int route_ent(int64_t E) { return E <= 256 ? 4 : E <= 320 ? 5 : E <= 512 ? 8 : 16; }

// Dispatch the router's experts per lane to a template parameter.
#define VYBDQ_DISPATCH_ENT(E, NAME, ...)                                       \
  switch (route_ent(E)) {                                                     \
    case 4: { constexpr int NAME = 4; __VA_ARGS__; } break;                   \
    case 5: { constexpr int NAME = 5; __VA_ARGS__; } break;                   \
    case 8: { constexpr int NAME = 8; __VA_ARGS__; } break;                   \
    default: { constexpr int NAME = 16; __VA_ARGS__; } break;                 \
  }

// At most 64 rows (T * topk <= 64): the same outputs as bucket_tiles from one wave with row i
// (token i / topk, slot i % topk) in lane i, and no LDS counts, scans or barriers: a row's place
// is the number of rows of lower expert ids plus the rows of its own expert before it (so rows
// keep token order inside an expert), and the first row of each expert writes the expert's
// m-tiles after those of the shared expert and of every lower expert id.
__device__ __forceinline__ void bucket_rows_wave(const int *idx_lds, int T, int topk, int BMr, int BMr2, int shared,
                                                 int *__restrict__ pos, int *__restrict__ row_map,
                                                 int4 *__restrict__ tiles, int *__restrict__ ntiles,
                                                 int4 *__restrict__ tiles2, int *__restrict__ ntiles2) {
  const int lane = threadIdx.x & 63;
  const int n = T * topk;
  const int id = lane < n ? idx_lds[lane] : 0x7fffffff;
  int below = 0, before = 0, cnt = 0;
  for (int j = 0; j < n; ++j) {
    const int o = __builtin_amdgcn_readlane(id, j);
    below += o < id;
    cnt += o == id;
    before += o == id && j < lane;
  }
  const bool first = lane < n && before == 0;  // this lane's row starts its expert's range
  const int mt = first ? (cnt + BMr - 1) / BMr : 0, mt2 = first ? (cnt + BMr2 - 1) / BMr2 : 0;
  const int tsh = shared ? (T + BMr - 1) / BMr : 0, tsh2 = shared ? (T + BMr2 - 1) / BMr2 : 0;
  int t = tsh, t2 = tsh2, tot = tsh, tot2 = tsh2;
  for (int j = 0; j < n; ++j) {
    const int o = __builtin_amdgcn_readlane(id, j);
    const int m = __builtin_amdgcn_readlane(mt, j), m2 = __builtin_amdgcn_readlane(mt2, j);
    if (o < id) { t += m; t2 += m2; }
    tot += m;
    tot2 += m2;
  }
  if (lane < n) {
    pos[lane] = below + before;
    row_map[below + before] = lane / topk;
  }
  for (int m = 0; m < mt; ++m) tiles[t + m] = make_int4(id, below, below + cnt, m);
  if (tiles2)
    for (int m = 0; m < mt2; ++m)
      tiles2[t2 + m] = make_int4(id, below + m * BMr2, below + (cnt < (m + 1) * BMr2 ? cnt : (m + 1) * BMr2), 0);
  if (lane == 0) {
    *ntiles = tot;
    if (ntiles2) *ntiles2 = tot2;
  }
  for (int j = lane; j < tsh; j += 64) tiles[j] = make_int4(-1, n, n + T, j);
  if (tiles2)
    for (int j = lane; j < tsh2; j += 64)
      tiles2[j] = make_int4(-1, n + j * BMr2, n + (T < (j + 1) * BMr2 ? T : (j + 1) * BMr2), 0);
  if (shared)
    for (int i = lane; i < T; i += 64) row_map[n + i] = i;
}

}  // namespace vybdq
