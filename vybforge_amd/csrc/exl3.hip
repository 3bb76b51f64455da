// EXL3 4-bpw trellis decode, full dequant and the fused GEMM (batch 1..16), gfx950.
//
// Format (native/exl3/README.md:24-49, native/exl3/exl3_ref.py:1-120): W [K, N] stored as
// 16x16 tiles, trellis uint16 [K/16][N/16][64] (256 nibbles per tile, LSB-first), suh fp16 [K],
// svh fp16 [N]. Tile slot (r, c) takes a 16-bit window of the tile's nibble stream through the
// tile-slot composition table and decodes it with the mcg codebook hash (exllamav3's
// decode_3inst at cb=1, the only codebook the reference implements: native/exl3/exl3_ref.py:19-22,
// native/kernels/exl3.vyb:15-19):
//   x = w * 0xCBAC1FED (mod 2^32);  y = (x & 0x8FFF8FFF) ^ 0x3B603B60;
//   value = fp16(fp16(y.lo) + fp16(y.hi))
// Both halves of y always lie in [0.125, 2), so their float32 sum is exact and one fp16 add
// (round to nearest even) equals the reference's float32-sum-then-round.
// W = diag(suh) (H/sqrt(128)) What (H/sqrt(128)) diag(svh) per 128x128 block, H = Sylvester
// Hadamard-128, so x W = FWHT(FWHT(x * suh)/sqrt(128) What)/sqrt(128) * svh per 128 chunk.
//
// Lane decomposition (exl3_slots.inc, generated and checked by gen_exl3_slots.py): 8 lanes share
// a tile; lane j owns columns j and j+8 (32 values), loads the tile's 16-byte chunk j (stream
// dwords 4j..4j+3) and takes dword 4j-1 from its neighbour by a shuffle; every window is one or
// two constant-offset funnel extracts of those 5 dwords. A wave covers 8 consecutive tiles along
// N (one 128-column Hadamard block) and reads 1 KB of contiguous trellis per step.
#include "exl3_dev.h"

#include <cstdlib>

namespace vybdq {

// LDS of the fused GEMM: the x' stage of a split (fp16, duplicated (x, x) pairs for batch <= 2),
// then for batches of 4..16 one kExl3WtBytes tile per wave. The per-wave partials
// [4 waves][BP rows][kExl3RedStride floats] reuse the stage after the loop (4 floats of padding
// per row put the 16-column groups of 4 batch rows on different banks).
constexpr int kExl3RedStride = 132;
// one launch (x rotation per workgroup, output rotation by the last split) up to batch 2; at
// batch 4..16 the per-workgroup rotation of every batch row costs more than the two extra
// launches (batch 16 measured 39 us with k_exl3_xprep / k_exl3_out, 68 us in one launch)
__host__ __device__ constexpr bool exl3_fused(int BP) { return BP <= 2; }
__host__ __device__ constexpr size_t exl3_xs_bytes(int BP, int kbs) {
  return BP <= 2 ? static_cast<size_t>(BP) * 16 * kbs * 4 : static_cast<size_t>(BP) * (16 * kbs + 8) * 2;
}
static size_t exl3_lds_bytes(int BP, int kbs) {
  const size_t main = exl3_xs_bytes(BP, kbs) + (BP >= 4 ? static_cast<size_t>(4) * kExl3WtBytes : 0);
  const size_t red = static_cast<size_t>(4) * BP * kExl3RedStride * 4;
  return main > red ? main : red;
}

// ---- decode-only: rotated basis What [K, N] ------------------------------------------------

template <int ODT>
__global__ void __launch_bounds__(256) k_exl3_decode(const uint16_t *__restrict__ trellis, void *__restrict__ out,
                                                     int64_t ntiles, int NB) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t tile = g >> 3;
  const int j = static_cast<int>(g & 7);
  const int64_t safe = tile < ntiles ? tile : 0;  // every lane joins the shuffle
  uint32_t w[6];
  lane_window(trellis, safe, j, w);
  _Float16 v[32];
  lane_decode(w, v);
  if (tile >= ntiles) return;
  const int64_t kb = tile / NB, nb = tile % NB;
  const int64_t N = static_cast<int64_t>(NB) * 16;
#pragma unroll
  for (int q = 0; q < 32; ++q) {
    const int64_t r = 16 * kb + (q & 15);
    const int64_t c = 16 * nb + j + (q >> 4) * 8;
    store_elem<ODT>(out, nullptr, r * N + c, static_cast<float>(v[q]));
  }
}

// ---- full dequant: W [K, N] = diag(suh) Hs What Hs diag(svh) -------------------------------
// One workgroup per 128x128 block: decode the 64 tiles into LDS (float, rows padded to 129),
// FWHT every row, then every column, scale, store.

template <int ODT>
__global__ void __launch_bounds__(256) k_exl3_dequant(const uint16_t *__restrict__ trellis,
                                                      const _Float16 *__restrict__ suh,
                                                      const _Float16 *__restrict__ svh, void *__restrict__ out,
                                                      int NB) {
  extern __shared__ float blk[];  // [128][129]
  const int bk = blockIdx.y, bn = blockIdx.x;
  const int64_t N = static_cast<int64_t>(NB) * 16;
  for (int task = threadIdx.x; task < 512; task += blockDim.x) {  // 64 tiles x 8 lanes
    const int tl = task >> 3, j = task & 7;
    const int tk = tl >> 3, tn = tl & 7;
    const int64_t tile = static_cast<int64_t>(8 * bk + tk) * NB + (8 * bn + tn);
    uint32_t w[6];
    lane_window(trellis, tile, j, w);
    _Float16 v[32];
    lane_decode(w, v);
#pragma unroll
    for (int q = 0; q < 32; ++q)
      blk[(16 * tk + (q & 15)) * 129 + 16 * tn + j + (q >> 4) * 8] = static_cast<float>(v[q]);
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int row = wave; row < 128; row += 4) {  // column transform: What_row . Hs
    float a0 = blk[row * 129 + 2 * lane], a1 = blk[row * 129 + 2 * lane + 1];
    fwht128_wave(a0, a1);
    blk[row * 129 + 2 * lane] = a0 * kRScale;
    blk[row * 129 + 2 * lane + 1] = a1 * kRScale;
  }
  __syncthreads();
  for (int col = wave; col < 128; col += 4) {  // row transform: Hs . (.)
    float a0 = blk[(2 * lane) * 129 + col], a1 = blk[(2 * lane + 1) * 129 + col];
    fwht128_wave(a0, a1);
    const float sv = static_cast<float>(svh[128 * bn + col]);
    const int64_t r0 = 128 * static_cast<int64_t>(bk) + 2 * lane;
    store_elem<ODT>(out, nullptr, r0 * N + 128 * bn + col, a0 * kRScale * static_cast<float>(suh[r0]) * sv);
    store_elem<ODT>(out, nullptr, (r0 + 1) * N + 128 * bn + col,
                    a1 * kRScale * static_cast<float>(suh[r0 + 1]) * sv);
  }
}

// ---- fused GEMM ------------------------------------------------------------------------------
// grid (N/128 column blocks, S k-splits), 4 waves per workgroup; a split's k-range is whole 128
// chunks.
// 1. x' [BP][k-range] = FWHT(x * suh) / sqrt(128) per 128 chunk. Batch <= 2: computed by the
//    GEMM workgroup itself for its k-range, in LDS; larger batches: by k_exl3_xprep into the
//    workspace (a workgroup would otherwise rotate BP chunks per wave before its first weight).
// 2. z[b][n] over the split's k-range = sum x'[b][k] What[k][n]: each wave a quarter of the
//    k-range on the block's 128 columns, the waves' partials summed in LDS in a fixed order.
// 3. y[b][n] = svh[n] * FWHT(sum_s z_s[b][.]) / sqrt(128), sums in split order. Batch <= 2: the
//    last split of a column block to arrive (a per-block arrival counter, reset by that last
//    arrival so the counters stay zero between calls) does it; larger batches: k_exl3_out.
//    The single-launch form publishes the partials with device-coherent stores (written
//    through the XCD's L2) that have completed (s_waitcnt vmcnt(0)) before the arrival is
//    counted, and the last arrival reads them with device-coherent loads issued after the
//    count has returned. An agent-scope release/acquire pair around the count would instead
//    write back and invalidate whole L2s: measured 17 us more per call at batch 1.

template <int XDT>
__global__ void __launch_bounds__(64) k_exl3_xprep(const void *__restrict__ X, const _Float16 *__restrict__ suh,
                                                   _Float16 *__restrict__ xp, int B, int64_t K) {
  const int chunk = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const int64_t k0 = 128 * static_cast<int64_t>(chunk) + 2 * lane;
  float a0 = 0.f, a1 = 0.f;
  if (b < B) {
    a0 = load_elem<XDT>(X, b * K + k0) * static_cast<float>(suh[k0]);
    a1 = load_elem<XDT>(X, b * K + k0 + 1) * static_cast<float>(suh[k0 + 1]);
  }
  fwht128_wave(a0, a1);
  xp[b * K + k0] = static_cast<_Float16>(a0 * kRScale);
  xp[b * K + k0 + 1] = static_cast<_Float16>(a1 * kRScale);
}

template <int BP>
__global__ void __launch_bounds__(256) k_exl3_gemm(const uint16_t *__restrict__ trellis, const void *__restrict__ X,
                                                   int xdt, const _Float16 *__restrict__ suh,
                                                   const _Float16 *__restrict__ svh, void *__restrict__ Y, int ydt,
                                                   int B, const _Float16 *__restrict__ xp, float *__restrict__ zpart,
                                                   uint32_t *__restrict__ arrivals, int64_t K, int NB,
                                                   int kb_per_split) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  __shared__ int is_last;
  const int g = blockIdx.x, s = blockIdx.y, S = gridDim.y;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)), lane = threadIdx.x & 63;
  const int t = lane >> 3, j = lane & 7;
  const int KB = static_cast<int>(K / 16);
  const int kb_begin = s * kb_per_split;
  const int kb_end = min(kb_begin + kb_per_split, KB);
  const int nkb = kb_end - kb_begin;
  // Small batches dot the two fp16 halves of each decoded value with (x, x) (one v_dot2 per weight
  // and batch row: x lo + x hi, the float32 sum the fp16 value rounds), which saves the half add
  // and the pairing of decoded values; x' is staged duplicated for that. Larger batches round
  // the value to fp16 once and share it across the batch rows.
  constexpr bool HALVES = BP <= 2;
  constexpr bool FUSED = exl3_fused(BP);  // x rotation and output rotation in this launch
  // Batches of 4..16 multiply on the matrix cores: each wave writes its decoded values of two
  // k-blocks into its own LDS tile [128 columns][32 k] (column stride kExl3WtStride bytes), then
  // runs one v_mfma_f32_16x16x32_f16 per 16-column fragment with the x' rows as the A operand
  // (rows past the batch read as zero). The VALU keeps only the decode.
  constexpr bool MMA = BP >= 4;
  // This wave's k-blocks and the first kD of its trellis chunks, loaded before anything else (they
  // do not depend on x); the loop keeps kD chunks in flight per lane (a register ring).
  constexpr int kD = 4;
  const int per_wave = (nkb + 3) / 4;
  const int w_begin = wave * per_wave;
  const int w_end = min(w_begin + per_wave, nkb);
  const int64_t nb = 8 * static_cast<int64_t>(g) + t;
  auto load_chunk = [&](int kk) {
    const int kc = kk < w_end ? kk : (w_end > w_begin ? w_end - 1 : 0);  // in range: re-read the last
    const int64_t tile = static_cast<int64_t>(kb_begin + kc) * NB + nb;
    return *reinterpret_cast<const u4 *>(trellis + tile * 64 + 8 * j);
  };
  // 1. x' rows of this split: [BP][16 * nkb] fp16 (HALVES: u32 pairs (x, x))
  const int rows = 16 * nkb;
  // x' row stride of the stage (elements): the matrix-core A reads take 16 batch rows at once,
  // so their rows are 16 B apart in the banks (a stride of whole 128-B lines would put all 16
  // reads on the same banks)
  const int xstride = MMA ? rows + 8 : rows;
  const int nch = nkb / 8;
  // Batch <= 2: each wave rotates the 128-chunks cb = wave, wave + 4, ... of x (batch row cb / nch).
  // The raw x and suh elements of its first kXP chunks are read before the trellis ring: loads
  // return in order, so the rotation then waits for these alone, not for the ring behind them.
  constexpr int kXP = 2;
  // (x elements k, k + 1 of the chunk's batch row: two f32 words, or one word of two 16-bit
  // halves; suh k, k + 1 as one word of halves. Kept raw: converting them here would wait.)
  auto x_raw = [&](int cb, uint32_t (&xv)[2], uint32_t &sv) {
    const int b = cb / nch, c = cb - b * nch;
    const int64_t k = 16 * static_cast<int64_t>(kb_begin) + 128 * c + 2 * lane;
    const int64_t i = static_cast<int64_t>(b < B ? b : 0) * K + k;
    if (xdt == VYBDQ_F32) __builtin_memcpy(xv, static_cast<const float *>(X) + i, 8);
    else __builtin_memcpy(xv, static_cast<const uint16_t *>(X) + i, 4);
    __builtin_memcpy(&sv, suh + k, 4);
  };
  uint32_t xw[kXP][2], sw[kXP];
  if constexpr (FUSED) {
#pragma unroll
    for (int it = 0; it < kXP; ++it)
      if (wave + 4 * it < BP * nch) x_raw(wave + 4 * it, xw[it], sw[it]);
  }
  // Batch > 2: the rotated x' rows are copied from the workspace in 16-byte chunks, four per
  // thread at a time; the first four are read before the trellis ring for the same reason.
  const int nc = BP * rows / 8;
  auto xp_chunk = [&](int i) {
    const int b = i / (rows / 8), c = i % (rows / 8);
    return *reinterpret_cast<const u4 *>(xp + b * K + 16 * static_cast<int64_t>(kb_begin) + 8 * c);
  };
  auto xs_store = [&](int i, const u4 v) {
    const int b = i / (rows / 8), c = i % (rows / 8);
    *reinterpret_cast<u4 *>(reinterpret_cast<_Float16 *>(smem) + b * xstride + 8 * c) = v;
  };
  u4 xv4[4];
  if constexpr (!FUSED) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = threadIdx.x + u * blockDim.x;
      if (i < nc) xv4[u] = xp_chunk(i);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  u4 ring[kD];
#pragma unroll
  for (int d = 0; d < kD; ++d) ring[d] = load_chunk(w_begin + d);
  if constexpr (!FUSED) {
    for (int i0 = threadIdx.x;;) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (i0 + u * blockDim.x < nc) xs_store(i0 + u * blockDim.x, xv4[u]);
      i0 += 4 * blockDim.x;
      if (i0 >= nc) break;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (i0 + u * blockDim.x < nc) xv4[u] = xp_chunk(i0 + u * blockDim.x);
    }
  }
  auto rotate = [&](int cb, const uint32_t (&xv)[2], uint32_t sv) {  // one 128-chunk, whole wave
    const int b = cb / nch, c = cb - b * nch;
    const int r = 128 * c + 2 * lane;
    float a0 = 0.f, a1 = 0.f;
    if (b < B) {
      if (xdt == VYBDQ_F32) { a0 = __uint_as_float(xv[0]); a1 = __uint_as_float(xv[1]); }
      else if (xdt == VYBDQ_F16) { a0 = half_bits_to_f32(xv[0] & 0xffffu); a1 = half_bits_to_f32(xv[0] >> 16); }
      else { a0 = __uint_as_float(xv[0] << 16); a1 = __uint_as_float(xv[0] & 0xffff0000u); }
      a0 *= half_bits_to_f32(sv & 0xffffu);
      a1 *= half_bits_to_f32(sv >> 16);
    }
    fwht128_wave(a0, a1);
    const uint32_t h0 = __builtin_bit_cast(uint16_t, static_cast<_Float16>(a0 * kRScale));
    const uint32_t h1 = __builtin_bit_cast(uint16_t, static_cast<_Float16>(a1 * kRScale));
    if constexpr (HALVES) {
      *reinterpret_cast<u2 *>(reinterpret_cast<uint32_t *>(smem) + b * rows + r) = u2{h0 | (h0 << 16), h1 | (h1 << 16)};
    } else {
      *reinterpret_cast<uint32_t *>(reinterpret_cast<_Float16 *>(smem) + b * rows + r) = h0 | (h1 << 16);
    }
  };
  if constexpr (FUSED) {
#pragma unroll
    for (int it = 0; it < kXP; ++it)
      if (wave + 4 * it < BP * nch) rotate(wave + 4 * it, xw[it], sw[it]);
    for (int cb = wave + 4 * kXP; cb < BP * nch; cb += 4) {
      uint32_t xv[2], sv;
      x_raw(cb, xv, sv);
      rotate(cb, xv, sv);
    }
  }
  __syncthreads();
  const _Float16 *xs = reinterpret_cast<const _Float16 *>(smem);

  // 2. this split's partial
  float acc[BP][2];
#pragma unroll
  for (int b = 0; b < BP; ++b) acc[b][0] = acc[b][1] = 0.f;
  f4 accm[MMA ? 8 : 1];
#pragma unroll
  for (int f = 0; f < (MMA ? 8 : 1); ++f) accm[f] = f4{0.f, 0.f, 0.f, 0.f};
  char *wt = smem + exl3_xs_bytes(BP, kb_per_split) + static_cast<size_t>(wave) * kExl3WtBytes;
  auto step = [&](int kk, const u4 c) {
    uint32_t w[6];
    chunk_window(c, w);
    if constexpr (HALVES) {
      // the 16 (x, x) pairs of this k-block per batch row: four 16-B LDS reads
      uint32_t xq[BP][16];
#pragma unroll
      for (int b = 0; b < BP; ++b) {
        const u4 *src = reinterpret_cast<const u4 *>(reinterpret_cast<const uint32_t *>(smem) + b * rows + 16 * kk);
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
      return;
    }
    if constexpr (MMA) {
      // The 32 slot words of this k-block as they are: word q holds the two fp16 halves of value q
      // (their sum is the value), q < 16 column c0 at k = 16 kk + q, q >= 16 column c0 + 8. Column
      // c's 16 words in k order make the tile row [c][k' = 2 k + h], and the MFMA with each x'
      // value twice in A adds x lo + x hi in float32: no fp16 add or packing of decoded values.
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
      // A = x'[m][16 kk + 4 g .. + 4], each value twice (k' = 8 g .. + 8); B = the tile
      const int m = lane & 15, gk = lane >> 4;
      u2 xv = u2{0u, 0u};
      if (m < BP) xv = *reinterpret_cast<const u2 *>(xs + m * xstride + 16 * kk + 4 * gk);
      const h8 a = __builtin_bit_cast(h8, u4{__builtin_amdgcn_perm(xv[0], xv[0], 0x01000100u),
                                             __builtin_amdgcn_perm(xv[0], xv[0], 0x03020302u),
                                             __builtin_amdgcn_perm(xv[1], xv[1], 0x01000100u),
                                             __builtin_amdgcn_perm(xv[1], xv[1], 0x03020302u)});
#pragma unroll
      for (int f = 0; f < 8; ++f) {
        const h8 b = *reinterpret_cast<const h8 *>(wt + (16 * f + m) * kExl3WtStride + 16 * gk);
        accm[f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, accm[f], 0, 0, 0);
      }
      return;
    }
    _Float16 v[32];
    lane_decode(w, v);
    h2 pj[8], pj8[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pj[i] = h2{v[2 * i], v[2 * i + 1]};
      pj8[i] = h2{v[16 + 2 * i], v[16 + 2 * i + 1]};
    }
#pragma unroll
    for (int b = 0; b < BP; ++b) {
      const u4 *xr = reinterpret_cast<const u4 *>(xs + b * rows + 16 * kk);
      const u4 x0 = xr[0], x1 = xr[1];
      const uint32_t xw[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const h2 xv = __builtin_bit_cast(h2, xw[i]);
        acc[b][0] = __builtin_amdgcn_fdot2(pj[i], xv, acc[b][0], false);
        acc[b][1] = __builtin_amdgcn_fdot2(pj8[i], xv, acc[b][1], false);
      }
    }
  };
  // Whole groups of kD k-blocks without conditions, each ring slot refilled right after the step
  // that consumed it (into the same registers): the loads stay in flight across groups. (A
  // per-block bound made every slot a merge of two paths, and a refill issued before the step
  // needed a second register set that was copied back at the loop end; both made the compiler
  // wait for every load once per group.) The last (fewer than kD) blocks are already in the ring.
  int k0 = w_begin;
  for (; k0 + kD <= w_end; k0 += kD) {
#pragma unroll
    for (int d = 0; d < kD; ++d) {
      step(k0 + d, ring[d]);
      ring[d] = load_chunk(k0 + d + kD);
      // keeps the refill here: sunk to the end of the group it would leave no load in flight
      // while the group's last step waits for its own
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int d = 0; d < kD - 1; ++d)
    if (k0 + d < w_end) step(k0 + d, ring[d]);
  // reduce the 4 waves (same columns, different k) in a fixed order
  __syncthreads();
  float *red = reinterpret_cast<float *>(smem);  // [4][BP][kExl3RedStride]
  if constexpr (MMA) {
    // accm[f][r] = z[batch 4 (lane >> 4) + r][column 16 f + (lane & 15)]
#pragma unroll
    for (int f = 0; f < 8; ++f)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int b = 4 * (lane >> 4) + r;
        if (b < BP) red[(wave * BP + b) * kExl3RedStride + 16 * f + (lane & 15)] = accm[f][r];
      }
  } else {
    const int c0 = 16 * t + j;  // this lane's columns: c0 and c0 + 8
#pragma unroll
    for (int b = 0; b < BP; ++b) {
      red[(wave * BP + b) * kExl3RedStride + c0] = acc[b][0];
      red[(wave * BP + b) * kExl3RedStride + c0 + 8] = acc[b][1];
    }
  }
  __syncthreads();
  const int64_t N = static_cast<int64_t>(NB) * 16;
  auto zp = [&](int split, int b, int c) {
    return reinterpret_cast<uint32_t *>(zpart) + (static_cast<int64_t>(split) * BP + b) * N + 128 * static_cast<int64_t>(g) + c;
  };
  for (int i = threadIdx.x; i < B * 128; i += blockDim.x) {
    const int b = i / 128, c = i % 128;
    const float z = ((red[(0 * BP + b) * kExl3RedStride + c] + red[(1 * BP + b) * kExl3RedStride + c]) +
                     red[(2 * BP + b) * kExl3RedStride + c]) + red[(3 * BP + b) * kExl3RedStride + c];
    if constexpr (FUSED) __hip_atomic_store(zp(s, b, c), __float_as_uint(z), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *zp(s, b, c) = __float_as_uint(z);
  }
  if constexpr (!FUSED) return;

  // 3. arrival; the last split of the block applies the output rotation
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partials are performed
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(arrivals + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = old == static_cast<uint32_t>(S - 1);
    if (is_last) __hip_atomic_store(arrivals + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!is_last) return;
  for (int b = wave; b < B; b += 4) {
    // the splits' partials (this lane's two columns as one 8-byte word) in groups of 8 independent
    // loads, one round trip per group, added in split order
    float a0 = 0.f, a1 = 0.f;
    for (int s0 = 0; s0 < S; s0 += 8) {
      uint64_t v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (s0 + u < S)
          v[u] = __hip_atomic_load(reinterpret_cast<uint64_t *>(zp(s0 + u, b, 2 * lane)), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (s0 + u < S) {
          a0 += __uint_as_float(static_cast<uint32_t>(v[u]));
          a1 += __uint_as_float(static_cast<uint32_t>(v[u] >> 32));
        }
    }
    fwht128_wave(a0, a1);
    const int64_t n0 = 128 * static_cast<int64_t>(g) + 2 * lane;
    const float y0 = a0 * kRScale * static_cast<float>(svh[n0]);
    const float y1 = a1 * kRScale * static_cast<float>(svh[n0 + 1]);
    if (ydt == VYBDQ_F32) { store_elem<VYBDQ_F32>(Y, nullptr, b * N + n0, y0); store_elem<VYBDQ_F32>(Y, nullptr, b * N + n0 + 1, y1); }
    else if (ydt == VYBDQ_F16) { store_elem<VYBDQ_F16>(Y, nullptr, b * N + n0, y0); store_elem<VYBDQ_F16>(Y, nullptr, b * N + n0 + 1, y1); }
    else { store_elem<VYBDQ_BF16>(Y, nullptr, b * N + n0, y0); store_elem<VYBDQ_BF16>(Y, nullptr, b * N + n0 + 1, y1); }
  }
}

// 3. (batch > 2) y[b][n] = svh[n] * FWHT(sum_s zpart[s][b][.]) / sqrt(128)

template <int YDT>
__global__ void __launch_bounds__(64) k_exl3_out(const float *__restrict__ zpart, const _Float16 *__restrict__ svh,
                                                 void *__restrict__ Y, int BP, int S, int64_t N) {
  const int blk = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const int64_t n0 = 128 * static_cast<int64_t>(blk) + 2 * lane;
  // the splits' partials in groups of 8 independent 8-byte loads, added in split order
  float a0 = 0.f, a1 = 0.f;
  for (int s0 = 0; s0 < S; s0 += 8) {
    f2 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (s0 + u < S) v[u] = *reinterpret_cast<const f2 *>(zpart + (static_cast<int64_t>(s0 + u) * BP + b) * N + n0);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (s0 + u < S) {
        a0 += v[u][0];
        a1 += v[u][1];
      }
  }
  fwht128_wave(a0, a1);
  store_elem<YDT>(Y, nullptr, b * N + n0, a0 * kRScale * static_cast<float>(svh[n0]));
  store_elem<YDT>(Y, nullptr, b * N + n0 + 1, a1 * kRScale * static_cast<float>(svh[n0 + 1]));
}

// ---- host --------------------------------------------------------------------------------

static int exl3_bp(int64_t B) { return B <= 1 ? 1 : B <= 2 ? 2 : B <= 4 ? 4 : B <= 8 ? 8 : 16; }

// K-splits: enough workgroups to fill the chip, bounded so partials stay small; a split's
// k-range is whole 128 chunks (the x rotation is done per chunk inside the GEMM)
struct Exl3Split {
  int S;    // splits
  int kbs;  // 16-row k-blocks per split (a multiple of 8)
};
static Exl3Split exl3_splits(int64_t K, int64_t N, int BP) {
  const int KB = static_cast<int>(K / 16);
  const int64_t groups = N / 128;
  int S;
  if (BP <= 2) {
    // about 24 k-blocks per split (6 per wave), at most ~8 workgroups per CU. Measured, batch 1:
    // K = 5120, N = 17408: 14 splits 20.2-20.9 us against 21.3-22.4 at 7-12; K = 10240: 14
    // splits 37.4 us against 41.0 at 7; K = 2560: 7 splits 13.0 us against 13.7 at 10; K = 17408,
    // N = 5120: 16 splits 24.8 us (12: 23.6, 7: 29.2). Fewer splits leave some CUs a workgroup
    // more than others for longer; more add x rotations and partials.
    S = (KB + 23) / 24;
    const int64_t fill = groups < 2048 ? 2048 / groups : 1;
    if (S > fill) S = static_cast<int>(fill);
  } else {
    // the matrix-core batches (4..16): ~2048 workgroups (K = 5120, N = 17408: batch 4 at 16 splits
    // 1294 against 1194 GB/s at 8; batch 16: 8, 12, 20 and 24 splits 9-11% slower)
    S = static_cast<int>((2048 + groups - 1) / groups);
  }
  if (S > 16) S = 16;
  if (S > KB / 4) S = KB / 4 > 0 ? KB / 4 : 1;
  if (const char *e = tuning_env("VYBDQ_EXL3_SPLITS")) S = atoi(e);  // tuning override
  if (S < 1) S = 1;
  int kbs = (KB + S - 1) / S;
  kbs = (kbs + 7) / 8 * 8;
  return {(KB + kbs - 1) / kbs, kbs};
}

// workspace: per-column-block arrival counters (zero between calls), x' (batch > 2), partials
static int64_t exl3_arrival_bytes(int64_t N) { return ((N / 128 * 4 + 255) / 256) * 256; }
static int64_t exl3_xp_bytes(int BP, int64_t K) { return exl3_fused(BP) ? 0 : ((BP * K * 2 + 255) / 256) * 256; }

static int64_t exl3_ws_bytes(int64_t B, int64_t K, int64_t N) {
  const int BP = exl3_bp(B);
  return exl3_arrival_bytes(N) + exl3_xp_bytes(BP, K) + static_cast<int64_t>(exl3_splits(K, N, BP).S) * BP * N * 4;
}

}  // namespace vybdq

using namespace vybdq;

static int exl3_check(uint64_t trellis, int64_t K, int64_t N, int codebook) {
  VYBDQ_REQUIRE(trellis, VYBDQ_ERR_ARG, "null trellis");
  VYBDQ_REQUIRE(codebook == VYBDQ_EXL3_MCG, VYBDQ_ERR_ARG,
                "unsupported codebook: only mcg (1) is implemented, as in the reference");
  VYBDQ_REQUIRE(K > 0 && N > 0 && K % 16 == 0 && N % 16 == 0, VYBDQ_ERR_SHAPE, "K and N must be positive multiples of 16");
  VYBDQ_REQUIRE((trellis & 15) == 0, VYBDQ_ERR_ALIGN, "trellis must be 16-byte aligned");
  VYBDQ_REQUIRE(N / 16 < (1 << 30) && K / 16 < (1 << 30), VYBDQ_ERR_SHAPE, "too many tiles");
  return VYBDQ_OK;
}

extern "C" int vybdq_exl3_decode_tiles(uint64_t trellis, uint64_t out, int64_t K, int64_t N, int codebook,
                                       int out_dt, uint64_t stream) {
  int rc = exl3_check(trellis, K, N, codebook);
  if (rc) return rc;
  VYBDQ_REQUIRE(out, VYBDQ_ERR_ARG, "null out");
  VYBDQ_REQUIRE(out_dt == VYBDQ_F32 || out_dt == VYBDQ_F16 || out_dt == VYBDQ_F64, VYBDQ_ERR_ARG,
                "out_dt must be F32, F16 or F64");
  const int NB = static_cast<int>(N / 16);
  const int64_t ntiles = (K / 16) * NB;
  const unsigned grid = static_cast<unsigned>((ntiles * 8 + 255) / 256);
  hipStream_t s = as_stream(stream);
  const auto *t = reinterpret_cast<const uint16_t *>(trellis);
  void *o = reinterpret_cast<void *>(out);
#define L(ODT) hipLaunchKernelGGL((k_exl3_decode<ODT>), dim3(grid), dim3(256), 0, s, t, o, ntiles, NB)
  if (out_dt == VYBDQ_F32) L(VYBDQ_F32); else if (out_dt == VYBDQ_F16) L(VYBDQ_F16); else L(VYBDQ_F64);
#undef L
  return check_launch("vybdq_exl3_decode_tiles");
}

extern "C" int vybdq_dequant_exl3(uint64_t trellis, uint64_t suh, uint64_t svh, uint64_t out, int64_t K, int64_t N,
                                  int codebook, int out_dt, uint64_t stream) {
  int rc = exl3_check(trellis, K, N, codebook);
  if (rc) return rc;
  VYBDQ_REQUIRE(suh && svh && out, VYBDQ_ERR_ARG, "null suh, svh or out");
  VYBDQ_REQUIRE(K % 128 == 0 && N % 128 == 0, VYBDQ_ERR_SHAPE, "K and N must be multiples of 128");
  VYBDQ_REQUIRE(out_dt == VYBDQ_F32 || out_dt == VYBDQ_F16 || out_dt == VYBDQ_F64, VYBDQ_ERR_ARG,
                "out_dt must be F32, F16 or F64");
  const int NB = static_cast<int>(N / 16);
  const dim3 grid(static_cast<unsigned>(N / 128), static_cast<unsigned>(K / 128));
  const size_t lds = 128 * 129 * 4;
  hipStream_t s = as_stream(stream);
  const auto *t = reinterpret_cast<const uint16_t *>(trellis);
  const auto *su = reinterpret_cast<const _Float16 *>(suh);
  const auto *sv = reinterpret_cast<const _Float16 *>(svh);
  void *o = reinterpret_cast<void *>(out);
#define L(ODT)                                                                                             \
  do {                                                                                                     \
    static std::atomic<uint64_t> raised{0};                                                                \
    const int rc = ensure_lds_limit(reinterpret_cast<const void *>(&k_exl3_dequant<ODT>),                  \
                                    static_cast<int>(lds), raised, "vybdq_dequant_exl3");                  \
    if (rc) return rc;                                                                                     \
    hipLaunchKernelGGL((k_exl3_dequant<ODT>), grid, dim3(256), lds, s, t, su, sv, o, NB);                 \
  } while (0)
  if (out_dt == VYBDQ_F32) L(VYBDQ_F32); else if (out_dt == VYBDQ_F16) L(VYBDQ_F16); else L(VYBDQ_F64);
#undef L
  return check_launch("vybdq_dequant_exl3");
}

extern "C" int64_t vybdq_exl3_workspace_size(int64_t B, int64_t K, int64_t N) {
  if (B < 1 || B > 16 || K <= 0 || N <= 0 || K % 128 || N % 128) return -1;
  return exl3_ws_bytes(B, K, N);
}

template <int BP>
static void exl3_gemm_launch(const uint16_t *t, const void *X, int xdt, const _Float16 *su, const _Float16 *sv,
                             void *Y, int ydt, int B, const _Float16 *xp, float *zp, uint32_t *arr, int64_t K,
                             int NB, const Exl3Split &sp, hipStream_t s) {
  const size_t lds = exl3_lds_bytes(BP, sp.kbs);  // <= 160 KB, checked by the caller
  if (lds > 64 * 1024) {
    static std::atomic<uint64_t> raised{0};
    if (ensure_lds_limit(reinterpret_cast<const void *>(&k_exl3_gemm<BP>), 160 * 1024, raised, "exl3 gemm"))
      return;  // the launch below then fails and check_launch reports it
  }
  hipLaunchKernelGGL((k_exl3_gemm<BP>), dim3(static_cast<unsigned>(NB / 8), static_cast<unsigned>(sp.S)),
                     dim3(256), lds, s, t, X, xdt, su, sv, Y, ydt, B, xp, zp, arr, K, NB, sp.kbs);
}

extern "C" int vybdq_exl3_gemm(uint64_t trellis, uint64_t suh, uint64_t svh, uint64_t X, uint64_t Y, int64_t B,
                               int64_t K, int64_t N, int codebook, int x_dt, int y_dt, uint64_t ws,
                               int64_t ws_bytes, uint64_t stream) {
  int rc = exl3_check(trellis, K, N, codebook);
  if (rc) return rc;
  VYBDQ_REQUIRE(suh && svh && X && Y, VYBDQ_ERR_ARG, "null suh, svh, X or Y");
  VYBDQ_REQUIRE(B >= 1 && B <= 16, VYBDQ_ERR_SHAPE, "B must be in [1, 16]");
  VYBDQ_REQUIRE(K % 128 == 0 && N % 128 == 0, VYBDQ_ERR_SHAPE, "K and N must be multiples of 128");
  VYBDQ_REQUIRE(dt_valid_in(x_dt), VYBDQ_ERR_ARG, "x_dt must be F32, F16 or BF16");
  VYBDQ_REQUIRE(dt_valid_in(y_dt), VYBDQ_ERR_ARG, "y_dt must be F32, F16 or BF16");
  VYBDQ_REQUIRE(ws && (ws & 255) == 0, VYBDQ_ERR_WORKSPACE, "workspace must be non-null and 256-byte aligned");
  VYBDQ_REQUIRE(ws_bytes >= exl3_ws_bytes(B, K, N), VYBDQ_ERR_WORKSPACE,
                "workspace smaller than vybdq_exl3_workspace_size");
  const int BP = exl3_bp(B);
  const Exl3Split sp = exl3_splits(K, N, BP);
  VYBDQ_REQUIRE(exl3_lds_bytes(BP, sp.kbs) <= 160 * 1024, VYBDQ_ERR_SHAPE,
                "K too large for one split's x' stage in LDS at this batch");
  const int NB = static_cast<int>(N / 16);
  hipStream_t s = as_stream(stream);
  auto *arr = reinterpret_cast<uint32_t *>(ws);
  auto *xp = reinterpret_cast<_Float16 *>(ws + exl3_arrival_bytes(N));
  auto *zp = reinterpret_cast<float *>(ws + exl3_arrival_bytes(N) + exl3_xp_bytes(BP, K));
  const auto *su = reinterpret_cast<const _Float16 *>(suh);
  const auto *sv = reinterpret_cast<const _Float16 *>(svh);
  const auto *t = reinterpret_cast<const uint16_t *>(trellis);
  const void *x = reinterpret_cast<const void *>(X);
  void *y = reinterpret_cast<void *>(Y);
  const int b = static_cast<int>(B);
  if (!exl3_fused(BP)) {
    const dim3 gx(static_cast<unsigned>(K / 128), static_cast<unsigned>(BP));
    VYBDQ_DISPATCH_IN(x_dt, XDT, hipLaunchKernelGGL((k_exl3_xprep<XDT>), gx, dim3(64), 0, s, x, su, xp, b, K));
  }
  switch (BP) {
    case 1: exl3_gemm_launch<1>(t, x, x_dt, su, sv, y, y_dt, b, xp, zp, arr, K, NB, sp, s); break;
    case 2: exl3_gemm_launch<2>(t, x, x_dt, su, sv, y, y_dt, b, xp, zp, arr, K, NB, sp, s); break;
    case 4: exl3_gemm_launch<4>(t, x, x_dt, su, sv, y, y_dt, b, xp, zp, arr, K, NB, sp, s); break;
    case 8: exl3_gemm_launch<8>(t, x, x_dt, su, sv, y, y_dt, b, xp, zp, arr, K, NB, sp, s); break;
    default: exl3_gemm_launch<16>(t, x, x_dt, su, sv, y, y_dt, b, xp, zp, arr, K, NB, sp, s); break;
  }
  if (!exl3_fused(BP)) {
    const dim3 go(static_cast<unsigned>(N / 128), static_cast<unsigned>(B));
    VYBDQ_DISPATCH_IN(y_dt, YDT, hipLaunchKernelGGL((k_exl3_out<YDT>), go, dim3(64), 0, s, zp, sv, y, BP, sp.S, N));
  }
  return check_launch("vybdq_exl3_gemm");
}
