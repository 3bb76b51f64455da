// VYBDQ_PB_EXL3DQ and VYBDQ_PB_EXL3INV: the reference's fused EXL3 decode + column transform
// (exl3dq1, native/kernels/exl3.vyb:258-316; its cooperative form exl3dq1s,
// native/kernels/exl3dq.vyb:1-113) and its inverse-map builder (exl3inv, exl3.vyb:318-333) on
// their own parameter blocks, gfx950.
//
// EXL3DQ block: +0 q (trellis tiles, 128 B per 16x16 tile, tile = (row / 16) (cw / 16) + col / 16)
//   +8 td (16-byte header, then the 256 x 16-byte tile-map body: 4 u16 nibble indices, 4 u8 nibble
//   positions, u16 row, u16 col per slot)  +16 H f32 [128][128]  +24 T f32 (out)  +32 cw
//   +40 inv (u32 [16 x 16]: the slot of each tile position, normally td + 16 + 4096).
// The launch's thread count (grid x block in the reference) is rows x cw, rows a multiple of 128
// (a trailing 64-row half band would address T past rows x cw floats). Element (row, col):
//   w16 = OR_i nibble(tile, nidx_i) << 4 pos_i over the slot inv[(row % 16) 16 + col % 16];
//   y = (w16 * 0xCBAC1FED mod 2^32 & 0x8FFF8FFF) ^ 0x3B603B60; w = f32(fp16(y.lo) + fp16(y.hi))
//   (both halves lie in [0.125, 2), so the f32 sum is exact);
//   T[(row / 128 * cw / 128 + col / 128) 16384 + row % 128 * 128 + d] =
//     sum over c = 0..127 ascending of w(row, col / 128 * 128 + c) * H[c][d]  (f32 fma chain).
// Here one persistent workgroup per CU keeps H (64 KB), the map and its inverse in LDS and walks
// 64-row x 128-column blocks: the block's 32 trellis tiles (4 KB) are staged, each element is
// decoded once into LDS, and every thread then runs the 128-step fma chains of 4 rows x 4 columns.
// A block whose words are out of range (or a map entry outside its tile) is not computed and the
// status word gets kPbBadExl3.
//
// EXL3INV block: +0 td, +8 nbody (the map body's size, 4096); writes inv[row 16 + col] = slot at
// td + 16 + nbody for each of the 256 slots.
//
// The separate stages of the reference's f64 and f32 EXL3 pipelines (exl3.vyb:36-256), each on its
// own block (T = double for the f64 kernels, float for the *32 ones):
//   HGEN (exl3hgen / exl3hgen32): +0 H; H[i][j] = (-1)^popcount(i & j) * T(0.08838834764831845).
//   HAD1 (exl3had1 / exl3had132): +0 W +8 Tmp +16 H +24 cw +32 nbc +40 nblocks; for block
//     = (kb, nb) = (block / nbc, block % nbc): Tmp[block 16384 + b 128 + d] =
//     sum over c = 0..127 ascending of W[(128 kb + b) cw + 128 nb + c] * H[c][d].
//   HAD2 (exl3had2 / exl3had232): +0 Tmp +8 O +16 H +24 suh +32 svh +40 cw +48 nbc +56 nblocks;
//     O[(128 kb + a) cw + 128 nb + d] = (sum over b ascending of H[a][b] * Tmp[block 16384 + b 128
//     + d]) * T(suh[128 kb + a]) * T(svh[128 nb + d]), suh / svh fp16.
//   CVT32 (exl3cvt32): +0 S (f32) +8 D (f64) +16 n; D[i] = S[i].
// The reference runs one thread per output over a 128-tap loop; here a persistent grid keeps H in
// LDS and each thread carries 4 x 4 outputs (fma chains in the same index order). The map-driven
// tile decode exl3deq / exl3deq32 (exl3.vyb:207-242, 375-422), launched with (q, tab, o) rather
// than a block, is vybdq_exl3_deq_map below.
#include "common.h"

namespace vybdq {

namespace {

constexpr uint32_t kPbBadExl3 = 16u;
constexpr int kXRows = 64;          // rows per block
constexpr int kXStride = 129;       // LDS row stride of the decoded block (floats): rows on distinct banks
constexpr int kXThreads = 512;
constexpr size_t kXLds = (128 * 128 + kXRows * kXStride) * 4 + 32 * 128 + 256 * 16 + 256 * 4;

__global__ void __launch_bounds__(kXThreads) k_pbexl3dq(const int64_t *__restrict__ pb, int64_t threads,
                                                       uint32_t *__restrict__ status) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  float *Hs = reinterpret_cast<float *>(lds);                    // [128][128]
  float *Ws = Hs + 128 * 128;                                    // [64][kXStride]
  uint8_t *qs = reinterpret_cast<uint8_t *>(Ws + kXRows * kXStride);  // 32 tiles x 128 B
  uint4 *map = reinterpret_cast<uint4 *>(qs + 32 * 128);         // 256 slots
  uint32_t *inv = reinterpret_cast<uint32_t *>(map + 256);       // 256 positions

  const int64_t Q = pb[0], TD = pb[1], HP = pb[2], TP = pb[3], cw = pb[4], IV = pb[5];
  const int t = threadIdx.x;
  bool ok = Q && TD && HP && TP && IV && ((HP | TP) & 15) == 0 && (TD & 3) == 0 && (IV & 3) == 0 && (Q & 15) == 0 &&
            cw >= 128 && cw % 128 == 0 && cw < (int64_t(1) << 30) && threads > 0 && threads % (cw * 128) == 0;
  if (!ok) {
    if (blockIdx.x == 0 && t == 0)
      __hip_atomic_fetch_or(status, kPbBadExl3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const int64_t rows = threads / cw;
  const int64_t nbc128 = cw / 128, nbc16 = cw / 16;
  const int64_t nblk = rows / kXRows * nbc128;

  // H, the map body and the inverse map, checked while they are staged
  for (int i = t; i < 128 * 128 / 4; i += kXThreads)
    reinterpret_cast<float4 *>(Hs)[i] = gptr<const float4>(HP)[i];
  bool bad = false;
  if (t < 256) {
    const uint8_t *rec = gptr<const uint8_t>(TD) + 16 + 16 * t;
    uint4 m;
    m.x = rec[0] | rec[1] << 8 | rec[2] << 16 | rec[3] << 24;
    m.y = rec[4] | rec[5] << 8 | rec[6] << 16 | rec[7] << 24;
    m.z = rec[8] | rec[9] << 8 | rec[10] << 16 | rec[11] << 24;
    m.w = rec[12] | rec[13] << 8 | rec[14] << 16 | rec[15] << 24;
    bad = (m.x & 0xff00ff00u) || (m.y & 0xff00ff00u) || (m.z & 0xfcfcfcfcu);  // nibble index < 256, pos < 4
    map[t] = m;
    const uint32_t v = gptr<const uint32_t>(IV)[t];
    bad = bad || v >= 256;
    inv[t] = v;
  }
  if (__syncthreads_or(bad)) {
    if (blockIdx.x == 0 && t == 0)
      __hip_atomic_fetch_or(status, kPbBadExl3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }

  const uint8_t *q = gptr<const uint8_t>(Q);
  float *T = gptr<float>(TP);
  const int tx = t & 31, ty = t >> 5;  // columns 4 tx .. 4 tx + 3, rows 4 ty .. 4 ty + 3
  for (int64_t blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
    const int64_t rb = blk / nbc128, nb = blk % nbc128;
    // 4 row bands of 8 consecutive tiles (1 KB each)
    if (t < 256) {
      const int band = t >> 6, part = t & 63;
      const int64_t tile = (rb * 4 + band) * nbc16 + nb * 8;
      reinterpret_cast<uint4 *>(qs)[band * 64 + part] = reinterpret_cast<const uint4 *>(q + tile * 128)[part];
    }
    __syncthreads();
    for (int e = t; e < kXRows * 128; e += kXThreads) {
      const int b = e >> 7, c = e & 127;
      const int slot = inv[(b & 15) * 16 + (c & 15)];
      const uint4 m = map[slot];
      const uint8_t *tq = qs + ((b >> 4) * 8 + (c >> 4)) * 128;
      uint32_t w16 = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t nidx = ((i < 2 ? m.x : m.y) >> (16 * (i & 1))) & 0xffu;
        const uint32_t pos = (m.z >> (8 * i)) & 3u;
        const uint32_t nib = (tq[nidx >> 1] >> (4 * (nidx & 1))) & 15u;
        w16 |= nib << (4 * pos);
      }
      const uint32_t x = w16 * 0xCBAC1FEDu;
      const uint32_t y = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
      const h2 v = __builtin_bit_cast(h2, y);
      Ws[b * kXStride + c] = static_cast<float>(v[0]) + static_cast<float>(v[1]);
    }
    __syncthreads();
    float acc[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int d = 0; d < 4; ++d) acc[r][d] = 0.f;
#pragma unroll 4
    for (int c = 0; c < 128; ++c) {
      const float4 h = *reinterpret_cast<const float4 *>(Hs + c * 128 + 4 * tx);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float wv = Ws[(4 * ty + r) * kXStride + c];
        acc[r][0] = fmaf(wv, h.x, acc[r][0]);
        acc[r][1] = fmaf(wv, h.y, acc[r][1]);
        acc[r][2] = fmaf(wv, h.z, acc[r][2]);
        acc[r][3] = fmaf(wv, h.w, acc[r][3]);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = rb * kXRows + 4 * ty + r;
      const int64_t o = ((row >> 7) * nbc128 + nb) * 16384 + (row & 127) * 128 + 4 * tx;
      *reinterpret_cast<float4 *>(T + o) = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
    }
    __syncthreads();
  }
}

__global__ void __launch_bounds__(256) k_pbexl3inv(const int64_t *__restrict__ pb, uint32_t *__restrict__ status) {
  const int64_t TD = pb[0], nbody = pb[1];
  const bool ok = TD && (TD & 3) == 0 && nbody >= 4096 && nbody % 4 == 0 && nbody < (int64_t(1) << 30);
  if (!ok) {
    if (threadIdx.x == 0)
      __hip_atomic_fetch_or(status, kPbBadExl3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const int slot = threadIdx.x;
  const uint8_t *rec = gptr<const uint8_t>(TD) + 16 + 16 * slot;
  const uint32_t r = rec[12] | rec[13] << 8, c = rec[14] | rec[15] << 8;
  if (r >= 16 || c >= 16) {
    __hip_atomic_fetch_or(status, kPbBadExl3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  gptr<uint32_t>(TD + 16 + nbody)[r * 16 + c] = static_cast<uint32_t>(slot);
}

// ---- exl3hgen / exl3had1 / exl3had2 (f64) and their *32 forms, exl3cvt32 ---------------------

constexpr double kHs = 0.08838834764831845;  // 1 / sqrt(128), the reference's constant

template <typename T>
__global__ void __launch_bounds__(256) k_pbhgen(const int64_t *__restrict__ pb, uint32_t *__restrict__ status) {
  const int64_t HP = pb[0];
  if (!HP || (HP & static_cast<int64_t>(sizeof(T) - 1))) {
    if (blockIdx.x == 0 && threadIdx.x == 0)
      __hip_atomic_fetch_or(status, kPbBadExl3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const int gid = blockIdx.x * 256 + threadIdx.x;  // 64 workgroups: the 16384 entries
  const int i = gid >> 7, j = gid & 127;
  const T v = static_cast<T>(kHs);
  gptr<T>(HP)[gid] = (__builtin_popcount(static_cast<unsigned>(i & j)) & 1) ? -v : v;
}

// four consecutive elements from 16-byte aligned memory (global or LDS)
template <typename T>
__device__ __forceinline__ void ld4(const T *p, T (&v)[4]) {
  if constexpr (sizeof(T) == 4) {
    const float4 t = *reinterpret_cast<const float4 *>(p);
    v[0] = t.x, v[1] = t.y, v[2] = t.z, v[3] = t.w;
  } else {
    const double2 a = reinterpret_cast<const double2 *>(p)[0], b = reinterpret_cast<const double2 *>(p)[1];
    v[0] = a.x, v[1] = a.y, v[2] = b.x, v[3] = b.y;
  }
}

template <typename T>
__device__ __forceinline__ void st4(T *p, const T (&v)[4]) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    reinterpret_cast<double2 *>(p)[0] = make_double2(v[0], v[1]);
    reinterpret_cast<double2 *>(p)[1] = make_double2(v[2], v[3]);
  }
}

constexpr int kHadThreads = 512;  // 16 x 32 threads, 4 x 4 outputs each: 64 rows per pass

__device__ __forceinline__ float fma_t(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fma_t(double a, double b, double c) { return __builtin_fma(a, b, c); }

__device__ __forceinline__ float half_to(uint16_t h, float) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }
__device__ __forceinline__ double half_to(uint16_t h, double) {
  return static_cast<double>(__builtin_bit_cast(_Float16, h));
}

// ROW = false: HAD1 (X = W, the column transform X_blk H); ROW = true: HAD2 (H X_blk, X = Tmp,
// then the suh / svh scales). H lives in LDS; X streams from global memory, four elements per load
// along the summed index, so each thread's 16 chains advance in lockstep over it.
template <typename T, bool ROW>
__global__ void __launch_bounds__(kHadThreads) k_pbhad(const int64_t *__restrict__ pb, uint32_t *__restrict__ status) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  T *Hs = reinterpret_cast<T *>(lds);  // [128][128]
  const int64_t XP = pb[0], OP = pb[1], HP = pb[2];
  const int64_t SU = ROW ? pb[3] : 0, SV = ROW ? pb[4] : 0;
  const int64_t cw = pb[ROW ? 5 : 3], nbc = pb[ROW ? 6 : 4], nblocks = pb[ROW ? 7 : 5];
  const bool ok = XP && OP && HP && ((XP | OP | HP) & 15) == 0 && (!ROW || (SU && SV && ((SU | SV) & 1) == 0)) &&
                  nbc >= 1 && cw >= 128 * nbc && cw % (16 / sizeof(T)) == 0 && cw < (int64_t(1) << 40) &&
                  nblocks >= 1 && nblocks < (int64_t(1) << 40);
  if (!ok) {
    if (blockIdx.x == 0 && threadIdx.x == 0)
      __hip_atomic_fetch_or(status, kPbBadExl3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const int t = threadIdx.x;
  for (int i = t; i < 128 * 128 / 4; i += kHadThreads) {
    T v[4];
    ld4(gptr<const T>(HP) + 4 * i, v);
    st4(Hs + 4 * i, v);
  }
  __syncthreads();
  const T *X = gptr<const T>(XP);
  T *O = gptr<T>(OP);
  const int tx = t & 31, ty = t >> 5;  // columns 4 tx .. 4 tx + 3, rows 4 ty .. 4 ty + 3 of a pass
  for (int64_t blk = blockIdx.x; blk < nblocks; blk += gridDim.x) {
    const int64_t kb = blk / nbc, nb = blk - kb * nbc;
#pragma unroll 1
    for (int pass = 0; pass < 2; ++pass) {
      const int r0 = 64 * pass + 4 * ty;
      T acc[4][4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[r][j] = T(0);
      if constexpr (!ROW) {
        // acc[r][j] += W[row r][c] * H[c][4 tx + j], c ascending
        const T *xr = X + (128 * kb + r0) * cw + 128 * nb;
#pragma unroll 2
        for (int c = 0; c < 128; c += 4) {
          T w[4][4], h[4][4];
#pragma unroll
          for (int r = 0; r < 4; ++r) ld4(xr + r * cw + c, w[r]);
#pragma unroll
          for (int k = 0; k < 4; ++k) ld4(Hs + (c + k) * 128 + 4 * tx, h[k]);
#pragma unroll
          for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
              for (int j = 0; j < 4; ++j) acc[r][j] = fma_t(w[r][k], h[k][j], acc[r][j]);
        }
        T *o = O + blk * 16384 + r0 * 128 + 4 * tx;
#pragma unroll
        for (int r = 0; r < 4; ++r) st4(o + r * 128, acc[r]);
      } else {
        // acc[r][j] += H[row r][b] * Tmp[b][4 tx + j], b ascending
        const T *xb = X + blk * 16384 + 4 * tx;
#pragma unroll 2
        for (int b = 0; b < 128; b += 4) {
          T h[4][4], x[4][4];
#pragma unroll
          for (int r = 0; r < 4; ++r) ld4(Hs + (r0 + r) * 128 + b, h[r]);
#pragma unroll
          for (int k = 0; k < 4; ++k) ld4(xb + (b + k) * 128, x[k]);
#pragma unroll
          for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
              for (int j = 0; j < 4; ++j) acc[r][j] = fma_t(h[r][k], x[k][j], acc[r][j]);
        }
        const uint16_t *su = gptr<const uint16_t>(SU), *sv = gptr<const uint16_t>(SV);
        T svc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) svc[j] = half_to(sv[128 * nb + 4 * tx + j], T(0));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t row = 128 * kb + r0 + r;
          const T sur = half_to(su[row], T(0));
          T v[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) v[j] = acc[r][j] * sur * svc[j];
          st4(O + row * cw + 128 * nb + 4 * tx, v);
        }
      }
    }
  }
}

__global__ void __launch_bounds__(256) k_pbcvt32(const int64_t *__restrict__ pb, uint32_t *__restrict__ status) {
  const int64_t SP = pb[0], DP = pb[1], n = pb[2];
  if (!SP || !DP || (SP & 3) || (DP & 7) || n < 0) {
    if (blockIdx.x == 0 && threadIdx.x == 0)
      __hip_atomic_fetch_or(status, kPbBadExl3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const float *S = gptr<const float>(SP);
  double *D = gptr<double>(DP);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
    D[i] = static_cast<double>(S[i]);
}

// exl3deq / exl3deq32: thread t of every workgroup owns slot t of the map (its record read once),
// the workgroups walk the tiles. tab: +0 cw, +8 ntiles, +16 the 256 x 16-byte map body.
template <typename T>
__global__ void __launch_bounds__(256) k_exl3_deq_map(const uint8_t *__restrict__ q, const int64_t *__restrict__ tab,
                                                      T *__restrict__ o, uint32_t *__restrict__ status) {
  const int t = threadIdx.x;
  const int64_t cw = tab[0], ntiles = tab[1];
  const uint32_t *rec = reinterpret_cast<const uint32_t *>(tab + 2) + 4 * t;
  const uint32_t m0 = rec[0], m1 = rec[1], m2 = rec[2], m3 = rec[3];
  const uint32_t r = m3 & 0xffffu, c = m3 >> 16;
  const bool bad = (m0 & 0xff00ff00u) || (m1 & 0xff00ff00u) || (m2 & 0xfcfcfcfcu) || r >= 16 || c >= 16;
  const bool shape_ok = cw >= 16 && cw % 16 == 0 && cw < (int64_t(1) << 40) && ntiles >= 0 && ntiles < (int64_t(1) << 40);
  if (__syncthreads_or(bad || !shape_ok)) {
    if (blockIdx.x == 0 && t == 0)
      __hip_atomic_fetch_or(status, kPbBadExl3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  uint32_t nidx[4], sh[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    nidx[i] = ((i < 2 ? m0 : m1) >> (16 * (i & 1))) & 0xffu;
    sh[i] = 4 * ((m2 >> (8 * i)) & 3u);
  }
  const int64_t nbc = cw / 16;
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const uint8_t *tq = q + tile * 128;
    uint32_t w16 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) w16 |= ((tq[nidx[i] >> 1] >> (4 * (nidx[i] & 1))) & 15u) << sh[i];
    const uint32_t y = ((w16 * 0xCBAC1FEDu) & 0x8FFF8FFFu) ^ 0x3B603B60u;
    const h2 v = __builtin_bit_cast(h2, y);
    // both halves lie in +-[0.125, 2): their float32 sum is exact, so it equals the f64 sum
    const float val = static_cast<float>(v[0]) + static_cast<float>(v[1]);
    const int64_t kb = tile / nbc, nb = tile - kb * nbc;
    o[(16 * kb + r) * cw + 16 * nb + c] = static_cast<T>(val);
  }
}

}  // namespace

int pb_exl3stage_launch(int kind, const int64_t *pb, uint32_t *status, hipStream_t s) {
  const unsigned cus = static_cast<unsigned>(device_cu_count());
  switch (kind) {
    case VYBDQ_PB_EXL3HGEN:
      hipLaunchKernelGGL(k_pbhgen<double>, dim3(64), dim3(256), 0, s, pb, status);
      return check_launch("p-block exl3hgen");
    case VYBDQ_PB_EXL3HGEN32:
      hipLaunchKernelGGL(k_pbhgen<float>, dim3(64), dim3(256), 0, s, pb, status);
      return check_launch("p-block exl3hgen32");
    case VYBDQ_PB_EXL3CVT32:
      hipLaunchKernelGGL(k_pbcvt32, dim3(4 * cus), dim3(256), 0, s, pb, status);
      return check_launch("p-block exl3cvt32");
    default: break;
  }
  static std::atomic<uint64_t> done[4];
  const bool row = kind == VYBDQ_PB_EXL3HAD2 || kind == VYBDQ_PB_EXL3HAD232;
  const bool f64 = kind == VYBDQ_PB_EXL3HAD1 || kind == VYBDQ_PB_EXL3HAD2;
  const void *fn = f64 ? (row ? reinterpret_cast<const void *>(k_pbhad<double, true>)
                              : reinterpret_cast<const void *>(k_pbhad<double, false>))
                       : (row ? reinterpret_cast<const void *>(k_pbhad<float, true>)
                              : reinterpret_cast<const void *>(k_pbhad<float, false>));
  const int lds = 128 * 128 * (f64 ? 8 : 4);
  const int rc = ensure_lds_limit(fn, lds, done[2 * f64 + row], "p-block exl3 Hadamard stage");
  if (rc) return rc;
  if (f64) {
    if (row) hipLaunchKernelGGL((k_pbhad<double, true>), dim3(cus), dim3(kHadThreads), lds, s, pb, status);
    else hipLaunchKernelGGL((k_pbhad<double, false>), dim3(cus), dim3(kHadThreads), lds, s, pb, status);
  } else {
    if (row) hipLaunchKernelGGL((k_pbhad<float, true>), dim3(cus), dim3(kHadThreads), lds, s, pb, status);
    else hipLaunchKernelGGL((k_pbhad<float, false>), dim3(cus), dim3(kHadThreads), lds, s, pb, status);
  }
  return check_launch("p-block exl3 Hadamard stage");
}

int exl3_deq_map_launch(const uint8_t *q, const int64_t *tab, void *o, int out_dt, uint32_t *status, hipStream_t s) {
  const unsigned grid = static_cast<unsigned>(8 * device_cu_count());
  if (out_dt == VYBDQ_F64)
    hipLaunchKernelGGL(k_exl3_deq_map<double>, dim3(grid), dim3(256), 0, s, q, tab, static_cast<double *>(o), status);
  else
    hipLaunchKernelGGL(k_exl3_deq_map<float>, dim3(grid), dim3(256), 0, s, q, tab, static_cast<float *>(o), status);
  return check_launch("exl3 map decode");
}

int pb_exl3dq_launch(const int64_t *pb, int64_t threads, uint32_t *status, hipStream_t s) {
  static std::atomic<uint64_t> lds_done{0};
  const int rc = ensure_lds_limit(reinterpret_cast<const void *>(k_pbexl3dq), static_cast<int>(kXLds), lds_done,
                                  "p-block exl3");
  if (rc) return rc;
  hipLaunchKernelGGL(k_pbexl3dq, dim3(static_cast<unsigned>(device_cu_count())), dim3(kXThreads), kXLds, s, pb,
                     threads, status);
  return check_launch("p-block exl3 decode + column transform");
}

int pb_exl3inv_launch(const int64_t *pb, uint32_t *status, hipStream_t s) {
  hipLaunchKernelGGL(k_pbexl3inv, dim3(1), dim3(256), 0, s, pb, status);
  return check_launch("p-block exl3 inverse map");
}

}  // namespace vybdq
