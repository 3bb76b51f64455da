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

}  // namespace

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
