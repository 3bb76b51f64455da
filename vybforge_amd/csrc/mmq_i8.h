// Prefill GEMM on Q8_0 rows with int8 MFMA against Q8 activations (xq8 layout), gfx950.
//
// Y[m, n] = RS[m, n] + sum_b dx[m, b] * dw[n, b] * sum_{k in block b} xq[m, k] * wq[n, k]
//
// The inner integer sum of one 32-weight block is one v_mfma_i32_16x16x32_i8 (exact, int32): its
// 32 k-slots are the block's 32 elements (lane group g = L >> 4 supplies elements 8g .. 8g+7).
// Every block's int32 tile is converted to float32 and accumulated with the product of its two
// scales, dx[m, b] * dw[n, b] (the xq8 row scale and the Q8_0 block scale): three VALU operations
// per output element per block, which bound this path (the MFMA itself is a small share).
//
// Workgroup = 8 waves (two per SIMD: a single wave issues VALU work at half the SIMD's rate),
// tile = 128 rows x F 16-column fragments: wave (h, n) owns rows 64 h .. 64 h + 63 and quarter n of
// the fragments. Each super-step covers 128 k (4 blocks). Everything the super-step reads is
// brought into LDS by coalesced direct-to-LDS loads, double buffered:
//   - the tile's weight rows: each row's 136-byte span of the super-step, as the 16-byte-aligned
//     144-byte window around it (9 global_load_lds_dwordx4 pieces per row, consecutive lanes on
//     consecutive pieces);
//   - Xq as 16-byte row pieces, 1 KB per (m-fragment, block pair), read back as MFMA fragments;
//   - the four xq8 scales of each row.
// Each lane then reads its 8 quant bytes and the block scale of every (fragment, block) from LDS.
#pragma once
#include "mmq.h"

namespace vybdq {

constexpr int kI8MT = 8;   // 128 rows per tile (4 m-fragments per wave)
constexpr int kI8Threads = 512;
constexpr int kI8NFX = 5;  // up to 20 fragments (320 columns) per tile
constexpr int kI8Pieces = 9;  // 16-byte pieces per row window (144 B)

struct I8Args {
  MmArgs m;            // weights, shape, tiling, output and split-K fields (m.X unused)
  const int8_t *Xq;    // [M][ldq] int8
  const float *Xs;     // [M][lds] float32 block scales
  int64_t ldq;         // bytes between Xq rows
  int64_t lds;         // floats between Xs rows
};

// LDS bytes of one stage for F fragments per tile
__host__ __device__ constexpr int i8_b_bytes(int F) { return ((F * 16 * kI8Pieces + kI8Threads - 1) / kI8Threads) * kI8Threads * 16; }
constexpr int kI8ABytes = kI8MT * 2 * 1024;     // Xq: (m-fragment, block pair) chunks
constexpr int kI8SBytes = kI8MT * 16 * 4 * 4;   // Xs: row x 4 blocks
constexpr int kI8StageBytes = kI8ABytes + kI8SBytes + i8_b_bytes(4 * kI8NFX);
constexpr int kI8JB = i8_b_bytes(4 * kI8NFX) / (kI8Threads * 16);  // weight DMA instructions per thread per super-step

template <int NF>
__device__ __forceinline__ void i8_body(const I8Args &ia, uint8_t *st0, uint8_t *st1, uint32_t *last, int tile, int split,
                                        int row0, int fb, int fb_tile, int s0, int s1) {
  constexpr int MT = kI8MT / 2;  // m-fragments of this wave
  constexpr int NFA = NF > 0 ? NF : 1;
  const MmArgs &a = ia.m;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int mh = w >> 2;  // which 64 rows of the tile
  const int g = lane >> 4, nl = lane & 15;
  const int R = a.F * 16;                    // weight rows of the tile
  const int rows_total = a.N;

  // Direct-to-LDS loads issued from asm: the compiler cannot tell that they never alias the LDS
  // reads of the other stage and would otherwise wait for all of them (vmcnt(0)) before the first
  // LDS read of every super-step. All global traffic of this kernel goes through here, so the
  // waits are explicit: vmcnt(0) before each barrier. M0 carries the wave-uniform LDS base.
  auto dma = [](const void *src, void *dst, auto size) {
    const uint32_t l = __builtin_amdgcn_readfirstlane(
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void *)dst)));
    if constexpr (decltype(size)::value == 16)
      asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(l) : "memory", "m0");
    else
      asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(l) : "memory", "m0");
  };
  using D4 = std::integral_constant<int, 4>;
  using D16 = std::integral_constant<int, 16>;
  // everything super-step s reads, into stage st
  auto issue = [&](int s, uint8_t *st) {
    s = s < s1 ? s : s1 - 1;
    // Xq: instruction (m-fragment i, block pair tp) = 1 KB of LDS: lane l fetches the 16 bytes at
    // k = 128 s + 64 tp + 16 (l / 16) of row 16 i + l % 16 (16 rows x 64 contiguous bytes); the
    // MFMA lane (row r, k-group g) of block t = 2 tp + u later reads 8 bytes at lane l = r + 16 (2u + g / 2),
    // offset 8 (g % 2). Instruction j = w + 4 jj covers (i, tp) = (j / 2, j % 2).
#pragma unroll
    for (int jj = 0; jj < kI8MT * 2 / 8; ++jj) {
      const int j = w + 8 * jj;
      const int i = j >> 1, tp = j & 1;
      int r = row0 + 16 * i + (lane & 15);
      r = r < a.M ? r : a.M - 1;
      const int8_t *src = ia.Xq + static_cast<int64_t>(r) * ia.ldq + 128 * s + 64 * tp + 16 * (lane >> 4);
      dma(src, st + j * 1024, D16{});
    }
    // Xs: [row][the 4 block scales of the super-step]; the even and the odd waves each fetch the same
    // 64 rows (identical bytes to the same place: no branch around the load)
    {
      int r = row0 + 64 * (w & 1) + lane;
      r = r < a.M ? r : a.M - 1;
      dma(ia.Xs + static_cast<int64_t>(r) * ia.lds + 4 * s, st + kI8ABytes + 64 * 16 * (w & 1), D16{});
    }
    // weight rows: piece p = 256 j + tid -> (row p / 9, piece p % 9)
    const int64_t span = (static_cast<int64_t>(s) * 136) & ~static_cast<int64_t>(15);
    // a fixed count (sized for the widest tile; narrower tiles re-read their last piece into the
    // unused part of the stage): a data-dependent trip count here costs the whole loop its registers
#pragma unroll
    for (int j = 0; j < kI8JB; ++j) {
      int p = kI8Threads * j + tid;
      p = p < R * kI8Pieces ? p : R * kI8Pieces - 1;
      int row = fb_tile * 16 + p / kI8Pieces;
      row = row < rows_total ? row : rows_total - 1;
      const uint8_t *src = a.W + static_cast<int64_t>(row) * a.rowbytes + span + 16 * (p % kI8Pieces);
      dma(src, st + kI8ABytes + kI8SBytes + kI8Threads * 16 * j + 64 * 16 * w, D16{});
    }
  };
  auto bar = [] {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
  };

  f4 acc[MT][NFA];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int f = 0; f < NFA; ++f) acc[i][f] = f4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int s, const uint8_t *st) {
    if constexpr (NF > 0) {
      const uint8_t *bq = st + kI8ABytes + kI8SBytes;
      const float *xs = reinterpret_cast<const float *>(st + kI8ABytes);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        // block t of the super-step: fences keep its loads from being hoisted into the previous
        // block's MFMAs and holding registers there
        __builtin_amdgcn_sched_barrier(0);
        long q[NFA];
        float dw[NFA];
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          const int row_l = (fb - fb_tile + f) * 16 + nl;
          const uint8_t *base = bq + row_l * (kI8Pieces * 16) + 8 * (s & 1);  // the span start
          uint32_t lo, hi, dwd;
          if (t % 2 == 0) {
            // block at a 4-aligned offset: quants start 2 bytes into a dword
            const uint32_t *p = reinterpret_cast<const uint32_t *>(base + 34 * t + 8 * g);
            const uint32_t w0 = p[0], w1 = p[1], w2 = p[2];
            lo = __builtin_amdgcn_alignbit(w1, w0, 16);
            hi = __builtin_amdgcn_alignbit(w2, w1, 16);
            dwd = *reinterpret_cast<const uint32_t *>(base + 34 * t) & 0xffffu;
          } else {
            // block at a 2-aligned offset: quants dword-aligned, scale in the high half of the
            // dword before the block
            const uint32_t *p = reinterpret_cast<const uint32_t *>(base + 34 * t + 2 + 8 * g);
            lo = p[0];
            hi = p[1];
            dwd = *reinterpret_cast<const uint32_t *>(base + 34 * t - 2) >> 16;
          }
          q[f] = static_cast<long>((static_cast<uint64_t>(hi) << 32) | lo);
          dw[f] = half_bits_to_f32(dwd);
        }
        typedef int i4 __attribute__((ext_vector_type(4)));
        // A fragment of (i, t): 8 bytes at lane (l % 16) + 16 (2 (t % 2) + g / 2) of chunk (i, t / 2)
        auto a_frag = [&](int i) {
          i += MT * mh;
          return *reinterpret_cast<const long *>(st + (i * 2 + t / 2) * 1024 +
                                                  ((lane & 15) + 16 * (2 * (t & 1) + (g >> 1))) * 16 + 8 * (g & 1));
        };
        auto mfmas = [&](long af, i4 (&c)[NFA]) {
#pragma unroll
          for (int f = 0; f < NF; ++f) c[f] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af, q[f], i4{0, 0, 0, 0}, 0, 0, 0);
        };
        // the MFMAs of m-fragment i + 1 are issued before m-fragment i's results are scaled
        i4 cc[2][NFA];
        mfmas(a_frag(0), cc[0]);
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          if (i + 1 < MT) mfmas(a_frag(i + 1), cc[(i + 1) & 1]);
          // xq8 scales of this lane's 4 output rows (16 i + 4 g + r) for block t
          float dx[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) dx[r] = xs[(16 * (i + MT * mh) + 4 * g + r) * 4 + t];
#pragma unroll
          for (int f = 0; f < NF; ++f)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              acc[i][f][r] = fmaf(static_cast<float>(cc[i & 1][f][r]), dx[r] * dw[f], acc[i][f][r]);
        }
      }
    }
  };

  if (s0 < s1) {
    issue(s0, st0);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  }
  __syncthreads();
  int s = s0;
  for (; s + 2 <= s1; s += 2) {
    issue(s + 1, st1);
    compute(s, st0);
    __builtin_amdgcn_s_waitcnt(0x0f70);
    bar();
    issue(s + 2, st0);
    compute(s + 1, st1);
    __builtin_amdgcn_s_waitcnt(0x0f70);
    bar();
  }
  if (s < s1) compute(s, st0);

  mm_finish<MT, kI8NFX, NF, 8>(a, last, tile, split, row0 + 64 * mh, fb, acc);
}

__global__ void __launch_bounds__(kI8Threads, 1) k_mmq_i8(I8Args ia) {
  __shared__ __attribute__((aligned(16))) uint8_t st0[kI8StageBytes];
  __shared__ __attribute__((aligned(16))) uint8_t st1[kI8StageBytes];
  __shared__ uint32_t last;
  const MmArgs &a = ia.m;
  const int units = a.m_tiles * a.n_tiles * a.splits;
  int id = blockIdx.x;
  if (a.xcd) id = (blockIdx.x & 7) * (units >> 3) + (blockIdx.x >> 3);
  const int mt = id % a.m_tiles;
  const int rest = id / a.m_tiles;
  const int ntile = rest % a.n_tiles;
  const int split = rest / a.n_tiles;
  const int tile = ntile * a.m_tiles + mt;
  const int s0 = split * a.sps;
  const int s1 = s0 + a.sps < a.S ? s0 + a.sps : a.S;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)) & 3;  // N quarter
  const int Fq = a.F >> 2, Fr = a.F & 3;
  const int fb_tile = ntile * a.F;
  const int fb = fb_tile + w * Fq + (w < Fr ? w : Fr);
  int nf = Fq + (w < Fr ? 1 : 0);
  const int left = (a.N >> 4) - fb;
  nf = nf < left ? nf : (left > 0 ? left : 0);
  const int row0 = mt * 16 * kI8MT;
  switch (nf) {
    case 5: i8_body<5>(ia, st0, st1, &last, tile, split, row0, fb, fb_tile, s0, s1); break;
    case 4: i8_body<4>(ia, st0, st1, &last, tile, split, row0, fb, fb_tile, s0, s1); break;
    case 3: i8_body<3>(ia, st0, st1, &last, tile, split, row0, fb, fb_tile, s0, s1); break;
    case 2: i8_body<2>(ia, st0, st1, &last, tile, split, row0, fb, fb_tile, s0, s1); break;
    case 1: i8_body<1>(ia, st0, st1, &last, tile, split, row0, fb, fb_tile, s0, s1); break;
    default: i8_body<0>(ia, st0, st1, &last, tile, split, row0, fb, fb_tile, s0, s1); break;
  }
}

}  // namespace vybdq
