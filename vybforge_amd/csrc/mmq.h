// Prefill dequant GEMM on packed GGUF rows with fp16 MFMA, gfx950, weights dequantized straight
// into MFMA operand registers.
//
// Y[m, n] = RS[m, n] + sum_k X[m, k] * W[n, k]   (W: q4_0 or Q8_0 rows, GGUF row layout)
//
// Workgroup = 4 waves, tile = BM (= 16 MT) rows x F 16-column fragments; the F fragments are
// split among the waves (wave w owns nf_w of them, nf_w = F/4 or F/4 + 1), so a wave's weight
// rows are private to it and never pass through LDS.
//
// K is walked in super-steps of 128 (four 32-weight blocks). The MFMA is
// v_mfma_f32_16x16x32_f16: lane L supplies B[k-slot 8(L>>4) .. +8][n = L & 15]. The k-slots of
// the four MFMAs of a super-step are assigned so that lane group g = L >> 4 covers block g of the
// super-step: in step t (0..3) its 8 slots hold elements 8t .. 8t+7 of block 4s + g. A lane thus
// loads whole blocks (one 20-byte (q4_0) or 36-byte (Q8_0) dword-aligned window per fragment per
// super-step), and only its own block scale applies to it. The A operand (X) uses the same
// k-slot assignment: it is staged into LDS in MFMA fragment order, chunk (m-fragment i, step t)
// = 64 lanes x 8 fp16, so every A fragment read is one conflict-free ds_read_b128 per lane.
//
// Dequantization: a quant byte v becomes the fp16 0x64vv = 1024 + v (v_perm_b32 with a 0x64 byte
// constant), then (h - OFF) is exact in fp16 (a small integer) and the multiply by the block's
// fp16 scale rounds once: the fp16 weight is round(d * q) exactly as in the decode. OFF = 1032
// for q4_0 nibbles (q - 8), 1152 for Q8_0 bytes biased by 128.
//
// Pipelining: each lane keeps D super-steps of weight windows in flight (a register ring),
// prefetches the next super-step's X chunks into registers before the MFMAs, and converts them
// into the other half of a double-buffered LDS tile afterwards; one barrier per super-step.
// Loads past the end of the K range re-read the last super-step, so every path through the loop
// issues the same loads and the waits stay exact.
//
// Split-K: a tile's super-steps may be split among `splits` workgroups. Each stores its f32
// partial tile (in fragment order); a second kernel sums the partials of every output in split
// order (fixed order: deterministic) and runs the epilogue.
#pragma once
#include "gemv_dev.h"
#include <type_traits>

namespace vybdq {

constexpr int kMmMT = 8;    // BM = 128
constexpr int kMmNFX = 5;   // up to 20 fragments (320 columns) per tile, 4 waves
constexpr int kMmNFX8 = 3;  // 8 waves: up to 24 fragments
constexpr int kMmPartFrags = 8 * kMmNFX8 > 4 * kMmNFX ? 8 * kMmNFX8 : 4 * kMmNFX;  // split partial slots per tile

typedef _Float16 hf8 __attribute__((ext_vector_type(8)));

struct MmArgs {
  const uint8_t *W;
  int64_t rowbytes;
  const void *X;
  int64_t ldx;            // elements between X rows
  const int *row_map;     // output row -> X row (null: identity)
  int M, N;
  int S;                  // super-steps (K / 128)
  int F;                  // 16-column fragments per tile
  int m_tiles, n_tiles, splits, sps;  // sps: super-steps per split
  int xcd;                // 1: consecutive units of one XCD share weight rows
  void *Y;
  int ydt;
  int64_t ldy;
  const void *RS;
  float *part;            // split partials [tile][split][waves][NFX][MT][64][4]
  const uint8_t *W2;      // SwiGLU: the up rows (W holds the gate rows, same layout)
  float limit;            // SwiGLU clamp
  const float *xscale;    // per X row: X row r was staged as X / xscale[r] (null: 1); output row m
                          // reads it at r = row_map[m] where a row map is given
};

__device__ __forceinline__ float mm_silu(float g) { return g / (1.0f + __expf(-g)); }

template <int FMT> struct MmFmt;
// D: weight super-steps in flight per lane (the register ring) with 4 waves; D8 with 8 waves
// (half the registers per wave)
template <> struct MmFmt<FMT_Q4_0> {
  static constexpr int BB = 18, WD = 5, D = 4, D8 = 2, SB = 0, HB = 0, QS = 0;
  static constexpr float OFF = 1032.0f;
};
template <> struct MmFmt<FMT_Q8_0> {
  static constexpr int BB = 34, WD = 9, D = 3, D8 = 2, SB = 0, HB = 0, QS = 0;
  static constexpr float OFF = 1152.0f;
};
// Q4_K: 144-byte super-blocks of 256 (d, dmin, 12 scale bytes, 128 nibble bytes); a 128-k super-step
// is half a super-block. A lane's window: the 32 nibble bytes of its sub-block's pair (sub-block
// j = 4 (s & 1) + g: low nibbles of qs[32 (j / 2) ..] for even j, high for odd). The 16-byte
// heads (d, dmin, scales) of the tile's rows go to LDS with the X stage (one direct load per wave
// and step), so the register ring holds only the nibbles.
template <> struct MmFmt<FMT_Q4_K> {
  static constexpr int BB = 0, WD = 8, D = 3, D8 = 2, SB = 144;
  static constexpr int HB = 16, QS = 16;  // bytes of each row's super-block head staged in LDS; nibble start
  static constexpr float OFF = 0.0f;
};
// Q5_K: 176-byte super-blocks (d, dmin, 12 scale bytes, 32 high-bit bytes, 128 nibble bytes): the
// same nibble windows, and the head staged in LDS is 48 bytes (with the high bits: bit j of
// qh[l] is the fifth bit of element l of sub-block j).
template <> struct MmFmt<FMT_Q5_K> {
  static constexpr int BB = 0, WD = 8, D = 3, D8 = 2, SB = 176;
  static constexpr int HB = 48, QS = 48;
  static constexpr float OFF = 0.0f;
};

// Q4_K sub-block j = 4 odd + g of the super-block with head hd: fp16(d * sc) and fp16(dmin * m) (the
// products in float32, get_scale_min_k4), packed as (ds, -dm). Both 6-bit forms are extracted and
// one is selected, so the wave-uniform parity costs no branch.
__device__ __forceinline__ uint32_t q4k_scales(const u4 hd, int g, bool odd) {
  const uint32_t o = 8u * static_cast<uint32_t>(g);
  const uint32_t a0 = __builtin_amdgcn_ubfe(hd[1], o, 6), b0 = __builtin_amdgcn_ubfe(hd[2], o, 6);
  const uint32_t a1 = __builtin_amdgcn_ubfe(hd[3], o, 4) | (__builtin_amdgcn_ubfe(hd[1], o + 6, 2) << 4);
  const uint32_t b1 = __builtin_amdgcn_ubfe(hd[3], o + 4, 4) | (__builtin_amdgcn_ubfe(hd[2], o + 6, 2) << 4);
  const float sc = static_cast<float>(odd ? a1 : a0), mn = static_cast<float>(odd ? b1 : b0);
  return __builtin_bit_cast(uint32_t, h2{static_cast<_Float16>(half_bits_to_f32(hd[0] & 0xffffu) * sc),
                                         static_cast<_Float16>(-(half_bits_to_f32(hd[0] >> 16) * mn))});
}

// The 8 fp16 weights of step t (elements 8t .. 8t+7 of the lane's sub-block; sh = 4 for the high
// nibbles): q exact in fp16 (0x64vv - 1024), then one fp16 fma q * ds - dm. (The decode and the
// super-block GEMM round the float32 value of the same expression once to fp16; this differs from
// it by the fp16 rounding of ds and dm, within one fp16 ulp of the weight's scale.)
// Q5_K: hb2 = the 8 high-bit bytes of the step's elements; bit j of each is the fifth bit.
template <bool Q5>
__device__ __forceinline__ _Float16 __attribute__((ext_vector_type(8))) q4k_step(const uint32_t (&w)[8], int t,
                                                                                 uint32_t sh, uint32_t sd,
                                                                                 u2 hb2 = u2{0u, 0u}, uint32_t j = 0) {
  const h2 v2 = __builtin_bit_cast(h2, sd);
  const h2 ds = {v2[0], v2[0]}, ndm = {v2[1], v2[1]};
  const h2 k1024 = {static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
  _Float16 __attribute__((ext_vector_type(8))) r;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t v = (w[2 * t + h] >> sh) & 0x0F0F0F0Fu;
    if constexpr (Q5) v |= ((hb2[h] >> j) << 4) & 0x10101010u;
    const h2 q0 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(C64, v, SEL_B01)) - k1024;
    const h2 q1 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(C64, v, SEL_B23)) - k1024;
    const h2 p0 = __builtin_elementwise_fma(q0, ds, ndm);
    const h2 p1 = __builtin_elementwise_fma(q1, ds, ndm);
    r[4 * h + 0] = p0[0];
    r[4 * h + 1] = p0[1];
    r[4 * h + 2] = p1[0];
    r[4 * h + 3] = p1[1];
  }
  return r;
}

// a WD-dword window starting at a 4-byte-aligned address
template <int WD>
__device__ __forceinline__ void load_window(const uint8_t *p, uint32_t (&w)[WD]) {
  const u4a4 *v = reinterpret_cast<const u4a4 *>(p);
#pragma unroll
  for (int i = 0; i < WD / 4; ++i) {
    const u4a4 t = v[i];
    w[4 * i + 0] = t[0];
    w[4 * i + 1] = t[1];
    w[4 * i + 2] = t[2];
    w[4 * i + 3] = t[3];
  }
  w[WD - 1] = reinterpret_cast<const uint32_t *>(p)[WD - 1];
}

// The same window as buffer loads: wave-uniform resource (base address in scalar registers) and
// super-step offset `soff`, 32-bit lane offset `voff`; one offset register per lane and fragment,
// where 64-bit lane pointers would take two per fragment plus their update arithmetic.
template <int WD>
__device__ __forceinline__ void load_window_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                                uint32_t (&w)[WD]) {
#pragma unroll
  for (int i = 0; i < WD / 4; ++i) {
    const u4 t = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff + 16 * i), static_cast<int>(soff), 0);
    w[4 * i + 0] = t[0];
    w[4 * i + 1] = t[1];
    w[4 * i + 2] = t[2];
    w[4 * i + 3] = t[3];
  }
  w[WD - 1] = __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(voff + 4 * (WD - 1)), static_cast<int>(soff), 0);
}

// The 8 fp16 weights of step t (elements 8t .. 8t+7 of the lane's block) from its window.
// sel: v_perm selector that extracts the quant dword j from window dwords (j, j+1) (depends on
// whether the block starts 0 or 2 bytes into the window); shd: bit offset of the scale.
template <int FMT>
__device__ __forceinline__ hf8 dequant_step(const uint32_t (&w)[MmFmt<FMT>::WD], int t, uint32_t sel, uint32_t shd) {
  const uint32_t d16 = __builtin_amdgcn_ubfe(w[0], shd, 16);
  const _Float16 d = __builtin_bit_cast(_Float16, static_cast<uint16_t>(d16));
  const h2 dd = {d, d};
  const h2 off = {static_cast<_Float16>(-MmFmt<FMT>::OFF), static_cast<_Float16>(-MmFmt<FMT>::OFF)};
  uint32_t v[2];
  if constexpr (FMT == FMT_Q8_0) {
    // elements 8t .. 8t+7 = quant dwords 2t, 2t+1 (block bytes 2 + 8t ..)
#pragma unroll
    for (int h = 0; h < 2; ++h) v[h] = __builtin_amdgcn_perm(w[2 * t + h + 1], w[2 * t + h], sel) ^ 0x80808080u;
  } else {
    // GGUF order: element j < 16 = low nibble of qs[j], j + 16 = high nibble; step t reads
    // qs dwords 2(t & 1), 2(t & 1) + 1, low nibbles for t < 2, high for t >= 2
    const int j0 = 2 * (t & 1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t q = __builtin_amdgcn_perm(w[j0 + h + 1], w[j0 + h], sel);
      v[h] = (t < 2 ? q : q >> 4) & 0x0F0F0F0Fu;
    }
  }
  hf8 r;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const h2 p0 = (__builtin_bit_cast(h2, __builtin_amdgcn_perm(C64, v[h], SEL_B01)) + off) * dd;
    const h2 p1 = (__builtin_bit_cast(h2, __builtin_amdgcn_perm(C64, v[h], SEL_B23)) + off) * dd;
    r[4 * h + 0] = p0[0];
    r[4 * h + 1] = p0[1];
    r[4 * h + 2] = p1[0];
    r[4 * h + 3] = p1[1];
  }
  return r;
}

// X chunk (8 elements) raw registers and its fp16 conversion
template <int XDT> struct XChunk { u4 r; };
template <> struct XChunk<VYBDQ_F32> { u4 r[2]; };

template <int XDT>
__device__ __forceinline__ void x_load(const void *X, uint32_t off, XChunk<XDT> &c) {
  if constexpr (XDT == VYBDQ_F32) {
    const u4 *p = reinterpret_cast<const u4 *>(static_cast<const float *>(X) + off);
    c.r[0] = p[0];
    c.r[1] = p[1];
  } else {
    c.r = *reinterpret_cast<const u4 *>(static_cast<const uint16_t *>(X) + off);
  }
}

template <int XDT>
__device__ __forceinline__ u4 x_to_f16(const XChunk<XDT> &c) {
  u4 o;
  if constexpr (XDT == VYBDQ_F16) {
    o = c.r;
  } else if constexpr (XDT == VYBDQ_BF16) {
    // bf16 -> fp16 is exact for |x| in the fp16 normal range, so truncation loses nothing there
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t v = c.r[j];
      o[j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(__uint_as_float(v << 16), __uint_as_float(v & 0xffff0000u)));
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u4 &s = c.r[j >> 1];
      const uint32_t a = s[2 * (j & 1)], b = s[2 * (j & 1) + 1];
      o[j] = __builtin_bit_cast(uint32_t, h2{static_cast<_Float16>(__uint_as_float(a)), static_cast<_Float16>(__uint_as_float(b))});
    }
  }
  return o;
}

// LDS: the X tile ring (one array per stage) and the split-K flag
template <int MT>
struct MmLds {
  uint8_t *a[4];
  uint32_t *last;
  uint8_t *h[4];  // Q4_K: the super-block heads of the tile's rows, one stage per X stage
};

// Split-K reduction (when the tile's super-steps were split) and the epilogue store of one wave's
// accumulators acc[i][f][r] = C[row0 + 16 i + 4 g + r][(fb + f) * 16 + nl]; NW waves per workgroup.
// SWI: the wave holds NF gate fragments then the NF up fragments of the same columns, and the
// output is silu(min(g, limit)) * clamp(u, -limit, limit) (no split-K).
template <int MT, int NFX, int NF, int NW = 4, bool SWI = false>
__device__ __forceinline__ void mm_finish(const MmArgs &a, uint32_t *last, int tile, int split, int row0, int fb,
                                          f4 (&acc)[MT][(SWI ? 2 : 1) * NF > 0 ? (SWI ? 2 : 1) * NF : 1]) {
  (void)last;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, nl = lane & 15;
  // ---- split-K: store the partial tile; k_mm_reduce sums the splits in order and stores Y
  if (!SWI && a.splits > 1) {
    constexpr int PER_WAVE = NFX * MT * 64 * 4;  // floats
    float *mine = a.part + ((static_cast<int64_t>(tile) * a.splits + split) * NW + w) * PER_WAVE;
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int i = 0; i < MT; ++i) *reinterpret_cast<f4 *>(mine + ((f * MT + i) * 64 + lane) * 4) = acc[i][f];
    return;
  }

  // ---- epilogue: acc[i][f][r] = C[row0 + 16 i + 4 g + r][(fb + f) * 16 + nl]
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const int64_t n = static_cast<int64_t>(fb + f) * 16 + nl;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = row0 + 16 * i + 4 * g + r;
        if (m >= a.M) continue;
        const int64_t idx = static_cast<int64_t>(m) * a.ldy + n;
        const float xs = a.xscale ? a.xscale[a.row_map ? a.row_map[m] : m] : 1.0f;
        float v = acc[i][f][r] * xs;
        if constexpr (SWI) {
          const float gt = fminf(v, a.limit);
          const float up = fminf(fmaxf(acc[i][NF + f][r] * xs, -a.limit), a.limit);
          v = mm_silu(gt) * up;
        }
        switch (a.ydt) {
          case VYBDQ_F32: store_elem<VYBDQ_F32>(a.Y, a.RS, idx, v); break;
          case VYBDQ_F16: store_elem<VYBDQ_F16>(a.Y, a.RS, idx, v); break;
          case VYBDQ_BF16: store_elem<VYBDQ_BF16>(a.Y, a.RS, idx, v); break;
          default: store_elem<VYBDQ_F64>(a.Y, a.RS, idx, v); break;
        }
      }
  }
}

// Per-wave body for NF owned fragments (NF wave-uniform; NF = 0 waves only stage X). SWI: each
// owned fragment is a pair, gate rows from W and the same up rows from W2 (2 NF B fragments).
template <int FMT, int XDT, int MT, int NFX, int NF, bool SWI = false, int NW = 4>
__device__ __forceinline__ void mm_body(const MmArgs &a, const MmLds<MT> &sm, int tile, int split, int row0, int fb,
                                        int s0, int s1) {
  constexpr int WD = MmFmt<FMT>::WD;
  constexpr int D = NW == 8 ? MmFmt<FMT>::D8 : MmFmt<FMT>::D;
  constexpr int BB = MmFmt<FMT>::BB;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, nl = lane & 15;

  constexpr int NB = (SWI ? 2 : 1) * NF;  // B fragments per step
  // ---- weight windows: lane (nl, g), fragment f -> row (fb + f) * 16 + nl, block 4s + g, read by
  // buffer loads: base = row fb * 16 (wave-uniform resource), super-step offset s * 4 BB (scalar),
  // lane offset (f * 16 + nl) rows + the block's dword-aligned start (NB * 16 rows of a K < 2^25
  // matrix stay below 2^32 bytes). Super-steps past the range re-read the last one.
  // With 4 waves (512 registers per lane) each lane keeps 64-bit row pointers instead.
  // Q4_K / Q5_K (KQ): the lane offset is the row start; the nibble run is placed per step.
  constexpr bool KQ = FMT == FMT_Q4_K || FMT == FMT_Q5_K;
  constexpr int HB = MmFmt<FMT>::HB, HC = HB / 16;  // head bytes per row in LDS, 16-byte loads per row
  static_assert(!KQ || !SWI, "super-block rows: plain GEMM only");
  const int lane_blk = KQ ? 0 : g * BB - 2 * (g & 1);
  uint32_t loff[NB > 0 ? NB : 1];
  const uint8_t *wrow[NB > 0 ? NB : 1];
#pragma unroll
  for (int f = 0; f < NB; ++f) {
    const int fr = f < NF ? f : f - NF;
    loff[f] = static_cast<uint32_t>((fr * 16 + nl) * a.rowbytes) + static_cast<uint32_t>(lane_blk);
    const int64_t n = static_cast<int64_t>(fb + fr) * 16 + nl;
    wrow[f] = (f < NF ? a.W : a.W2) + n * a.rowbytes + lane_blk;
  }
  const uint32_t qg = MmFmt<FMT>::QS + 32 * (g >> 1);  // the lane group's nibble run in a half super-block
  const __amdgpu_buffer_rsrc_t wr0 = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(a.W + static_cast<int64_t>(fb) * 16 * a.rowbytes), 0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t wr1 = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>((SWI ? a.W2 : a.W) + static_cast<int64_t>(fb) * 16 * a.rowbytes), 0, 0x7fffffff, 0x00020000);
  const uint32_t sel = (g & 1) ? 0x07060504u : 0x05040302u;  // quant dword j from (w[j+1], w[j])
  const uint32_t shd = (g & 1) ? 16u : 0u;
  auto wload = [&](int f, int s, uint32_t (&dst)[WD]) {
    s = s < s1 ? s : s1 - 1;
    if constexpr (KQ) {
      // the 32 nibble bytes of half s & 1 of super-block s / 2, lane group g
      const uint32_t qo = static_cast<uint32_t>(s >> 1) * MmFmt<FMT>::SB + 64u * static_cast<uint32_t>(s & 1);
      const u4 q0 = __builtin_amdgcn_raw_buffer_load_b128(wr0, static_cast<int>(loff[f] + qg), static_cast<int>(qo), 0);
      const u4 q1 = __builtin_amdgcn_raw_buffer_load_b128(wr0, static_cast<int>(loff[f] + qg + 16), static_cast<int>(qo), 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dst[i] = q0[i];
        dst[4 + i] = q1[i];
      }
    } else if constexpr (NW == 8) {
      load_window_buf<WD>(f < NF ? wr0 : wr1, loff[f], static_cast<uint32_t>(s) * (4 * BB), dst);
    } else {
      load_window<WD>(wrow[f] + static_cast<int64_t>(s) * (4 * BB), dst);
    }
  };

  // ---- X chunks: the MT x 4 chunks (m-fragment i, step t) of a super-step are split among the
  // NW waves: thread (w, lane) stages chunks (i = ib + j, t = w % 4) for j < XC: row
  // row0 + 16 i + nl, k = 128 s + 32 g + 8 t
  static_assert(NW == 4 || NW == 8, "waves per workgroup");
  constexpr int XC = MT * 4 / NW;
  const int xt = w & 3, ib = (w >> 2) * XC;
  uint32_t xoff[XC];
#pragma unroll
  for (int j = 0; j < XC; ++j) {
    int r = row0 + 16 * (ib + j) + nl;
    r = r < a.M ? r : a.M - 1;
    const int xr = a.row_map ? a.row_map[r] : r;
    xoff[j] = static_cast<uint32_t>(static_cast<int64_t>(xr) * a.ldx) + 32 * g + 8 * xt;
  }
  auto xk = [&](int s) {
    s = s < s1 ? s : s1 - 1;
    return static_cast<uint32_t>(s) * 128u;
  };
  // fp16 X goes straight from global memory into an LDS stage (global_load_lds_dwordx4: lane L
  // of the wave writes chunk base + 16 L, the fragment-order slot of its chunk), NA - 1 stages
  // ahead; other types pass through registers one stage ahead and are converted to fp16 before
  // the LDS store
  constexpr bool DMA = XDT == VYBDQ_F16;
  constexpr int NA = D;  // X stages in LDS (the register path uses them one stage ahead)
  static_assert(D % NA == 0, "ring slot and LDS stage advance together");
  XChunk<XDT> xc[DMA ? 1 : XC];
  auto x_dma = [&](int s, uint8_t *dst) {
    const uint32_t k = xk(s);
    const uint16_t *xb = static_cast<const uint16_t *>(a.X) + k;
#pragma unroll
    for (int j = 0; j < XC; ++j) {
      uint8_t *d = dst + ((ib + j) * 4 + xt) * 1024;
      if constexpr (NW == 8) {
        // two ring stages: the compiler's own bookkeeping of direct-to-LDS loads would drain every
        // load at the loop head, so these are issued untracked (the waits below are explicit)
        lds_dma16_s(xb, 2 * xoff[j], d);
      } else {
        __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1))) *)(xb + xoff[j]),
                                         (void __attribute__((address_space(3))) *)d, 16, 0, 0);
      }
    }
  };
  // Super-block heads: the first HB bytes of each tile row's super-block, row r at r * HB in LDS;
  // 16-byte chunk c = 64 (HC w + i) + lane (load i of wave w) is byte 16 (c % HC) of row c / HC
  // (rows past the tile clamped to its last row)
  static_assert(!KQ || (NW == 8 && DMA), "super-block rows: 8-wave body with fp16 X only");
  const int tile_row0 = KQ ? (tile / a.m_tiles) * a.F * 16 : 0;
  const int tile_rows = KQ ? (a.N - tile_row0 < a.F * 16 ? a.N - tile_row0 : a.F * 16) : 1;
  uint32_t hoff[HC > 0 ? HC : 1];
#pragma unroll
  for (int i = 0; i < HC; ++i) {
    const int c = 64 * (HC * w + i) + lane;
    const int r = c / HC < tile_rows ? c / HC : tile_rows - 1;
    hoff[i] = static_cast<uint32_t>(r * a.rowbytes) + 16u * static_cast<uint32_t>(c % HC);
  }
  const uint8_t *hbase0 = a.W + static_cast<int64_t>(tile_row0) * a.rowbytes;
  auto h_dma = [&](int s, uint8_t *dst) {
    s = s < s1 ? s : s1 - 1;
#pragma unroll
    for (int i = 0; i < HC; ++i)
      lds_dma16_s(hbase0 + static_cast<int64_t>(s >> 1) * MmFmt<FMT>::SB, hoff[i], dst + (HC * w + i) * 1024);
  };
  auto x_regs = [&](int s) {
    const uint32_t k = xk(s);
#pragma unroll
    for (int j = 0; j < XC; ++j) x_load<XDT>(a.X, xoff[j] + k, xc[j]);
  };
  auto x_stage = [&](uint8_t *dst) {
#pragma unroll
    for (int j = 0; j < XC; ++j)
      *reinterpret_cast<u4 *>(dst + (((ib + j) * 4 + xt) * 64 + lane) * 16) = x_to_f16<XDT>(xc[j]);
  };
  // Workgroup barrier without memory fences: each wave has already waited for the memory
  // operations the other waves depend on (its X DMA by vmcnt, its LDS stores by lgkmcnt), and
  // __syncthreads()' release fence would wait for every weight load in flight as well. The empty
  // asm and sched_barriers keep the compiler from moving memory operations across it.
  auto bar = [] {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
  };
  // vmcnt wait that leaves the N most recent loads in flight (expcnt and lgkmcnt not waited)
  auto wait_vm = [](auto n) {
    constexpr int N = decltype(n)::value;
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  };
  constexpr int LPW = KQ ? 2 : WD / 4 + 1;  // load instructions per weight window
  constexpr int XL = XC + HC;               // X-side loads per wave and step (+ the super-block heads)
  // Loads younger than X(s + 1) when step s ends in the steady state: W(s + 2 - NA + D), then per
  // step X(.) and W(.) for the NA - 2 steps after it. Earlier steps have at least as many, so
  // waiting for this many is safe everywhere (it may wait a little longer in the first steps).
  constexpr int YOUNGER = (NA - 2) * (XL + NB * LPW) + NB * LPW;

  f4 acc[MT][NB > 0 ? NB : 1];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int f = 0; f < (NB > 0 ? NB : 1); ++f) acc[i][f] = f4{0.f, 0.f, 0.f, 0.f};

  uint32_t ring[D][NB > 0 ? NB : 1][WD];

  // ---- prologue: X(s0 .. s0 + NA - 2) and weights s0 .. s0 + D - 1, interleaved as the steady
  // state issues them
  if (s0 < s1) {
    if constexpr (DMA) {
#pragma unroll
      for (int j = 0; j < D; ++j) {
        if (j < NA - 1) {
          x_dma(s0 + j, sm.a[j]);
          if constexpr (KQ) h_dma(s0 + j, sm.h[j]);
        }
#pragma unroll
        for (int f = 0; f < NB; ++f) wload(f, s0 + j, ring[j][f]);
        __builtin_amdgcn_sched_barrier(0);
      }
      wait_vm(std::integral_constant<int, (NA - 2) * (XL + NB * LPW) + 2 * NB * LPW < 64
                                              ? (NA - 2) * (XL + NB * LPW) + 2 * NB * LPW : 63>{});
      if constexpr ((NA - 2) * (XL + NB * LPW) + 2 * NB * LPW >= 64) wait_vm(std::integral_constant<int, 0>{});
    } else {
      x_regs(s0);
#pragma unroll
      for (int d = 0; d < D; ++d) {
#pragma unroll
        for (int f = 0; f < NB; ++f) wload(f, s0 + d, ring[d][f]);
        __builtin_amdgcn_sched_barrier(0);
      }
      x_stage(sm.a[0]);
    }
  }
  __syncthreads();

  // MFMAs of one super-step: A fragments of step t + 1 and the B fragment after the current one
  // are produced while the current MFMAs run
  auto compute = [&](const uint32_t (&slot)[NB > 0 ? NB : 1][WD], const uint8_t *abase, const uint8_t *hb, int s) {
    if constexpr (NB > 0) {
      // Q4_K: the lane's sub-block scale and min per fragment, once per super-step, from the
      // row heads staged with this step's X
      uint32_t sd[KQ ? NB : 1];
      const uint32_t jq = 4u * static_cast<uint32_t>(s & 1) + static_cast<uint32_t>(g);  // the lane's sub-block
      if constexpr (KQ) {
        const bool odd = (s & 1) != 0;
#pragma unroll
        for (int f = 0; f < NB; ++f)
          sd[f] = q4k_scales(*reinterpret_cast<const u4 *>(hb + ((fb + f) * 16 + nl - tile_row0) * HB), g, odd);
      }
      const uint32_t nsh = 4u * static_cast<uint32_t>(g & 1);
      auto bstep = [&](int f, int t) {
        if constexpr (FMT == FMT_Q5_K)
          return q4k_step<true>(slot[f], t, nsh, sd[f],
                                *reinterpret_cast<const u2 *>(hb + ((fb + f) * 16 + nl - tile_row0) * HB + 16 + 8 * t), jq);
        else if constexpr (KQ) return q4k_step<false>(slot[f], t, nsh, sd[f]);
        else return dequant_step<FMT>(slot[f], t, sel, shd);
      };
      // ABUF = 2: the A fragments of step t + 1 are read into the other buffer at the start of
      // step t; ABUF = 1 (8 waves, 256 registers per lane): fragment i of step t + 1 is read into
      // af[0][i] right after the last MFMA of step t that reads it
      constexpr int ABUF = NW == 4 ? 2 : 1;
      hf8 af[ABUF][MT];
#pragma unroll
      for (int i = 0; i < MT; ++i) af[0][i] = *reinterpret_cast<const hf8 *>(abase + (i * 4 * 64 + lane) * 16);
      hf8 bcur = bstep(0, 0);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (ABUF == 2 && t < 3) {
#pragma unroll
          for (int i = 0; i < MT; ++i)
            af[(t + 1) % ABUF][i] = *reinterpret_cast<const hf8 *>(abase + ((i * 4 + t + 1) * 64 + lane) * 16);
        }
#pragma unroll
        for (int f = 0; f < NB; ++f) {
          const bool last = t == 3 && f == NB - 1;
          const int fn = f + 1 < NB ? f + 1 : 0;
          const int tn = f + 1 < NB ? t : t + 1;
          hf8 bnext = bcur;
          if (!last) bnext = bstep(fn, tn);
#pragma unroll
          for (int i = 0; i < MT; ++i) {
            acc[i][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t % ABUF][i], bcur, acc[i][f], 0, 0, 0);
            if (ABUF == 1 && t < 3 && f == NB - 1)
              af[0][i] = *reinterpret_cast<const hf8 *>(abase + ((i * 4 + t + 1) * 64 + lane) * 16);
          }
          bcur = bnext;
        }
      }
    }
  };

  // one super-step s from ring slot DC = (s - s0) % D (a compile-time constant; the LDS stage is
  // DC % NA); REFILL issues the weights of s + D into the slot
  auto step = [&](auto dc, auto refill, int s) {
    constexpr int d = decltype(dc)::value;
    if constexpr (DMA) {
      x_dma(s + NA - 1, sm.a[(d + NA - 1) % NA]);
      if constexpr (KQ) h_dma(s + NA - 1, sm.h[(d + NA - 1) % NA]);
    } else {
      x_regs(s + 1);
    }
    __builtin_amdgcn_sched_barrier(0);
    compute(ring[d], sm.a[d % NA], sm.h[d % NA], s);
    if constexpr (decltype(refill)::value) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int f = 0; f < NB; ++f) wload(f, s + D, ring[d][f]);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (DMA) wait_vm(std::integral_constant<int, YOUNGER>{});
    } else {
      if constexpr (DMA) wait_vm(std::integral_constant<int, 0>{});
    }
    if constexpr (!DMA) {
      x_stage(sm.a[(d + 1) % NA]);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the LDS stores are done
    }
    bar();
  };
  using Yes = std::true_type;
  using No = std::false_type;
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  static_assert(D >= 2 && D <= 4, "ring depth");
  int s = s0;
  for (; s + D <= s1; s += D) {
    step(I0{}, Yes{}, s);
    step(I1{}, Yes{}, s + 1);
    if constexpr (D >= 3) step(I2{}, Yes{}, s + 2);
    if constexpr (D >= 4) step(I3{}, Yes{}, s + 3);
  }
  if (s < s1) step(I0{}, No{}, s);
  if (s + 1 < s1) step(I1{}, No{}, s + 1);
  if constexpr (D >= 4) {
    if (s + 2 < s1) step(I2{}, No{}, s + 2);
  }

  mm_finish<MT, NFX, NF, NW, SWI>(a, sm.last, tile, split, row0, fb, acc);
}

// One work unit (m-tile, n-tile, K split) of the GEMM; every wave of the workgroup calls it. The
// tile's F fragments are split among the NW waves (F / NW each, the first F % NW waves one more).
template <int FMT, int XDT, int MT, int NFX, int NW = 4>
__device__ __forceinline__ void mmq_unit(const MmArgs &a, const MmLds<MT> &sm, int id) {
  const int mt = id % a.m_tiles;
  const int rest = id / a.m_tiles;
  const int ntile = rest % a.n_tiles;
  const int split = rest / a.n_tiles;
  const int tile = ntile * a.m_tiles + mt;
  const int s0 = split * a.sps;
  const int s1 = s0 + a.sps < a.S ? s0 + a.sps : a.S;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int Fq = a.F / NW, Fr = a.F % NW;
  const int fb = ntile * a.F + w * Fq + (w < Fr ? w : Fr);
  int nf = Fq + (w < Fr ? 1 : 0);
  const int left = (a.N >> 4) - fb;
  nf = nf < left ? nf : (left > 0 ? left : 0);
  const int row0 = mt * 16 * MT;
  static_assert(NFX <= 5, "fragment variants");
  switch (nf) {
    case 5: if constexpr (NFX >= 5) mm_body<FMT, XDT, MT, NFX, 5, false, NW>(a, sm, tile, split, row0, fb, s0, s1); break;
    case 4: if constexpr (NFX >= 4) mm_body<FMT, XDT, MT, NFX, 4, false, NW>(a, sm, tile, split, row0, fb, s0, s1); break;
    case 3: if constexpr (NFX >= 3) mm_body<FMT, XDT, MT, NFX, 3, false, NW>(a, sm, tile, split, row0, fb, s0, s1); break;
    case 2: mm_body<FMT, XDT, MT, NFX, 2, false, NW>(a, sm, tile, split, row0, fb, s0, s1); break;
    case 1: mm_body<FMT, XDT, MT, NFX, 1, false, NW>(a, sm, tile, split, row0, fb, s0, s1); break;
    default: mm_body<FMT, XDT, MT, NFX, 0, false, NW>(a, sm, tile, split, row0, fb, s0, s1); break;
  }
}

#define VYBDQ_MMQ_LDS(FMT, MT)                                                        \
  constexpr int NA_ = MmFmt<FMT>::D;                                                  \
  __shared__ __attribute__((aligned(16))) uint8_t a0[MT * 4096];                      \
  __shared__ __attribute__((aligned(16))) uint8_t a1[MT * 4096];                      \
  __shared__ __attribute__((aligned(16))) uint8_t a2[NA_ > 2 ? MT * 4096 : 16];       \
  __shared__ __attribute__((aligned(16))) uint8_t a3[NA_ > 3 ? MT * 4096 : 16];       \
  __shared__ uint32_t last;                                                           \
  constexpr int NH_ = MmFmt<FMT>::HB > 0 ? 512 * MmFmt<FMT>::HB : 16;                \
  __shared__ __attribute__((aligned(16))) uint8_t h0[NH_];                            \
  __shared__ __attribute__((aligned(16))) uint8_t h1[NH_];                            \
  __shared__ __attribute__((aligned(16))) uint8_t h2_[NA_ > 2 ? NH_ : 16];            \
  __shared__ __attribute__((aligned(16))) uint8_t h3[NA_ > 3 ? NH_ : 16];             \
  const MmLds<MT> sm{{a0, a1, a2, a3}, &last, {h0, h1, h2_, h3}}

template <int FMT, int XDT, int MT, int NFX, int NW = 4>
__global__ void __launch_bounds__(64 * NW, 1) k_mmq(MmArgs a) {
  VYBDQ_MMQ_LDS(FMT, MT);
  const int units = a.m_tiles * a.n_tiles * a.splits;
  int id = blockIdx.x;
  if (a.xcd) id = (blockIdx.x & 7) * (units >> 3) + (blockIdx.x >> 3);
  mmq_unit<FMT, XDT, MT, NFX, NW>(a, sm, id);
}

// Split-K reduction: Y = RS + sum over splits (in split order) of the partial tiles, one float4
// (4 rows of one column) per thread. Partial layout [tile][split][wave][fragment][m-fragment]
// [lane][4]; NW waves per workgroup, MT m-fragments per wave, MH = 2 when waves w and w + 4 own the
// two 64-row halves of the tile (int8 path), 1 when every wave owns all the tile's rows.
template <int NW, int MT, int NFX, int MH>
__global__ void __launch_bounds__(256) k_mm_reduce(MmArgs a) {
  constexpr int PER_WAVE = NFX * MT * 64 * 4;
  constexpr int CHUNKS = NW * NFX * MT * 64;  // float4 per tile
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int tile = static_cast<int>(c / CHUNKS);
  if (tile >= a.m_tiles * a.n_tiles) return;
  int e = static_cast<int>(c % CHUNKS);
  const int lane = e & 63;
  e >>= 6;
  const int i = e % MT;
  e /= MT;
  const int f = e % NFX;
  const int w = e / NFX;
  const int mt = tile % a.m_tiles, ntile = tile / a.m_tiles;
  constexpr int NQ = NW / MH;  // fragment groups
  const int q = w % NQ;         // fragment group of this wave
  const int mh = w / NQ;
  const int Fq = a.F / NQ, Fr = a.F % NQ;
  const int fb = ntile * a.F + q * Fq + (q < Fr ? q : Fr);
  int nf = Fq + (q < Fr ? 1 : 0);
  const int left = (a.N >> 4) - fb;
  nf = nf < left ? nf : (left > 0 ? left : 0);
  if (f >= nf) return;
  const float *p = a.part + (static_cast<int64_t>(tile) * a.splits * NW + w) * PER_WAVE + ((f * MT + i) * 64 + lane) * 4;
  f4 tot = *reinterpret_cast<const f4 *>(p);
  for (int j = 1; j < a.splits; ++j) tot += *reinterpret_cast<const f4 *>(p + static_cast<int64_t>(j) * NW * PER_WAVE);
  const int64_t n = static_cast<int64_t>(fb + f) * 16 + (lane & 15);
  const int row0 = mt * 16 * MT * MH + mh * 16 * MT + 16 * i + 4 * (lane >> 4);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = row0 + r;
    if (m >= a.M) continue;
    const int64_t idx = static_cast<int64_t>(m) * a.ldy + n;
    const float v = a.xscale ? tot[r] * a.xscale[a.row_map ? a.row_map[m] : m] : tot[r];
    switch (a.ydt) {
      case VYBDQ_F32: store_elem<VYBDQ_F32>(a.Y, a.RS, idx, v); break;
      case VYBDQ_F16: store_elem<VYBDQ_F16>(a.Y, a.RS, idx, v); break;
      case VYBDQ_BF16: store_elem<VYBDQ_BF16>(a.Y, a.RS, idx, v); break;
      default: store_elem<VYBDQ_F64>(a.Y, a.RS, idx, v); break;
    }
  }
}

template <int NW, int MT, int NFX, int MH>
int mm_reduce_launch(const MmArgs &a, hipStream_t s) {
  if (a.splits <= 1) return VYBDQ_OK;
  const int64_t chunks = static_cast<int64_t>(a.m_tiles) * a.n_tiles * NW * NFX * MT * 64;
  hipLaunchKernelGGL((k_mm_reduce<NW, MT, NFX, MH>), dim3(static_cast<unsigned>((chunks + 255) / 256)), dim3(256), 0, s, a);
  return check_launch("mmq split-K reduce");
}

// X [M][K] (f32 or bf16, 16-byte aligned, K % 8 == 0) -> xh [M][K] fp16 and xscale[M], one
// workgroup per row (mmq_host.hip)
// One row of X (K elements, bf16 or f32) -> fp16 with a power-of-two scale that brings the row's
// largest |x| into [2^14, 2^15), and that scale (the body of x_rows_to_f16; 256 threads, wmax: 4
// floats of LDS). CH > 0: the row (at most 256 CH chunks of 8) is loaded once into registers, all
// loads issued before the first use; CH = 0: two passes over the row (any K).
template <int XDT, int CH>
__device__ __forceinline__ void x_row_to_f16(const void *__restrict__ X, u4 *__restrict__ Xh,
                                             float *__restrict__ xscale, int64_t K, int64_t row, float *wmax) {
  const int64_t n8 = K / 8;
  // the row's base in 64-bit arithmetic (M * K may exceed 2^32 elements); offsets inside the row
  // are 32-bit (every caller bounds K below 2^24)
  const void *Xr = static_cast<const char *>(X) + row * K * (XDT == VYBDQ_F32 ? 4 : 2);
  auto chunk_max = [](const XChunk<XDT> &c, float m) {
    if constexpr (XDT == VYBDQ_F32) {
#pragma unroll
      for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(__uint_as_float(c.r[j >> 2][j & 3])));
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t v = c.r[j];
        m = fmaxf(m, fmaxf(fabsf(__uint_as_float(v << 16)), fabsf(__uint_as_float(v & 0xffff0000u))));
      }
    }
    return m;
  };
  auto chunk_f16 = [](const XChunk<XDT> &c, float inv) {
    u4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float a, b;
      if constexpr (XDT == VYBDQ_F32) {
        a = __uint_as_float(c.r[j >> 1][2 * (j & 1)]);
        b = __uint_as_float(c.r[j >> 1][2 * (j & 1) + 1]);
      } else {
        a = __uint_as_float(c.r[j] << 16);
        b = __uint_as_float(c.r[j] & 0xffff0000u);
      }
      o[j] = __builtin_bit_cast(uint32_t, h2{static_cast<_Float16>(a * inv), static_cast<_Float16>(b * inv)});
    }
    return o;
  };
  float amax = 0.f;
  XChunk<XDT> cc[CH > 0 ? CH : 1];
  if constexpr (CH > 0) {
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int64_t i = threadIdx.x + 256 * j;
      if (i < n8) x_load<XDT>(Xr, static_cast<uint32_t>(i * 8), cc[j]);
    }
#pragma unroll
    for (int j = 0; j < CH; ++j)
      if (threadIdx.x + 256 * j < n8) amax = chunk_max(cc[j], amax);
  } else {
    for (int64_t i = threadIdx.x; i < n8; i += 256) {
      XChunk<XDT> c;
      x_load<XDT>(Xr, static_cast<uint32_t>(i * 8), c);
      amax = chunk_max(c, amax);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  float inv;
  const float scale = block_scale(amax, inv);
  if (threadIdx.x == 0) xscale[row] = scale;
  if constexpr (CH > 0) {
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int64_t i = threadIdx.x + 256 * j;
      if (i < n8) Xh[row * n8 + i] = chunk_f16(cc[j], inv);
    }
  } else {
    for (int64_t i = threadIdx.x; i < n8; i += 256) {
      XChunk<XDT> c;
      x_load<XDT>(Xr, static_cast<uint32_t>(i * 8), c);
      Xh[row * n8 + i] = chunk_f16(c, inv);
    }
  }
}

// chunks of 8 per thread of a 256-thread row conversion; CH = 2, 4, 8, 12 when it is at most that, else 0
inline int x_row_chunks(int64_t K) { return static_cast<int>((K / 8 + 255) / 256); }

int x_rows_to_f16(const void *X, int xdt, int64_t M, int64_t K, void *xh, float *xscale, hipStream_t s);

// fp16 X (streamed into LDS by direct loads): 8 waves per workgroup, two per SIMD, so that one
// wave's dequantization issues while the other's MFMAs run; every wave owns at most kMmNFX8
// fragments (F <= 4 kMmNFX = 8 kMmNFX8 - 4). Other X types: 4 waves (the register X path needs the
// registers of one wave per SIMD).
template <int FMT, int XDT>
int mmq_launch(MmArgs &a, hipStream_t s) {
  const int64_t units = static_cast<int64_t>(a.m_tiles) * a.n_tiles * a.splits;
  a.xcd = units % 8 == 0 ? 1 : 0;
  bool eight = XDT == VYBDQ_F16;
  if (const char *e = tuning_env("VYBDQ_MMQ_WAVES")) eight = eight && e[0] != '4';
  constexpr bool KQ = FMT == FMT_Q4_K || FMT == FMT_Q5_K;
  static_assert(!KQ || XDT == VYBDQ_F16, "super-block rows: fp16 X (the 8-wave body) only");
  if constexpr (XDT == VYBDQ_F16) {
    if (eight || KQ) {
      constexpr int NFX8 = KQ ? 2 : kMmNFX8;  // super-block rows: F <= 16 (the planner's limit)
      hipLaunchKernelGGL((k_mmq<FMT, XDT, kMmMT, NFX8, 8>), dim3(static_cast<unsigned>(units)), dim3(512), 0, s, a);
      const int rc = check_launch("mmq gemm");
      if (rc) return rc;
      return mm_reduce_launch<8, kMmMT, NFX8, 1>(a, s);
    }
  }
  if constexpr (!KQ) {
    hipLaunchKernelGGL((k_mmq<FMT, XDT, kMmMT, kMmNFX>), dim3(static_cast<unsigned>(units)), dim3(256), 0, s, a);
    const int rc = check_launch("mmq gemm");
    if (rc) return rc;
    return mm_reduce_launch<4, kMmMT, kMmNFX, 1>(a, s);
  }
  return VYBDQ_OK;
}

}  // namespace vybdq
