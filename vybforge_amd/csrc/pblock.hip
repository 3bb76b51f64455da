// vybdq_launch_pblock: the library's kernels launched on the reference's own parameter blocks,
// gfx950.
//
// The reference launches every GEMV / prefill GEMM with one pointer to a device-resident block of
// little-endian int64 words (lk(h, gx, bx, p), native/host/ridge_decode.vyb:204-227), and under its
// captured decode graph it rewrites words of those blocks with asynchronous copies between replays
// (put_ia, ridge_decode.vyb:168-180). So nothing here reads a block on the host: every word is
// read by the kernel when the launch runs, shapes included, and the work split is planned on the
// device from them.
//   GEMV (set_gemv, ridge_decode.vyb:264-270): the persistent chain kernel of chain.hip with one
//     stage, reading the block in the reference layout (x f32, GGUF nibble order).
//   GEMM (set_gemm, ridge_decode.vyb:272-275; gen_rpf.py:2-8): q4_0 / Q8_0 run the register-operand
//     MFMA tile body of mmq.h in a persistent grid (one workgroup per CU) over the tiles of a plan
//     made on the device with the host planner's cost model (no split-K: the block has no
//     workspace word); the super-block types run the LDS-staged kernel of kqgemm.hip likewise.
// A block whose words violate a kernel's preconditions is not computed: the launch writes nothing
// and sets a bit of this device's status word, which vybdq_pblock_status() reports and clears.
#include "mmq.h"

#include <mutex>
#include <string>

namespace vybdq {

// defined in chain.hip / kqgemm.hip
int pb_gemv_dispatch(int wtype, uint64_t P, int64_t maxK, uint32_t *status, hipStream_t s);
int kq_gemm_pblock(int wtype, int xdt, const int64_t *pb, uint32_t *status, hipStream_t s);
// pblock_moe.hip / pblock_exl3.hip
int pb_moe_launch(const int64_t *pb, uint32_t *status, hipStream_t s);
int pb_exl3dq_launch(const int64_t *pb, int64_t threads, uint32_t *status, hipStream_t s);
int pb_exl3inv_launch(const int64_t *pb, uint32_t *status, hipStream_t s);
int pb_exl3stage_launch(int kind, const int64_t *pb, uint32_t *status, hipStream_t s);
int exl3_deq_map_launch(const uint8_t *q, const int64_t *tab, void *o, int out_dt, uint32_t *status, hipStream_t s);

// status word bits (word 0 of the per-device status array; word 1 is the chain's stage counter)
constexpr uint32_t kPbWaitTimeout = 1u, kPbBadGemv = 2u, kPbBadGemm = 4u, kPbBadMoe = 8u, kPbBadExl3 = 16u;
// largest K of a GEMV block (the chain's LDS x stage is sized for it: 48.6 KB, 3 workgroups per CU)
constexpr int64_t kPbMaxK = 20480;

static __device__ __align__(256) uint32_t pb_status[64] = {0};

namespace {
std::mutex g_pb_mu;
uint64_t g_pb_status[64];  // device address of pb_status per device
}  // namespace

// the current device's status array (hipGetSymbolAddress once per device)
int pb_status_address(uint64_t &ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return set_error(VYBDQ_ERR_HIP, "vybdq_launch_pblock: no current HIP device");
  std::lock_guard<std::mutex> lock(g_pb_mu);
  if (!g_pb_status[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(pb_status));
    if (e != hipSuccess || !p)
      return set_error(VYBDQ_ERR_HIP, std::string("vybdq_launch_pblock: hipGetSymbolAddress failed: ") +
                                          hipGetErrorString(e));
    g_pb_status[dev] = reinterpret_cast<uint64_t>(p);
  }
  ptr = g_pb_status[dev];
  return VYBDQ_OK;
}

// The host planner's tile choice (mmq_host.hip mm_plan) without K splits, for `grid` workgroups:
// fragments per tile F minimising rounds x super-steps x (fixed + per-fragment cycles).
__device__ __forceinline__ void mmq_pb_plan(int M, int N, int S, int grid, int &F, int &m_tiles, int &n_tiles) {
  m_tiles = (M + 16 * kMmMT - 1) / (16 * kMmMT);
  const int Ftot = N / 16;
  double best = -1.0;
  F = 1;
  n_tiles = Ftot;
  for (int f = 1; f <= 4 * kMmNFX && f <= Ftot; ++f) {
    const int nt = (Ftot + f - 1) / f;
    if ((nt - 1) * f >= Ftot) continue;
    const int64_t units = static_cast<int64_t>(m_tiles) * nt;
    const int64_t rounds = (units + grid - 1) / grid;
    const double t = static_cast<double>(rounds) * S * (1440.0 + 1584.0 * ((f + 3) / 4));
    if (best < 0 || t < best - 1e-9) {
      best = t;
      F = f;
      n_tiles = nt;
    }
  }
}

// set_gemm block: W@0 X@8 Y@16 S@24 N@32 K@40 LDY@48 RS@56 (G@64, NMT@72: the reference's grid,
// not used). LDY >= 0: Y f64, row stride LDY, RS f64 (or 0); LDY < 0: Y f32, row stride -LDY, RS
// ignored.
template <int FMT, int XDT>
__global__ void __launch_bounds__(256, 1) k_mmq_pb(const int64_t *__restrict__ pb, uint32_t *__restrict__ status) {
  VYBDQ_MMQ_LDS(FMT, kMmMT);
  const int64_t W = pb[0], X = pb[1], Y = pb[2], M = pb[3], N = pb[4], K = pb[5], LDY = pb[6], RS = pb[7];
  const int64_t ldy = LDY < 0 ? -LDY : LDY;
  const bool ok = W && X && Y && M >= 1 && M < (1 << 24) && N >= 16 && N % 16 == 0 && N < (1 << 24) && K >= 256 &&
                  K % 256 == 0 && K < (1 << 24) && M * K < (int64_t(1) << 31) && ldy >= N && (W & 3) == 0 &&
                  (X & 15) == 0;
  if (!ok) {
    if (blockIdx.x == 0 && threadIdx.x == 0)
      __hip_atomic_fetch_or(status, kPbBadGemm, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  MmArgs a{};
  a.W = gptr<const uint8_t>(W);
  a.rowbytes = (K / 32) * MmFmt<FMT>::BB;
  a.X = gptr<const void>(X);
  a.ldx = K;
  a.M = static_cast<int>(M);
  a.N = static_cast<int>(N);
  a.S = static_cast<int>(K / 128);
  mmq_pb_plan(a.M, a.N, a.S, gridDim.x, a.F, a.m_tiles, a.n_tiles);
  a.splits = 1;
  a.sps = a.S;
  a.xcd = 0;
  a.Y = gptr<void>(Y);
  a.ydt = LDY < 0 ? VYBDQ_F32 : VYBDQ_F64;
  a.ldy = ldy;
  a.RS = LDY < 0 ? nullptr : gptr<const void>(RS);
  const int units = a.m_tiles * a.n_tiles;
  for (int u = blockIdx.x; u < units; u += gridDim.x) mmq_unit<FMT, XDT, kMmMT, kMmNFX>(a, sm, u);
}

template <int FMT, int XDT>
static int mmq_pb_launch(const int64_t *pb, uint32_t *status, hipStream_t s) {
  hipLaunchKernelGGL((k_mmq_pb<FMT, XDT>), dim3(static_cast<unsigned>(device_cu_count())), dim3(256), 0, s, pb, status);
  return check_launch("p-block gemm");
}

}  // namespace vybdq

using namespace vybdq;

extern "C" int vybdq_launch_pblock(int kind, uint64_t P, uint64_t stream) {
  VYBDQ_REQUIRE(P, VYBDQ_ERR_ARG, "null parameter block");
  VYBDQ_REQUIRE((P & 7) == 0, VYBDQ_ERR_ALIGN, "the parameter block must be 8-byte aligned");
  if (kind == VYBDQ_PB_MOE || kind == VYBDQ_PB_EXL3INV) {
    uint64_t st = 0;
    const int rc = pb_status_address(st);
    if (rc) return rc;
    const auto *pb = reinterpret_cast<const int64_t *>(P);
    auto *status = reinterpret_cast<uint32_t *>(st);
    return kind == VYBDQ_PB_MOE ? pb_moe_launch(pb, status, as_stream(stream))
                                : pb_exl3inv_launch(pb, status, as_stream(stream));
  }
  if (kind == VYBDQ_PB_EXL3HGEN || kind == VYBDQ_PB_EXL3HGEN32 || kind == VYBDQ_PB_EXL3HAD1 ||
      kind == VYBDQ_PB_EXL3HAD132 || kind == VYBDQ_PB_EXL3HAD2 || kind == VYBDQ_PB_EXL3HAD232 ||
      kind == VYBDQ_PB_EXL3CVT32) {
    uint64_t st = 0;
    const int rc = pb_status_address(st);
    if (rc) return rc;
    return pb_exl3stage_launch(kind, reinterpret_cast<const int64_t *>(P), reinterpret_cast<uint32_t *>(st),
                               as_stream(stream));
  }
  VYBDQ_REQUIRE(kind != VYBDQ_PB_EXL3DQ, VYBDQ_ERR_ARG,
                "VYBDQ_PB_EXL3DQ takes its extent from the grid: use vybdq_launch_pblock_grid");
  const int op = kind & ~0xff, ty = kind & 0xff;
  VYBDQ_REQUIRE(op == VYBDQ_PB_GEMV || op == VYBDQ_PB_GEMM || op == VYBDQ_PB_GEMM_XH, VYBDQ_ERR_ARG,
                "kind must be VYBDQ_PB_GEMV, VYBDQ_PB_GEMM or VYBDQ_PB_GEMM_XH plus a GGML type id, or "
                "VYBDQ_PB_MOE or one of the VYBDQ_PB_EXL3* kinds");
  VYBDQ_REQUIRE(ty == 2 || ty == 8 || ty == 12 || ty == 13 || ty == 14 || ty == 22, VYBDQ_ERR_ARG,
                "the type id must be 2 (q4_0), 8 (Q8_0), 12 (Q4_K), 13 (Q5_K), 14 (Q6_K) or 22 (IQ2_S)");
  uint64_t st = 0;
  const int rc = pb_status_address(st);
  if (rc) return rc;
  hipStream_t s = as_stream(stream);
  if (op == VYBDQ_PB_GEMV) return pb_gemv_dispatch(ty, P, kPbMaxK, reinterpret_cast<uint32_t *>(st), s);
  const int xdt = op == VYBDQ_PB_GEMM ? VYBDQ_F32 : VYBDQ_F16;
  const auto *pb = reinterpret_cast<const int64_t *>(P);
  auto *status = reinterpret_cast<uint32_t *>(st);
  if (ty >= 12) return kq_gemm_pblock(ty, xdt, pb, status, s);
  if (ty == 2) return xdt == VYBDQ_F32 ? mmq_pb_launch<FMT_Q4_0, VYBDQ_F32>(pb, status, s)
                                       : mmq_pb_launch<FMT_Q4_0, VYBDQ_F16>(pb, status, s);
  return xdt == VYBDQ_F32 ? mmq_pb_launch<FMT_Q8_0, VYBDQ_F32>(pb, status, s)
                          : mmq_pb_launch<FMT_Q8_0, VYBDQ_F16>(pb, status, s);
}

extern "C" int vybdq_launch_pblock_grid(int kind, uint64_t P, uint32_t grid_x, uint32_t block_x, uint64_t stream) {
  if (kind != VYBDQ_PB_EXL3DQ) return vybdq_launch_pblock(kind, P, stream);
  VYBDQ_REQUIRE(P, VYBDQ_ERR_ARG, "null parameter block");
  VYBDQ_REQUIRE((P & 7) == 0, VYBDQ_ERR_ALIGN, "the parameter block must be 8-byte aligned");
  const int64_t threads = static_cast<int64_t>(grid_x) * block_x;
  VYBDQ_REQUIRE(threads > 0, VYBDQ_ERR_SHAPE, "the grid has no threads");
  uint64_t st = 0;
  const int rc = pb_status_address(st);
  if (rc) return rc;
  return pb_exl3dq_launch(reinterpret_cast<const int64_t *>(P), threads, reinterpret_cast<uint32_t *>(st),
                          as_stream(stream));
}

extern "C" int vybdq_exl3_deq_map(uint64_t q, uint64_t tab, uint64_t out, int out_dt, uint64_t stream) {
  VYBDQ_REQUIRE(q && tab && out, VYBDQ_ERR_ARG, "null pointer");
  VYBDQ_REQUIRE(out_dt == VYBDQ_F32 || out_dt == VYBDQ_F64, VYBDQ_ERR_ARG, "out_dt must be VYBDQ_F32 or VYBDQ_F64");
  VYBDQ_REQUIRE((tab & 7) == 0 && (out & (out_dt == VYBDQ_F64 ? 7 : 3)) == 0, VYBDQ_ERR_ALIGN,
                "tab must be 8-byte and out element aligned");
  uint64_t st = 0;
  const int rc = pb_status_address(st);
  if (rc) return rc;
  return exl3_deq_map_launch(reinterpret_cast<const uint8_t *>(q), reinterpret_cast<const int64_t *>(tab),
                             reinterpret_cast<void *>(out), out_dt, reinterpret_cast<uint32_t *>(st), as_stream(stream));
}

extern "C" int vybdq_pblock_status(void) {
  uint64_t st = 0;
  const int rc = pb_status_address(st);
  if (rc) return rc;
  uint32_t v = 0;
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(&v, reinterpret_cast<const void *>(st), 4, hipMemcpyDeviceToHost);
  if (e == hipSuccess && v) {
    const uint32_t zero = 0;
    e = hipMemcpy(reinterpret_cast<void *>(st), &zero, 4, hipMemcpyHostToDevice);
  }
  if (e != hipSuccess) return set_error(VYBDQ_ERR_HIP, std::string("vybdq_pblock_status: ") + hipGetErrorString(e));
  if (v & kPbBadGemv) return set_error(VYBDQ_ERR_SHAPE, "a GEMV parameter block was invalid (M != 1, K, N or pointers)");
  if (v & kPbBadGemm) return set_error(VYBDQ_ERR_SHAPE, "a GEMM parameter block was invalid (S, N, K, LDY or pointers)");
  if (v & kPbBadMoe) return set_error(VYBDQ_ERR_SHAPE, "a MoE parameter block was invalid (S or pointers)");
  if (v & kPbBadExl3)
    return set_error(VYBDQ_ERR_SHAPE,
                     "an EXL3 parameter block or map was invalid (cw, nbc, nblocks, the grid, pointers or the tile map)");
  if (v & kPbWaitTimeout) return set_error(VYBDQ_ERR_HIP, "a GEMV parameter block launch timed out");
  return VYBDQ_OK;
}
