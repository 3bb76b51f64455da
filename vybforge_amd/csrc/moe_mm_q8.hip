// Instantiations of the grouped MoE expert GEMM for Q8_0 weights (own translation unit: parallel build).
#include "moe_mm.h"

namespace vybdq {

int moe_mm_q8(int xdt, int mt, bool swi, const MoeMmArgs &g, int max_tiles, hipStream_t s) {
  if (g.tile_rows == 4) return set_error(VYBDQ_ERR_SHAPE, "moe grouped gemm: 4-row tiles are q4_0 only");
  if (swi) {
    switch (xdt) {
      case VYBDQ_F32: return mt == 1 ? moe_mm_launch<FMT_Q8_0, VYBDQ_F32, 1, true>(g, max_tiles, s)
                                     : moe_mm_launch<FMT_Q8_0, VYBDQ_F32, 2, true>(g, max_tiles, s);
      case VYBDQ_F16: return mt == 1 ? moe_mm_launch<FMT_Q8_0, VYBDQ_F16, 1, true>(g, max_tiles, s)
                                     : moe_mm_launch<FMT_Q8_0, VYBDQ_F16, 2, true>(g, max_tiles, s);
      default: return mt == 1 ? moe_mm_launch<FMT_Q8_0, VYBDQ_BF16, 1, true>(g, max_tiles, s)
                              : moe_mm_launch<FMT_Q8_0, VYBDQ_BF16, 2, true>(g, max_tiles, s);
    }
  }
  // down: X is the fp16 activations
  return mt == 1 ? moe_mm_launch<FMT_Q8_0, VYBDQ_F16, 1, false>(g, max_tiles, s)
                 : moe_mm_launch<FMT_Q8_0, VYBDQ_F16, 2, false>(g, max_tiles, s);
}

}  // namespace vybdq
