// Instantiations of the grouped MoE expert GEMM for q4_0 weights (own translation unit: parallel build).
#include "moe_mm.h"

namespace vybdq {

int moe_mm_q4(int xdt, int mt, bool swi, const MoeMmArgs &g, int max_tiles, hipStream_t s) {
  // 16-row m-tiles with fp16 X (the converted tokens, the activations): the weights are staged
  // through LDS (VYBDQ_MOE_LDS=0 under VYBDQ_TUNING keeps the register-operand body)
  const char *e = tuning_env("VYBDQ_MOE_LDS");
  const bool lds_off = e && e[0] == '0';
  if (g.tile_rows == 4) {  // 4-row tiles: the LDS-staged body with four stages
    if (mt != 1 || !moe_mm_lds_ok(FMT_Q4_0, xdt, swi, g))
      return set_error(VYBDQ_ERR_SHAPE, "moe grouped gemm: 4-row tiles need the LDS-staged body");
    return swi ? moe_mm_lds_launch<128, 1, true, 4>(g, max_tiles, s) : moe_mm_lds_launch<128, 1, false, 4>(g, max_tiles, s);
  }
  if (!lds_off && mt == 1 && moe_mm_lds_ok(FMT_Q4_0, xdt, swi, g))
    return swi ? moe_mm_lds_launch<128, 1, true>(g, max_tiles, s) : moe_mm_lds_launch<128, 1, false>(g, max_tiles, s);
  if (swi) {
    switch (xdt) {
      case VYBDQ_F32: return mt == 1 ? moe_mm_launch<FMT_Q4_0, VYBDQ_F32, 1, true>(g, max_tiles, s)
                                     : moe_mm_launch<FMT_Q4_0, VYBDQ_F32, 2, true>(g, max_tiles, s);
      case VYBDQ_F16: return mt == 1 ? moe_mm_launch<FMT_Q4_0, VYBDQ_F16, 1, true>(g, max_tiles, s)
                                     : moe_mm_launch<FMT_Q4_0, VYBDQ_F16, 2, true>(g, max_tiles, s);
      default: return mt == 1 ? moe_mm_launch<FMT_Q4_0, VYBDQ_BF16, 1, true>(g, max_tiles, s)
                              : moe_mm_launch<FMT_Q4_0, VYBDQ_BF16, 2, true>(g, max_tiles, s);
    }
  }
  // down: X is the fp16 activations
  return mt == 1 ? moe_mm_launch<FMT_Q4_0, VYBDQ_F16, 1, false>(g, max_tiles, s)
                 : moe_mm_launch<FMT_Q4_0, VYBDQ_F16, 2, false>(g, max_tiles, s);
}

}  // namespace vybdq
