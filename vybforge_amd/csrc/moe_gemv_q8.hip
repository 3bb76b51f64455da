// Instantiations of the grouped MoE expert GEMV for Q8_0 weights (own translation unit: parallel build).
#include "moe_gemv.h"

namespace vybdq {

int moe_gemv_q8(bool swi, const MoeGvArgs &a, int max_groups, hipStream_t s) {
  return moe_gemv_launch<FMT_Q8_0>(swi, a, max_groups, s);
}

}  // namespace vybdq
