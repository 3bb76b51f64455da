// One instantiation of the MFMA dequant GEMM kernel (compiled in parallel with its siblings).
#include "mmq.h"

namespace vybdq {
template int mmq_launch<FMT_Q8_0, VYBDQ_BF16>(MmArgs &, hipStream_t);
}  // namespace vybdq
