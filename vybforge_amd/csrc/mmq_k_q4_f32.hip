// One instantiation of the MFMA dequant GEMM kernel (compiled in parallel with its siblings).
#include "mmq.h"

namespace vybdq {
template int mmq_launch<FMT_Q4_0, VYBDQ_F32>(MmArgs &, hipStream_t);
}  // namespace vybdq
