// One instantiation of the MFMA dequant GEMM kernel (compiled in parallel with its siblings).
#include "mmq.h"

namespace vybdq {
template int mmq_launch<FMT_Q5_K, VYBDQ_F16>(MmArgs &, hipStream_t);
}  // namespace vybdq
