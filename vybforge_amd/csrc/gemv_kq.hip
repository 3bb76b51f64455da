// Super-block (Q4_K, Q5_K, Q6_K, IQ2_S) instantiations of the pair GEMV (gemv_pair.h, kquant_dev.h).
#include "gemv_pair.h"

namespace vybdq {

int gemv_kq_dispatch(int fmt, const void *X, int64_t M, int64_t K, int x_dt, const Segs &segs, hipStream_t s) {
  if (fmt == FMT_Q4_K) return launch_pair_chunks<FMT_Q4_K, VYBDQ_Q4_GGML>(X, M, K, x_dt, segs, s);
  if (fmt == FMT_Q5_K) return launch_pair_chunks<FMT_Q5_K, VYBDQ_Q4_GGML>(X, M, K, x_dt, segs, s);
  if (fmt == FMT_IQ2_S) return launch_pair_chunks<FMT_IQ2_S, VYBDQ_Q4_GGML>(X, M, K, x_dt, segs, s);
  return launch_pair_chunks<FMT_Q6_K, VYBDQ_Q4_GGML>(X, M, K, x_dt, segs, s);
}

}  // namespace vybdq
