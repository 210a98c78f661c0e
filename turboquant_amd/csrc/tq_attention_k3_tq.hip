// tq_attention_k3_tq.hip -- the fused decode kernels for 3-bit
// TQ (PQ records with the QJL correction) records: every head_dim, head-group and
// workgroup shape, with the inline split-K merge and for the reference
// ABI's separate merge launch.  One unit per bit width and cache mode, so
// that the kernels build in parallel.
#include "tq_decode_kernel.h"

namespace tqa {
template void launch_stream_bm<3, kModeTq, true>(AttnArgs &, int, int, dim3, hipStream_t);
template void launch_stream_bm<3, kModeTq, false>(AttnArgs &, int, int, dim3, hipStream_t);
}  // namespace tqa
