// Instances of the streaming GEMV for one weight format (WF_FP8).
#include "bz_gemv_kernel.h"

namespace bz {
int launch_fp8(const GemvParams& p, const Launch& l, hipStream_t st) { return launch_m<WF_FP8>(p, l, st); }
}  // namespace bz
