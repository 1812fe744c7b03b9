// Instances of the streaming GEMV for one weight format (WF_BF16).
#include "bz_gemv_kernel.h"

namespace bz {
int launch_bf16(const GemvParams& p, const Launch& l, hipStream_t st) { return launch_m<WF_BF16>(p, l, st); }
}  // namespace bz
