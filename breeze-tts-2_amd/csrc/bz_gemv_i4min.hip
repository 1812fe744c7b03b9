// Instances of the streaming GEMV for one weight format (WF_I4MIN).
#include "bz_gemv_kernel.h"

namespace bz {
int launch_i4min(const GemvParams& p, const Launch& l, hipStream_t st) { return launch_m<WF_I4MIN>(p, l, st); }
}  // namespace bz
