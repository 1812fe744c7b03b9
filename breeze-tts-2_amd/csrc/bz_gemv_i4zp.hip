// Instances of the streaming GEMV for one weight format (WF_I4ZP).
#include "bz_gemv_kernel.h"

namespace bz {
int launch_i4zp(const GemvParams& p, const Launch& l, hipStream_t st) { return launch_m<WF_I4ZP>(p, l, st); }
}  // namespace bz
