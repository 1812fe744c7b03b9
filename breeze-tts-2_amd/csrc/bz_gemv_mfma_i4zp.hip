// Matrix-core instances of the streaming GEMV for one weight format (WF_I4ZP).
#include "bz_gemv_mfma.h"

namespace bz {
int launch_mfma_i4zp(const GemvParams& p, const Launch& l, hipStream_t st) { return launch_mfma_m<WF_I4ZP>(p, l, st); }
}  // namespace bz
