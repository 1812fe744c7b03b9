// Matrix-core instances of the streaming GEMV for one weight format (WF_BF16).
#include "bz_gemv_mfma.h"

namespace bz {
int launch_mfma_bf16(const GemvParams& p, const Launch& l, hipStream_t st) { return launch_mfma_m<WF_BF16>(p, l, st); }
}  // namespace bz
