// Instances of the several-block streaming GEMV for one weight format (WF_I4TP).
#include "bz_gemv_wide.h"

namespace bz {
int launch_wide_i4tp(const StreamParams& p, const WideLaunch& l, int nblk, hipStream_t st) {
    return launch_wide_wf<WF_I4TP>(p, l, nblk, st);
}
}  // namespace bz
