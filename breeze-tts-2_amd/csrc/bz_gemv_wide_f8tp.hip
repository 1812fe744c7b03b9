// Instances of the several-block streaming GEMV for one weight format (WF_F8TP).
#include "bz_gemv_wide.h"

namespace bz {
int launch_wide_f8tp(const StreamParams& p, const WideLaunch& l, int nblk, hipStream_t st) {
    return launch_wide_wf<WF_F8TP>(p, l, nblk, st);
}
}  // namespace bz
