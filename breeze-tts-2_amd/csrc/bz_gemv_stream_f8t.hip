// Instances of the tiled streaming GEMV for one weight format (WF_F8T).
#include "bz_gemv_stream.h"

namespace bz {
int launch_stream_f8t(const StreamParams& p, const StreamLaunch& l, hipStream_t st) {
    return launch_stream_wf<WF_F8T>(p, l, st);
}
}  // namespace bz
