// Instances of the tiled streaming GEMV for one weight format (WF_I4TP).
#include "bz_gemv_stream.h"

namespace bz {
int launch_stream_i4tp(const StreamParams& p, const StreamLaunch& l, hipStream_t st) {
    return launch_stream_wf<WF_I4TP>(p, l, st);
}
}  // namespace bz
