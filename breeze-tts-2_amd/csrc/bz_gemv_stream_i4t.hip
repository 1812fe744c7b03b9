// Instances of the tiled streaming GEMV for one weight format (WF_I4T).
#include "bz_gemv_stream.h"

namespace bz {
int launch_stream_i4t(const StreamParams& p, const StreamLaunch& l, hipStream_t st) {
    return launch_stream_wf<WF_I4T>(p, l, st);
}
}  // namespace bz
