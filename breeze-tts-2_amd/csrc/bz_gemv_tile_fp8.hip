// Several-row tile kernel instances for one weight format (WF_FP8).
#include "bz_gemv_tile.h"

namespace bz {
int launch_tile_fp8(const TileParams& tp, const TileLaunch& l, hipStream_t st) { return launch_tile_wf<WF_FP8>(tp, l, st); }
}  // namespace bz
