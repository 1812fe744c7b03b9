// Several-row tile kernel instances for one weight format (BZ_W_FP8_TILED).
#include "bz_gemv_tile.h"

namespace bz {
int launch_tile_f8t(const TileParams& tp, const TileLaunch& l, hipStream_t st) { return launch_tile_wf<BZ_W_FP8_TILED>(tp, l, st); }
}  // namespace bz
