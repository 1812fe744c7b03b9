// Several-row tile kernel instances for one weight format (WF_I4ZP).
#include "bz_gemv_tile.h"

namespace bz {
int launch_tile_i4zp(const TileParams& tp, const TileLaunch& l, hipStream_t st) { return launch_tile_wf<WF_I4ZP>(tp, l, st); }
}  // namespace bz
