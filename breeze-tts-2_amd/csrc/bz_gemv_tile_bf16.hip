// Several-row tile kernel instances for one weight format (WF_BF16).
#include "bz_gemv_tile.h"

namespace bz {
int launch_tile_bf16(const TileParams& tp, const TileLaunch& l, hipStream_t st) { return launch_tile_wf<WF_BF16>(tp, l, st); }
}  // namespace bz
