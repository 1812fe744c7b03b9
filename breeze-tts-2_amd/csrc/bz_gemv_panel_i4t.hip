// Instances of the several-row panel GEMV for one weight format (WF_I4T).
#include "bz_gemv_panel.h"

namespace bz {
int launch_panel_i4t(const PanelParams& p, const PanelLaunch& l, hipStream_t st) {
    return launch_panel_wf<WF_I4T>(p, l, st);
}
}  // namespace bz
