// Instances of the several-row panel GEMV for one weight format (WF_F8T).
#include "bz_gemv_panel.h"

namespace bz {
int launch_panel_f8t(const PanelParams& p, const PanelLaunch& l, hipStream_t st) {
    return launch_panel_wf<WF_F8T>(p, l, st);
}
}  // namespace bz
