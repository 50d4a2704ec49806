// qr_panel_wide8.hip — configurations of the blocked path's panel kernel: 64 columns on 8 waves, 128 columns
// (one translation unit per group, so that they compile in parallel).
#include "panel_kernel.hpp"

namespace fastqr {

FASTQR_PANEL_LAUNCHER(panel_launch_wide8) {
  FASTQR_PANEL(2, 4, 8)
  FASTQR_PANEL(4, 4, 8)
  FASTQR_PANEL(8, 4, 8)
  FASTQR_PANEL(8, 8, 4)
  FASTQR_PANEL(8, 6, 4)
  FASTQR_PANEL(8, 5, 4)
  FASTQR_PANEL(8, 7, 4)
  return hipSuccess;
}

}  // namespace fastqr
