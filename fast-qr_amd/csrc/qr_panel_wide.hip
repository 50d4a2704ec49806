// qr_panel_wide.hip — configurations of the blocked path's panel kernel: 64 columns on up to 4 waves
// (one translation unit per group, so that they compile in parallel).
#include "panel_kernel.hpp"

namespace fastqr {

FASTQR_PANEL_LAUNCHER(panel_launch_wide) {
  FASTQR_PANEL(1, 4, 4)
  FASTQR_PANEL(4, 4, 4)
  FASTQR_PANEL(4, 8, 4)
  FASTQR_PANEL(4, 6, 4)
  FASTQR_PANEL(4, 2, 4)
  FASTQR_PANEL(4, 3, 4)
  FASTQR_PANEL(4, 5, 4)
  FASTQR_PANEL(4, 7, 4)
  return hipSuccess;
}

}  // namespace fastqr
