// qr_panel_tall.hip — configurations of the blocked path's panel kernel: 16 and 32 columns on 8 waves
// (one translation unit per group, so that they compile in parallel).
#include "panel_kernel.hpp"

namespace fastqr {

FASTQR_PANEL_LAUNCHER(panel_launch_tall) {
  FASTQR_PANEL(8, 16, 2)
  FASTQR_PANEL(8, 24, 2)
  FASTQR_PANEL(8, 16, 1)
  FASTQR_PANEL(8, 32, 1)
  FASTQR_PANEL(8, 8, 2)
  FASTQR_PANEL(8, 6, 2)
  FASTQR_PANEL(8, 12, 2)
  FASTQR_PANEL(8, 5, 2)
  FASTQR_PANEL(8, 7, 2)
  FASTQR_PANEL(8, 10, 2)
  FASTQR_PANEL(8, 14, 2)
  FASTQR_PANEL(8, 20, 2)
  FASTQR_PANEL(8, 28, 1)
  FASTQR_PANEL(8, 18, 2)
  FASTQR_PANEL(8, 22, 2)
  FASTQR_PANEL(8, 26, 1)
  FASTQR_PANEL(8, 30, 1)
  return hipSuccess;
}

}  // namespace fastqr
