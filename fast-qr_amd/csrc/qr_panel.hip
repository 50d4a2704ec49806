// qr_panel.hip — panel factorisation of the blocked path (16- or 32-column
// panels, up to 4096 rows), one workgroup per matrix, the panel in global H.
// The factorisation itself is panel_body (panel.hpp).
//
// Reference counterpart: blocked{n}_panel_factor_kernel and the T formation of
// blocked{n}_trailing_update_kernel (submissions/candidate.py:2404-2505,
// 2544-2584).
#include "panel_kernel.hpp"

namespace fastqr {

// 32-column panels up to 3072 rows ((8, 24, 2): 14 registers spill in the
// 16-byte-load variant, still 64 fewer panels and narrow updates per 4096
// matrix than 16 columns above 2048 rows: 2 x 4096 15.5 -> 14.5 ms on MI355X).
int panel_width_for(int m) { return m > 3072 ? 16 : 32; }

// Panels of the strip-resident path.  A 64-column panel updates its blocks
// inside the kernel, which saves narrow trailing-update launches on the
// critical path; it needs twice the registers of a 32-column one, so one
// workgroup per CU.  With enough matrices to keep every CU busy twice over,
// the narrow updates are cheap and occupancy wins: 32 columns (measured on
// MI355X: 640 x 512 is 13% faster with 32, 60 x 1024 4% faster with 64).
int panel_width_wide(int m, int64_t batch) { return (batch < 512 && m <= 1024) ? 64 : 32; }

int panel_max_rows() { return 4096; }

// (waves, tiles per wave) configurations, by panel width and rows
hipError_t launch_panel_cfg(int nw, int tpw, float* H, int64_t batch, int64_t hs0, int64_t ldh, float* tau,
                            int64_t ts0, int64_t ts1, float* Tws, int n, int k0, int nb, int slot, bool vec,
                            hipStream_t stream) {
  const int m = n - k0;
  if (m > 16 * nw * tpw) return hipErrorInvalidValue;
  const bool v4 = vec && (m & 3) == 0;
  const dim3 grid((unsigned)batch);
  bool done = false;
  hipError_t e = panel_launch_narrow(nw, tpw, nb, v4, grid, H, hs0, ldh, tau, ts0, ts1, Tws, n, k0, slot, stream, &done);
  if (!done) e = panel_launch_tall(nw, tpw, nb, v4, grid, H, hs0, ldh, tau, ts0, ts1, Tws, n, k0, slot, stream, &done);
  if (!done) e = panel_launch_wide(nw, tpw, nb, v4, grid, H, hs0, ldh, tau, ts0, ts1, Tws, n, k0, slot, stream, &done);
  if (!done) e = panel_launch_wide8(nw, tpw, nb, v4, grid, H, hs0, ldh, tau, ts0, ts1, Tws, n, k0, slot, stream, &done);
  return done ? e : hipErrorInvalidValue;
}

FASTQR_PANEL_LAUNCHER(panel_launch_narrow) {
  FASTQR_PANEL(1, 4, 2)
  FASTQR_PANEL(2, 4, 2)
  FASTQR_PANEL(4, 4, 2)
  FASTQR_PANEL(4, 5, 2)
  FASTQR_PANEL(4, 6, 2)
  FASTQR_PANEL(4, 7, 2)
  FASTQR_PANEL(4, 8, 2)
  FASTQR_PANEL(4, 16, 2)
  return hipSuccess;
}

hipError_t launch_panel(float* H, int64_t batch, int64_t hs0, int64_t ldh, float* tau, int64_t ts0, int64_t ts1,
                        float* Tws, int n, int k0, int nb, int m_cap, int slot, bool vec, hipStream_t stream) {
  // configuration chosen for m_cap >= n - k0 rows and width nb; rows covered = 16 * NW * TPW
  const int m = m_cap;
  int nw = 0, tpw = 0;
  // measured best per height (one workgroup per matrix; MI355X)
  if (nb == 128) {
    if (m <= 64) {
      nw = 1, tpw = 4, nb = 64;  // at most 64 columns remain
    } else if (m <= 128) {
      nw = 2, tpw = 4;
    } else if (m <= 256) {
      nw = 4, tpw = 4;
    } else if (m <= 512) {
      nw = 8, tpw = 4;
    }
  } else if (nb == 64) {
    if (m <= 64) {
      nw = 1, tpw = 4;
    } else if (m <= 128) {
      nw = 4, tpw = 2;
    } else if (m <= 192) {
      nw = 4, tpw = 3;
    } else if (m <= 256) {
      nw = 4, tpw = 4;
    } else if (m <= 320) {
      nw = 4, tpw = 5;
    } else if (m <= 384) {
      nw = 4, tpw = 6;
    } else if (m <= 448) {
      nw = 4, tpw = 7;
    } else if (m <= 512) {
      nw = 4, tpw = 8;
    } else if (m <= 640) {
      nw = 8, tpw = 5;
    } else if (m <= 768) {
      nw = 8, tpw = 6;
    } else if (m <= 896) {
      nw = 8, tpw = 7;
    } else if (m <= 1024) {
      nw = 8, tpw = 8;
    }
  } else if (nb == 32) {
    if (m <= 64) {
      nw = 1, tpw = 4;
    } else if (m <= 128) {
      nw = 2, tpw = 4;
    } else if (m <= 256) {
      nw = 4, tpw = 4;
    } else if (m <= 320) {
      nw = 4, tpw = 5;
    } else if (m <= 384) {
      nw = 4, tpw = 6;
    } else if (m <= 448) {
      nw = 4, tpw = 7;
    } else if (m <= 512) {
      nw = 4, tpw = 8;
    } else if (m <= 640) {
      nw = 8, tpw = 5;
    } else if (m <= 768) {
      nw = 8, tpw = 6;
    } else if (m <= 896) {
      nw = 8, tpw = 7;
    } else if (m <= 1024) {
      nw = 8, tpw = 8;
    } else if (m <= 1280) {
      nw = 8, tpw = 10;
    } else if (m <= 1536) {
      nw = 8, tpw = 12;
    } else if (m <= 1792) {
      nw = 8, tpw = 14;
    } else if (m <= 2048) {
      nw = 8, tpw = 16;
    } else if (m <= 2304) {
      nw = 8, tpw = 18;
    } else if (m <= 2560) {
      nw = 8, tpw = 20;
    } else if (m <= 2816) {
      nw = 8, tpw = 22;
    } else if (m <= 3072) {
      nw = 8, tpw = 24;
    }
  } else if (nb == 16) {
    if (m <= 2048) {
      nw = 8, tpw = 16;
    } else if (m <= 3328) {
      nw = 8, tpw = 26;
    } else if (m <= 3584) {
      nw = 8, tpw = 28;
    } else if (m <= 3840) {
      nw = 8, tpw = 30;
    } else if (m <= 4096) {
      nw = 8, tpw = 32;
    }
  }
  if (nw == 0) return hipErrorInvalidValue;
  return launch_panel_cfg(nw, tpw, H, batch, hs0, ldh, tau, ts0, ts1, Tws, n, k0, nb, slot, vec, stream);
}

}  // namespace fastqr
