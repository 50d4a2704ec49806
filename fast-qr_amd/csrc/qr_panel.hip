// qr_panel.hip — panel factorisation of the blocked path (16- or 32-column
// panels, up to 4096 rows), one workgroup per matrix, the panel in global H.
// The factorisation itself is panel_body (panel.hpp).
//
// Reference counterpart: blocked{n}_panel_factor_kernel and the T formation of
// blocked{n}_trailing_update_kernel (submissions/candidate.py:2404-2505,
// 2544-2584).
#include "kernels.hpp"
#include "panel.hpp"

namespace fastqr {

namespace {

// Panel storage in global H (matrix b): element (row r, column c) of the panel
// at byte offset 4 * ((k0 + c) * ldh + k0 + r) through the matrix's buffer
// descriptor; T to the matrix's workspace slot, tau at column k0.
struct GlobalPanelIO {
  rsrc_t rs;
  uint32_t base;
  int64_t ldh;
  float* T;
  float* tau;
  int64_t ts1;
  __device__ __forceinline__ uint32_t off(int r, int c) const { return base + 4u * (uint32_t)(c * ldh + r); }
  __device__ __forceinline__ f32x4 load4(int r, int c, bool ok) const { return buf_load4(rs, ok ? off(r, c) : kOffNone); }
  __device__ __forceinline__ float load1(int r, int c, bool ok) const { return buf_load(rs, ok ? off(r, c) : kOffNone); }
  __device__ __forceinline__ void store4(int r, int c, bool ok, f32x4 v) const {
    buf_store4(rs, ok ? off(r, c) : kOffNone, v);
  }
  __device__ __forceinline__ void store1(int r, int c, bool ok, float v) const {
    buf_store(rs, ok ? off(r, c) : kOffNone, v);
  }
  __device__ __forceinline__ void store_T(int slot, int r, int c, float v) const { T[slot * 1024 + r * 32 + c] = v; }
  __device__ __forceinline__ void store_tau(int c, float v) const { tau[(int64_t)c * ts1] = v; }
  __device__ __forceinline__ void barrier() const { __syncthreads(); }
};

}  // namespace

// Occupancy: (4, 8, 2) is held to 168 registers (three waves per SIMD, three
// workgroups per CU), so 640 matrices of 512 rows run in one round on 256 CUs
// instead of two.
template <int NW, int TPW, int NBLK, bool VEC>
__global__ void __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu((NW == 4 && TPW == 8 && NBLK == 2 && VEC) ? 3 : (NW + 3) / 4, 8)))
panel_kernel(float* __restrict__ H, int64_t hs0, int64_t ldh, float* __restrict__ tau, int64_t ts0, int64_t ts1,
             float* __restrict__ Tws, int n, int k0, int slot) {
  // the panel is the critical path: its waves win issue arbitration against
  // trailing-update waves running concurrently on the same SIMDs
  __builtin_amdgcn_s_setprio(3);
  const int64_t b = blockIdx.x;
  GlobalPanelIO io;
  io.rs = make_rsrc(H + b * hs0, (uint32_t)(4 * ldh * n));
  io.base = 4u * (uint32_t)(k0 * ldh + k0);
  io.ldh = ldh;
  io.T = Tws + (b * kMaxSlots + slot) * 32 * 32;
  io.tau = tau + b * ts0 + (int64_t)k0 * ts1;
  io.ts1 = ts1;
  panel_body<NW, TPW, NBLK, VEC>(io, n - k0, (int)threadIdx.x);
}

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
#define FASTQR_PANEL(NW, TPW, NBLK)                                                                             \
  if (nw == NW && tpw == TPW && nb == 16 * NBLK) {                                                              \
    if (v4)                                                                                                     \
      hipLaunchKernelGGL((panel_kernel<NW, TPW, NBLK, true>), grid, dim3(NW * 64), 0, stream, H, hs0, ldh, tau, \
                         ts0, ts1, Tws, n, k0, slot);                                                           \
    else                                                                                                        \
      hipLaunchKernelGGL((panel_kernel<NW, TPW, NBLK, false>), grid, dim3(NW * 64), 0, stream, H, hs0, ldh,     \
                         tau, ts0, ts1, Tws, n, k0, slot);                                                      \
    return hipGetLastError();                                                                                   \
  }
  FASTQR_PANEL(1, 4, 2)
  FASTQR_PANEL(2, 4, 2)
  FASTQR_PANEL(4, 4, 2)
  FASTQR_PANEL(4, 8, 2)
  FASTQR_PANEL(4, 16, 2)
  FASTQR_PANEL(8, 16, 2)
  FASTQR_PANEL(8, 24, 2)
  FASTQR_PANEL(8, 16, 1)
  FASTQR_PANEL(8, 32, 1)
  FASTQR_PANEL(8, 8, 2)
  FASTQR_PANEL(1, 4, 4)
  FASTQR_PANEL(2, 4, 8)
  FASTQR_PANEL(4, 4, 8)
  FASTQR_PANEL(8, 4, 8)
  FASTQR_PANEL(4, 4, 4)
  FASTQR_PANEL(4, 8, 4)
  FASTQR_PANEL(8, 8, 4)
  FASTQR_PANEL(4, 6, 2)
  FASTQR_PANEL(8, 6, 2)
  FASTQR_PANEL(8, 12, 2)
  FASTQR_PANEL(4, 6, 4)
  FASTQR_PANEL(8, 6, 4)
  FASTQR_PANEL(4, 2, 4)
  FASTQR_PANEL(4, 3, 4)
#undef FASTQR_PANEL
  return hipErrorInvalidValue;
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
    } else if (m <= 384) {
      nw = 4, tpw = 6;
    } else if (m <= 512) {
      nw = 4, tpw = 8;
    } else if (m <= 768) {
      nw = 8, tpw = 6;
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
    } else if (m <= 384) {
      nw = 4, tpw = 6;
    } else if (m <= 512) {
      nw = 4, tpw = 8;
    } else if (m <= 768) {
      nw = 8, tpw = 6;
    } else if (m <= 1024) {
      nw = 8, tpw = 8;
    } else if (m <= 1536) {
      nw = 8, tpw = 12;
    } else if (m <= 2048) {
      nw = 8, tpw = 16;
    } else if (m <= 3072) {
      nw = 8, tpw = 24;
    }
  } else if (nb == 16) {
    if (m <= 2048) {
      nw = 8, tpw = 16;
    } else if (m <= 4096) {
      nw = 8, tpw = 32;
    }
  }
  if (nw == 0) return hipErrorInvalidValue;
  return launch_panel_cfg(nw, tpw, H, batch, hs0, ldh, tau, ts0, ts1, Tws, n, k0, nb, slot, vec, stream);
}

}  // namespace fastqr
