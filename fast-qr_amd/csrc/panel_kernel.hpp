// panel_kernel.hpp — the blocked path's panel kernel (panel in global H),
// included by the translation units that instantiate its configurations
// (qr_panel*.hip: split so that they compile in parallel).
#pragma once

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

// One configuration's launch: returns from the enclosing launcher when
// (nw, tpw, nb) is this configuration.
#define FASTQR_PANEL(NW, TPW, NBLK)                                                                             \
  if (nw == NW && tpw == TPW && nb == 16 * NBLK) {                                                              \
    if (v4)                                                                                                     \
      hipLaunchKernelGGL((panel_kernel<NW, TPW, NBLK, true>), grid, dim3(NW * 64), 0, stream, H, hs0, ldh, tau, \
                         ts0, ts1, Tws, n, k0, slot);                                                           \
    else                                                                                                        \
      hipLaunchKernelGGL((panel_kernel<NW, TPW, NBLK, false>), grid, dim3(NW * 64), 0, stream, H, hs0, ldh,     \
                         tau, ts0, ts1, Tws, n, k0, slot);                                                      \
    *done = true;                                                                                               \
    return hipGetLastError();                                                                                   \
  }

// The configurations of each translation unit; `done` is set when (nw, tpw,
// nb) was one of them.
#define FASTQR_PANEL_LAUNCHER(NAME)                                                                              \
  hipError_t NAME(int nw, int tpw, int nb, bool v4, dim3 grid, float* H, int64_t hs0, int64_t ldh, float* tau,   \
                  int64_t ts0, int64_t ts1, float* Tws, int n, int k0, int slot, hipStream_t stream, bool* done)
FASTQR_PANEL_LAUNCHER(panel_launch_narrow);  // 32 columns, up to 4 waves (qr_panel.hip)
FASTQR_PANEL_LAUNCHER(panel_launch_tall);    // 16 and 32 columns, 8 waves (qr_panel_tall.hip)
FASTQR_PANEL_LAUNCHER(panel_launch_wide);    // 64 columns, up to 4 waves (qr_panel_wide.hip)
FASTQR_PANEL_LAUNCHER(panel_launch_wide8);   // 64 columns on 8 waves, 128 columns (qr_panel_wide8.hip)

}  // namespace fastqr
