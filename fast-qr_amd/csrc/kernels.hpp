// kernels.hpp — host-side launchers of the QR kernels (internal to libfastqr).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fastqr {

// n <= 64: one wave64 per matrix (qr_wave.hip).
hipError_t launch_qr_wave(const float* A, int64_t batch, int n, int64_t as0, int64_t as1, int64_t as2,
                          float* H, int64_t hs0, int64_t hs1, int64_t hs2, float* tau, int64_t ts0,
                          int64_t ts1, hipStream_t stream);

// Blocked path (qr_blocked.hip).
hipError_t launch_copy_colmajor(const float* A, int64_t batch, int n, int64_t as0, int64_t as1, int64_t as2,
                                float* H, int64_t hs0, int64_t ldh, hipStream_t stream);
int panel_width_for(int m);
hipError_t launch_panel(float* H, int64_t batch, int64_t hs0, int64_t ldh, float* tau, int64_t ts0,
                        int64_t ts1, float* Tws, int n, int k0, hipStream_t stream);
hipError_t launch_update(float* H, int64_t batch, int64_t hs0, int64_t ldh, const float* Tws, int n, int k0,
                         int nb, bool vec, hipStream_t stream);

// Largest panel width used by the blocked path (sizes the T workspace).
constexpr int kMaxPanel = 32;

}  // namespace fastqr
