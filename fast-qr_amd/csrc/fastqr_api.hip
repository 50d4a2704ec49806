// fastqr_api.hip — the C ABI declared in include/fastqr.h.
//
// Argument validation mirrors the reference's pybind shims
// (submissions/candidate.py:111-124, 251-270, 508-527, 1333-1353): shapes,
// strides and pointers are checked before anything is launched; failures
// return a negative status and a message instead of raising.  The shape
// switch replaces custom_kernel's dispatch (submissions/candidate.py:8383-8415)
// and depends on n only — never on the data.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "../../include/fastqr.h"
#include "kernels.hpp"

namespace {

thread_local char g_last_error[512] = "";
thread_local int g_forced_error = 0;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail((int)e, "%s: %s", what, hipGetErrorString(e));
}

constexpr int64_t kMaxN = 8192;
constexpr int kWaveMaxN = 64;

bool ranges_overlap(const float* a, int64_t a_elems, const float* b, int64_t b_elems) {
  const uintptr_t a0 = (uintptr_t)a, a1 = a0 + (uintptr_t)a_elems * 4;
  const uintptr_t b0 = (uintptr_t)b, b1 = b0 + (uintptr_t)b_elems * 4;
  return a0 < b1 && b0 < a1;
}

int64_t span_elems(int64_t batch, int64_t n, int64_t s0, int64_t s1, int64_t s2) {
  return (batch - 1) * s0 + (n - 1) * s1 + (n - 1) * s2 + 1;
}

}  // namespace

extern "C" {

int fastqr_version(void) { return 1; }

const char* fastqr_last_error(void) { return g_last_error; }

void fastqr_debug_force_error(int code) { g_forced_error = code; }

const char* fastqr_path_name(int64_t n) {
  if (n <= kWaveMaxN) return "wave64";
  return "blocked";
}

size_t fastqr_workspace_bytes(int64_t batch, int64_t n) {
  if (batch <= 0 || n <= kWaveMaxN) return 0;
  const size_t t_bytes = (size_t)batch * fastqr::kMaxPanel * fastqr::kMaxPanel * sizeof(float);
  return (t_bytes + 255) & ~(size_t)255;
}

int fastqr_geqrf_f32(const float* A, int64_t batch, int64_t n, int64_t a_s0, int64_t a_s1, int64_t a_s2,
                     float* H, int64_t h_s0, int64_t h_s1, int64_t h_s2, float* tau, int64_t tau_s0,
                     int64_t tau_s1, void* workspace, size_t workspace_bytes, void* stream_ptr) {
  g_last_error[0] = '\0';
  if (g_forced_error != 0) {
    const int code = g_forced_error;
    g_forced_error = 0;
    return fail(code, "forced error %d (test hook)", code);
  }
  if (batch < 0 || n < 0) return fail(FASTQR_EINVAL, "batch and n must be non-negative (got %lld, %lld)",
                                      (long long)batch, (long long)n);
  if (batch == 0 || n == 0) return FASTQR_OK;
  if (n > kMaxN) return fail(FASTQR_EINVAL, "n=%lld exceeds the supported maximum %lld", (long long)n,
                             (long long)kMaxN);
  if (batch > 2147483647LL) return fail(FASTQR_EINVAL, "batch too large");
  if (!A || !H || !tau) return fail(FASTQR_EINVAL, "A, H and tau must be non-null device pointers");
  if (a_s0 < 0 || a_s1 < 0 || a_s2 < 0 || h_s0 < 0 || h_s1 < 0 || h_s2 < 0 || tau_s0 < 0 || tau_s1 < 0)
    return fail(FASTQR_EINVAL, "negative strides are not supported");
  if (batch > 1 && (h_s0 == 0 || tau_s0 == 0))
    return fail(FASTQR_EINVAL, "H and tau batch strides must be non-zero when batch > 1");
  if (n > 1 && tau_s1 == 0) return fail(FASTQR_EINVAL, "tau column stride must be non-zero");

  const hipStream_t stream = (hipStream_t)stream_ptr;
  const int ni = (int)n;

  if (n <= kWaveMaxN) {
    if (h_s1 == 0 || h_s2 == 0) return fail(FASTQR_ELAYOUT, "H strides must be non-zero");
    const bool same = (A == H && a_s0 == h_s0 && a_s1 == h_s1 && a_s2 == h_s2);
    if (!same && ranges_overlap(A, span_elems(batch, n, a_s0, a_s1, a_s2), H, span_elems(batch, n, h_s0, h_s1, h_s2)))
      return fail(FASTQR_EOVERLAP, "A and H overlap with different layouts");
    const hipError_t e = fastqr::launch_qr_wave(A, batch, ni, a_s0, a_s1, a_s2, H, h_s0, h_s1, h_s2, tau,
                                                tau_s0, tau_s1, stream);
    return e == hipSuccess ? FASTQR_OK : hip_fail(e, "qr_wave launch");
  }

  // Blocked path: columns of H must be contiguous.
  if (h_s1 != 1 || h_s2 < n)
    return fail(FASTQR_ELAYOUT,
                "H must have contiguous columns (stride (*, 1, >=n)); got (%lld, %lld, %lld)",
                (long long)h_s0, (long long)h_s1, (long long)h_s2);
  if (batch > 1 && h_s0 < h_s2 * n)
    return fail(FASTQR_ELAYOUT, "H batch stride %lld smaller than one matrix (%lld)", (long long)h_s0,
                (long long)(h_s2 * n));
  const size_t need = fastqr_workspace_bytes(batch, n);
  if (workspace_bytes < need || (need > 0 && workspace == nullptr))
    return fail(FASTQR_EWORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
  if (((uintptr_t)workspace & 15) != 0) return fail(FASTQR_EWORKSPACE, "workspace must be 16-byte aligned");
  const bool same = (A == H && a_s0 == h_s0 && a_s1 == h_s1 && a_s2 == h_s2);
  if (!same && ranges_overlap(A, span_elems(batch, n, a_s0, a_s1, a_s2), H, span_elems(batch, n, h_s0, h_s1, h_s2)))
    return fail(FASTQR_EOVERLAP, "A and H overlap with different layouts");

  float* Tws = (float*)workspace;
  const bool vec = ((uintptr_t)H % 16 == 0) && (h_s0 % 4 == 0) && (h_s2 % 4 == 0) && (n % 4 == 0);
  hipError_t e = hipSuccess;
  if (!same) {
    e = fastqr::launch_copy_colmajor(A, batch, ni, a_s0, a_s1, a_s2, H, h_s0, h_s2, stream);
    if (e != hipSuccess) return hip_fail(e, "copy launch");
  }
  for (int k0 = 0; k0 < ni;) {
    const int nb = fastqr::panel_width_for(ni - k0);
    e = fastqr::launch_panel(H, batch, h_s0, h_s2, tau, tau_s0, tau_s1, Tws, ni, k0, stream);
    if (e != hipSuccess) return hip_fail(e, "panel launch");
    e = fastqr::launch_update(H, batch, h_s0, h_s2, Tws, ni, k0, nb, vec, stream);
    if (e != hipSuccess) return hip_fail(e, "update launch");
    k0 += nb;
  }
  return FASTQR_OK;
}

}  // extern "C"
