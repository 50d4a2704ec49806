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

#include <vector>

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

// ---- opt-in per-launch profiling (fastqr_profile_*) ----------------------
enum Kind { kCopy = 0, kPanel = 1, kUpdate = 2, kWave = 3, kLds = 4 };
const char* const kKindNames[FASTQR_PROFILE_KINDS] = {"copy", "panel", "update", "wave64", "lds"};

struct Record {
  int kind;
  hipEvent_t start, stop;
  double flops, bytes;
};

struct Totals {
  int64_t launches = 0;
  double ms = 0.0, flops = 0.0, bytes = 0.0;
};

struct Profiler {
  bool on = false;
  std::vector<Record> pending;
  std::vector<hipEvent_t> pool;
  Totals totals[FASTQR_PROFILE_KINDS];

  hipEvent_t take() {
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }

  hipError_t drain() {
    hipError_t err = hipSuccess;
    for (Record& r : pending) {
      float ms = 0.0f;
      hipError_t e = hipEventSynchronize(r.stop);
      if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.start, r.stop);
      if (e != hipSuccess && err == hipSuccess) err = e;
      Totals& t = totals[r.kind];
      t.launches += 1;
      t.ms += ms;
      t.flops += r.flops;
      t.bytes += r.bytes;
      pool.push_back(r.start);
      pool.push_back(r.stop);
    }
    pending.clear();
    return err;
  }
};

thread_local Profiler g_prof;

// Launch `fn` (returning hipError_t), bracketed by events when profiling.
template <class F>
hipError_t timed(int kind, double flops, double bytes, hipStream_t stream, F&& fn) {
  if (!g_prof.on) return fn();
  hipEvent_t a = g_prof.take(), b = g_prof.take();
  if (!a || !b) return fn();
  (void)hipEventRecord(a, stream);
  const hipError_t e = fn();
  (void)hipEventRecord(b, stream);
  g_prof.pending.push_back(Record{kind, a, b, flops, bytes});
  return e;
}

}  // namespace

extern "C" {

int fastqr_profile_enable(int on) {
  if (on) {
    (void)g_prof.drain();
    for (Totals& t : g_prof.totals) t = Totals{};
  }
  g_prof.on = on != 0;
  return FASTQR_OK;
}

int fastqr_profile_collect(int kind, int64_t* launches, double* milliseconds, double* flops, double* bytes) {
  if (kind < 0 || kind >= FASTQR_PROFILE_KINDS) return fail(FASTQR_EINVAL, "profile kind %d out of range", kind);
  const hipError_t e = g_prof.drain();
  const Totals& t = g_prof.totals[kind];
  if (launches) *launches = t.launches;
  if (milliseconds) *milliseconds = t.ms;
  if (flops) *flops = t.flops;
  if (bytes) *bytes = t.bytes;
  return e == hipSuccess ? FASTQR_OK : hip_fail(e, "profile collect");
}

const char* fastqr_profile_kind_name(int kind) {
  return (kind >= 0 && kind < FASTQR_PROFILE_KINDS) ? kKindNames[kind] : "";
}

int fastqr_version(void) { return 1; }

const char* fastqr_last_error(void) { return g_last_error; }

void fastqr_debug_force_error(int code) { g_forced_error = code; }

const char* fastqr_path_name(int64_t n) {
  if (n <= kWaveMaxN) return "wave64";
  return "blocked";
}

size_t fastqr_workspace_bytes(int64_t batch, int64_t n) {
  if (batch <= 0 || n <= kWaveMaxN) return 0;
  const size_t t_bytes = (size_t)batch * fastqr::kMaxSlots * 32 * 32 * sizeof(float);
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
    const double nn = (double)n;
    const hipError_t e = timed(kWave, batch * 4.0 * nn * nn * nn / 3.0, batch * (8.0 * nn * nn + 4.0 * nn), stream,
                               [&] {
                                 return fastqr::launch_qr_wave(A, batch, ni, a_s0, a_s1, a_s2, H, h_s0, h_s1, h_s2,
                                                               tau, tau_s0, tau_s1, stream);
                               });
    return e == hipSuccess ? FASTQR_OK : hip_fail(e, "qr_wave launch");
  }

  // Blocked path: columns of H must be contiguous.
  if (h_s1 != 1 || h_s2 < n)
    return fail(FASTQR_ELAYOUT,
                "H must have contiguous columns (stride (*, 1, >=n)); got (%lld, %lld, %lld)",
                (long long)h_s0, (long long)h_s1, (long long)h_s2);
  if (h_s2 * n * 4 >= (int64_t)1 << 31)
    return fail(FASTQR_ELAYOUT, "one matrix of H spans %lld bytes; the blocked path addresses at most 2 GiB",
                (long long)(h_s2 * n * 4));
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
  const double bd = (double)batch;
  if (!same) {
    e = timed(kCopy, 0.0, bd * 8.0 * (double)n * (double)n, stream, [&] {
      return fastqr::launch_copy_colmajor(A, batch, ni, a_s0, a_s1, a_s2, H, h_s0, h_s2, stream);
    });
    if (e != hipSuccess) return hip_fail(e, "copy launch");
  }
  // Panels are processed in groups of up to kMaxWY: each panel is followed by
  // a narrow update of the rest of its group's columns; after the group, one
  // wide update applies all of the group's transforms to the trailing columns.
  for (int g0 = 0; g0 < ni;) {
    const int mg = ni - g0;
    const int nb = fastqr::panel_width_for(mg);
    const int g_end = (g0 + fastqr::kMaxWY * nb < ni) ? g0 + fastqr::kMaxWY * nb : ni;
    int npan = 0;
    for (int pk = g0; pk < g_end; pk += nb, ++npan) {
      const double m = ni - pk;
      const double wd = (m < nb) ? m : nb;
      e = timed(kPanel, bd * (2.0 * m * wd * wd - 2.0 * wd * wd * wd / 3.0), bd * 8.0 * m * wd, stream, [&] {
        return fastqr::launch_panel(H, batch, h_s0, h_s2, tau, tau_s0, tau_s1, Tws, ni, pk, nb, mg, npan, vec,
                                    stream);
      });
      if (e != hipSuccess) return hip_fail(e, "panel launch");
      const int c0 = pk + (int)wd;
      if (c0 < g_end) {
        const double c = g_end - c0;
        e = timed(kUpdate, bd * 4.0 * m * wd * c, bd * (8.0 * m * c + 4.0 * m * wd), stream, [&] {
          return fastqr::launch_wy_update(H, batch, h_s0, h_s2, Tws, ni, pk, nb, npan, 1, c0, g_end, vec, stream);
        });
        if (e != hipSuccess) return hip_fail(e, "update launch");
      }
    }
    if (g_end < ni) {
      const double m = mg;
      const double wg = g_end - g0;
      const double c = ni - g_end;
      e = timed(kUpdate, bd * 4.0 * m * wg * c, bd * (8.0 * m * c + 4.0 * m * wg), stream, [&] {
        return fastqr::launch_wy_update(H, batch, h_s0, h_s2, Tws, ni, g0, nb, 0, npan, g_end, ni, vec, stream);
      });
      if (e != hipSuccess) return hip_fail(e, "update launch");
    }
    g0 = g_end;
  }
  return FASTQR_OK;
}

}  // extern "C"
