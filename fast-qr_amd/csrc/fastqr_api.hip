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

#include <algorithm>
#include <atomic>
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

constexpr int64_t kMaxN = 4096;
// Largest n of the mixed-precision variant (its panels and Q^T C calls).
constexpr int64_t kMixedMaxN = 2048;
constexpr int kWaveMaxN = 64;
// Tall matrices use the row-split trailing update (a 32-column strip of more
// than 2048 rows does not fit in one workgroup's registers, and small batches
// leave most of the GPU idle with one workgroup per strip).
constexpr int64_t kRowSplitMinN = 2049;

bool use_rowsplit(int64_t /*batch*/, int64_t n) { return n >= kRowSplitMinN; }

// Panel groups per factorisation: at least 64 columns each, n <= kMaxN.
constexpr int kMaxGroups = (int)(kMaxN / 64);

// Strip-resident path, small batches of tall matrices (8 x 2048): the narrow
// update after a 32-column panel taller than kWyrNarrowMinRows runs on the
// row-split kernels (partial products over row blocks, then the apply), which
// spread it over hundreds of one-wave workgroups instead of one workgroup per
// (matrix, strip).  Its partials and W need scratch beyond the T slots.
constexpr int64_t kWyrNarrowMaxBatch = 16;
constexpr int kWyrNarrowMinRows = 1024;
bool use_wyr_narrow(int64_t batch, int64_t n) { return batch <= kWyrNarrowMaxBatch && n > kWyrNarrowMinRows; }

bool ranges_overlap(const float* a, int64_t a_elems, const float* b, int64_t b_elems) {
  const uintptr_t a0 = (uintptr_t)a, a1 = a0 + (uintptr_t)a_elems * 4;
  const uintptr_t b0 = (uintptr_t)b, b1 = b0 + (uintptr_t)b_elems * 4;
  return a0 < b1 && b0 < a1;
}

int64_t span_elems(int64_t batch, int64_t n, int64_t s0, int64_t s1, int64_t s2) {
  return (batch - 1) * s0 + (n - 1) * s1 + (n - 1) * s2 + 1;
}

// ---- opt-in per-launch profiling (fastqr_profile_*) ----------------------
enum Kind { kCopy = 0, kPanel = 1, kUpdate = 2, kWave = 3, kLds = 4, kUpdateRows = 5 };
const char* const kKindNames[FASTQR_PROFILE_KINDS] = {"copy", "panel", "update", "wave64", "lds", "update_rowsplit"};

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

// ---- side stream and events for panel look-ahead (one set per device) ------
struct DeviceAux {
  hipStream_t side = nullptr;
  std::vector<hipEvent_t> events;
  size_t next = 0;
  hipEvent_t take() {
    if (next == events.size()) {
      hipEvent_t e = nullptr;
      if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) return nullptr;
      events.push_back(e);
    }
    return events[next++];
  }
};

thread_local std::vector<DeviceAux> g_aux;

DeviceAux* device_aux() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return nullptr;
  if ((size_t)dev >= g_aux.size()) g_aux.resize(dev + 1);
  DeviceAux& a = g_aux[dev];
  if (!a.side && hipStreamCreateWithFlags(&a.side, hipStreamNonBlocking) != hipSuccess) {
    a.side = nullptr;
    return nullptr;
  }
  a.next = 0;
  return &a;
}

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


// Blocked QR with the row-split trailing update (tall matrices).  Panels are
// grouped (up to kMaxWY panels, at most kWyrMaxK columns).  On the side stream:
// each panel, then a row-split update of the rest of its group by that panel;
// after the group its T factors and Gram matrix are joined into the group T and
// the group is applied to the next group's columns (look-ahead).  On the
// caller's stream the group is applied to everything right of the next group,
// overlapping the next group's panels.  Two scratch areas (one per stream) and
// two banks of T slots and group T alternate by group parity.
int run_rowsplit(float* H, int64_t batch, int64_t hs0, int64_t ldh, float* tau, int64_t ts0, int64_t ts1, float* Tws,
                 int n, bool vec, bool single_stream, hipStream_t stream) {
  using fastqr::WyrCall;
  const int64_t slot_floats = batch * fastqr::kMaxSlots * 1024;
  float* Tg0 = Tws + slot_floats;
  // one scratch area per stream (a single stream needs one)
  float* area[2] = {Tg0 + 2 * batch * fastqr::kWyrTgStride, nullptr};
  area[1] = single_stream ? area[0] : area[0] + fastqr::wyr_workspace_floats(batch, n);
  const double bd = (double)batch;

  struct Group {
    int g0, nb, g_end, npan, slot_base;
  };
  Group groups[kMaxGroups];
  int ngroups = 0;
  for (int g0 = 0; g0 < n; ++ngroups) {
    const int nb = fastqr::panel_width_for(n - g0);
    const int span = fastqr::kMaxWY * nb < fastqr::kWyrMaxK ? fastqr::kMaxWY * nb : fastqr::kWyrMaxK;
    const int g_end = (g0 + span < n) ? g0 + span : n;
    if (ngroups == kMaxGroups) return fail(FASTQR_EINVAL, "too many panel groups for n=%d", n);
    groups[ngroups] = Group{g0, nb, g_end, (g_end - g0 + nb - 1) / nb, (ngroups & 1) * fastqr::kMaxWY};
    g0 = g_end;
  }
  // Single stream: the side stream's work (panels, narrow and look-ahead
  // updates) is issued on the caller's stream in the same order, so each
  // group's wide update simply runs before the next group's panels.
  DeviceAux* aux = single_stream ? nullptr : device_aux();
  if (!single_stream && !aux) return fail(FASTQR_EINVAL, "cannot create the side stream");
  const hipStream_t side = single_stream ? stream : aux->side;
  auto join = [&](hipStream_t waiter, hipStream_t signaller) -> hipError_t {
    if (single_stream) return hipSuccess;
    hipEvent_t ev = aux->take();
    if (!ev) return hipErrorOutOfMemory;
    hipError_t e = hipEventRecord(ev, signaller);
    if (e == hipSuccess) e = hipStreamWaitEvent(waiter, ev, 0);
    return e;
  };
  auto base_call = [&](int kv, int k, int c_begin, int c_end, float* scratch) {
    WyrCall c{};
    c.H = H;
    c.hs0 = hs0;
    c.ldh = (int)ldh;
    c.n = n;
    c.batch = batch;
    c.kv = kv;
    c.k = k;
    c.c_begin = c_begin;
    c.c_end = c_end;
    c.Tws = Tws;
    c.scratch = scratch;
    c.rows_per_blk = fastqr::wyr_rows_per_block(n - kv, batch, c_end - c_begin);
    c.vec = vec;
    return c;
  };
  auto run_wyr = [&](const WyrCall& c, hipStream_t st) -> hipError_t {
    const double m = n - c.kv, k = c.k;
    const double cx = c.c_end - c.c_begin - (c.gram ? 32.0 * ((c.k + 31) / 32) : 0.0);
    return timed(kUpdateRows, bd * 4.0 * m * k * cx, bd * (12.0 * m * cx + 8.0 * m * k), st,
                 [&] { return fastqr::launch_wyr(c, st); });
  };

  hipError_t e = join(side, stream);  // the side stream starts after the copy
  if (e != hipSuccess) return hip_fail(e, "stream join");
  bool rest_done[kMaxGroups] = {};
  for (int gi = 0; gi < ngroups; ++gi) {
    const Group& G = groups[gi];
    for (int i = 0; i < G.npan; ++i) {
      const int pk = G.g0 + i * G.nb;
      const double m = n - pk;
      const int w = (n - pk < G.nb) ? n - pk : G.nb;
      e = timed(kPanel, bd * (2.0 * m * w * w - 2.0 * w * w * w / 3.0), bd * 8.0 * m * w, side, [&] {
        return fastqr::launch_panel(H, batch, hs0, ldh, tau, ts0, ts1, Tws, n, pk, G.nb, n - pk, G.slot_base + i, vec,
                                    side);
      });
      if (e != hipSuccess) return hip_fail(e, "panel launch");
      if (pk + w < G.g_end) {
        WyrCall c = base_call(pk, w, pk + w, G.g_end, area[0]);
        c.Tslot = Tws + (G.slot_base + i) * 1024;
        c.hi_prio = true;
        if ((e = run_wyr(c, side)) != hipSuccess) return hip_fail(e, "narrow update launch");
      }
    }
    if (gi + 1 == ngroups) break;
    const Group& Nx = groups[gi + 1];
    float* Tg = Tg0 + (int64_t)(gi & 1) * batch * fastqr::kWyrTgStride;
    // the next group's columns last received the previous group's wide update
    if (gi >= 1 && rest_done[gi - 1] && (e = join(side, stream)) != hipSuccess) return hip_fail(e, "stream join");
    WyrCall c = base_call(G.g0, G.g_end - G.g0, G.g0, Nx.g_end, area[0]);
    c.gram = true;
    c.use_tg = true;
    c.q = G.npan;
    c.nb = G.nb;
    c.slot0 = G.slot_base;
    c.Tg = Tg;
    c.hi_prio = true;
    if ((e = run_wyr(c, side)) != hipSuccess) return hip_fail(e, "look-ahead update launch");
    if (Nx.g_end < n) {
      if ((e = join(stream, side)) != hipSuccess) return hip_fail(e, "stream join");
      WyrCall r = base_call(G.g0, G.g_end - G.g0, Nx.g_end, n, area[1]);
      r.use_tg = true;
      r.Tg = Tg;
      if ((e = run_wyr(r, stream)) != hipSuccess) return hip_fail(e, "trailing update launch");
      rest_done[gi] = true;
    }
  }
  if ((e = join(stream, side)) != hipSuccess) return hip_fail(e, "stream join");
  return FASTQR_OK;
}

// Workspace of the blocked path: the T slots; for tall matrices (row-split
// update) two group-T banks and the partial products of each stream.
size_t workspace_bytes_for(int64_t batch, int64_t n, bool single_stream) {
  if (batch <= 0 || n <= fastqr::kLdsMaxN || n > kMaxN) return 0;
  size_t floats = (size_t)batch * fastqr::kMaxSlots * 32 * 32;
  if (use_rowsplit(batch, n))
    floats += 2 * (size_t)batch * fastqr::kWyrTgStride +
              (single_stream ? 1 : 2) * fastqr::wyr_workspace_floats(batch, (int)n);
  else if (use_wyr_narrow(batch, n))
    floats += fastqr::wyr_workspace_floats(batch, (int)n);
  return (floats * sizeof(float) + 255) & ~(size_t)255;
}

// fastqr_geqrf_f32 after the test hook.  `single_stream` keeps every launch
// on the caller's stream (no side stream, no events: nothing is created).
int geqrf_impl(const float* A, int64_t batch, int64_t n, int64_t a_s0, int64_t a_s1, int64_t a_s2, float* H,
               int64_t h_s0, int64_t h_s1, int64_t h_s2, float* tau, int64_t tau_s0, int64_t tau_s1, void* workspace,
               size_t workspace_bytes, bool single_stream, void* stream_ptr) {
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

  if (n <= fastqr::kLdsMaxN) {
    // one workgroup (or wave) per matrix reads A once and writes H once: any H strides
    if (h_s1 == 0 || h_s2 == 0) return fail(FASTQR_ELAYOUT, "H strides must be non-zero");
    const bool same = (A == H && a_s0 == h_s0 && a_s1 == h_s1 && a_s2 == h_s2);
    if (!same && ranges_overlap(A, span_elems(batch, n, a_s0, a_s1, a_s2), H, span_elems(batch, n, h_s0, h_s1, h_s2)))
      return fail(FASTQR_EOVERLAP, "A and H overlap with different layouts");
    const double nn = (double)n;
    const double fl = batch * 4.0 * nn * nn * nn / 3.0, by = batch * (8.0 * nn * nn + 4.0 * nn);
    if (n <= kWaveMaxN) {
      const hipError_t e = timed(kWave, fl, by, stream, [&] {
        return fastqr::launch_qr_wave(A, batch, ni, a_s0, a_s1, a_s2, H, h_s0, h_s1, h_s2, tau, tau_s0, tau_s1, stream);
      });
      return e == hipSuccess ? FASTQR_OK : hip_fail(e, "qr_wave launch");
    }
    const hipError_t e = timed(kLds, fl, by, stream, [&] {
      return fastqr::launch_qr_lds(A, batch, ni, a_s0, a_s1, a_s2, H, h_s0, h_s1, h_s2, tau, tau_s0, tau_s1, stream);
    });
    return e == hipSuccess ? FASTQR_OK : hip_fail(e, "qr_lds launch");
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
  const size_t need = workspace_bytes_for(batch, n, single_stream);
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
  // A -> H, columns [c0, c1)
  auto copy_cols = [&](int c0, int c1, int max_wgs = 0) -> hipError_t {
    if (same || c1 <= c0) return hipSuccess;
    return timed(kCopy, 0.0, bd * 8.0 * (double)n * (double)(c1 - c0), stream, [&] {
      return fastqr::launch_copy_colmajor(A, batch, ni, a_s0, a_s1, a_s2, H, h_s0, h_s2, c0, c1, stream, max_wgs);
    });
  };
  if (use_rowsplit(batch, n)) {
    if ((e = copy_cols(0, ni)) != hipSuccess) return hip_fail(e, "copy launch");
    return run_rowsplit(H, batch, h_s0, h_s2, tau, tau_s0, tau_s1, Tws, ni, vec, single_stream, stream);
  }

  // Panels are processed in groups of up to 128 columns (kMaxWY transforms
  // of 32 columns, one T slot each).  A group is two panels of 64 columns or
  // four of 32 (panel_width_wide); each panel but the group's last is followed by a narrow update
  // of the group's remaining columns.  The group's transforms are then applied
  // together to the columns right of it.  Look-ahead: that wide update is
  // split into the next group's columns (first) and the rest; the next
  // group's panels run on a side stream while the rest is updated on the
  // caller's stream.  T slots rotate over three banks.
  struct Group {
    int g0, pw, g_end, slot_base;
  };
  constexpr int kTw = 32;  // transform width of the strip-resident update
  Group groups[kMaxGroups];
  int ngroups = 0;
  for (int g0 = 0; g0 < ni; ++ngroups) {
    const int g_end = (g0 + fastqr::kMaxWY * kTw < ni) ? g0 + fastqr::kMaxWY * kTw : ni;
    groups[ngroups] = Group{g0, fastqr::panel_width_wide(ni - g0, batch), g_end, (ngroups % 3) * fastqr::kMaxWY};
    g0 = g_end;
  }
  // narrow updates on the row-split kernels (small batches of tall matrices);
  // one scratch area: narrow updates run one at a time, on the side stream
  const bool wyr_narrow = use_wyr_narrow(batch, n);
  float* const wyr_scratch = Tws + (size_t)batch * fastqr::kMaxSlots * 1024;
  // Narrow updates inside a group, left-looking: after each panel only the
  // next panel's columns are updated, by all of the group's transforms so far
  // in one launch (the later columns wait for their own turn), so the launch
  // on the critical path covers one panel instead of the rest of the group and
  // loads its columns once for several transforms.  Groups whose narrow
  // updates run on the row-split kernels keep one transform per launch over
  // the rest of the group (those kernels join several transforms only with a
  // group T).
  // a_first: the group's columns right of its first panel are not in H yet
  // (row-major input, only the first panel copied): each narrow update reads
  // the next panel's columns from A, their first touch.
  auto run_panels = [&](const Group& G, hipStream_t st, bool a_first = false) -> hipError_t {
    const bool left_looking = !(wyr_narrow && ni - G.g0 > kWyrNarrowMinRows);
    for (int pk = G.g0; pk < G.g_end; pk += G.pw) {
      const double m = ni - pk;
      const int wi = (G.g_end - pk < G.pw) ? G.g_end - pk : G.pw;
      const double wd = wi;
      const int slot = G.slot_base + (pk - G.g0) / kTw;
      hipError_t err = timed(kPanel, bd * (2.0 * m * wd * wd - 2.0 * wd * wd * wd / 3.0), bd * 8.0 * m * wd, st, [&] {
        return fastqr::launch_panel(H, batch, h_s0, h_s2, tau, tau_s0, tau_s1, Tws, ni, pk, G.pw, ni - pk, slot, vec,
                                    st);
      });
      if (err != hipSuccess) return err;
      const int c0 = pk + wi;
      if (c0 < G.g_end && left_looking) {
        const int c1 = (G.g_end - c0 < G.pw) ? G.g_end : c0 + G.pw;  // the next panel's columns
        const int nwy = (c0 - G.g0) / kTw;                              // transforms of the group so far
        double fl = 0.0;
        for (int j = 0; j < nwy; ++j) fl += 4.0 * (ni - G.g0 - kTw * j) * kTw * (c1 - c0);
        const double mg = ni - G.g0;
        err = timed(kUpdate, bd * fl, bd * (8.0 * mg * (c1 - c0) + 4.0 * mg * (c0 - G.g0)), st, [&] {
          return fastqr::launch_wy_update(H, batch, h_s0, h_s2, Tws, ni, G.g0, kTw, G.slot_base, nwy, c0, c1, vec,
                                          true, 0, st, false, a_first ? A : nullptr, a_s0, a_s1);
        });
        if (err != hipSuccess) return err;
      } else if (c0 < G.g_end) {
        const double c = G.g_end - c0;
        if (wyr_narrow && wi <= kTw && ni - pk > kWyrNarrowMinRows) {
          fastqr::WyrCall wc{};
          wc.H = H;
          wc.hs0 = h_s0;
          wc.ldh = (int)h_s2;
          wc.n = ni;
          wc.batch = batch;
          wc.kv = pk;
          wc.k = wi;
          wc.c_begin = c0;
          wc.c_end = G.g_end;
          wc.Tws = Tws;
          wc.Tslot = Tws + slot * 1024;
          wc.scratch = wyr_scratch;
          wc.rows_per_blk = fastqr::wyr_rows_per_block(ni - pk, batch, G.g_end - c0);
          wc.vec = vec;
          wc.hi_prio = true;
          err = timed(kUpdateRows, bd * 4.0 * m * wd * c, bd * (8.0 * m * c + 4.0 * m * wd), st,
                      [&] { return fastqr::launch_wyr(wc, st); });
        } else {
          err = timed(kUpdate, bd * 4.0 * m * wd * c, bd * (8.0 * m * c + 4.0 * m * wd), st, [&] {
            return fastqr::launch_wy_update(H, batch, h_s0, h_s2, Tws, ni, pk, kTw, slot, (wi + kTw - 1) / kTw, c0,
                                            G.g_end, vec, true, 0, st);
          });
        }
        if (err != hipSuccess) return err;
      }
    }
    return hipSuccess;
  };
  // The wide update that overlaps the next group's panels leaves one CU per
  // matrix to them when the batch is smaller than the GPU: each panel
  // workgroup needs most of a CU's registers and would otherwise wait for a
  // CU to drain behind the update's workgroups.  Small batches leave four, so
  // the narrow update after each panel (one workgroup per matrix and strip)
  // runs beside the wide update too; the wide update has slack (measured on
  // MI355X: 8 x 2048 5% faster; eight CUs per matrix gain nothing more).
  // Small matrices run every launch on the caller's stream: their trailing
  // updates are short, and the side stream's event hand-offs cost more than
  // the overlap gains (measured on MI355X, side stream -> one stream: 40 x 352
  // 363 -> 343 us, 40 x 320 315 -> 272, 40 x 448 483 -> 455, 256 x 352 567 ->
  // 558, 640 x 256 593 -> 581; but 40 x 512 561 -> 579 and 640 x 352 1,075 ->
  // 1,125).
  const bool one_stream = single_stream || n <= 256 || (n <= 448 && batch <= 256);
  DeviceAux* aux = (ngroups > 2 && !one_stream) ? device_aux() : nullptr;
  int num_cus = 0, dev = 0;
  if (!aux && ngroups > 2) {
    num_cus = 0;  // one stream: the wide update has the whole GPU
  } else if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&num_cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    num_cus = 0;
  int rest_cus = 0;
  if (num_cus > 0 && batch < num_cus / 2)
    rest_cus = (4 * batch <= num_cus / 2) ? num_cus - 4 * (int)batch : num_cus - (int)batch;
  else if (num_cus > 0)
    // Large batches: every CU keeps one workgroup slot free, so the next
    // group's panels share the SIMDs with the wide update instead of waiting
    // for its workgroups to drain (measured on MI355X: 640 x 512 2,410 -> 2,352 us,
    // 60 x 1024 2,095 -> 2,084 us; two slots free was slower).
    rest_cus = fastqr::kWyLeaveOneSlot;
  // from_a: the columns are read from the row-major input A (their first update; not copied)
  auto run_update = [&](const Group& G, int c_begin, int c_end, bool critical, hipStream_t st,
                        bool from_a = false) -> hipError_t {
    if (c_end <= c_begin) return hipSuccess;
    const double m = ni - G.g0, wg = G.g_end - G.g0, c = c_end - c_begin;
    return timed(kUpdate, bd * 4.0 * m * wg * c, bd * (8.0 * m * c + 4.0 * m * wg), st, [&] {
      return fastqr::launch_wy_update(H, batch, h_s0, h_s2, Tws, ni, G.g0, kTw, G.slot_base,
                                      (G.g_end - G.g0 + kTw - 1) / kTw, c_begin, c_end, vec, critical,
                                      critical ? 0 : rest_cus, st, false, from_a ? A : nullptr, a_s0, a_s1);
    });
  };

  // Only the first group's columns are copied before its panels start.  A
  // row-major input is not copied any further: the first group's look-ahead
  // and wide updates, the first kernels that touch the other columns, read
  // them from A and write them to H (one read of A and no extra pass over H;
  // a copy beside the first group's panels takes HBM and CU slots from them).
  // Other layouts copy the rest: with the side stream on the caller's stream
  // beside those panels, ahead of the first look-ahead update; on one stream
  // up front.
  const bool from_a = !same && a_s2 == 1 && a_s1 >= n && 4 * ((n - 1) * a_s1 + n) < ((int64_t)1 << 31);
  const int c_first = (aux || from_a) ? groups[0].g_end : ni;
  // With left-looking narrow updates in the first group, only its first
  // panel's columns are copied: the narrow updates read the next panels'
  // columns from A (the copy is on the critical path before the first panel;
  // 640 x 512: 128 columns 52 us, 32 columns 13 us).
  const bool first_from_a =
      from_a && !(wyr_narrow && ni - groups[0].g0 > kWyrNarrowMinRows) && groups[0].pw < groups[0].g_end;
  if ((e = copy_cols(0, first_from_a ? groups[0].pw : c_first)) != hipSuccess) return hip_fail(e, "copy launch");
  if (!aux) {
    for (int g = 0; g < ngroups; ++g) {
      const Group& G = groups[g];
      e = run_panels(G, stream, g == 0 && first_from_a);
      if (e == hipSuccess) e = run_update(G, G.g_end, ni, false, stream, g == 0 && from_a);
      if (e != hipSuccess) return hip_fail(e, "blocked launch");
    }
    return FASTQR_OK;
  }
  // The panels and the look-ahead updates (the critical path) run in order on
  // the side stream.  The wide update of group g runs on the caller's stream
  // after g's look-ahead update (not beside it: the look-ahead is on the
  // critical path), overlapping the next group's panels, in two parts: first
  // the columns of group g+2, which the next look-ahead update reads (it waits
  // for that part only), then everything right of them.  T slots rotate over
  // three banks: group g+1's panels overwrite the bank of group g-2, so they
  // wait for g-2's wide update to end (long done in practice).
  const hipStream_t side = aux->side;
  auto record = [&](hipStream_t st) -> hipEvent_t {
    hipEvent_t evt = aux->take();
    if (evt && hipEventRecord(evt, st) != hipSuccess) evt = nullptr;
    return evt;
  };
  hipEvent_t ev = record(stream);  // the side stream must not run ahead of work already queued on `stream`
  if (!ev) return fail(FASTQR_EINVAL, "cannot record HIP events");
  if ((e = hipStreamWaitEvent(side, ev, 0)) != hipSuccess) return hip_fail(e, "stream join");
  if ((e = run_panels(groups[0], side, first_from_a)) != hipSuccess) return hip_fail(e, "panel launch");
  // Four workgroups per CU keep the copy at HBM speed and leave the CUs' other
  // slots to the first group's panels: uncapped, its tens of thousands of
  // small workgroups fill every CU and the panels wait for the copy to drain
  // (640 x 512: the first panel 46 -> 196 us beside it).
  if (!from_a && (e = copy_cols(c_first, ni, num_cus > 0 ? 4 * num_cus : 0)) != hipSuccess)
    return hip_fail(e, "copy launch");
  // columns of the next look-ahead update ready (first: the copy)
  hipEvent_t ev_near = (c_first < ni && !from_a) ? record(stream) : nullptr;
  if (c_first < ni && !from_a && !ev_near) return fail(FASTQR_EINVAL, "cannot record HIP events");
  hipEvent_t ev_rest[kMaxGroups] = {};  // group g's wide update ended
  for (int g = 0; g + 1 < ngroups; ++g) {
    const Group& G = groups[g];
    const Group& Nx = groups[g + 1];
    if (ev_near && (e = hipStreamWaitEvent(side, ev_near, 0)) != hipSuccess) return hip_fail(e, "stream join");
    if ((e = run_update(G, Nx.g0, Nx.g_end, true, side, from_a && g == 0)) != hipSuccess)
      return hip_fail(e, "update launch");
    hipEvent_t ev_la = record(side);
    if (!ev_la) return fail(FASTQR_EINVAL, "cannot record HIP events");
    if (g >= 2 && (e = hipStreamWaitEvent(side, ev_rest[g - 2], 0)) != hipSuccess) return hip_fail(e, "stream join");
    if ((e = run_panels(Nx, side)) != hipSuccess) return hip_fail(e, "panel launch");
    if ((e = hipStreamWaitEvent(stream, ev_la, 0)) != hipSuccess) return hip_fail(e, "stream join");
    ev_near = nullptr;
    if (g + 2 < ngroups) {
      const Group& N2 = groups[g + 2];
      if ((e = run_update(G, N2.g0, N2.g_end, false, stream, from_a && g == 0)) != hipSuccess)
        return hip_fail(e, "update launch");
      if (!(ev_near = record(stream))) return fail(FASTQR_EINVAL, "cannot record HIP events");
      if ((e = run_update(G, N2.g_end, ni, false, stream, from_a && g == 0)) != hipSuccess)
        return hip_fail(e, "update launch");
    }
    if (!(ev_rest[g] = record(stream))) return fail(FASTQR_EINVAL, "cannot record HIP events");
  }
  hipEvent_t ev_end = record(side);
  if (!ev_end) return fail(FASTQR_EINVAL, "cannot record HIP events");
  if ((e = hipStreamWaitEvent(stream, ev_end, 0)) != hipSuccess) return hip_fail(e, "stream join");
  return FASTQR_OK;
}

// ---- fastqr_geqrf_f32_noalloc: scratch in a static device array ------------
// The blocked path's T factors (and the row-split partial products) live in
// `scratch`, one copy per GPU, held until the process ends.  Its device address
// is taken once per device with hipGetSymbolAddress (the array's name is only a
// host-side stand-in) and kept in g_scratch_ptr; kernels only ever see that
// address.  Every call on a GPU shares the array: calls that overlap in time on
// one GPU (two streams, two threads) race on it.  Nothing in it has to start at
// zero: every T slot and partial product is written before it is read.
__device__ __align__(256) unsigned char scratch[FASTQR_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// Device address of the current device's `scratch`.
int noalloc_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(FASTQR_EINVAL, "device %d beyond the %d supported", dev, kMaxDevices);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (p == nullptr) return fail(FASTQR_EWORKSPACE, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return FASTQR_OK;
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
  if (n <= fastqr::kLdsMaxN) return "lds";
  return "blocked";
}

size_t fastqr_workspace_bytes(int64_t batch, int64_t n) { return workspace_bytes_for(batch, n, false); }

size_t fastqr_orgqr_workspace_bytes(int64_t batch, int64_t n) {
  if (batch <= 0 || n <= 0 || n > kMaxN) return 0;
  // the batch is processed in chunks of at most kMaxGridY matrices
  const int64_t chunk = batch < fastqr::kMaxGridY ? batch : fastqr::kMaxGridY;
  return (fastqr::orgqr_workspace_floats(chunk, (int)n) * sizeof(float) + 255) & ~(size_t)255;
}

int fastqr_orgqr_f32(const float* H, int64_t batch, int64_t n, int64_t h_s0, int64_t h_s1, int64_t h_s2,
                     const float* tau, int64_t tau_s0, int64_t tau_s1, float* Q, int64_t q_s0, int64_t q_s1,
                     int64_t q_s2, void* workspace, size_t workspace_bytes, void* stream_ptr) {
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
  if (!H || !tau || !Q) return fail(FASTQR_EINVAL, "H, tau and Q must be non-null device pointers");
  if (h_s0 < 0 || h_s1 < 0 || h_s2 < 0 || q_s0 < 0 || q_s2 < 0 || tau_s0 < 0 || tau_s1 < 0)
    return fail(FASTQR_EINVAL, "negative strides are not supported");
  if (batch > 1 && (q_s0 == 0 || tau_s0 == 0))
    return fail(FASTQR_EINVAL, "Q and tau batch strides must be non-zero when batch > 1");
  if (n > 1 && (tau_s1 == 0 || h_s1 == 0 || h_s2 == 0)) return fail(FASTQR_EINVAL, "H and tau strides must be non-zero");
  if (q_s1 != 1 || q_s2 < n)
    return fail(FASTQR_ELAYOUT, "Q must have contiguous columns (stride (*, 1, >=n)); got (%lld, %lld, %lld)",
                (long long)q_s0, (long long)q_s1, (long long)q_s2);
  if (q_s2 * n * 4 >= (int64_t)1 << 31)
    return fail(FASTQR_ELAYOUT, "one matrix of Q spans %lld bytes; at most 2 GiB are addressed",
                (long long)(q_s2 * n * 4));
  if (batch > 1 && q_s0 < q_s2 * n)
    return fail(FASTQR_ELAYOUT, "Q batch stride %lld smaller than one matrix (%lld)", (long long)q_s0,
                (long long)(q_s2 * n));
  const size_t need = fastqr_orgqr_workspace_bytes(batch, n);
  if (workspace_bytes < need || (need > 0 && workspace == nullptr))
    return fail(FASTQR_EWORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
  if (((uintptr_t)workspace & 15) != 0) return fail(FASTQR_EWORKSPACE, "workspace must be 16-byte aligned");
  const bool same = ((const float*)Q == H && q_s0 == h_s0 && q_s1 == h_s1 && q_s2 == h_s2);
  const int64_t q_span = span_elems(batch, n, q_s0, 1, q_s2);
  if (!same && ranges_overlap(H, span_elems(batch, n, h_s0, h_s1, h_s2), Q, q_span))
    return fail(FASTQR_EOVERLAP, "H and Q overlap with different layouts");
  if (ranges_overlap(tau, span_elems(batch, n, tau_s0, tau_s1, 0), Q, q_span))
    return fail(FASTQR_EOVERLAP, "tau and Q overlap");
  const bool vec = ((uintptr_t)Q % 16 == 0) && (q_s0 % 4 == 0) && (q_s2 % 4 == 0) && (n % 4 == 0);
  // chunks of at most kMaxGridY matrices (its kernels put the batch in grid.y),
  // one after another on the stream, sharing the workspace
  for (int64_t b0 = 0; b0 < batch; b0 += fastqr::kMaxGridY) {
    const int64_t nb = (batch - b0 < fastqr::kMaxGridY) ? batch - b0 : fastqr::kMaxGridY;
    const hipError_t e = fastqr::launch_orgqr(H + b0 * h_s0, nb, (int)n, h_s0, h_s1, h_s2, tau + b0 * tau_s0, tau_s0,
                                              tau_s1, Q + b0 * q_s0, q_s0, q_s2, (float*)workspace, vec,
                                              (hipStream_t)stream_ptr);
    if (e != hipSuccess) return hip_fail(e, "orgqr launch");
  }
  return FASTQR_OK;
}

size_t fastqr_ormqr_workspace_bytes(int64_t batch, int64_t m, int64_t r, int64_t k) {
  if (batch <= 0 || r <= 0 || k <= 0 || m < r || m > kMaxN || k > 2147483647LL) return 0;
  const int64_t chunk = batch < fastqr::kMaxGridY ? batch : fastqr::kMaxGridY;
  return (fastqr::ormqr_workspace_floats(chunk, (int)m, (int)r, (int)k) * sizeof(float) + 255) & ~(size_t)255;
}

int fastqr_ormqr_f32(const float* H, int64_t batch, int64_t m, int64_t r, int64_t h_s0, int64_t h_s1, int64_t h_s2,
                     const float* tau, int64_t tau_s0, int64_t tau_s1, float* C, int64_t k, int64_t c_s0,
                     int64_t c_s1, int64_t c_s2, int transpose, void* workspace, size_t workspace_bytes,
                     void* stream_ptr) {
  g_last_error[0] = '\0';
  if (g_forced_error != 0) {
    const int code = g_forced_error;
    g_forced_error = 0;
    return fail(code, "forced error %d (test hook)", code);
  }
  if (batch < 0 || m < 0 || r < 0 || k < 0)
    return fail(FASTQR_EINVAL, "batch, m, r and k must be non-negative (got %lld, %lld, %lld, %lld)",
                (long long)batch, (long long)m, (long long)r, (long long)k);
  if (r > m) return fail(FASTQR_EINVAL, "r=%lld reflectors exceed m=%lld rows", (long long)r, (long long)m);
  if (batch == 0 || m == 0 || k == 0 || r == 0) return FASTQR_OK;  // nothing to apply (Q = I when r == 0)
  if (m > kMaxN) return fail(FASTQR_EINVAL, "m=%lld exceeds the supported maximum %lld", (long long)m,
                             (long long)kMaxN);
  if (batch > 2147483647LL || k > 2147483647LL) return fail(FASTQR_EINVAL, "batch or k too large");
  if (!H || !tau || !C) return fail(FASTQR_EINVAL, "H, tau and C must be non-null device pointers");
  if (h_s0 < 0 || h_s2 < 0 || c_s0 < 0 || c_s2 < 0 || tau_s0 < 0 || tau_s1 < 0)
    return fail(FASTQR_EINVAL, "negative strides are not supported");
  if (batch > 1 && c_s0 == 0) return fail(FASTQR_EINVAL, "C batch stride must be non-zero when batch > 1");
  if (r > 1 && tau_s1 == 0) return fail(FASTQR_EINVAL, "tau column stride must be non-zero");
  if (h_s1 != 1 || h_s2 < m)
    return fail(FASTQR_ELAYOUT, "H must have contiguous columns (stride (*, 1, >=m)); got (%lld, %lld, %lld)",
                (long long)h_s0, (long long)h_s1, (long long)h_s2);
  if (c_s1 != 1 || c_s2 < m)
    return fail(FASTQR_ELAYOUT, "C must have contiguous columns (stride (*, 1, >=m)); got (%lld, %lld, %lld)",
                (long long)c_s0, (long long)c_s1, (long long)c_s2);
  // 32-bit byte offsets up to the end of the last (partial) 32-column block
  if (h_s2 * ((r + 31) & ~31LL) * 4 >= (int64_t)1 << 31 || c_s2 * ((k + 31) & ~31LL) * 4 >= (int64_t)1 << 31)
    return fail(FASTQR_ELAYOUT, "one matrix of H or C spans more than the 2 GiB a launch addresses");
  if (batch > 1 && c_s0 < c_s2 * k)
    return fail(FASTQR_ELAYOUT, "C batch stride %lld smaller than one matrix (%lld)", (long long)c_s0,
                (long long)(c_s2 * k));
  const size_t need = fastqr_ormqr_workspace_bytes(batch, m, r, k);
  if (workspace_bytes < need || (need > 0 && workspace == nullptr))
    return fail(FASTQR_EWORKSPACE, "workspace of %zu bytes required, %zu given", need, workspace_bytes);
  if (((uintptr_t)workspace & 15) != 0) return fail(FASTQR_EWORKSPACE, "workspace must be 16-byte aligned");
  const int64_t c_span = span_elems(batch, m, c_s0, 1, 0) + (k - 1) * c_s2;
  if (ranges_overlap(H, span_elems(batch, m, h_s0, 1, 0) + (r - 1) * h_s2, C, c_span))
    return fail(FASTQR_EOVERLAP, "H and C overlap");
  if (ranges_overlap(tau, span_elems(batch, r, tau_s0, tau_s1, 0), C, c_span))
    return fail(FASTQR_EOVERLAP, "tau and C overlap");
  // 16-byte column segments when every column of H and C starts 16-byte aligned and m rows fill them
  const bool vec = ((uintptr_t)H % 16 == 0) && (h_s0 % 4 == 0) && (h_s2 % 4 == 0) && ((uintptr_t)C % 16 == 0) &&
                   (c_s0 % 4 == 0) && (c_s2 % 4 == 0) && (m % 4 == 0);
  // chunks of at most kMaxGridY matrices (the T kernel puts the batch in grid.y)
  for (int64_t b0 = 0; b0 < batch; b0 += fastqr::kMaxGridY) {
    const int64_t nb = (batch - b0 < fastqr::kMaxGridY) ? batch - b0 : fastqr::kMaxGridY;
    const hipError_t e = fastqr::launch_ormqr(H + b0 * h_s0, nb, (int)m, (int)r, h_s0, h_s2, tau + b0 * tau_s0, tau_s0,
                                              tau_s1, C + b0 * c_s0, c_s0, c_s2, (int)k, transpose != 0,
                                              (float*)workspace, vec, (hipStream_t)stream_ptr);
    if (e != hipSuccess) return hip_fail(e, "ormqr launch");
  }
  return FASTQR_OK;
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
  return geqrf_impl(A, batch, n, a_s0, a_s1, a_s2, H, h_s0, h_s1, h_s2, tau, tau_s0, tau_s1, workspace,
                    workspace_bytes, false, stream_ptr);
}

int fastqr_geqrf_f32_noalloc(const float* A, int64_t batch, int64_t n, int64_t a_s0, int64_t a_s1, int64_t a_s2,
                             float* H, int64_t h_s0, int64_t h_s1, int64_t h_s2, float* tau, int64_t tau_s0,
                             int64_t tau_s1, void* stream_ptr) {
  g_last_error[0] = '\0';
  if (g_forced_error != 0) {
    const int code = g_forced_error;
    g_forced_error = 0;
    return fail(code, "forced error %d (test hook)", code);
  }
  const size_t need = workspace_bytes_for(batch, n, true);
  if (need > (size_t)FASTQR_NOALLOC_SCRATCH_BYTES)
    return fail(FASTQR_EWORKSPACE,
                "batch=%lld n=%lld needs %zu bytes of scratch; fastqr_geqrf_f32_noalloc holds at most %zu "
                "(split the batch, or call fastqr_geqrf_f32 with a workspace)",
                (long long)batch, (long long)n, need, (size_t)FASTQR_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = noalloc_scratch(&ws);
    if (rc != FASTQR_OK) return rc;
  }
  return geqrf_impl(A, batch, n, a_s0, a_s1, a_s2, H, h_s0, h_s1, h_s2, tau, tau_s0, tau_s1, ws,
                    need > 0 ? (size_t)FASTQR_NOALLOC_SCRATCH_BYTES : 0, true, stream_ptr);
}

}  // extern "C"

// ---- mixed-precision variant (tools/blocked_qr_reference.py:193-262) ------

namespace {

// Workspace of fastqr_geqrf_mixed_f32, 256-byte aligned regions: the panel T
// slots, the repair buffer C (column-major, leading dimension n: A's columns
// k.. for R maintenance, the panel's for the refresh) and the workspace of
// the fp32 Q^T C calls that recompute them.
struct MixedLayout {
  size_t t_bytes = 0, c_bytes = 0, q_bytes = 0;
  int64_t c_cols = 0;
  size_t total() const { return t_bytes + c_bytes + q_bytes; }
};

size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

bool mixed_layout(int64_t batch, int64_t n, int64_t pw, int flags, MixedLayout* L) {
  if (batch <= 0 || n <= 0 || n > kMixedMaxN || batch > fastqr::kMaxGridY || (pw != 16 && pw != 32) ||
      (flags & ~(FASTQR_MIXED_R_MAINTENANCE | FASTQR_MIXED_PANEL_REFRESH)) != 0)
    return false;
  L->t_bytes = round256((size_t)batch * fastqr::kMaxSlots * 32 * 32 * sizeof(float));
  const bool rm = flags & FASTQR_MIXED_R_MAINTENANCE, pr = flags & FASTQR_MIXED_PANEL_REFRESH;
  L->c_cols = rm ? n : pr ? pw : 0;
  L->c_bytes = round256((size_t)batch * n * L->c_cols * sizeof(float));
  size_t q = 0;
  for (int64_t k = 0; k < n; k += pw) {
    const int64_t w = n - k < pw ? n - k : pw;
    if (pr && k > 0) q = std::max(q, fastqr_ormqr_workspace_bytes(batch, n, k, w));
    if (rm) q = std::max(q, fastqr_ormqr_workspace_bytes(batch, n, k + w, n - k));
  }
  L->q_bytes = round256(q);
  return true;
}

}  // namespace

extern "C" {

size_t fastqr_geqrf_mixed_workspace_bytes(int64_t batch, int64_t n, int64_t panel_width, int flags) {
  MixedLayout L;
  return mixed_layout(batch, n, panel_width, flags, &L) ? L.total() : 0;
}

int fastqr_geqrf_mixed_f32(const float* A, int64_t batch, int64_t n, int64_t a_s0, int64_t a_s1, int64_t a_s2,
                           float* H, int64_t h_s0, int64_t h_s1, int64_t h_s2, float* tau, int64_t tau_s0,
                           int64_t tau_s1, int64_t panel_width, int precision, int flags, void* workspace,
                           size_t workspace_bytes, void* stream_ptr) {
  g_last_error[0] = '\0';
  if (g_forced_error != 0) {
    const int code = g_forced_error;
    g_forced_error = 0;
    return fail(code, "forced error %d (test hook)", code);
  }
  if (batch < 0 || n < 0) return fail(FASTQR_EINVAL, "batch and n must be non-negative (got %lld, %lld)",
                                      (long long)batch, (long long)n);
  if (panel_width != 16 && panel_width != 32)
    return fail(FASTQR_EINVAL, "panel_width must be 16 or 32 (got %lld)", (long long)panel_width);
  if (precision < FASTQR_PREC_FP32 || precision > FASTQR_PREC_BF16_INPUT)
    return fail(FASTQR_EINVAL, "precision must be one of FASTQR_PREC_* (got %d)", precision);
  if ((flags & ~(FASTQR_MIXED_R_MAINTENANCE | FASTQR_MIXED_PANEL_REFRESH)) != 0)
    return fail(FASTQR_EINVAL, "unknown flags 0x%x", flags);
  if (batch == 0 || n == 0) return FASTQR_OK;
  if (n > kMixedMaxN) return fail(FASTQR_EINVAL, "n=%lld exceeds the mixed variant's maximum %lld", (long long)n,
                                  (long long)kMixedMaxN);
  if (batch > fastqr::kMaxGridY) return fail(FASTQR_EINVAL, "batch=%lld exceeds %lld", (long long)batch,
                                             (long long)fastqr::kMaxGridY);
  if (!A || !H || !tau) return fail(FASTQR_EINVAL, "A, H and tau must be non-null device pointers");
  if (a_s0 < 0 || a_s1 < 0 || a_s2 < 0 || h_s0 < 0 || h_s2 < 0 || tau_s0 < 0 || tau_s1 < 0)
    return fail(FASTQR_EINVAL, "negative strides are not supported");
  if (batch > 1 && (h_s0 == 0 || tau_s0 == 0))
    return fail(FASTQR_EINVAL, "H and tau batch strides must be non-zero when batch > 1");
  if (n > 1 && tau_s1 == 0) return fail(FASTQR_EINVAL, "tau column stride must be non-zero");
  if (h_s1 != 1 || h_s2 < n)
    return fail(FASTQR_ELAYOUT, "H must have contiguous columns (stride (*, 1, >=n)); got (%lld, %lld, %lld)",
                (long long)h_s0, (long long)h_s1, (long long)h_s2);
  if (h_s2 * n * 4 >= (int64_t)1 << 31)
    return fail(FASTQR_ELAYOUT, "one matrix of H spans %lld bytes; at most 2 GiB are addressed",
                (long long)(h_s2 * n * 4));
  if (batch > 1 && h_s0 < h_s2 * n)
    return fail(FASTQR_ELAYOUT, "H batch stride %lld smaller than one matrix (%lld)", (long long)h_s0,
                (long long)(h_s2 * n));
  const int64_t h_span = span_elems(batch, n, h_s0, 1, h_s2);
  if (ranges_overlap(A, span_elems(batch, n, a_s0, a_s1, a_s2), H, h_span))
    return fail(FASTQR_EOVERLAP, "A and H overlap (the repair steps read A again)");
  if (ranges_overlap(tau, span_elems(batch, n, tau_s0, tau_s1, 0), H, h_span))
    return fail(FASTQR_EOVERLAP, "tau and H overlap");
  MixedLayout L;
  if (!mixed_layout(batch, n, panel_width, flags, &L)) return fail(FASTQR_EINVAL, "invalid mixed-precision arguments");
  if (workspace_bytes < L.total() || workspace == nullptr)
    return fail(FASTQR_EWORKSPACE, "workspace of %zu bytes required, %zu given", L.total(), workspace_bytes);
  if (((uintptr_t)workspace & 255) != 0) return fail(FASTQR_EWORKSPACE, "workspace must be 256-byte aligned");

  hipStream_t stream = (hipStream_t)stream_ptr;
  float* Tws = (float*)workspace;
  float* C = (float*)((char*)workspace + L.t_bytes);
  void* qws = (char*)workspace + L.t_bytes + L.c_bytes;
  const int ni = (int)n, pw = (int)panel_width;
  const int64_t c_s0 = n * L.c_cols;
  const bool vec = ((uintptr_t)H % 16 == 0) && (h_s0 % 4 == 0) && (h_s2 % 4 == 0) && (n % 4 == 0);
  const bool rm = flags & FASTQR_MIXED_R_MAINTENANCE, pr = flags & FASTQR_MIXED_PANEL_REFRESH;
  hipError_t e = fastqr::launch_copy_colmajor(A, batch, ni, a_s0, a_s1, a_s2, H, h_s0, h_s2, 0, ni, stream);
  if (e != hipSuccess) return hip_fail(e, "copy launch");
  for (int k = 0; k < ni; k += pw) {
    const int w = ni - k < pw ? ni - k : pw;
    if (pr && k > 0) {
      // panel rows k.. <- rows k.. of Q_k^T A[:, k:k+w], Q_k = H_0 ... H_{k-1}, in fp32
      if ((e = fastqr::launch_block_copy(A + k * a_s2, batch, a_s0, a_s1, a_s2, C, c_s0, 1, n, ni, w, 0, 0, false,
                                         stream)) != hipSuccess)
        return hip_fail(e, "refresh copy launch");
      int rc = fastqr_ormqr_f32(H, batch, n, k, h_s0, 1, h_s2, tau, tau_s0, tau_s1, C, w, c_s0, 1, n, 1, qws,
                                L.q_bytes, stream_ptr);
      if (rc != FASTQR_OK) return rc;
      if ((e = fastqr::launch_block_copy(C + k, batch, c_s0, 1, n, H + k * h_s2 + k, h_s0, 1, h_s2, ni - k, w, k, k,
                                         false, stream)) != hipSuccess)
        return hip_fail(e, "refresh copy launch");
    }
    if ((e = fastqr::launch_panel(H, batch, h_s0, h_s2, tau, tau_s0, tau_s1, Tws, ni, k, pw, ni - k, 0, vec,
                                  stream)) != hipSuccess)
      return hip_fail(e, "panel launch");
    if (k + w < ni &&
        (e = fastqr::launch_mixed_update(precision, H, batch, h_s0, h_s2, Tws, ni, k, w, k + w, vec, stream)) != hipSuccess)
      return hip_fail(e, "mixed update launch");
    if (rm) {
      // rows k .. k+w-1 of columns k.. (upper triangle) <- Q_{k+w}^T A[:, k:], in fp32
      if ((e = fastqr::launch_block_copy(A + k * a_s2, batch, a_s0, a_s1, a_s2, C, c_s0, 1, n, ni, ni - k, 0, 0,
                                         false, stream)) != hipSuccess)
        return hip_fail(e, "repair copy launch");
      int rc = fastqr_ormqr_f32(H, batch, n, k + w, h_s0, 1, h_s2, tau, tau_s0, tau_s1, C, n - k, c_s0, 1, n, 1, qws,
                                L.q_bytes, stream_ptr);
      if (rc != FASTQR_OK) return rc;
      if ((e = fastqr::launch_block_copy(C + k, batch, c_s0, 1, n, H + k * h_s2 + k, h_s0, 1, h_s2, w, ni - k, k, k,
                                         true, stream)) != hipSuccess)
        return hip_fail(e, "repair copy launch");
    }
  }
  return FASTQR_OK;
}

}  // extern "C"
