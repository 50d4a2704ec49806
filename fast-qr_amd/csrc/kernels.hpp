// kernels.hpp — host-side launchers of the QR kernels (internal to libfastqr).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fastqr {

// n <= 64: one wave64 per matrix (qr_wave.hip).
hipError_t launch_qr_wave(const float* A, int64_t batch, int n, int64_t as0, int64_t as1, int64_t as2,
                          float* H, int64_t hs0, int64_t hs1, int64_t hs2, float* tau, int64_t ts0,
                          int64_t ts1, hipStream_t stream);

// 64 < n <= kLdsMaxN: one workgroup per matrix, the matrix resident in LDS (qr_lds.hip).
constexpr int kLdsMaxN = 176;
hipError_t launch_qr_lds(const float* A, int64_t batch, int n, int64_t as0, int64_t as1, int64_t as2, float* H,
                         int64_t hs0, int64_t hs1, int64_t hs2, float* tau, int64_t ts0, int64_t ts1,
                         hipStream_t stream);

// Largest grid.y (and grid.z) extent a launch uses: kernels that put the
// batch there are launched in chunks of this many matrices.
constexpr int64_t kMaxGridY = 65535;

// Blocked path (qr_blocked.hip).
// Copy columns [c0, c1) of A (any strides) into H (columns contiguous); c0 a
// multiple of 64.  max_wgs > 0 caps the grid (the workgroups loop over the
// 64 x 64 tiles).
hipError_t launch_copy_colmajor(const float* A, int64_t batch, int n, int64_t as0, int64_t as1, int64_t as2,
                                float* H, int64_t hs0, int64_t ldh, int c0, int c1, hipStream_t stream,
                                int max_wgs = 0);
// Panel width (32, or 16 above 2048 rows) and the tallest panel supported (qr_panel.hip).
int panel_width_for(int m);
// Panel width of the strip-resident path (64 or 32; T slots of 32 columns).
int panel_width_wide(int m, int64_t batch);
int panel_max_rows();
// Panel of width nb at column k0, template sized for m_cap >= n - k0 rows;
// its T factors go to workspace slots `slot` .. (one 32 x 32 slot per 32
// columns; a 16-column panel uses one slot).
// Explicit (waves, tiles per wave) variant of launch_panel, for tuning.
hipError_t launch_panel_cfg(int nw, int tpw, float* H, int64_t batch, int64_t hs0, int64_t ldh, float* tau,
                            int64_t ts0, int64_t ts1, float* Tws, int n, int k0, int nb, int slot, bool vec,
                            hipStream_t stream);
hipError_t launch_panel(float* H, int64_t batch, int64_t hs0, int64_t ldh, float* tau, int64_t ts0,
                        int64_t ts1, float* Tws, int n, int k0, int nb, int m_cap, int slot, bool vec,
                        hipStream_t stream);
// Apply nwy compact-WY transforms (panels k0 + i*nb, T slots slot0 + i) to
// columns [c_begin, c_end), rows [k0, n), first to last (last to first with
// `reverse`).  max_cus > 0 caps the grid at that many CUs' worth of resident
// workgroups (the workgroups then loop over the work), leaving the other CUs
// to kernels on another stream; kWyLeaveOneSlot caps it at one workgroup per
// CU fewer than fit, leaving a slot on every CU.
constexpr int kWyLeaveOneSlot = -1;

// Mixed-precision variant (qr_mixed.hip).  Operand precision of its trailing
// update (the values of FASTQR_PREC_* in the C header).
constexpr int kPrecF32 = 0, kPrecTf32 = 1, kPrecF16 = 2, kPrecBf16 = 3;
// Columns [c_begin, n), rows [k0, n) <- minus V r(r(T)^T r(r(V)^T r(X))) for
// the panel of width w at column k0 (its T in workspace slot 0).  vec: 16-byte
// column segments (H 16-byte aligned, ldh, batch stride and n multiples of 4).
hipError_t launch_mixed_update(int prec, float* H, int64_t batch, int64_t hs0, int64_t ldh, const float* Tws, int n,
                               int k0, int w, int c_begin, bool vec, hipStream_t stream);
// dst[b, dr0 + i, dc0 + j] = src[b, i, j], i < rows, j < cols (pointers at
// their first element); `upper`: only where dr0 + i <= dc0 + j.
hipError_t launch_block_copy(const float* src, int64_t batch, int64_t s0, int64_t s1, int64_t s2, float* dst,
                             int64_t d0, int64_t d1, int64_t d2, int rows, int cols, int dr0, int dc0, bool upper,
                             hipStream_t stream);
// With A (row-major, leading dimension lda, batch stride as0) the columns
// [c_begin, c_end) are read from A instead of H and written to H (their first
// update, when the blocked path did not copy them); strips of at most 2048
// rows.
hipError_t launch_wy_update(float* H, int64_t batch, int64_t hs0, int64_t ldh, const float* Tws, int n,
                            int k0, int nb, int slot0, int nwy, int c_begin, int c_end, bool vec, bool hi_prio,
                            int max_cus, hipStream_t stream, bool reverse = false, const float* A = nullptr,
                            int64_t as0 = 0, int64_t lda = 0);
// The same transforms applied to a matrix C of its own (ormqr): V from the
// first vcols columns of the factors (leading dimension ldv, m rows), C with
// ccols columns (leading dimension ldc, m rows), every column of C updated.
hipError_t launch_wy_apply(const float* V, int64_t batch, int64_t vs0, int64_t ldv, int vcols, float* C, int64_t cs0,
                           int64_t ldc, int ccols, const float* Tws, int m, int k0, int nb, int slot0, int nwy,
                           bool vec, hipStream_t stream, bool reverse);

// Row-split compact-WY update (qr_update.hip): for tall matrices and small
// batches the trailing update is split over row blocks as well as column
// strips (partial V^T X per row block, W = -T^T P, X += V W).
constexpr int kWyrMaxBlk = 4;                  // reflector blocks of 32 per update
constexpr int kWyrMaxK = 32 * kWyrMaxBlk;      // reflectors per update (a group of panels)
constexpr int kWyrTgLd = kWyrMaxK;             // leading dimension of a group T
constexpr int64_t kWyrTgStride = (int64_t)kWyrMaxK * kWyrMaxK;  // floats per matrix per group-T bank

struct WyrCall {
  float* H;
  int64_t hs0;
  int ldh, n;
  int64_t batch;
  int kv, k;            // reflectors: columns [kv, kv + k) of H, rows [kv, n)
  int c_begin, c_end;   // columns to read; with gram the first ceil(k/32) strips are the group's own
  bool gram;            // form the group T (Gram V^T V + panel T join) into Tg
  bool use_tg;          // take T from Tg (k x k) instead of the single panel slot Tslot
  int q, nb, slot0;     // the group's panels (count, width, first T slot) for the join
  const float* Tws;     // T slots (kMaxSlots per matrix)
  const float* Tslot;   // T of a single panel: slot base, per-matrix stride kMaxSlots * 1024
  float* Tg;            // group T bank, per-matrix stride kWyrTgStride
  float* scratch;       // partial products and W (wyr_workspace_floats(batch, n) floats)
  int rows_per_blk;     // multiple of 32
  bool vec;
  bool hi_prio;         // critical path: the waves win issue arbitration on shared SIMDs
  // ormqr: the updated columns [c_begin, c_end) are columns of a matrix X of
  // their own (xcols columns, leading dimension ldx, n rows); V is then read
  // from H's first vcols columns.  Not with gram.
  float* X = nullptr;
  int64_t xs0 = 0;
  int ldx = 0, xcols = 0, vcols = 0;
  bool t_trans = false;  // apply X - V T V^T X (T of the slot / Tg read transposed)
};
hipError_t launch_wyr(const WyrCall& c, hipStream_t stream);
int wyr_rows_per_block(int m, int64_t batch, int cols);
size_t wyr_workspace_floats(int64_t batch, int n);

// Panels per group: the wide trailing update applies this many transforms at once.
constexpr int kMaxWY = 4;
// T-factor slots per matrix in the workspace (32 x 32 floats each): three
// groups' worth, so a group's panels can run while the wide updates of the
// two groups before it are still being applied.
constexpr int kMaxSlots = 3 * kMaxWY;

// Explicit Q from (H, tau) (qr_orgqr.hip): backward accumulation over
// 32-column panels in place in Q.  Above kOrgqrRowSplitMinN rows the panel
// updates run on the row-split kernels.
constexpr int kOrgqrRowSplitMinN = 2048;
constexpr int64_t kOrgqrGroupMinBatch = 48;  // panels grouped per update from this batch on
// from this batch on, a group's narrow updates are left-looking (one column
// block per launch, every earlier transform of the group at once)
constexpr int64_t kOrgqrLeftLookingMinBatch = 256;
size_t orgqr_workspace_floats(int64_t batch, int n);
hipError_t launch_orgqr(const float* H, int64_t batch, int n, int64_t hs0, int64_t hs1, int64_t hs2, const float* tau,
                        int64_t ts0, int64_t ts1, float* Q, int64_t qs0, int64_t ldq, float* ws, bool vec,
                        hipStream_t stream);

// Q C or Q^T C in place in C (qr_orgqr.hip), Q = H_0 ... H_{r-1} from r
// reflectors of m rows (H columns contiguous), C m x k (columns contiguous):
// T of every 32-column panel, then the panels' transforms applied to C in
// groups of kMaxWY (first to last for Q^T C, last to first for Q C); groups
// taller than a strip fits run on the row-split kernels.
size_t ormqr_workspace_floats(int64_t batch, int m, int r, int k);
hipError_t launch_ormqr(const float* H, int64_t batch, int m, int r, int64_t hs0, int64_t ldh, const float* tau,
                        int64_t ts0, int64_t ts1, float* C, int64_t cs0, int64_t ldc, int k, bool transpose, float* ws,
                        bool vec, hipStream_t stream);

}  // namespace fastqr
