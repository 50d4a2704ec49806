/*
 * hhqr.c — CPU restatement of the reference's batched Householder QR.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path (fast-qr_amd/) links,
 * loads or calls this file; it is the checker that tests/, the smoke test and
 * bench.py's CPU-baseline leg compare the HIP kernels against.
 *
 * What it restates (reference files, relative to the reference repo root):
 *   - reflector convention  submissions/candidate.py:654-668 and 2084-2098
 *     (LAPACK slarfg without the safmin rescaling loop):
 *         active = sigma > 0
 *         beta   = alpha >= 0 ? -sqrt(alpha^2 + sigma) : +sqrt(alpha^2 + sigma)
 *         tau    = (beta - alpha) / beta
 *         v      = x / (alpha - beta),   v_k = 1
 *         inactive: beta = alpha, tau = 0, v = 0
 *   - unblocked column loop  submissions/candidate.py:146-226 (geqrf32_kernel)
 *     and 2404-2505 (blocked panel factor): sigma over rows > k, reflector,
 *     normalise, then for every later column j: dot = v^T a_j over rows >= k,
 *     a_j -= tau * v * dot.
 *   - T factor (forward, column-wise, LAPACK slarft)  tools/blocked_qr_reference.py:98-109
 *     and submissions/candidate.py:2544-2584:
 *         T_jj = tau_j ;  T[0:j, j] = T[0:j, 0:j] * ( -tau_j * V[:, 0:j]^T v_j )
 *   - compact-WY trailing update  tools/blocked_qr_reference.py:112-122 and
 *     submissions/candidate.py:2593-2672:  A2 <- A2 - V * (T^T * (V^T * A2))
 *   - panel loop  tools/blocked_qr_reference.py:192-262 (panel factored by the
 *     unblocked routine here instead of torch.geqrf).
 *
 * Layouts: A is read through arbitrary element strides (as0, as1, as2) like the
 * reference kernels (submissions/candidate.py:150-158).  H is written
 * column-major, stride (n*n, 1, n), as allocate_column_major_H does
 * (submissions/candidate.py:3752-3769).  tau is (b, n) contiguous.
 *
 * `mutation` lets the tests plant a known mistake in the oracle (on the CPU
 * only) to show that the checks catch it:
 *   0 none; 1 flip the sign of beta; 2 use T instead of T^T in the update;
 *   3 drop the unit diagonal of v in the trailing dot.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_OK 0
#define ORC_EINVAL -1
#define ORC_ENOMEM -2

int orc_version(void) { return 1; }

/* ---- reflector (submissions/candidate.py:654-668) ---------------------- */
void orc_reflector_f32(float alpha, float sigma, int mutation,
                       float* beta, float* tau, float* denom, int* active) {
    *active = sigma > 0.0f;
    if (*active) {
        const float norm = sqrtf(alpha * alpha + sigma);
        float b = (alpha >= 0.0f) ? -norm : norm;
        if (mutation == 1) b = -b;
        *beta = b;
        *tau = (b - alpha) / b;
        *denom = alpha - b;
    } else {
        *beta = alpha;
        *tau = 0.0f;
        *denom = 1.0f;
    }
}

static void reflector_f64(double alpha, double sigma, double* beta, double* tau,
                          double* denom, int* active) {
    *active = sigma > 0.0;
    if (*active) {
        const double norm = sqrt(alpha * alpha + sigma);
        *beta = (alpha >= 0.0) ? -norm : norm;
        *tau = (*beta - alpha) / *beta;
        *denom = alpha - *beta;
    } else {
        *beta = alpha;
        *tau = 0.0;
        *denom = 1.0;
    }
}

/* ---- unblocked factor of columns [c0, c1) over rows [c0, m) of a
 * column-major m x ncols block (leading dimension ld).  Columns >= c1 up to
 * upd_end are updated with every reflector (reference "reflector" mode).
 * submissions/candidate.py:177-219 / 2437-2504. ------------------------- */
static void factor_cols_f32(float* a, int64_t ld, int64_t m, int64_t c0, int64_t c1,
                            int64_t upd_end, float* tau, int mutation) {
    for (int64_t k = c0; k < c1; ++k) {
        float* ak = a + k * ld;
        float sigma = 0.0f;
        for (int64_t i = k + 1; i < m; ++i) sigma += ak[i] * ak[i];
        float beta, tk, denom;
        int active;
        orc_reflector_f32(ak[k], sigma, mutation, &beta, &tk, &denom, &active);
        tau[k] = tk;
        for (int64_t i = k + 1; i < m; ++i) ak[i] = active ? ak[i] / denom : 0.0f;
        for (int64_t j = k + 1; j < upd_end; ++j) {
            float* aj = a + j * ld;
            float dot = aj[k];
            for (int64_t i = k + 1; i < m; ++i) dot += ak[i] * aj[i];
            aj[k] -= tk * dot;
            for (int64_t i = k + 1; i < m; ++i) aj[i] -= tk * ak[i] * dot;
        }
        ak[k] = beta;
    }
}

static void factor_cols_f64(double* a, int64_t ld, int64_t m, int64_t c0, int64_t c1,
                            int64_t upd_end, double* tau) {
    for (int64_t k = c0; k < c1; ++k) {
        double* ak = a + k * ld;
        double sigma = 0.0;
        for (int64_t i = k + 1; i < m; ++i) sigma += ak[i] * ak[i];
        double beta, tk, denom;
        int active;
        reflector_f64(ak[k], sigma, &beta, &tk, &denom, &active);
        tau[k] = tk;
        for (int64_t i = k + 1; i < m; ++i) ak[i] = active ? ak[i] / denom : 0.0;
        for (int64_t j = k + 1; j < upd_end; ++j) {
            double* aj = a + j * ld;
            double dot = aj[k];
            for (int64_t i = k + 1; i < m; ++i) dot += ak[i] * aj[i];
            aj[k] -= tk * dot;
            for (int64_t i = k + 1; i < m; ++i) aj[i] -= tk * ak[i] * dot;
        }
        ak[k] = beta;
    }
}

static void load_colmajor_f32(const float* A, int64_t n, int64_t s1, int64_t s2, float* w) {
    for (int64_t j = 0; j < n; ++j)
        for (int64_t i = 0; i < n; ++i) w[j * n + i] = A[i * s1 + j * s2];
}

/* Unblocked batched QR in fp32. */
int orc_geqrf_unblocked_f32(int64_t b, int64_t n, const float* A, int64_t as0, int64_t as1,
                            int64_t as2, float* H, float* tau, int mutation) {
    if (b < 0 || n < 0 || (b > 0 && n > 0 && (!A || !H || !tau))) return ORC_EINVAL;
    for (int64_t bi = 0; bi < b; ++bi) {
        float* h = H + bi * n * n;
        load_colmajor_f32(A + bi * as0, n, as1, as2, h);
        factor_cols_f32(h, n, n, 0, n, n, tau + bi * n, mutation);
    }
    return ORC_OK;
}

/* Same algorithm in fp64 (input fp32, output fp64); used as an
 * independent-precision cross-check. */
int orc_geqrf_unblocked_f64(int64_t b, int64_t n, const float* A, int64_t as0, int64_t as1,
                            int64_t as2, double* H, double* tau) {
    if (b < 0 || n < 0 || (b > 0 && n > 0 && (!A || !H || !tau))) return ORC_EINVAL;
    for (int64_t bi = 0; bi < b; ++bi) {
        double* h = H + bi * n * n;
        const float* a = A + bi * as0;
        for (int64_t j = 0; j < n; ++j)
            for (int64_t i = 0; i < n; ++i) h[j * n + i] = (double)a[i * as1 + j * as2];
        factor_cols_f64(h, n, n, 0, n, n, tau + bi * n);
    }
    return ORC_OK;
}

/* ---- T factor, forward column-wise (slarft), nb x nb column-major upper.
 * V is m x nb column-major (ld), unit diagonal implicit and zeros above it are
 * implied: V[i][j] for i < j is ignored, V[j][j] is taken as 1.
 * tools/blocked_qr_reference.py:98-109; submissions/candidate.py:2544-2584. */
int orc_larft_f32(int64_t m, int64_t nb, const float* V, int64_t ldv, const float* tau,
                  float* T) {
    if (m < nb || nb < 0) return ORC_EINVAL;
    float* y = (float*)malloc(sizeof(float) * (size_t)(nb > 0 ? nb : 1));
    if (!y) return ORC_ENOMEM;
    memset(T, 0, sizeof(float) * (size_t)(nb * nb));
    for (int64_t j = 0; j < nb; ++j) {
        T[j * nb + j] = tau[j];
        for (int64_t i = 0; i < j; ++i) {
            /* v_i^T v_j over rows >= j (v_j is zero above row j, one at row j) */
            float dot = V[i * ldv + j];
            for (int64_t r = j + 1; r < m; ++r) dot += V[i * ldv + r] * V[j * ldv + r];
            y[i] = -tau[j] * dot;
        }
        for (int64_t i = 0; i < j; ++i) {
            float acc = 0.0f;
            for (int64_t p = 0; p < j; ++p) acc += T[p * nb + i] * y[p];
            T[j * nb + i] = acc;
        }
    }
    free(y);
    return ORC_OK;
}

/* A2 (m x c, column-major ld2) <- A2 - V T^T V^T A2, V m x nb (unit lower
 * trapezoidal, implicit).  tools/blocked_qr_reference.py:112-122. */
static int apply_compact_wy_f32(int64_t m, int64_t nb, int64_t c, const float* V, int64_t ldv,
                                const float* T, float* A2, int64_t ld2, int mutation) {
    float* P = (float*)malloc(sizeof(float) * (size_t)(nb * (c > 0 ? c : 1)));
    float* W = (float*)malloc(sizeof(float) * (size_t)(nb * (c > 0 ? c : 1)));
    if (!P || !W) { free(P); free(W); return ORC_ENOMEM; }
    for (int64_t col = 0; col < c; ++col) {
        const float* a = A2 + col * ld2;
        for (int64_t j = 0; j < nb; ++j) {
            float acc = (mutation == 3) ? 0.0f : a[j];
            for (int64_t r = j + 1; r < m; ++r) acc += V[j * ldv + r] * a[r];
            P[col * nb + j] = acc;
        }
        for (int64_t j = 0; j < nb; ++j) {
            float acc = 0.0f;
            for (int64_t i = 0; i < nb; ++i) {
                /* W = T^T P : W[j] = sum_i T[i][j] P[i]; mutation 2 uses T[j][i]. */
                const float t = (mutation == 2) ? T[i * nb + j] : T[j * nb + i];
                acc += t * P[col * nb + i];
            }
            W[col * nb + j] = acc;
        }
        float* aw = A2 + col * ld2;
        for (int64_t r = 0; r < m; ++r) {
            float acc = 0.0f;
            const int64_t jmax = r < nb ? r : nb - 1;
            for (int64_t j = 0; j <= jmax; ++j) {
                const float v = (r == j) ? 1.0f : V[j * ldv + r];
                acc += v * W[col * nb + j];
            }
            aw[r] -= acc;
        }
    }
    free(P);
    free(W);
    return ORC_OK;
}

/* Blocked batched QR in fp32 with panel width nb: unblocked panel factor,
 * slarft T, compact-WY trailing update.  tools/blocked_qr_reference.py:192-262. */
int orc_geqrf_blocked_f32(int64_t b, int64_t n, int64_t nb, const float* A, int64_t as0,
                          int64_t as1, int64_t as2, float* H, float* tau, int mutation) {
    if (b < 0 || n < 0 || nb <= 0 || (b > 0 && n > 0 && (!A || !H || !tau))) return ORC_EINVAL;
    float* T = (float*)malloc(sizeof(float) * (size_t)(nb * nb));
    if (!T) return ORC_ENOMEM;
    for (int64_t bi = 0; bi < b; ++bi) {
        float* h = H + bi * n * n;
        float* tb = tau + bi * n;
        load_colmajor_f32(A + bi * as0, n, as1, as2, h);
        for (int64_t k = 0; k < n; k += nb) {
            const int64_t w = (n - k < nb) ? n - k : nb;
            /* panel: columns [k, k+w), rows [k, n); updates only inside the panel */
            factor_cols_f32(h, n, n, k, k + w, k + w, tb, mutation);
            if (k + w < n) {
                float* panel = h + k * n + k; /* rows k.., ld n */
                int rc = orc_larft_f32(n - k, w, panel, n, tb + k, T);
                if (rc == ORC_OK)
                    rc = apply_compact_wy_f32(n - k, w, n - k - w, panel, n, T,
                                              h + (k + w) * n + k, n, mutation);
                if (rc != ORC_OK) { free(T); return rc; }
            }
        }
    }
    free(T);
    return ORC_OK;
}
