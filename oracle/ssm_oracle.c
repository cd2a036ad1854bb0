/*
 * TEST INFRASTRUCTURE ONLY -- the float64 CPU oracle for the selective-scan
 * path.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load this library, and only as the checker.  The product path
 * (mamba_windows_cuda + libmwc_ssm.so) never calls it.
 *
 * What it restates (reference = zouyuanqing/mamba-windows-cuda):
 *   oracle_ssm_fwd   <- selective_scan_ref, mamba_windows_cuda/mamba_cuda.py:875-946
 *                       dA = exp(delta*A) (no clamp, mamba_cuda.py:910-911),
 *                       h_t = dA_t*h_{t-1} + delta_t*u_t*B_t (915-922),
 *                       y = sum_n C*h + D*u (928-929), h_{-1} = h_prev or 0 (905-906).
 *                       Optional clamp of delta*A to [-88, 88] restates the
 *                       kernels' safe_exp (mamba_cuda.py:65-70).
 *   oracle_ssm_bwd   <- the gradients torch autograd takes through
 *                       selective_scan_ref (the reference's own gradient oracle,
 *                       tests/test_selective_scan.py:361-364), written as the
 *                       reverse-time adjoint:
 *                         g_t   = dout_t*C_t + dA_{t+1}*g_{t+1},  g_{L-1} includes dh_last
 *                         dC    = sum_d dout*h_t          dB = sum_d g_t*delta_t*u_t
 *                         du    = D*dout + delta*sum_n g*B
 *                         ddelta= sum_n g*(A*dA_t*h_{t-1} + u*B)
 *                         dA    = sum_{b,t} g*delta*dA_t*h_{t-1}
 *                         dD    = sum_{b,t} dout*u        dh_prev = dA_0*g_0
 *                       plus, when not NULL, the running-error magnitudes of dA,
 *                       ddelta and du (conditioning measures for tests, not
 *                       gradients): the same sums with every term replaced by its
 *                       magnitude and h, g by the recurrences run on magnitudes,
 *                         H_t = dA_t*H_{t-1} + |delta*u*B|,  H_{-1} = |h_prev|
 *                         G_t = |dout_t*C_t| + dA_{t+1}*G_{t+1}, G_{L-1} incl. |dh_last|
 *                         dA_abs     = sum_{b,t} |delta|*G*dA_t*H_{t-1}
 *                         ddelta_abs = sum_n |A|*G*dA_t*H_{t-1} + |u|*sum_n G*|B|
 *                         du_abs     = |D*dout| + |delta|*sum_n G*|B|
 *                       (bounds of |h| and |g| free of cancellation: an fp32
 *                       evaluation's error in each output is a few eps32 times its
 *                       magnitude sum, whatever the cancellation in h, g or the sum).
 *   oracle_pscan_fwd <- parallel_scan_ref, mamba_windows_cuda/pscan.py:153-171
 *                       (H_0 = X_0, A_0 ignored; H_t = A_t*H_{t-1} + X_t)
 *   oracle_pscan_bwd <- its adjoint: G~_t = dH_t + A_{t+1}*G~_{t+1};
 *                       dX_t = G~_t; dA_t = G~_t*H_{t-1} (t >= 1); dA_0 = 0.
 *
 * Pins (tests/test_oracle.py): torch autograd through a float64 restatement
 * of selective_scan_ref, torch.autograd.gradcheck (finite differences), the
 * cumsum closed form of tests/test_selective_scan.py:8-36, brute-force loops,
 * and special cases (A=0 -> cumsum, delta=0 -> constant state, L=1, B=0,
 * pscan with A=1 -> cumsum, A=0 -> X, constant a -> geometric sum).
 *
 * Layouts follow the reference: u, delta, out, du, ddelta (B,L,D); A, dA (D,N);
 * B, C, dB, dC (B,L,N); D, dD (D,); h_prev, h_last, dh_last, dh_prev (B,D,N).
 * Results are deterministic for any OpenMP thread count: every reduction over
 * channels is summed in a fixed block order.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef int64_t i64;

#define OR_DBLK 16 /* channels per forward work item */
#define OR_BBLK 64 /* channels per backward work item (bounds the partial buffers) */
#define OR_NMAX 64 /* largest state size the forward stack buffer holds */

static inline double clamp88(double x, int clamp) {
    if (!clamp) return x;
    return x < -88.0 ? -88.0 : (x > 88.0 ? 88.0 : x);
}

void oracle_ssm_fwd(i64 Bsz, i64 L, i64 Dm, i64 N, const double* u, const double* delta,
                    const double* A, const double* Bm, const double* Cm, const double* Dv,
                    const double* h_prev, int clamp, double* out, double* h_last) {
    if (N > OR_NMAX) return;
    const i64 nblk = (Dm + OR_DBLK - 1) / OR_DBLK;
#pragma omp parallel for schedule(dynamic, 1)
    for (i64 item = 0; item < Bsz * nblk; ++item) {
        const i64 b = item / nblk, d0 = (item % nblk) * OR_DBLK;
        const i64 d1 = d0 + OR_DBLK < Dm ? d0 + OR_DBLK : Dm;
        double h[OR_DBLK * OR_NMAX];
        for (i64 d = d0; d < d1; ++d)
            for (i64 n = 0; n < N; ++n)
                h[(d - d0) * N + n] = h_prev ? h_prev[(b * Dm + d) * N + n] : 0.0;
        for (i64 t = 0; t < L; ++t) {
            const i64 row = (b * L + t) * Dm;
            const double* Bt = Bm + (b * L + t) * N;
            const double* Ct = Cm + (b * L + t) * N;
            for (i64 d = d0; d < d1; ++d) {
                const double dt = delta[row + d], ut = u[row + d];
                double y = 0.0;
                double* hd = h + (d - d0) * N;
                for (i64 n = 0; n < N; ++n) {
                    const double dA = exp(clamp88(dt * A[d * N + n], clamp));
                    hd[n] = dA * hd[n] + dt * ut * Bt[n];
                    y += Ct[n] * hd[n];
                }
                out[row + d] = y + Dv[d] * ut;
            }
        }
        if (h_last)
            for (i64 d = d0; d < d1; ++d)
                for (i64 n = 0; n < N; ++n) h_last[(b * Dm + d) * N + n] = h[(d - d0) * N + n];
    }
}

void oracle_ssm_bwd(i64 Bsz, i64 L, i64 Dm, i64 N, const double* u, const double* delta,
                    const double* A, const double* Bm, const double* Cm, const double* Dv,
                    const double* h_prev, const double* dout, const double* dh_last, int clamp,
                    double* du, double* ddelta, double* dA, double* dB, double* dC, double* dD,
                    double* dh_prev, double* dA_abs, double* ddelta_abs, double* du_abs) {
    const i64 nblk = (Dm + OR_BBLK - 1) / OR_BBLK;
    const i64 nitems = Bsz * nblk;
    /* per-item partials, summed afterwards in item order (deterministic) */
    double* pBC = (double*)calloc((size_t)nitems * L * N * 2, sizeof(double));
    double* pA = (double*)calloc((size_t)nitems * OR_BBLK * N, sizeof(double));
    double* pAa = (double*)calloc((size_t)nitems * OR_BBLK * N, sizeof(double));
    double* pD = (double*)calloc((size_t)nitems * OR_BBLK, sizeof(double));
#pragma omp parallel for schedule(dynamic, 1)
    for (i64 item = 0; item < nitems; ++item) {
        const i64 b = item / nblk, d0 = (item % nblk) * OR_BBLK;
        const i64 d1 = d0 + OR_BBLK < Dm ? d0 + OR_BBLK : Dm;
        const i64 nd = d1 - d0;
        /* full state history of this block: hist[t][d][n] = h_t; eA[t][d][n] = dA_t */
        double* hist = (double*)malloc((size_t)L * nd * N * sizeof(double));
        double* eA = (double*)malloc((size_t)L * nd * N * sizeof(double));
        double* g = (double*)malloc((size_t)nd * N * sizeof(double));
        double* hp = (double*)malloc((size_t)nd * N * sizeof(double));
        /* the magnitude recurrences H, G of the running-error sums */
        double* hista = (double*)malloc((size_t)L * nd * N * sizeof(double));
        double* ga = (double*)malloc((size_t)nd * N * sizeof(double));
        for (i64 d = d0; d < d1; ++d)
            for (i64 n = 0; n < N; ++n) hp[(d - d0) * N + n] = h_prev ? h_prev[(b * Dm + d) * N + n] : 0.0;
        for (i64 t = 0; t < L; ++t) {
            const i64 row = (b * L + t) * Dm;
            const double* Bt = Bm + (b * L + t) * N;
            for (i64 d = d0; d < d1; ++d) {
                const double dt = delta[row + d], ut = u[row + d];
                for (i64 n = 0; n < N; ++n) {
                    const i64 k = (d - d0) * N + n;
                    const double prev = t ? hist[((t - 1) * nd) * N + k] : hp[k];
                    const double e = exp(clamp88(dt * A[d * N + n], clamp));
                    eA[(t * nd) * N + k] = e;
                    hist[(t * nd) * N + k] = e * prev + dt * ut * Bt[n];
                    const double preva = t ? hista[((t - 1) * nd) * N + k] : fabs(hp[k]);
                    hista[(t * nd) * N + k] = e * preva + fabs(dt * ut * Bt[n]);
                }
            }
        }
        for (i64 k = 0; k < nd * N; ++k) {
            const i64 d = d0 + k / N, n = k % N;
            g[k] = dh_last ? dh_last[(b * Dm + d) * N + n] : 0.0; /* carried part dA_{t+1} g_{t+1} */
            ga[k] = fabs(g[k]);
        }
        double* myBC = pBC + (size_t)item * L * N * 2;
        double* myA = pA + (size_t)item * OR_BBLK * N;
        double* myAa = pAa + (size_t)item * OR_BBLK * N;
        double* myD = pD + (size_t)item * OR_BBLK;
        for (i64 t = L - 1; t >= 0; --t) {
            const i64 row = (b * L + t) * Dm;
            const double* Bt = Bm + (b * L + t) * N;
            const double* Ct = Cm + (b * L + t) * N;
            for (i64 d = d0; d < d1; ++d) {
                const double dt = delta[row + d], ut = u[row + d], yo = dout[row + d];
                double r1 = 0.0, r2 = 0.0, r1a = 0.0, r2a = 0.0;
                for (i64 n = 0; n < N; ++n) {
                    const i64 k = (d - d0) * N + n;
                    const double ht = hist[(t * nd) * N + k];
                    const double prev = t ? hist[((t - 1) * nd) * N + k] : hp[k];
                    const double e = eA[(t * nd) * N + k];
                    const double gt = g[k] + yo * Ct[n];
                    myBC[(t * N + n) * 2 + 1] += yo * ht;      /* dC */
                    myBC[(t * N + n) * 2 + 0] += gt * dt * ut; /* dB */
                    r1 += gt * Bt[n];
                    const double s = gt * e * prev;
                    r2 += A[d * N + n] * s;
                    myA[(d - d0) * N + n] += dt * s;
                    g[k] = e * gt;
                    /* magnitudes */
                    const double gta = ga[k] + fabs(yo * Ct[n]);
                    const double sa = gta * e * (t ? hista[((t - 1) * nd) * N + k] : fabs(hp[k]));
                    r1a += gta * fabs(Bt[n]);
                    r2a += fabs(A[d * N + n]) * sa;
                    myAa[(d - d0) * N + n] += fabs(dt) * sa;
                    ga[k] = e * gta;
                }
                du[row + d] = Dv[d] * yo + dt * r1;
                ddelta[row + d] = r2 + ut * r1;
                if (ddelta_abs) ddelta_abs[row + d] = r2a + fabs(ut) * r1a;
                if (du_abs) du_abs[row + d] = fabs(Dv[d] * yo) + fabs(dt) * r1a;
                myD[d - d0] += yo * ut;
            }
        }
        if (dh_prev)
            for (i64 k = 0; k < nd * N; ++k) {
                const i64 d = d0 + k / N, n = k % N;
                dh_prev[(b * Dm + d) * N + n] = g[k];
            }
        free(hist);
        free(eA);
        free(g);
        free(hp);
        free(hista);
        free(ga);
    }
    /* deterministic reductions */
    for (i64 b = 0; b < Bsz; ++b)
        for (i64 i = 0; i < L * N; ++i) {
            double sb = 0.0, sc = 0.0;
            for (i64 blk = 0; blk < nblk; ++blk) {
                const double* p = pBC + (size_t)(b * nblk + blk) * L * N * 2;
                sb += p[i * 2 + 0];
                sc += p[i * 2 + 1];
            }
            dB[b * L * N + i] = sb;
            dC[b * L * N + i] = sc;
        }
    for (i64 d = 0; d < Dm; ++d) {
        const i64 blk = d / OR_BBLK, off = d % OR_BBLK;
        double sd = 0.0;
        for (i64 n = 0; n < N; ++n) {
            double sa = 0.0, saa = 0.0;
            for (i64 b = 0; b < Bsz; ++b) {
                sa += pA[(size_t)(b * nblk + blk) * OR_BBLK * N + off * N + n];
                saa += pAa[(size_t)(b * nblk + blk) * OR_BBLK * N + off * N + n];
            }
            dA[d * N + n] = sa;
            if (dA_abs) dA_abs[d * N + n] = saa;
        }
        for (i64 b = 0; b < Bsz; ++b) sd += pD[(size_t)(b * nblk + blk) * OR_BBLK + off];
        dD[d] = sd;
    }
    free(pBC);
    free(pA);
    free(pAa);
    free(pD);
}

/* H[s][t][c] for s < nseq, t < L, c < ncols (the scan runs over t). */
void oracle_pscan_fwd(i64 nseq, i64 L, i64 ncols, const double* A, const double* X, double* H) {
#pragma omp parallel for schedule(static)
    for (i64 s = 0; s < nseq; ++s) {
        const i64 base = s * L * ncols;
        for (i64 c = 0; c < ncols; ++c) H[base + c] = X[base + c];
        for (i64 t = 1; t < L; ++t)
            for (i64 c = 0; c < ncols; ++c) {
                const i64 i = base + t * ncols + c;
                H[i] = A[i] * H[i - ncols] + X[i];
            }
    }
}

void oracle_pscan_bwd(i64 nseq, i64 L, i64 ncols, const double* A, const double* H,
                      const double* dH, double* dA, double* dX) {
#pragma omp parallel for schedule(static)
    for (i64 s = 0; s < nseq; ++s) {
        const i64 base = s * L * ncols;
        for (i64 t = L - 1; t >= 0; --t)
            for (i64 c = 0; c < ncols; ++c) {
                const i64 i = base + t * ncols + c;
                const double carry = (t + 1 < L) ? A[i + ncols] * dX[i + ncols] : 0.0;
                dX[i] = dH[i] + carry;
                dA[i] = t ? dX[i] * H[i - ncols] : 0.0;
            }
    }
}
