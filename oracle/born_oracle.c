/*
 * Brute-force scalar restatement of Born attention, forward and backward, in
 * double precision.
 *
 * TEST INFRASTRUCTURE ONLY: built by oracle/Makefile into
 * oracle/_build/libborn_oracle.so and loaded solely by tests/ to pin the
 * vectorised numpy oracle (oracle/born_oracle.py).  Nothing in the product
 * library links or calls it.
 *
 * Semantics follow the reference's flash_born.py (Vengo/QuantumDLBlocks,
 * src/qdlblocks/kernels/flash_born.py):
 *   visibility  causal j <= i (169-170), window i - j < W (173-174),
 *               same document (175-177)
 *   weight      a = max(0, scale_h * (q_i . k_j)), p = a * a (166-180)
 *   normaliser  Z_i = sum_j p_ij + eps, O_i = sum_j p_ij v_j / Z_i (182-192)
 *   backward    dP = (dO_i . v_j - dO_i . O_i) / Z_i, dS = 2 a dP,
 *               dq = s dS k, dk = s dS^T q, dv = (p / Z)^T dO,
 *               dscale = sum dS (q . k)                           (270-322, 387-427)
 * It is written as plain loops, one (b, h, i) row at a time, so that it shares
 * no code or vectorisation structure with the numpy statement.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

static int visible(int64_t i, int64_t j, int is_causal, int64_t window,
                   const int32_t *doc_row) {
    if (is_causal && j > i) return 0;
    if (window > 0 && (i - j) >= window) return 0;
    if (doc_row && doc_row[i] != doc_row[j]) return 0;
    return 1;
}

static double dot(const double *x, const double *y, int64_t n) {
    double s = 0.0;
    for (int64_t d = 0; d < n; ++d) s += x[d] * y[d];
    return s;
}

/* q, k, v, out: (B, H, T, D) contiguous; z: (B, H, T); scale: n_scale values
 * (1 or H); doc_ids: (B, T) or NULL. */
void born_oracle_fwd(int64_t B, int64_t H, int64_t T, int64_t D,
                     const double *q, const double *k, const double *v,
                     const double *scale, int64_t n_scale,
                     const int32_t *doc_ids, int is_causal, int64_t window,
                     double eps, double *out, double *z) {
    double *p = (double *)malloc(sizeof(double) * (size_t)(T > 0 ? T : 1));
    for (int64_t b = 0; b < B; ++b) {
        const int32_t *doc_row = doc_ids ? doc_ids + b * T : NULL;
        for (int64_t h = 0; h < H; ++h) {
            double s = scale[n_scale > 1 ? h : 0];
            const int64_t base = (b * H + h) * T;
            for (int64_t i = 0; i < T; ++i) {
                double zsum = 0.0;
                for (int64_t j = 0; j < T; ++j) {
                    double a = 0.0;
                    if (visible(i, j, is_causal, window, doc_row)) {
                        a = s * dot(q + (base + i) * D, k + (base + j) * D, D);
                        if (a < 0.0) a = 0.0;
                    }
                    p[j] = a * a;
                    zsum += p[j];
                }
                zsum += eps;
                z[base + i] = zsum;
                for (int64_t d = 0; d < D; ++d) {
                    double acc = 0.0;
                    for (int64_t j = 0; j < T; ++j) acc += p[j] * v[(base + j) * D + d];
                    out[(base + i) * D + d] = acc / zsum;
                }
            }
        }
    }
    free(p);
}

/* Gradients of sum(out * dout).  dq, dk, dv: (B, H, T, D); dscale: n_scale
 * values (summed over heads when n_scale == 1). */
void born_oracle_bwd(int64_t B, int64_t H, int64_t T, int64_t D,
                     const double *q, const double *k, const double *v,
                     const double *scale, int64_t n_scale,
                     const int32_t *doc_ids, int is_causal, int64_t window,
                     double eps, const double *dout, double *dq, double *dk,
                     double *dv, double *dscale) {
    const size_t n = (size_t)(B * H * T * D);
    double *out = (double *)malloc(sizeof(double) * (n ? n : 1));
    double *z = (double *)malloc(sizeof(double) * (size_t)((B * H * T) > 0 ? (B * H * T) : 1));
    born_oracle_fwd(B, H, T, D, q, k, v, scale, n_scale, doc_ids, is_causal, window, eps, out, z);
    for (size_t e = 0; e < n; ++e) dq[e] = dk[e] = dv[e] = 0.0;
    for (int64_t e = 0; e < n_scale; ++e) dscale[e] = 0.0;
    for (int64_t b = 0; b < B; ++b) {
        const int32_t *doc_row = doc_ids ? doc_ids + b * T : NULL;
        for (int64_t h = 0; h < H; ++h) {
            double s = scale[n_scale > 1 ? h : 0];
            const int64_t base = (b * H + h) * T;
            for (int64_t i = 0; i < T; ++i) {
                const double *qi = q + (base + i) * D;
                const double *doi = dout + (base + i) * D;
                double delta = dot(doi, out + (base + i) * D, D);
                double zi = z[base + i];
                for (int64_t j = 0; j < T; ++j) {
                    if (!visible(i, j, is_causal, window, doc_row)) continue;
                    const double *kj = k + (base + j) * D;
                    const double *vj = v + (base + j) * D;
                    double r = dot(qi, kj, D);
                    double a = s * r;
                    if (a <= 0.0) continue;
                    double p = a * a;
                    double dp = (dot(doi, vj, D) - delta) / zi;
                    double ds = 2.0 * a * dp;
                    for (int64_t d = 0; d < D; ++d) {
                        dq[(base + i) * D + d] += s * ds * kj[d];
                        dk[(base + j) * D + d] += s * ds * qi[d];
                        dv[(base + j) * D + d] += (p / zi) * doi[d];
                    }
                    dscale[n_scale > 1 ? h : 0] += ds * r;
                }
            }
        }
    }
    free(out);
    free(z);
}
