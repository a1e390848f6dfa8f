/* Brute-force periodic pair list with ASE neighbor_list("ijS") semantics (oracle).
 *
 * Restates the pair set produced by ase.neighborlist.neighbor_list (ase 3.29.0, pinned at
 * requirements.txt:5, called at face/neighbors.py:12 and face/datasets.py:51): all (i, j, S)
 * with |pos[j] - pos[i] + S . cell| < rc in fp64, S integer, S_c = 0 on non-periodic axes,
 * (i, i, 0) excluded, positions used as given (not wrapped).
 *
 * Arithmetic order (compiled with -ffp-contract=off, no FMA):
 *   shift_c = (S0*cell[0][c] + S1*cell[1][c]) + S2*cell[2][c]
 *   d_c     = (pos[j][c] - pos[i][c]) + shift_c
 *   r       = sqrt((d0*d0 + d1*d1) + d2*d2),  kept iff r < rc
 * Output order is canonical: i ascending, then j ascending, then S lexicographic.
 *
 * Every pair (i, j) is tested against every image S in the interval that can contain a
 * hit: along reciprocal axis c, |(f_j - f_i + S)_c| * face_dist_c <= |d| < rc, widened by one
 * image on each side against rounding.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static void inv3(const double* m, double* o) {
    double a = m[0], b = m[1], c = m[2], d = m[3], e = m[4], f = m[5], g = m[6], h = m[7], k = m[8];
    double det = a * (e * k - f * h) - b * (d * k - f * g) + c * (d * h - e * g);
    o[0] = (e * k - f * h) / det; o[1] = (c * h - b * k) / det; o[2] = (b * f - c * e) / det;
    o[3] = (f * g - d * k) / det; o[4] = (a * k - c * g) / det; o[5] = (c * d - a * f) / det;
    o[6] = (d * h - e * g) / det; o[7] = (b * g - a * h) / det; o[8] = (a * e - b * d) / det;
}

/* cell: 3x3 row-major, row r = lattice vector r. pbc[3] in {0,1}.
 * Writes at most cap pairs (i, j, S[3]); returns the total number of pairs. */
int64_t oracle_pair_list(const double* pos, int32_t n, const double* cell, const int32_t* pbc, double rc,
                         int32_t* out_i, int32_t* out_j, int32_t* out_S, int64_t cap) {
    double inv[9] = {0};
    double fd[3] = {1, 1, 1};
    int any_pbc = pbc[0] || pbc[1] || pbc[2];
    if (any_pbc) {
        inv3(cell, inv);
        for (int c = 0; c < 3; c++) {   /* reciprocal vector c = column c of inv(cell) */
            double l = sqrt(inv[0 * 3 + c] * inv[0 * 3 + c] + inv[1 * 3 + c] * inv[1 * 3 + c] +
                            inv[2 * 3 + c] * inv[2 * 3 + c]);
            fd[c] = 1.0 / l;
        }
    }
    int64_t cnt = 0;
    for (int32_t i = 0; i < n; i++) {
        double fi[3] = {0, 0, 0};
        if (any_pbc)
            for (int c = 0; c < 3; c++)
                fi[c] = pos[i * 3 + 0] * inv[0 * 3 + c] + pos[i * 3 + 1] * inv[1 * 3 + c] + pos[i * 3 + 2] * inv[2 * 3 + c];
        for (int32_t j = 0; j < n; j++) {
            int lo[3] = {0, 0, 0}, hi[3] = {0, 0, 0};
            for (int c = 0; c < 3; c++) {
                if (!pbc[c]) continue;
                double fj = pos[j * 3 + 0] * inv[0 * 3 + c] + pos[j * 3 + 1] * inv[1 * 3 + c] + pos[j * 3 + 2] * inv[2 * 3 + c];
                double df = fj - fi[c], w = rc / fd[c];
                lo[c] = (int)floor(-df - w) - 1;
                hi[c] = (int)ceil(-df + w) + 1;
            }
            for (int s0 = lo[0]; s0 <= hi[0]; s0++)
                for (int s1 = lo[1]; s1 <= hi[1]; s1++)
                    for (int s2 = lo[2]; s2 <= hi[2]; s2++) {
                        if (i == j && s0 == 0 && s1 == 0 && s2 == 0) continue;
                        double d[3];
                        for (int c = 0; c < 3; c++) {
                            double sh = 0.0;
                            if (any_pbc) sh = ((double)s0 * cell[0 * 3 + c] + (double)s1 * cell[1 * 3 + c]) + (double)s2 * cell[2 * 3 + c];
                            d[c] = (pos[j * 3 + c] - pos[i * 3 + c]) + sh;
                        }
                        double r = sqrt((d[0] * d[0] + d[1] * d[1]) + d[2] * d[2]);
                        if (r < rc) {
                            if (cnt < cap) {
                                out_i[cnt] = i; out_j[cnt] = j;
                                out_S[cnt * 3 + 0] = s0; out_S[cnt * 3 + 1] = s1; out_S[cnt * 3 + 2] = s2;
                            }
                            cnt++;
                        }
                    }
        }
    }
    return cnt;
}

/* The same pairs, in the same order and from the same arithmetic as oracle_pair_list, for cells
 * periodic on all three axes, with the j loop narrowed to candidates from a bin grid: along
 * reciprocal axis c a pair within rc has |(f_j - f_i + S)_c| < w_c = rc / face_dist_c, so with
 * bins of width >= w_c (1 + 1e-6) over the wrapped fractional coordinate every such j lies in
 * i's bin or a cyclically adjacent one (the margin covers the rounding of f, ~1e-16). Axes with
 * fewer than three such bins are one bin. Each candidate j (ascending) runs the brute-force
 * image loop, skipping only images that provably hold no pair. Returns -1 when some axis is not
 * periodic. */
static int cmp_i32(const void* a, const void* b) {
    int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
    return (x > y) - (x < y);
}

int64_t oracle_pair_list_cells(const double* pos, int32_t n, const double* cell, const int32_t* pbc, double rc,
                               int32_t* out_i, int32_t* out_j, int32_t* out_S, int64_t cap) {
    if (!(pbc[0] && pbc[1] && pbc[2])) return -1;
    double inv[9], fd[3], w[3];
    int nb[3];
    inv3(cell, inv);
    for (int c = 0; c < 3; c++) {
        double l = sqrt(inv[0 * 3 + c] * inv[0 * 3 + c] + inv[1 * 3 + c] * inv[1 * 3 + c] +
                        inv[2 * 3 + c] * inv[2 * 3 + c]);
        fd[c] = 1.0 / l;
        w[c] = rc / fd[c];
        double m = floor(1.0 / (w[c] * (1.0 + 1e-6)));
        nb[c] = m < 3.0 ? 1 : (m > 1024.0 ? 1024 : (int)m);
    }
    const int64_t nbins = (int64_t)nb[0] * nb[1] * nb[2];
    int32_t* bin_of = (int32_t*)malloc(sizeof(int32_t) * (n > 0 ? n : 1));
    int64_t* start = (int64_t*)calloc(nbins + 1, sizeof(int64_t));
    int32_t* members = (int32_t*)malloc(sizeof(int32_t) * (n > 0 ? n : 1));
    int32_t* cand = (int32_t*)malloc(sizeof(int32_t) * (n > 0 ? n : 1));
    double* frac = (double*)malloc(sizeof(double) * 3 * (n > 0 ? n : 1));
    if (!bin_of || !start || !members || !cand || !frac) {
        free(bin_of); free(start); free(members); free(cand); free(frac);
        return -2;
    }
    for (int32_t a = 0; a < n; a++) {
        int b[3];
        for (int c = 0; c < 3; c++) {
            double f = pos[a * 3 + 0] * inv[0 * 3 + c] + pos[a * 3 + 1] * inv[1 * 3 + c] + pos[a * 3 + 2] * inv[2 * 3 + c];
            frac[a * 3 + c] = f;
            double u = f - floor(f);
            int k = (int)floor(u * nb[c]);
            b[c] = k < 0 ? 0 : (k >= nb[c] ? nb[c] - 1 : k);
        }
        bin_of[a] = (b[0] * nb[1] + b[1]) * nb[2] + b[2];
        start[bin_of[a] + 1]++;
    }
    for (int64_t k = 0; k < nbins; k++) start[k + 1] += start[k];
    {
        int64_t* fill = (int64_t*)malloc(sizeof(int64_t) * (nbins > 0 ? nbins : 1));
        if (!fill) {
            free(bin_of); free(start); free(members); free(cand); free(frac);
            return -2;
        }
        memcpy(fill, start, sizeof(int64_t) * nbins);
        for (int32_t a = 0; a < n; a++) members[fill[bin_of[a]]++] = a;
        free(fill);
    }
    int64_t cnt = 0;
    for (int32_t i = 0; i < n; i++) {
        const int32_t bi = bin_of[i];
        const int b0 = bi / (nb[1] * nb[2]), b1 = (bi / nb[2]) % nb[1], b2 = bi % nb[2];
        int32_t nc = 0;
        for (int d0 = (nb[0] > 1 ? -1 : 0); d0 <= (nb[0] > 1 ? 1 : 0); d0++)
            for (int d1 = (nb[1] > 1 ? -1 : 0); d1 <= (nb[1] > 1 ? 1 : 0); d1++)
                for (int d2 = (nb[2] > 1 ? -1 : 0); d2 <= (nb[2] > 1 ? 1 : 0); d2++) {
                    const int c0 = (b0 + d0 + nb[0]) % nb[0], c1 = (b1 + d1 + nb[1]) % nb[1],
                              c2 = (b2 + d2 + nb[2]) % nb[2];
                    const int64_t k = ((int64_t)c0 * nb[1] + c1) * nb[2] + c2;
                    for (int64_t m = start[k]; m < start[k + 1]; m++) cand[nc++] = members[m];
                }
        qsort(cand, nc, sizeof(int32_t), cmp_i32);
        const double* fi = frac + i * 3;
        for (int32_t t = 0; t < nc; t++) {
            const int32_t j = cand[t];
            int lo[3], hi[3];
            double dfs[3];
            for (int c = 0; c < 3; c++) {
                double fj = pos[j * 3 + 0] * inv[0 * 3 + c] + pos[j * 3 + 1] * inv[1 * 3 + c] + pos[j * 3 + 2] * inv[2 * 3 + c];
                double df = fj - fi[c], wc = rc / fd[c];
                dfs[c] = df;
                lo[c] = (int)floor(-df - wc) - 1;
                hi[c] = (int)ceil(-df + wc) + 1;
            }
            /* images with |df_c + s_c| >= w_c (1 + 1e-6) cannot hold a pair within rc: skipped
             * (the brute-force loop tests and rejects them); the rest in the same order */
            for (int s0 = lo[0]; s0 <= hi[0]; s0++) {
                if (fabs(dfs[0] + s0) >= w[0] * (1.0 + 1e-6)) continue;
                for (int s1 = lo[1]; s1 <= hi[1]; s1++) {
                    if (fabs(dfs[1] + s1) >= w[1] * (1.0 + 1e-6)) continue;
                    for (int s2 = lo[2]; s2 <= hi[2]; s2++) {
                        if (fabs(dfs[2] + s2) >= w[2] * (1.0 + 1e-6)) continue;
                        if (i == j && s0 == 0 && s1 == 0 && s2 == 0) continue;
                        double d[3];
                        for (int c = 0; c < 3; c++) {
                            double sh = ((double)s0 * cell[0 * 3 + c] + (double)s1 * cell[1 * 3 + c]) + (double)s2 * cell[2 * 3 + c];
                            d[c] = (pos[j * 3 + c] - pos[i * 3 + c]) + sh;
                        }
                        double r = sqrt((d[0] * d[0] + d[1] * d[1]) + d[2] * d[2]);
                        if (r < rc) {
                            if (cnt < cap) {
                                out_i[cnt] = i; out_j[cnt] = j;
                                out_S[cnt * 3 + 0] = s0; out_S[cnt * 3 + 1] = s1; out_S[cnt * 3 + 2] = s2;
                            }
                            cnt++;
                        }
                    }
                }
            }
        }
    }
    free(bin_of); free(start); free(members); free(cand); free(frac);
    return cnt;
}
