/*
 * lloyd_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement of scikit-learn 1.7.2's dense Lloyd k-means (the CPU
 * path skmetal dispatches KMeans to), used by tests/, by the smoke check and
 * by bench.py's cpu_baseline leg as the checker.  It is never linked into,
 * loaded by, or called from the product library (skmetal_amd/).
 *
 * What it follows (sklearn sources, read as text):
 *   - centring:        sklearn/cluster/_kmeans.py:1477-1484 (X -= X.mean(0),
 *                      init -= X_mean) and :1534-1537 (centers += X_mean)
 *   - E-step:          sklearn/cluster/_k_means_lloyd.pyx:168-212
 *                      (||c||^2 - 2 x.c, strict '<' argmin, lowest index wins)
 *   - M-step sums:     _k_means_lloyd.pyx:214-218 (unit weights)
 *   - relocation:      sklearn/cluster/_k_means_common.pyx:167-211
 *   - averaging:       _k_means_common.pyx:274-295 (incl. the in-order copy of
 *                      the heaviest cluster's row into still-empty clusters)
 *   - centre shift:    _k_means_common.pyx:298-311
 *   - loop/stopping:   sklearn/cluster/_kmeans.py:624-752 (strict label
 *                      convergence, sum(shift^2) <= tol, final E-step)
 *   - inertia:         _k_means_common.pyx:94-124
 *   - skmetal's known-answer vector: tests/test_kernels.py:93-99
 *
 * Precision: inputs and stored centres are fp32 exactly where sklearn stores
 * fp32 (centred X, centres after every M-step); distances, sums, shifts and
 * inertia are evaluated in fp64, so the oracle is a tighter "truth" than
 * sklearn's own fp32 BLAS/OpenMP arithmetic.  Centring reproduces numpy's
 * float32 X.mean(axis=0) bit for bit (sequential fp32 sum over rows, then one
 * fp32 divide).
 *
 * Relocation order: sklearn takes np.argpartition(dist, -n_empty)[::-1],
 * whose order among the n_empty farthest points is numpy-internal for
 * n_empty >= 3.  The oracle assigns empty clusters (ascending id) to points in
 * descending distance, ties to the lower row index; this coincides with
 * sklearn for n_empty <= 2.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

typedef int64_t i64;

/* numpy float32 X.mean(axis=0): out[c] = (sum_r X[r,c] in fp32, row order) / n (fp32). */
void oracle_mean_f32(const float* X, i64 n, i64 d, float* mean_out)
{
    for (i64 c = 0; c < d; ++c) mean_out[c] = 0.0f;
    for (i64 r = 0; r < n; ++r) {
        const float* row = X + r * d;
        for (i64 c = 0; c < d; ++c) mean_out[c] = mean_out[c] + row[c];
    }
    for (i64 c = 0; c < d; ++c) mean_out[c] = mean_out[c] / (float)n;
}

/* ||c_j||^2 in fp64. */
static void cnorms_f64(const float* C, i64 k, i64 d, double* out)
{
    for (i64 j = 0; j < k; ++j) {
        double s = 0.0;
        for (i64 c = 0; c < d; ++c) s += (double)C[j * d + c] * (double)C[j * d + c];
        out[j] = s;
    }
}

/*
 * E-step (_k_means_lloyd.pyx:196-212): label_i = argmin_j ||c_j||^2 - 2 x_i.c_j,
 * strict '<' so the lowest index wins ties.  Optionally returns, per row, the
 * best and second-best values of ||x||^2 + ||c||^2 - 2 x.c (true squared
 * distances, fp64) so callers can apply a near-tie rule.
 */
void oracle_assign(const float* X, i64 n, i64 d, const float* C, i64 k,
                   int32_t* labels, double* best_out, double* second_out)
{
    double* cn = (double*)malloc(sizeof(double) * (size_t)k);
    double* Cd = (double*)malloc(sizeof(double) * (size_t)(k * d));
    cnorms_f64(C, k, d, cn);
    for (i64 t = 0; t < k * d; ++t) Cd[t] = (double)C[t];

#pragma omp parallel
    {
        double* xr = (double*)malloc(sizeof(double) * (size_t)d);
#pragma omp for schedule(static)
        for (i64 i = 0; i < n; ++i) {
            const float* row = X + i * d;
            double xx = 0.0;
            for (i64 c = 0; c < d; ++c) { xr[c] = (double)row[c]; xx += xr[c] * xr[c]; }
            double best = INFINITY, second = INFINITY;
            int32_t lab = 0;
            for (i64 j = 0; j < k; ++j) {
                const double* cj = Cd + j * d;
                double dot = 0.0;
                for (i64 c = 0; c < d; ++c) dot += xr[c] * cj[c];
                double v = cn[j] - 2.0 * dot;
                if (v < best) { second = best; best = v; lab = (int32_t)j; }
                else if (v < second) { second = v; }
            }
            labels[i] = lab;
            if (best_out) best_out[i] = best + xx;
            if (second_out) second_out[i] = second + xx;
        }
        free(xr);
    }
    free(cn);
    free(Cd);
}

/* Per-cluster fp64 sums and counts of X rows by label (_k_means_lloyd.pyx:214-218). */
void oracle_sums(const float* X, i64 n, i64 d, const int32_t* labels, i64 k,
                 double* sums, i64* counts)
{
    memset(sums, 0, sizeof(double) * (size_t)(k * d));
    memset(counts, 0, sizeof(i64) * (size_t)k);
    for (i64 i = 0; i < n; ++i) {
        i64 j = labels[i];
        counts[j] += 1;
        const float* row = X + i * d;
        double* s = sums + j * d;
        for (i64 c = 0; c < d; ++c) s[c] += (double)row[c];
    }
}

/* ||x_i - c_{label_i}||^2 per row, fp64 direct form. */
void oracle_mindists(const float* X, i64 n, i64 d, const float* C, const int32_t* labels,
                     double* out)
{
#pragma omp parallel for schedule(static)
    for (i64 i = 0; i < n; ++i) {
        const float* row = X + i * d;
        const float* c = C + (i64)labels[i] * d;
        double s = 0.0;
        for (i64 f = 0; f < d; ++f) {
            double t = (double)row[f] - (double)c[f];
            s += t * t;
        }
        out[i] = s;
    }
}

/* Inertia (_k_means_common.pyx:94-124), fp64, unit weights. */
double oracle_inertia(const float* X, i64 n, i64 d, const float* C, const int32_t* labels)
{
    double total = 0.0;
#pragma omp parallel for schedule(static) reduction(+ : total)
    for (i64 i = 0; i < n; ++i) {
        const float* row = X + i * d;
        const float* c = C + (i64)labels[i] * d;
        double s = 0.0;
        for (i64 f = 0; f < d; ++f) {
            double t = (double)row[f] - (double)c[f];
            s += t * t;
        }
        total += s;
    }
    return total;
}

typedef struct { double dist; i64 idx; } far_t;

static int far_cmp(const void* a, const void* b)
{
    const far_t* x = (const far_t*)a;
    const far_t* y = (const far_t*)b;
    if (x->dist > y->dist) return -1;
    if (x->dist < y->dist) return 1;
    return (x->idx < y->idx) ? -1 : (x->idx > y->idx);
}

/*
 * One M-step from given labels: sums, relocation of empty clusters
 * (_k_means_common.pyx:167-211), averaging (:274-295) and shift (:298-311).
 * centers_old/new are fp32 [k x d]; shift_out is fp64 [k].
 * Returns the number of clusters that were empty before relocation.
 */
int oracle_mstep(const float* X, i64 n, i64 d, const int32_t* labels,
                 const float* centers_old, i64 k, float* centers_new, double* shift_out)
{
    double* sums = (double*)malloc(sizeof(double) * (size_t)(k * d));
    i64* counts = (i64*)malloc(sizeof(i64) * (size_t)k);
    oracle_sums(X, n, d, labels, k, sums, counts);

    int n_empty = 0;
    for (i64 j = 0; j < k; ++j) n_empty += (counts[j] == 0);

    if (n_empty > 0) {
        double* dist = (double*)malloc(sizeof(double) * (size_t)n);
        oracle_mindists(X, n, d, centers_old, labels, dist);
        double dmax = 0.0;
        for (i64 i = 0; i < n; ++i) if (dist[i] > dmax) dmax = dist[i];
        if (dmax > 0.0) {
            far_t* fr = (far_t*)malloc(sizeof(far_t) * (size_t)n);
            for (i64 i = 0; i < n; ++i) { fr[i].dist = dist[i]; fr[i].idx = i; }
            qsort(fr, (size_t)n, sizeof(far_t), far_cmp);
            /* the empty set is fixed before any point moves (pyx:176) */
            i64* empties = (i64*)malloc(sizeof(i64) * (size_t)n_empty);
            int ne = 0;
            for (i64 j = 0; j < k; ++j) if (counts[j] == 0) empties[ne++] = j;
            for (int e = 0; e < n_empty; ++e) {
                i64 j = empties[e];
                i64 far = fr[e].idx;
                i64 old = labels[far];
                const float* row = X + far * d;
                for (i64 c = 0; c < d; ++c) {
                    sums[old * d + c] -= (double)row[c];
                    sums[j * d + c] = (double)row[c];
                }
                counts[j] = 1;
                counts[old] -= 1;
            }
            free(empties);
            free(fr);
        }
        free(dist);
    }

    /* _average_centers: argmax over weights first, then rows in order. */
    i64 amax = 0;
    for (i64 j = 1; j < k; ++j) if (counts[j] > counts[amax]) amax = j;
    double* cur = (double*)malloc(sizeof(double) * (size_t)(k * d));
    memcpy(cur, sums, sizeof(double) * (size_t)(k * d));
    for (i64 j = 0; j < k; ++j) {
        if (counts[j] > 0) {
            for (i64 c = 0; c < d; ++c) cur[j * d + c] = cur[j * d + c] / (double)counts[j];
        } else {
            /* copies the heaviest row as it stands at this point of the loop:
             * averaged if amax < j, still a raw sum if amax > j. */
            for (i64 c = 0; c < d; ++c) cur[j * d + c] = cur[amax * d + c];
        }
    }
    for (i64 t = 0; t < k * d; ++t) centers_new[t] = (float)cur[t];

    for (i64 j = 0; j < k; ++j) {
        double s = 0.0;
        for (i64 c = 0; c < d; ++c) {
            double t = (double)centers_new[j * d + c] - (double)centers_old[j * d + c];
            s += t * t;
        }
        shift_out[j] = sqrt(s);
    }
    free(cur);
    free(sums);
    free(counts);
    return n_empty;
}

/*
 * Full KMeans.fit(X, init=C_init, n_init=1, algorithm="lloyd") with unit
 * weights (_kmeans.py:1454-1554 + _kmeans_single_lloyd :624-752).
 *   X_raw     [n x d] fp32, caller coordinates (not modified)
 *   C_init    [k x d] fp32, caller coordinates
 *   tol_abs   sklearn's _tol (mean variance x tol); 0 disables the shift test
 *   C_out     [k x d] final centres, caller coordinates
 *   labels    [n] final labels
 *   trace     optional [max_iter x k x d]: centres (caller coordinates) after
 *             each M-step
 * Returns n_iter_ (>= 1), or -1 on allocation failure.
 */
int oracle_lloyd(const float* X_raw, i64 n, i64 d, const float* C_init, i64 k,
                 int max_iter, double tol_abs, float* C_out, int32_t* labels,
                 double* inertia_out, float* trace)
{
    float* X = (float*)malloc(sizeof(float) * (size_t)(n * d));
    float* mean = (float*)malloc(sizeof(float) * (size_t)d);
    float* cen = (float*)malloc(sizeof(float) * (size_t)(k * d));
    float* cen_new = (float*)malloc(sizeof(float) * (size_t)(k * d));
    int32_t* old = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    double* shift = (double*)malloc(sizeof(double) * (size_t)k);
    if (!X || !mean || !cen || !cen_new || !old || !shift) return -1;

    oracle_mean_f32(X_raw, n, d, mean);
    for (i64 r = 0; r < n; ++r)
        for (i64 c = 0; c < d; ++c) X[r * d + c] = X_raw[r * d + c] - mean[c];
    for (i64 j = 0; j < k; ++j)
        for (i64 c = 0; c < d; ++c) cen[j * d + c] = C_init[j * d + c] - mean[c];
    for (i64 i = 0; i < n; ++i) old[i] = -1;

    int strict = 0;
    int it = 0;
    for (it = 0; it < max_iter; ++it) {
        oracle_assign(X, n, d, cen, k, labels, NULL, NULL);
        oracle_mstep(X, n, d, labels, cen, k, cen_new, shift);
        memcpy(cen, cen_new, sizeof(float) * (size_t)(k * d));
        if (trace) {
            float* tr = trace + (i64)it * k * d;
            for (i64 j = 0; j < k; ++j)
                for (i64 c = 0; c < d; ++c) tr[j * d + c] = cen[j * d + c] + mean[c];
        }
        int same = 1;
        for (i64 i = 0; i < n; ++i) if (labels[i] != old[i]) { same = 0; break; }
        if (same) { strict = 1; break; }
        double tot = 0.0;
        for (i64 j = 0; j < k; ++j) tot += shift[j] * shift[j];
        if (tot <= tol_abs) break;
        memcpy(old, labels, sizeof(int32_t) * (size_t)n);
    }
    int n_iter = (it < max_iter) ? it + 1 : max_iter;
    if (!strict) oracle_assign(X, n, d, cen, k, labels, NULL, NULL);
    if (inertia_out) *inertia_out = oracle_inertia(X, n, d, cen, labels);
    for (i64 j = 0; j < k; ++j)
        for (i64 c = 0; c < d; ++c) C_out[j * d + c] = cen[j * d + c] + mean[c];

    free(X); free(mean); free(cen); free(cen_new); free(old); free(shift);
    return n_iter;
}

int oracle_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
