/*
 * tsan_driver.c -- runs every OpenMP-parallel function of the fp64 checker
 * (race_oracle.c) on 8 streams with several threads, twice, under
 * ThreadSanitizer, and checks the two runs agree bit for bit.  Test
 * infrastructure only (make -C oracle sanitize builds and runs it): the
 * checker's parallel loops write disjoint per-stream slices and per-stream
 * partial sums that one thread adds afterwards; TSan (with LLVM's libomp and
 * its Archer tool, which tell TSan about OpenMP's own synchronisation) reports
 * any access that breaks that.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

int oracle_race_forward(const double *, const double *, const double *, const double *, const int64_t *,
                        int64_t, int64_t, int64_t, int, int, int, double, double, double *);
int oracle_race_backward(const double *, const double *, const double *, const double *, const double *,
                         const int64_t *, int64_t, int64_t, int64_t, int, int, int, double, double, double *,
                         double *, double *, double *, double *);
int oracle_race_global_forward(const double *, const double *, const double *, const double *, const int64_t *,
                               int64_t, int64_t, int64_t, int, int, double, double, double *, double *);
int oracle_race_global_backward(const double *, const double *, const double *, const double *, const double *,
                                const double *, const int64_t *, int64_t, int64_t, int64_t, int, int, double,
                                double, double *, double *, double *, double *, double *);
int oracle_race_forward_ex(const double *, const double *, const double *, const double *, const double *,
                           const int64_t *, int64_t, int64_t, int64_t, int, int, int, double, double, double *,
                           double *);
int oracle_race_backward_ex(const double *, const double *, const double *, const double *, const double *,
                            const double *, const double *, const int64_t *, int64_t, int64_t, int64_t, int, int,
                            int, double, double, double *, double *, double *, double *, double *);
int oracle_race_probs(const double *, const double *, const int64_t *, int64_t, int64_t, int64_t, int, int,
                      double, double *);
int oracle_race_probs_bwd(const double *, const double *, const double *, const int64_t *, int64_t, int64_t,
                          int64_t, int, int, double, double *, double *, double *);
void oracle_prefix_mean_flat(const float *, const float *, int64_t, int64_t, int64_t, double, float *);
void oracle_prefix_mean_flat_bw(const float *, const float *, const float *, int64_t, int64_t, int64_t, double,
                                float *, float *);

enum { N = 8, T = 67, D = 64, L = 4, K = 3, S = L << K };

static double urand(uint64_t *s) {
    *s = *s * 6364136223846793005ull + 1442695040888963407ull;
    return (double)(*s >> 11) / 9007199254740992.0 * 2.0 - 1.0;
}

static double *arr(size_t n, uint64_t *s) {
    double *a = malloc(n * sizeof(double));
    for (size_t j = 0; j < n; ++j) a[j] = urand(s);
    return a;
}

/* every function once into slot r (r = 0, 1) of the output buffers */
static void run_all(int r, double **in, int64_t *plane_of, double **out, float **fout, float **fin) {
    const size_t o = (size_t)N * T * D;
    double *q = in[0], *k = in[1], *v = in[2], *g = in[3], *pl = in[4], *kw = in[5], *dden = in[6], *dP = in[7];
    double *y = out[r];
    double g1, g2;
    oracle_race_forward(q, k, v, pl, plane_of, N, T, D, L, K, 1, 1e-6, 0.7, y);
    oracle_race_backward(q, k, v, g, pl, plane_of, N, T, D, L, K, 1, 1e-6, 0.7, y + o, y + 2 * o, y + 3 * o, &g1, &g2);
    y[4 * o] = g1;
    oracle_race_global_forward(q, k, v, pl, plane_of, N, T, D, L, K, 1e-6, 1.3, y + 5 * o, y + 6 * o);
    oracle_race_global_backward(q, k, v, g, dden, pl, plane_of, N, T, D, L, K, 1e-6, 1.3, y + 7 * o, y + 8 * o,
                                y + 9 * o, &g1, &g2);
    y[10 * o] = g1;
    oracle_race_forward_ex(q, k, v, kw, pl, plane_of, N, T, D, L, K, 0, 1e-6, 0.9, y + 11 * o, y + 12 * o);
    oracle_race_backward_ex(q, k, v, kw, g, dden, pl, plane_of, N, T, D, L, K, 0, 1e-6, 0.9, y + 13 * o,
                            y + 14 * o, y + 15 * o, &g1, &g2);
    y[16 * o] = g1;
    oracle_race_probs(q, pl, plane_of, N, T, D, L, K, 0.9, y + 17 * o);
    oracle_race_probs_bwd(q, dP, pl, plane_of, N, T, D, L, K, 0.9, y + 18 * o, &g1, &g2);
    y[19 * o] = g1;
    oracle_prefix_mean_flat(fin[0], fin[1], N, T, D, 1e-6, fout[r]);
    oracle_prefix_mean_flat_bw(fin[0], fin[1], fin[2], N, T, D, 1e-6, fout[r] + o, fout[r] + 2 * o);
}

int main(void) {
    uint64_t s = 12345;
    const size_t o = (size_t)N * T * D;
    double *in[8] = {arr(o, &s), arr(o, &s), arr(o, &s), arr(o, &s), arr((size_t)2 * L * K * D, &s),
                     arr((size_t)N * T, &s), arr((size_t)N * T, &s), arr((size_t)N * T * S, &s)};
    for (size_t j = 0; j < (size_t)N * T; ++j) in[5][j] = 0.5 * (in[5][j] + 1.0);  /* key weights in [0, 1] */
    int64_t plane_of[N];
    for (int n = 0; n < N; ++n) plane_of[n] = n & 1;  /* two estimators' planes */
    float *fin[3];
    for (int j = 0; j < 3; ++j) {
        fin[j] = malloc(o * sizeof(float));
        for (size_t e = 0; e < o; ++e) fin[j][e] = (float)(j == 0 ? 0.5 * (urand(&s) + 1.0) : urand(&s));
    }
    double *out[2];
    float *fout[2];
    const size_t nout = 20 * o + 1;
    for (int r = 0; r < 2; ++r) {
        out[r] = calloc(nout, sizeof(double));
        fout[r] = calloc(3 * o, sizeof(float));
        run_all(r, in, plane_of, out, fout, fin);
    }
    int bad = memcmp(out[0], out[1], nout * sizeof(double)) != 0 || memcmp(fout[0], fout[1], 3 * o * sizeof(float)) != 0;
    printf("tsan_driver: %s\n", bad ? "runs differ" : "two runs bit-identical");
    return bad;
}
