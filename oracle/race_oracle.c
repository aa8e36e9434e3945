/*
 * race_oracle.c -- CPU fp64 restatement of the RACE attention operator ("F1",
 * per-bucket normalised; "F2", one normaliser per token) and of the reference
 * CPU prefix-mean kernel.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP path of
 * race_attention_amd is compared against.  Only tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py may load it.  The product never links,
 * imports or falls back to it.
 *
 * Reference semantics restated (paths relative to the reference repository):
 *   misc/race.py:63-142      causal BatchedACE.forward
 *   misc/vit.py:918-978      non-causal BatchedACE.forward
 *   misc/race.py:54-58       corner prototypes = itertools.product([-1,+1], K)
 *   misc/race.py:101-105     logits = (tanh(proj)/scale) @ protos_T ; softmax over R
 *   misc/race.py:107-110     A = cumsum P_K ; B = cumsum P_K*v ; E = B/(A+1e-6)
 *   misc/race.py:135-138     out_t = sum over all S=L*R buckets of P_Q * E
 *   kernels/cpu/race_pref.cpp:36-101   prefix mean forward (fp64 accumulators)
 *   kernels/cpu/race_pref.cpp:104-220  prefix mean backward (two passes)
 *   misc/elsaa_causal_complete.py:438-586, misc/race_kernel.py:8-124
 *                            F2 causal readout num/max(den, 1e-6)
 *   misc/classification.py:576-592, :641-659, misc/vit.py:1452-1510
 *                            padding mask on P_K and the den output (F1)
 *
 * Layout used here: streams are independent; every per-stream tensor is
 * [T][D] row-major double.  planes are [NP][L][K][D]; stream n uses planes
 * block plane_of[n].  All arithmetic is double.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_MAX_K 16

/* Corner r of {-1,+1}^K in itertools.product order: the last coordinate
 * varies fastest, so coordinate k is +1 iff bit (K-1-k) of r is set
 * (misc/race.py:54-58). */
static inline double corner_sign(int r, int k, int K)
{
    return ((r >> (K - 1 - k)) & 1) ? 1.0 : -1.0;
}

/* Soft hash of one token (misc/race.py:79-105): th[l*K+k] = tanh(<x, w_lk>),
 * u = th*inv_temp, P[l*R+r] = softmax_r(sum_k c[r,k] u_k).  The softmax is the
 * max-subtracted exponential form of F.softmax. */
static void soft_hash(const double *x, const double *pl, int64_t D, int L, int K,
                      double inv_temp, double *th, double *P)
{
    const int R = 1 << K;
    for (int l = 0; l < L; ++l) {
        double u[ORACLE_MAX_K];
        for (int k = 0; k < K; ++k) {
            const double *w = pl + ((int64_t)l * K + k) * D;
            double acc = 0.0;
            for (int64_t d = 0; d < D; ++d)
                acc += x[d] * w[d];
            th[l * K + k] = tanh(acc);
            u[k] = th[l * K + k] * inv_temp;
        }
        double mx = -INFINITY;
        for (int r = 0; r < R; ++r) {
            double z = 0.0;
            for (int k = 0; k < K; ++k)
                z += corner_sign(r, k, K) * u[k];
            P[l * R + r] = z;
            if (z > mx)
                mx = z;
        }
        double sum = 0.0;
        for (int r = 0; r < R; ++r) {
            P[l * R + r] = exp(P[l * R + r] - mx);
            sum += P[l * R + r];
        }
        for (int r = 0; r < R; ++r)
            P[l * R + r] /= sum;
    }
}

/* Backward of soft_hash given dP: softmax backward, corner matmul backward,
 * tanh backward, projection backward.  Adds into dx[D]; adds
 * sum(du * th) into *g_inv_temp (du/d inv_temp = th) and sum |du * th| into
 * *g_abs (the magnitude of the summands, the scale of that reduction). */
static void soft_hash_bwd(const double *P, const double *th, const double *dP,
                          const double *pl, int64_t D, int L, int K,
                          double inv_temp, double *dx, double *g_inv_temp,
                          double *g_abs)
{
    const int R = 1 << K;
    for (int l = 0; l < L; ++l) {
        double dot = 0.0;
        for (int r = 0; r < R; ++r)
            dot += P[l * R + r] * dP[l * R + r];
        for (int k = 0; k < K; ++k) {
            double du = 0.0;
            for (int r = 0; r < R; ++r)
                du += P[l * R + r] * (dP[l * R + r] - dot) * corner_sign(r, k, K);
            const double t = th[l * K + k];
            *g_inv_temp += du * t;
            *g_abs += fabs(du * t);
            const double dproj = du * inv_temp * (1.0 - t * t);
            const double *w = pl + ((int64_t)l * K + k) * D;
            for (int64_t d = 0; d < D; ++d)
                dx[d] += dproj * w[d];
        }
    }
}

/* Forward of one stream.  Causal: per-token prefix state (misc/race.py:107-110,
 * kernels/cpu/race_pref.cpp:82-98).  Non-causal: full-sequence state
 * (misc/vit.py:962-975). */
static void stream_forward(const double *q, const double *k, const double *v,
                           const double *pl, int64_t T, int64_t D, int L, int K,
                           int causal, double eps, double inv_temp, double *o)
{
    const int R = 1 << K;
    const int64_t S = (int64_t)L * R;
    double *A = calloc((size_t)S, sizeof(double));
    double *B = calloc((size_t)(S * D), sizeof(double));
    double *th = malloc(sizeof(double) * (size_t)(L * K));
    double *PK = malloc(sizeof(double) * (size_t)S);
    double *PQ = malloc(sizeof(double) * (size_t)S);

    if (!causal) {
        for (int64_t t = 0; t < T; ++t) {
            soft_hash(k + t * D, pl, D, L, K, inv_temp, th, PK);
            for (int64_t s = 0; s < S; ++s) {
                A[s] += PK[s];
                for (int64_t d = 0; d < D; ++d)
                    B[s * D + d] += PK[s] * v[t * D + d];
            }
        }
    }
    for (int64_t t = 0; t < T; ++t) {
        if (causal) {
            soft_hash(k + t * D, pl, D, L, K, inv_temp, th, PK);
            for (int64_t s = 0; s < S; ++s) {
                A[s] += PK[s];
                for (int64_t d = 0; d < D; ++d)
                    B[s * D + d] += PK[s] * v[t * D + d];
            }
        }
        soft_hash(q + t * D, pl, D, L, K, inv_temp, th, PQ);
        double *ot = o + t * D;
        for (int64_t d = 0; d < D; ++d)
            ot[d] = 0.0;
        for (int64_t s = 0; s < S; ++s) {
            const double w = PQ[s] / (A[s] + eps);
            for (int64_t d = 0; d < D; ++d)
                ot[d] += w * B[s * D + d];
        }
    }
    free(A); free(B); free(th); free(PK); free(PQ);
}

/* Backward of one stream.  With W = P_Q/(A+eps) and G[t,s] = g_t . B_s(t):
 *   dP_Q[t,s] = G/(A+eps)
 *   dA[t,s]   = -W G/(A+eps)
 *   alpha_s(tau) = sum_{t>=tau} dA[t,s],  U_s(tau) = sum_{t>=tau} W[t,s] g_t
 *   dP_K[tau,s]  = alpha_s(tau) + v_tau . U_s(tau)
 *   dv_tau       = sum_s P_K[tau,s] U_s(tau)
 * (the two-pass alpha/beta scheme of kernels/cpu/race_pref.cpp:154-216 applied
 * to every bucket; non-causal sums run over the whole sequence). */
static void stream_backward(const double *q, const double *k, const double *v,
                            const double *g, const double *pl, int64_t T,
                            int64_t D, int L, int K, int causal, double eps,
                            double inv_temp, double *dq, double *dk, double *dv,
                            double *g_it, double *g_abs)
{
    const int R = 1 << K;
    const int64_t S = (int64_t)L * R;
    double *A = calloc((size_t)S, sizeof(double));
    double *B = calloc((size_t)(S * D), sizeof(double));
    double *dA = malloc(sizeof(double) * (size_t)(T * S));
    double *W = malloc(sizeof(double) * (size_t)(T * S));
    double *th = malloc(sizeof(double) * (size_t)(L * K));
    double *PK = malloc(sizeof(double) * (size_t)S);
    double *PQ = malloc(sizeof(double) * (size_t)S);
    double *dP = malloc(sizeof(double) * (size_t)S);
    double *alpha = calloc((size_t)S, sizeof(double));
    double *U = calloc((size_t)(S * D), sizeof(double));

    memset(dq, 0, sizeof(double) * (size_t)(T * D));
    memset(dk, 0, sizeof(double) * (size_t)(T * D));
    memset(dv, 0, sizeof(double) * (size_t)(T * D));

    if (!causal) {
        for (int64_t t = 0; t < T; ++t) {
            soft_hash(k + t * D, pl, D, L, K, inv_temp, th, PK);
            for (int64_t s = 0; s < S; ++s) {
                A[s] += PK[s];
                for (int64_t d = 0; d < D; ++d)
                    B[s * D + d] += PK[s] * v[t * D + d];
            }
        }
    }
    /* pass 1 (forward in t): state, dP_Q -> dq, dA and W per token */
    for (int64_t t = 0; t < T; ++t) {
        if (causal) {
            soft_hash(k + t * D, pl, D, L, K, inv_temp, th, PK);
            for (int64_t s = 0; s < S; ++s) {
                A[s] += PK[s];
                for (int64_t d = 0; d < D; ++d)
                    B[s * D + d] += PK[s] * v[t * D + d];
            }
        }
        soft_hash(q + t * D, pl, D, L, K, inv_temp, th, PQ);
        const double *gt = g + t * D;
        for (int64_t s = 0; s < S; ++s) {
            const double inv = 1.0 / (A[s] + eps);
            double G = 0.0;
            for (int64_t d = 0; d < D; ++d)
                G += gt[d] * B[s * D + d];
            dP[s] = G * inv;
            W[t * S + s] = PQ[s] * inv;
            dA[t * S + s] = -PQ[s] * inv * G * inv;
        }
        soft_hash_bwd(PQ, th, dP, pl, D, L, K, inv_temp, dq + t * D, g_it, g_abs);
    }
    if (!causal) {
        for (int64_t t = 0; t < T; ++t) {
            const double *gt = g + t * D;
            for (int64_t s = 0; s < S; ++s) {
                alpha[s] += dA[t * S + s];
                for (int64_t d = 0; d < D; ++d)
                    U[s * D + d] += W[t * S + s] * gt[d];
            }
        }
    }
    /* pass 2 (reverse in t): suffix sums alpha, U -> dP_K -> dk, dv */
    for (int64_t t = T - 1; t >= 0; --t) {
        const double *gt = g + t * D;
        const double *vt = v + t * D;
        if (causal) {
            for (int64_t s = 0; s < S; ++s) {
                alpha[s] += dA[t * S + s];
                for (int64_t d = 0; d < D; ++d)
                    U[s * D + d] += W[t * S + s] * gt[d];
            }
        }
        soft_hash(k + t * D, pl, D, L, K, inv_temp, th, PK);
        double *dvt = dv + t * D;
        for (int64_t s = 0; s < S; ++s) {
            double vu = 0.0;
            for (int64_t d = 0; d < D; ++d) {
                vu += vt[d] * U[s * D + d];
                dvt[d] += PK[s] * U[s * D + d];
            }
            dP[s] = alpha[s] + vu;
        }
        soft_hash_bwd(PK, th, dP, pl, D, L, K, inv_temp, dk + t * D, g_it, g_abs);
    }
    free(A); free(B); free(dA); free(W); free(th); free(PK); free(PQ);
    free(dP); free(alpha); free(U);
}

/* ---------------------------------------------------------------- exports */

int oracle_race_forward(const double *q, const double *k, const double *v,
                        const double *planes, const int64_t *plane_of,
                        int64_t N, int64_t T, int64_t D, int L, int K,
                        int causal, double eps, double inv_temp, double *out)
{
    if (K < 1 || K > ORACLE_MAX_K || L < 1 || N < 0 || T < 0 || D < 1)
        return -1;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t n = 0; n < N; ++n) {
        const double *pl = planes + plane_of[n] * (int64_t)L * K * D;
        stream_forward(q + n * T * D, k + n * T * D, v + n * T * D, pl, T, D,
                       L, K, causal, eps, inv_temp, out + n * T * D);
    }
    return 0;
}

int oracle_race_backward(const double *q, const double *k, const double *v,
                         const double *dout, const double *planes,
                         const int64_t *plane_of, int64_t N, int64_t T,
                         int64_t D, int L, int K, int causal, double eps,
                         double inv_temp, double *dq, double *dk, double *dv,
                         double *grad_inv_temp, double *grad_inv_temp_l1)
{
    if (K < 1 || K > ORACLE_MAX_K || L < 1 || N < 0 || T < 0 || D < 1)
        return -1;
    double *part = calloc((size_t)(N > 0 ? N : 1), sizeof(double));
    double *pabs = calloc((size_t)(N > 0 ? N : 1), sizeof(double));
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t n = 0; n < N; ++n) {
        const double *pl = planes + plane_of[n] * (int64_t)L * K * D;
        const int64_t o = n * T * D;
        stream_backward(q + o, k + o, v + o, dout + o, pl, T, D, L, K, causal,
                        eps, inv_temp, dq + o, dk + o, dv + o, &part[n], &pabs[n]);
    }
    double tot = 0.0, tabs = 0.0;
    for (int64_t n = 0; n < N; ++n) {
        tot += part[n];
        tabs += pabs[n];
    }
    if (grad_inv_temp)
        *grad_inv_temp = tot;
    if (grad_inv_temp_l1)
        *grad_inv_temp_l1 = tabs;
    free(part);
    free(pabs);
    return 0;
}

/* Restatement of race_prefix_mean_flat (kernels/cpu/race_pref.cpp:36-101):
 * w [NS][T], v [NS][T][D] float; E[ns,t,:] = B_t/(A_t+eps) with fp64 running
 * sums A_t = sum_{tau<=t} w, B_t = sum_{tau<=t} w v. */
void oracle_prefix_mean_flat(const float *w, const float *v, int64_t NS,
                             int64_t T, int64_t D, double eps, float *E)
{
#pragma omp parallel for schedule(static)
    for (int64_t ns = 0; ns < NS; ++ns) {
        double A = 0.0;
        double *B = calloc((size_t)D, sizeof(double));
        const float *wn = w + ns * T;
        const float *vn = v + ns * T * D;
        float *en = E + ns * T * D;
        for (int64_t t = 0; t < T; ++t) {
            const double wt = (double)wn[t];
            A += wt;
            const double inv = 1.0 / (A + eps);
            for (int64_t d = 0; d < D; ++d) {
                B[d] += wt * (double)vn[t * D + d];
                en[t * D + d] = (float)(B[d] * inv);
            }
        }
        free(B);
    }
}

/* Restatement of race_prefix_mean_flat_bw (kernels/cpu/race_pref.cpp:104-220):
 * pass 1 forward builds invA[t] and alpha[t] = -invA^2 (g_t . B_t); pass 2
 * reverse keeps suffix sums beta = sum g invA and a = sum alpha, giving
 * gW[t] = a + beta . v_t and gV[t] = w_t beta. */
void oracle_prefix_mean_flat_bw(const float *w, const float *v, const float *gE,
                                int64_t NS, int64_t T, int64_t D, double eps,
                                float *gW, float *gV)
{
#pragma omp parallel for schedule(static)
    for (int64_t ns = 0; ns < NS; ++ns) {
        const float *wn = w + ns * T;
        const float *vn = v + ns * T * D;
        const float *gn = gE + ns * T * D;
        double *invA = malloc(sizeof(double) * (size_t)(T > 0 ? T : 1));
        double *al = malloc(sizeof(double) * (size_t)(T > 0 ? T : 1));
        double *B = calloc((size_t)D, sizeof(double));
        double *beta = calloc((size_t)D, sizeof(double));
        double A = 0.0;
        for (int64_t t = 0; t < T; ++t) {
            const double wt = (double)wn[t];
            A += wt;
            double gb = 0.0;
            for (int64_t d = 0; d < D; ++d) {
                B[d] += wt * (double)vn[t * D + d];
                gb += (double)gn[t * D + d] * B[d];
            }
            invA[t] = 1.0 / (A + eps);
            al[t] = -invA[t] * invA[t] * gb;
        }
        double asuf = 0.0;
        for (int64_t t = T - 1; t >= 0; --t) {
            double bv = 0.0;
            for (int64_t d = 0; d < D; ++d) {
                beta[d] += (double)gn[t * D + d] * invA[t];
                bv += beta[d] * (double)vn[t * D + d];
            }
            asuf += al[t];
            gW[ns * T + t] = (float)(asuf + bv);
            const double wt = (double)wn[t];
            for (int64_t d = 0; d < D; ++d)
                gV[(ns * T + t) * D + d] = (float)(wt * beta[d]);
        }
        free(invA); free(al); free(B); free(beta);
    }
}

/* ------------------------------------------------- global normalisation (F2)
 *
 * Causal RACE with one normaliser per token instead of one per bucket
 * (CausalRACEAttention, misc/elsaa_causal_complete.py:438-586; the Triton
 * readout misc/race_kernel.py:8-124; its autograd
 * misc/elsaa_causal_complete.py:384-436):
 *   P = softmax_r(beta * sum_k c[r,k] tanh(<x, w_lk>))        (:483-490)
 *   num_t = sum_s P_Q[t,s] B_s(t),  den_t = sum_s P_Q[t,s] A_s(t)
 *           (sums over all L tables, race_kernel.py:108-123)
 *   out_t = num_t / max(den_t, floor)                           (:537)
 * with A, B the inclusive prefixes of P_K and P_K v.  beta enters exactly as
 * inv_temp does in F1, so soft_hash / soft_hash_bwd serve both. */
static void stream_forward_global(const double *q, const double *k, const double *v,
                                  const double *pl, int64_t T, int64_t D, int L, int K,
                                  double floor_, double beta, double *o, double *den)
{
    const int R = 1 << K;
    const int64_t S = (int64_t)L * R;
    double *A = calloc((size_t)S, sizeof(double));
    double *B = calloc((size_t)(S * D), sizeof(double));
    double *th = malloc(sizeof(double) * (size_t)(L * K));
    double *PK = malloc(sizeof(double) * (size_t)S);
    double *PQ = malloc(sizeof(double) * (size_t)S);
    for (int64_t t = 0; t < T; ++t) {
        soft_hash(k + t * D, pl, D, L, K, beta, th, PK);
        for (int64_t s = 0; s < S; ++s) {
            A[s] += PK[s];
            for (int64_t d = 0; d < D; ++d)
                B[s * D + d] += PK[s] * v[t * D + d];
        }
        soft_hash(q + t * D, pl, D, L, K, beta, th, PQ);
        double *ot = o + t * D, dn = 0.0;
        for (int64_t d = 0; d < D; ++d)
            ot[d] = 0.0;
        for (int64_t s = 0; s < S; ++s) {
            dn += PQ[s] * A[s];
            for (int64_t d = 0; d < D; ++d)
                ot[d] += PQ[s] * B[s * D + d];
        }
        den[t] = dn;
        const double dc = dn > floor_ ? dn : floor_;
        for (int64_t d = 0; d < D; ++d)
            ot[d] /= dc;
    }
    free(A); free(B); free(th); free(PK); free(PQ);
}

/* Backward of stream_forward_global for upstream gradients g (of out) and h
 * (of den, may be NULL).  With dc = max(den, floor):
 *   gd_t      = h_t - [den_t >= floor] (g_t . out_t) / dc_t
 *   dP_Q[t,s] = (g_t . B_s(t)) / dc_t + gd_t A_s(t)
 *   W[t,s]    = P_Q[t,s] / dc_t,     dA[t,s] = gd_t P_Q[t,s]
 * and then, as in F1, alpha_s(tau) = sum_{t>=tau} dA[t,s],
 * U_s(tau) = sum_{t>=tau} W[t,s] g_t, dP_K[tau,s] = alpha_s(tau) + v_tau . U_s(tau),
 * dv_tau = sum_s P_K[tau,s] U_s(tau). */
static void stream_backward_global(const double *q, const double *k, const double *v,
                                   const double *g, const double *h, const double *pl,
                                   int64_t T, int64_t D, int L, int K, double floor_,
                                   double beta, double *dq, double *dk, double *dv,
                                   double *g_beta, double *g_abs)
{
    const int R = 1 << K;
    const int64_t S = (int64_t)L * R;
    double *A = calloc((size_t)S, sizeof(double));
    double *B = calloc((size_t)(S * D), sizeof(double));
    double *dA = malloc(sizeof(double) * (size_t)(T * S));
    double *W = malloc(sizeof(double) * (size_t)(T * S));
    double *th = malloc(sizeof(double) * (size_t)(L * K));
    double *PK = malloc(sizeof(double) * (size_t)S);
    double *PQ = malloc(sizeof(double) * (size_t)S);
    double *dP = malloc(sizeof(double) * (size_t)S);
    double *alpha = calloc((size_t)S, sizeof(double));
    double *U = calloc((size_t)(S * D), sizeof(double));
    double *num = malloc(sizeof(double) * (size_t)D);

    memset(dq, 0, sizeof(double) * (size_t)(T * D));
    memset(dk, 0, sizeof(double) * (size_t)(T * D));
    memset(dv, 0, sizeof(double) * (size_t)(T * D));
    for (int64_t t = 0; t < T; ++t) {
        soft_hash(k + t * D, pl, D, L, K, beta, th, PK);
        for (int64_t s = 0; s < S; ++s) {
            A[s] += PK[s];
            for (int64_t d = 0; d < D; ++d)
                B[s * D + d] += PK[s] * v[t * D + d];
        }
        soft_hash(q + t * D, pl, D, L, K, beta, th, PQ);
        const double *gt = g + t * D;
        double dn = 0.0;
        for (int64_t d = 0; d < D; ++d)
            num[d] = 0.0;
        for (int64_t s = 0; s < S; ++s) {
            dn += PQ[s] * A[s];
            for (int64_t d = 0; d < D; ++d)
                num[d] += PQ[s] * B[s * D + d];
        }
        const double dc = dn > floor_ ? dn : floor_;
        double go = 0.0;
        for (int64_t d = 0; d < D; ++d)
            go += gt[d] * num[d] / dc;
        const double gd = (h ? h[t] : 0.0) - (dn >= floor_ ? go / dc : 0.0);
        for (int64_t s = 0; s < S; ++s) {
            double G = 0.0;
            for (int64_t d = 0; d < D; ++d)
                G += gt[d] * B[s * D + d];
            dP[s] = G / dc + gd * A[s];
            W[t * S + s] = PQ[s] / dc;
            dA[t * S + s] = gd * PQ[s];
        }
        soft_hash_bwd(PQ, th, dP, pl, D, L, K, beta, dq + t * D, g_beta, g_abs);
    }
    for (int64_t t = T - 1; t >= 0; --t) {
        const double *gt = g + t * D;
        const double *vt = v + t * D;
        for (int64_t s = 0; s < S; ++s) {
            alpha[s] += dA[t * S + s];
            for (int64_t d = 0; d < D; ++d)
                U[s * D + d] += W[t * S + s] * gt[d];
        }
        soft_hash(k + t * D, pl, D, L, K, beta, th, PK);
        double *dvt = dv + t * D;
        for (int64_t s = 0; s < S; ++s) {
            double vu = 0.0;
            for (int64_t d = 0; d < D; ++d) {
                vu += vt[d] * U[s * D + d];
                dvt[d] += PK[s] * U[s * D + d];
            }
            dP[s] = alpha[s] + vu;
        }
        soft_hash_bwd(PK, th, dP, pl, D, L, K, beta, dk + t * D, g_beta, g_abs);
    }
    free(A); free(B); free(dA); free(W); free(th); free(PK); free(PQ);
    free(dP); free(alpha); free(U); free(num);
}

int oracle_race_global_forward(const double *q, const double *k, const double *v,
                               const double *planes, const int64_t *plane_of,
                               int64_t N, int64_t T, int64_t D, int L, int K,
                               double floor_, double beta, double *out, double *den)
{
    if (K < 1 || K > ORACLE_MAX_K || L < 1 || N < 0 || T < 0 || D < 1)
        return -1;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t n = 0; n < N; ++n) {
        const double *pl = planes + plane_of[n] * (int64_t)L * K * D;
        stream_forward_global(q + n * T * D, k + n * T * D, v + n * T * D, pl, T, D,
                              L, K, floor_, beta, out + n * T * D, den + n * T);
    }
    return 0;
}

int oracle_race_global_backward(const double *q, const double *k, const double *v,
                                const double *dout, const double *dden,
                                const double *planes, const int64_t *plane_of,
                                int64_t N, int64_t T, int64_t D, int L, int K,
                                double floor_, double beta, double *dq, double *dk,
                                double *dv, double *grad_beta, double *grad_beta_l1)
{
    if (K < 1 || K > ORACLE_MAX_K || L < 1 || N < 0 || T < 0 || D < 1)
        return -1;
    double *part = calloc((size_t)(N > 0 ? N : 1), sizeof(double));
    double *pabs = calloc((size_t)(N > 0 ? N : 1), sizeof(double));
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t n = 0; n < N; ++n) {
        const double *pl = planes + plane_of[n] * (int64_t)L * K * D;
        const int64_t o = n * T * D;
        stream_backward_global(q + o, k + o, v + o, dout + o, dden ? dden + n * T : NULL, pl,
                               T, D, L, K, floor_, beta, dq + o, dk + o, dv + o,
                               &part[n], &pabs[n]);
    }
    double tot = 0.0, tabs = 0.0;
    for (int64_t n = 0; n < N; ++n) {
        tot += part[n];
        tabs += pabs[n];
    }
    if (grad_beta)
        *grad_beta = tot;
    if (grad_beta_l1)
        *grad_beta_l1 = tabs;
    free(part);
    free(pabs);
    return 0;
}

/* ------------------------------------------- key weights and den (F1 extras)
 *
 * The padded-batch forms of the non-causal operator
 * (misc/classification.py:576-592, BatchedACE.forward with mask;
 * :641-659 and misc/vit.py:1452-1510, _ace_with_denom):
 *   P_K'[t,s] = w_t P_K[t,s]   (w: per-token key weight, the mask)
 *   A, B from P_K' (V is masked by the caller), out as in F1,
 *   den_t = sum_s P_Q[t,s] A_s(t)   (unclamped; the caller clamps).
 * Causal and non-causal, like stream_forward.  w and den may be NULL. */
static void stream_forward_ex(const double *q, const double *k, const double *v,
                              const double *w, const double *pl, int64_t T, int64_t D,
                              int L, int K, int causal, double eps, double inv_temp,
                              double *o, double *den)
{
    const int R = 1 << K;
    const int64_t S = (int64_t)L * R;
    double *A = calloc((size_t)S, sizeof(double));
    double *B = calloc((size_t)(S * D), sizeof(double));
    double *th = malloc(sizeof(double) * (size_t)(L * K));
    double *PK = malloc(sizeof(double) * (size_t)S);
    double *PQ = malloc(sizeof(double) * (size_t)S);
    for (int64_t pass = causal ? 1 : 0; pass < 2; ++pass) {
        for (int64_t t = 0; t < T; ++t) {
            if (pass == 0 || causal) {
                soft_hash(k + t * D, pl, D, L, K, inv_temp, th, PK);
                const double wt = w ? w[t] : 1.0;
                for (int64_t s = 0; s < S; ++s) {
                    A[s] += wt * PK[s];
                    for (int64_t d = 0; d < D; ++d)
                        B[s * D + d] += wt * PK[s] * v[t * D + d];
                }
            }
            if (pass == 0)
                continue;
            soft_hash(q + t * D, pl, D, L, K, inv_temp, th, PQ);
            double *ot = o + t * D, dn = 0.0;
            for (int64_t d = 0; d < D; ++d)
                ot[d] = 0.0;
            for (int64_t s = 0; s < S; ++s) {
                dn += PQ[s] * A[s];
                const double ws = PQ[s] / (A[s] + eps);
                for (int64_t d = 0; d < D; ++d)
                    ot[d] += ws * B[s * D + d];
            }
            if (den)
                den[t] = dn;
        }
    }
    free(A); free(B); free(th); free(PK); free(PQ);
}

/* Backward of stream_forward_ex for upstream gradients g (out) and h (den,
 * may be NULL): F1's formulas with P_K' = w P_K, plus
 *   dP_Q[t,s] += h_t A_s(t),  dA[t,s] += h_t P_Q[t,s],
 * and dP_K = w (alpha + v . U) through the weight. */
static void stream_backward_ex(const double *q, const double *k, const double *v,
                               const double *w, const double *g, const double *h,
                               const double *pl, int64_t T, int64_t D, int L, int K,
                               int causal, double eps, double inv_temp, double *dq,
                               double *dk, double *dv, double *g_it, double *g_abs)
{
    const int R = 1 << K;
    const int64_t S = (int64_t)L * R;
    double *A = calloc((size_t)S, sizeof(double));
    double *B = calloc((size_t)(S * D), sizeof(double));
    double *dA = malloc(sizeof(double) * (size_t)(T * S));
    double *W = malloc(sizeof(double) * (size_t)(T * S));
    double *th = malloc(sizeof(double) * (size_t)(L * K));
    double *PK = malloc(sizeof(double) * (size_t)S);
    double *PQ = malloc(sizeof(double) * (size_t)S);
    double *dP = malloc(sizeof(double) * (size_t)S);
    double *alpha = calloc((size_t)S, sizeof(double));
    double *U = calloc((size_t)(S * D), sizeof(double));

    memset(dq, 0, sizeof(double) * (size_t)(T * D));
    memset(dk, 0, sizeof(double) * (size_t)(T * D));
    memset(dv, 0, sizeof(double) * (size_t)(T * D));
    for (int64_t pass = causal ? 1 : 0; pass < 2; ++pass) {
        for (int64_t t = 0; t < T; ++t) {
            if (pass == 0 || causal) {
                soft_hash(k + t * D, pl, D, L, K, inv_temp, th, PK);
                const double wt = w ? w[t] : 1.0;
                for (int64_t s = 0; s < S; ++s) {
                    A[s] += wt * PK[s];
                    for (int64_t d = 0; d < D; ++d)
                        B[s * D + d] += wt * PK[s] * v[t * D + d];
                }
            }
            if (pass == 0)
                continue;
            soft_hash(q + t * D, pl, D, L, K, inv_temp, th, PQ);
            const double *gt = g + t * D;
            const double ht = h ? h[t] : 0.0;
            for (int64_t s = 0; s < S; ++s) {
                const double inv = 1.0 / (A[s] + eps);
                double G = 0.0;
                for (int64_t d = 0; d < D; ++d)
                    G += gt[d] * B[s * D + d];
                dP[s] = G * inv + ht * A[s];
                W[t * S + s] = PQ[s] * inv;
                dA[t * S + s] = -PQ[s] * inv * G * inv + ht * PQ[s];
            }
            soft_hash_bwd(PQ, th, dP, pl, D, L, K, inv_temp, dq + t * D, g_it, g_abs);
        }
    }
    if (!causal) {
        for (int64_t t = 0; t < T; ++t) {
            const double *gt = g + t * D;
            for (int64_t s = 0; s < S; ++s) {
                alpha[s] += dA[t * S + s];
                for (int64_t d = 0; d < D; ++d)
                    U[s * D + d] += W[t * S + s] * gt[d];
            }
        }
    }
    for (int64_t t = T - 1; t >= 0; --t) {
        const double *gt = g + t * D;
        const double *vt = v + t * D;
        if (causal) {
            for (int64_t s = 0; s < S; ++s) {
                alpha[s] += dA[t * S + s];
                for (int64_t d = 0; d < D; ++d)
                    U[s * D + d] += W[t * S + s] * gt[d];
            }
        }
        soft_hash(k + t * D, pl, D, L, K, inv_temp, th, PK);
        const double wt = w ? w[t] : 1.0;
        double *dvt = dv + t * D;
        for (int64_t s = 0; s < S; ++s) {
            double vu = 0.0;
            for (int64_t d = 0; d < D; ++d) {
                vu += vt[d] * U[s * D + d];
                dvt[d] += wt * PK[s] * U[s * D + d];
            }
            dP[s] = wt * (alpha[s] + vu);
        }
        soft_hash_bwd(PK, th, dP, pl, D, L, K, inv_temp, dk + t * D, g_it, g_abs);
    }
    free(A); free(B); free(dA); free(W); free(th); free(PK); free(PQ);
    free(dP); free(alpha); free(U);
}

int oracle_race_forward_ex(const double *q, const double *k, const double *v,
                           const double *kw, const double *planes, const int64_t *plane_of,
                           int64_t N, int64_t T, int64_t D, int L, int K, int causal,
                           double eps, double inv_temp, double *out, double *den)
{
    if (K < 1 || K > ORACLE_MAX_K || L < 1 || N < 0 || T < 0 || D < 1)
        return -1;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t n = 0; n < N; ++n) {
        const double *pl = planes + plane_of[n] * (int64_t)L * K * D;
        stream_forward_ex(q + n * T * D, k + n * T * D, v + n * T * D, kw ? kw + n * T : NULL,
                          pl, T, D, L, K, causal, eps, inv_temp, out + n * T * D,
                          den ? den + n * T : NULL);
    }
    return 0;
}

int oracle_race_backward_ex(const double *q, const double *k, const double *v,
                            const double *kw, const double *dout, const double *dden,
                            const double *planes, const int64_t *plane_of, int64_t N,
                            int64_t T, int64_t D, int L, int K, int causal, double eps,
                            double inv_temp, double *dq, double *dk, double *dv,
                            double *grad_inv_temp, double *grad_inv_temp_l1)
{
    if (K < 1 || K > ORACLE_MAX_K || L < 1 || N < 0 || T < 0 || D < 1)
        return -1;
    double *part = calloc((size_t)(N > 0 ? N : 1), sizeof(double));
    double *pabs = calloc((size_t)(N > 0 ? N : 1), sizeof(double));
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t n = 0; n < N; ++n) {
        const double *pl = planes + plane_of[n] * (int64_t)L * K * D;
        const int64_t o = n * T * D;
        stream_backward_ex(q + o, k + o, v + o, kw ? kw + n * T : NULL, dout + o,
                           dden ? dden + n * T : NULL, pl, T, D, L, K, causal, eps, inv_temp,
                           dq + o, dk + o, dv + o, &part[n], &pabs[n]);
    }
    double tot = 0.0, tabs = 0.0;
    for (int64_t n = 0; n < N; ++n) {
        tot += part[n];
        tabs += pabs[n];
    }
    if (grad_inv_temp)
        *grad_inv_temp = tot;
    if (grad_inv_temp_l1)
        *grad_inv_temp_l1 = tabs;
    free(part);
    free(pabs);
    return 0;
}

/* ------------------------------------------------ bucket probabilities
 * P[n][t][s] of one input (misc/arxiv_64K.py:1580-1644,
 * misc/vit.py:3193-3262: projection, tanh, /temperature, corner logits,
 * softmax per table) and the backward dP -> dx, d inv_temp. */
int oracle_race_probs(const double *x, const double *planes, const int64_t *plane_of,
                      int64_t N, int64_t T, int64_t D, int L, int K, double inv_temp,
                      double *P)
{
    if (K < 1 || K > ORACLE_MAX_K || L < 1 || N < 0 || T < 0 || D < 1)
        return -1;
    const int64_t S = (int64_t)L << K;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t n = 0; n < N; ++n) {
        const double *pl = planes + plane_of[n] * (int64_t)L * K * D;
        double *th = malloc(sizeof(double) * (size_t)(L * K));
        for (int64_t t = 0; t < T; ++t)
            soft_hash(x + (n * T + t) * D, pl, D, L, K, inv_temp, th, P + (n * T + t) * S);
        free(th);
    }
    return 0;
}

int oracle_race_probs_bwd(const double *x, const double *dP, const double *planes,
                          const int64_t *plane_of, int64_t N, int64_t T, int64_t D, int L,
                          int K, double inv_temp, double *dx, double *grad_inv_temp,
                          double *grad_inv_temp_l1)
{
    if (K < 1 || K > ORACLE_MAX_K || L < 1 || N < 0 || T < 0 || D < 1)
        return -1;
    const int64_t S = (int64_t)L << K;
    double *part = calloc((size_t)(N > 0 ? N : 1), sizeof(double));
    double *pabs = calloc((size_t)(N > 0 ? N : 1), sizeof(double));
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t n = 0; n < N; ++n) {
        const double *pl = planes + plane_of[n] * (int64_t)L * K * D;
        double *th = malloc(sizeof(double) * (size_t)(L * K));
        double *P = malloc(sizeof(double) * (size_t)S);
        for (int64_t t = 0; t < T; ++t) {
            double *dxt = dx + (n * T + t) * D;
            memset(dxt, 0, sizeof(double) * (size_t)D);
            soft_hash(x + (n * T + t) * D, pl, D, L, K, inv_temp, th, P);
            soft_hash_bwd(P, th, dP + (n * T + t) * S, pl, D, L, K, inv_temp, dxt, &part[n], &pabs[n]);
        }
        free(th);
        free(P);
    }
    double tot = 0.0, tabs = 0.0;
    for (int64_t n = 0; n < N; ++n) {
        tot += part[n];
        tabs += pabs[n];
    }
    if (grad_inv_temp)
        *grad_inv_temp = tot;
    if (grad_inv_temp_l1)
        *grad_inv_temp_l1 = tabs;
    free(part);
    free(pabs);
    return 0;
}
