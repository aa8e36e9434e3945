// prefix_mean.hip -- gfx950 kernels of the flat causal prefix mean, the
// operator of the reference CPU extension (kernels/cpu/race_pref.cpp:36-220):
//   E[n,t,:] = B_t / (A_t + eps),  A_t = sum_{tau<=t} w,  B_t = sum_{tau<=t} w v
// and its backward.  Accumulation is fp64 as in the reference.  Streams are
// split into token segments; a three-phase scan (segment sums, segment
// prefix, per-segment walk) carries (A, B) across segments.  One 64-lane wave
// per (segment, stream); lane l owns columns l, l+64, ... (D <= 512).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace race {

constexpr int PM_MAXC = 8;  // columns per lane -> D <= 512

__device__ __forceinline__ double wave_sum(double x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

// per-segment sums of (B, A): delta[ns][seg][0..D) = B, [D] = A
__global__ __launch_bounds__(64) void k_pm_reduce(const float *__restrict__ w, const float *__restrict__ v,
                                                  double *__restrict__ delta, int64_t T, int D, int64_t tseg,
                                                  int nseg) {
    const int64_t ns = blockIdx.y;
    const int seg = blockIdx.x, lane = threadIdx.x;
    const int64_t t0 = seg * tseg, t1 = min(T, t0 + tseg);
    double B[PM_MAXC], A = 0.0;
    for (int c = 0; c < PM_MAXC; ++c) B[c] = 0.0;
    for (int64_t t = t0; t < t1; ++t) {
        const double wt = (double)w[ns * T + t];
        A += wt;
        const float *vt = v + (ns * T + t) * D;
        for (int c = 0; c < PM_MAXC; ++c) {
            const int d = lane + 64 * c;
            if (d < D) B[c] += wt * (double)vt[d];
        }
    }
    double *o = delta + (ns * nseg + seg) * (int64_t)(D + 1);
    for (int c = 0; c < PM_MAXC; ++c) {
        const int d = lane + 64 * c;
        if (d < D) o[d] = B[c];
    }
    if (lane == 0) o[D] = A;
}

// exclusive prefix over segments: state[ns][seg] (seg <= nseg)
__global__ void k_pm_scan(double *state, const double *delta, int nseg, int elems) {
    const int64_t ns = blockIdx.y;
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= elems) return;
    double acc = 0.0;
    for (int s = 0; s < nseg; ++s) {
        state[(ns * (nseg + 1) + s) * elems + e] = acc;
        acc += delta[(ns * nseg + s) * elems + e];
    }
    state[(ns * (nseg + 1) + nseg) * elems + e] = acc;
}

// exclusive suffix over segments: rstate[ns][seg] = sum of rdelta over later segments
__global__ void k_pm_rscan(double *rstate, const double *rdelta, int nseg, int elems) {
    const int64_t ns = blockIdx.y;
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= elems) return;
    double acc = 0.0;
    for (int s = nseg - 1; s >= 0; --s) {
        rstate[(ns * nseg + s) * elems + e] = acc;
        acc += rdelta[(ns * nseg + s) * elems + e];
    }
}

// forward walk: E (race_pref.cpp:82-98 order: A += w; inv; B += w v; E = B inv)
__global__ __launch_bounds__(64) void k_pm_out(const float *__restrict__ w, const float *__restrict__ v,
                                               float *__restrict__ E, const double *__restrict__ state, int64_t T,
                                               int D, int64_t tseg, int nseg, double eps) {
    const int64_t ns = blockIdx.y;
    const int seg = blockIdx.x, lane = threadIdx.x;
    const int64_t t0 = seg * tseg, t1 = min(T, t0 + tseg);
    const double *st = state + (ns * (nseg + 1) + seg) * (int64_t)(D + 1);
    double B[PM_MAXC], A = st[D];
    for (int c = 0; c < PM_MAXC; ++c) B[c] = (lane + 64 * c < D) ? st[lane + 64 * c] : 0.0;
    for (int64_t t = t0; t < t1; ++t) {
        const double wt = (double)w[ns * T + t];
        A += wt;
        const double inv = 1.0 / (A + eps);
        const float *vt = v + (ns * T + t) * D;
        float *et = E + (ns * T + t) * D;
        for (int c = 0; c < PM_MAXC; ++c) {
            const int d = lane + 64 * c;
            if (d < D) {
                B[c] += wt * (double)vt[d];
                et[d] = (float)(B[c] * inv);
            }
        }
    }
}

// backward pass 1 (forward walk, race_pref.cpp:161-182): invA[t], alpha[t];
// per-segment sums rdelta[..][0..D) = sum g invA, [D] = sum alpha
__global__ __launch_bounds__(64) void k_pm_bw_fwd(const float *__restrict__ w, const float *__restrict__ v,
                                                  const float *__restrict__ gE, const double *__restrict__ state,
                                                  double *__restrict__ invA, double *__restrict__ alpha,
                                                  double *__restrict__ rdelta, int64_t T, int D, int64_t tseg,
                                                  int nseg, double eps) {
    const int64_t ns = blockIdx.y;
    const int seg = blockIdx.x, lane = threadIdx.x;
    const int64_t t0 = seg * tseg, t1 = min(T, t0 + tseg);
    const double *st = state + (ns * (nseg + 1) + seg) * (int64_t)(D + 1);
    double B[PM_MAXC], bsum[PM_MAXC], A = st[D], asum = 0.0;
    for (int c = 0; c < PM_MAXC; ++c) {
        B[c] = (lane + 64 * c < D) ? st[lane + 64 * c] : 0.0;
        bsum[c] = 0.0;
    }
    for (int64_t t = t0; t < t1; ++t) {
        const double wt = (double)w[ns * T + t];
        A += wt;
        const float *vt = v + (ns * T + t) * D;
        const float *gt = gE + (ns * T + t) * D;
        double dot = 0.0;
        for (int c = 0; c < PM_MAXC; ++c) {
            const int d = lane + 64 * c;
            if (d < D) {
                B[c] += wt * (double)vt[d];
                dot += (double)gt[d] * B[c];
            }
        }
        dot = wave_sum(dot);
        const double iA = 1.0 / (A + eps);
        const double al = -(iA * iA) * dot;
        if (lane == 0) {
            invA[ns * T + t] = iA;
            alpha[ns * T + t] = al;
        }
        asum += al;
        for (int c = 0; c < PM_MAXC; ++c) {
            const int d = lane + 64 * c;
            if (d < D) bsum[c] += (double)gt[d] * iA;
        }
    }
    double *o = rdelta + (ns * nseg + seg) * (int64_t)(D + 1);
    for (int c = 0; c < PM_MAXC; ++c) {
        const int d = lane + 64 * c;
        if (d < D) o[d] = bsum[c];
    }
    if (lane == 0) o[D] = asum;
}

// backward pass 2 (reverse walk, race_pref.cpp:188-216): gW, gV
__global__ __launch_bounds__(64) void k_pm_bw_rev(const float *__restrict__ w, const float *__restrict__ v,
                                                  const float *__restrict__ gE, const double *__restrict__ invA,
                                                  const double *__restrict__ alpha,
                                                  const double *__restrict__ rstate, float *__restrict__ gW,
                                                  float *__restrict__ gV, int64_t T, int D, int64_t tseg,
                                                  int nseg) {
    const int64_t ns = blockIdx.y;
    const int seg = blockIdx.x, lane = threadIdx.x;
    const int64_t t0 = seg * tseg, t1 = min(T, t0 + tseg);
    const double *rs = rstate + (ns * nseg + seg) * (int64_t)(D + 1);
    double beta[PM_MAXC], asuf = rs[D];
    for (int c = 0; c < PM_MAXC; ++c) beta[c] = (lane + 64 * c < D) ? rs[lane + 64 * c] : 0.0;
    for (int64_t t = t1 - 1; t >= t0; --t) {
        const double iA = invA[ns * T + t];
        const float *vt = v + (ns * T + t) * D;
        const float *gt = gE + (ns * T + t) * D;
        float *gvt = gV + (ns * T + t) * D;
        asuf += alpha[ns * T + t];
        const double wt = (double)w[ns * T + t];
        double dot = 0.0;
        for (int c = 0; c < PM_MAXC; ++c) {
            const int d = lane + 64 * c;
            if (d < D) {
                beta[c] += (double)gt[d] * iA;
                dot += beta[c] * (double)vt[d];
                gvt[d] = (float)(wt * beta[c]);
            }
        }
        dot = wave_sum(dot);
        if (lane == 0) gW[ns * T + t] = (float)(asuf + dot);
    }
}

} // namespace race
