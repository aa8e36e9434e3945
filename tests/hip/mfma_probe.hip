// Test-only probe of the MFMA fragment helpers in race_device.h: computes
// C = A . B^T for one 16x16 tile with 64-deep k (two 32-deep steps) from LDS,
// plus the strided-B and transposed-store variants.  In-bounds by
// construction: one 64-lane wave, fixed 16x64 operands.
#include "../../race_attention_amd/csrc/race_device.h"
using namespace race;

template <typename T>
__global__ __launch_bounds__(64) void k_probe(const T *A, const T *B, float *C, float *Cbt, float *Ct) {
    constexpr int LD = ld_of<T>(64);
    __shared__ __align__(16) T sA[16 * LD], sB[16 * LD], sBkn[64 * ld_of<T>(16)];
    for (int idx = threadIdx.x; idx < 16 * 64; idx += 64) {
        const int r = idx / 64, c = idx % 64;
        sA[r * LD + c] = A[idx];
        sB[r * LD + c] = B[idx];
        sBkn[c * ld_of<T>(16) + r] = B[idx];  // B stored [k][n]
    }
    __syncthreads();
    f32x4 acc = zero4();
    tile_mma(acc, sA, LD, sB, LD, 2);
    f32x4 acc2 = zero4();
    tile_mma_bT(acc2, sA, LD, sBkn, ld_of<T>(16), 2);
    const int i = lane_id() & 15, g = lane_id() >> 4;
    for (int e = 0; e < 4; ++e) {
        C[(4 * g + e) * 16 + i] = acc[e];
        Cbt[(4 * g + e) * 16 + i] = acc2[e];
    }
    __shared__ float sT[16 * 20];
    st_tile_T(sT, 20, acc);
    __syncthreads();
    for (int idx = threadIdx.x; idx < 256; idx += 64) Ct[idx] = sT[(idx / 16) * 20 + idx % 16];
}

extern "C" int probe_mfma(int bf16, const void *A, const void *B, float *C, float *Cbt, float *Ct) {
    if (bf16)
        k_probe<race::bf16><<<1, 64>>>((const race::bf16 *)A, (const race::bf16 *)B, C, Cbt, Ct);
    else
        k_probe<float><<<1, 64>>>((const float *)A, (const float *)B, C, Cbt, Ct);
    return hipDeviceSynchronize() == hipSuccess ? 0 : -1;
}

// Row (16-lane) DPP scans: out[0..63] prefix, [64..127] suffix, [128..191] row
// sum, [192..255] lane 0 of the row broadcast to the row.
__global__ __launch_bounds__(64) void k_probe_rows(const float *x, float *out) {
    const float v = x[threadIdx.x];
    out[threadIdx.x] = row_prefix(v);
    out[64 + threadIdx.x] = row_suffix(v);
    out[128 + threadIdx.x] = row_sum(v);
    out[192 + threadIdx.x] = row_bcast0(v);
}

// MFMA chain with pi-ordered k: X = A . Bm^T (32 x 16, two tiles) kept in
// registers, then D = E . X (B operand from the accumulators) and
// Dt = X^T . E^T (A operand from the accumulators), E read with ld_frag_pi.
template <typename T>
__global__ __launch_bounds__(64) void k_probe_chain(const T *A, const T *Bm, const T *E, float *Dout, float *Dtout) {
    constexpr int LD = ld_of<T>(64), LDE = ld_of<T>(32);
    __shared__ __align__(16) T sA[32 * LD], sB[16 * LD], sE[16 * LDE];
    for (int idx = threadIdx.x; idx < 32 * 64; idx += 64) sA[(idx / 64) * LD + idx % 64] = A[idx];
    for (int idx = threadIdx.x; idx < 16 * 64; idx += 64) sB[(idx / 64) * LD + idx % 64] = Bm[idx];
    for (int idx = threadIdx.x; idx < 16 * 32; idx += 64) sE[(idx / 32) * LDE + idx % 32] = E[idx];
    __syncthreads();
    f32x4 x0 = zero4(), x1 = zero4();
    tile_mma(x0, sA, LD, sB, LD, 2);
    tile_mma(x1, sA + 16 * LD, LD, sB, LD, 2);
    const Frag<T> xf = frag_acc<T>(x0, x1);
    const int i = lane_id() & 15, g = lane_id() >> 4;
    const Frag<T> ef = ld_frag_pi(sE + i * LDE);
    f32x4 d = zero4(), dt = zero4();
    mma(d, ef, xf);
    mma(dt, xf, ef);
    for (int e = 0; e < 4; ++e) {
        Dout[(4 * g + e) * 16 + i] = d[e];
        Dtout[(4 * g + e) * 16 + i] = dt[e];
    }
}

extern "C" int probe_rows(const float *x, float *out) {
    k_probe_rows<<<1, 64>>>(x, out);
    return hipDeviceSynchronize() == hipSuccess ? 0 : -1;
}

extern "C" int probe_chain(int bf16, const void *A, const void *Bm, const void *E, float *D, float *Dt) {
    if (bf16)
        k_probe_chain<race::bf16><<<1, 64>>>((const race::bf16 *)A, (const race::bf16 *)Bm, (const race::bf16 *)E, D, Dt);
    else
        k_probe_chain<float><<<1, 64>>>((const float *)A, (const float *)Bm, (const float *)E, D, Dt);
    return hipDeviceSynchronize() == hipSuccess ? 0 : -1;
}

// 16-deep chained product: X = A . Bm^T (16 x 16, one tile) kept in registers,
// D = E . X with X as the B operand (k = row of X) and E read with ld_frag16.
template <typename T>
__global__ __launch_bounds__(64) void k_probe_chain16(const T *A, const T *Bm, const T *E, float *Dout, float *Dtout) {
    constexpr int LD = ld_of<T>(64), LDE = ld_of<T>(16);
    __shared__ __align__(16) T sA[16 * LD], sB[16 * LD], sE[16 * LDE];
    for (int idx = threadIdx.x; idx < 16 * 64; idx += 64) {
        sA[(idx / 64) * LD + idx % 64] = A[idx];
        sB[(idx / 64) * LD + idx % 64] = Bm[idx];
    }
    for (int idx = threadIdx.x; idx < 16 * 16; idx += 64) sE[(idx / 16) * LDE + idx % 16] = E[idx];
    __syncthreads();
    f32x4 x = zero4();
    tile_mma(x, sA, LD, sB, LD, 2);
    const Frag4<T> xf = frag16_acc<T>(x);
    const int i = lane_id() & 15, g = lane_id() >> 4;
    const Frag4<T> ef = ld_frag16(sE + i * LDE);
    f32x4 d = zero4(), dt = zero4();
    mma16(d, ef, xf);
    mma16(dt, xf, ef);
    for (int e = 0; e < 4; ++e) {
        Dout[(4 * g + e) * 16 + i] = d[e];
        Dtout[(4 * g + e) * 16 + i] = dt[e];
    }
}

extern "C" int probe_chain16(int bf16, const void *A, const void *Bm, const void *E, float *D, float *Dt) {
    if (bf16)
        k_probe_chain16<race::bf16><<<1, 64>>>((const race::bf16 *)A, (const race::bf16 *)Bm, (const race::bf16 *)E, D, Dt);
    else
        k_probe_chain16<float><<<1, 64>>>((const float *)A, (const float *)Bm, (const float *)E, D, Dt);
    return hipDeviceSynchronize() == hipSuccess ? 0 : -1;
}

// cross-row sums with the gfx950 permlane swaps: out[0:64] = x + x[l^16],
// out[64:128] = x + x[l^32]
__global__ __launch_bounds__(64) void k_probe_xor(const float *x, float *out) {
    const float v = x[threadIdx.x];
    out[threadIdx.x] = xor16_sum(v);
    out[64 + threadIdx.x] = xor32_sum(v);
}

extern "C" int probe_xor(const float *x, float *out) {
    k_probe_xor<<<1, 64>>>(x, out);
    return hipDeviceSynchronize() == hipSuccess ? 0 : -1;
}
