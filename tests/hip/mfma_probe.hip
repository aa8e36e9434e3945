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
