// Test helper: fills every CU's LDS with one 32-bit pattern, so that a kernel
// that reads LDS it has not written sees that pattern (all-ones bytes: NaN as
// fp32 and as bf16) instead of whatever finite values an earlier kernel left.
// Each workgroup holds 160 KiB, one workgroup per CU at a time; the caller
// launches several per CU.
#include <hip/hip_runtime.h>

__global__ __launch_bounds__(1024) void lds_fill_kernel(unsigned pattern, unsigned *sink) {
    __shared__ unsigned lds[40960];
    for (int k = threadIdx.x; k < 40960; k += 1024) lds[k] = pattern;
    asm volatile("" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = lds[(blockIdx.x * 977) % 40960];
}

// sink: at least `blocks` unsigned words of device memory
extern "C" int lds_fill(unsigned pattern, int blocks, unsigned *sink, void *stream) {
    if (blocks < 1) return -1;
    lds_fill_kernel<<<blocks, 1024, 0, (hipStream_t)stream>>>(pattern, sink);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}
