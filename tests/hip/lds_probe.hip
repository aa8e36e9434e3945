// LDS bank-conflict probe: 16 waves issue one LDS access shape with per-lane
// byte offsets (< 8192 - 40), 8 independent accesses per iteration whose bases
// are 8 KiB apart (the same bank pattern); returns clock cycles of the loop.
// Every address stays inside the 64 KiB shared array.
#include <hip/hip_runtime.h>

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef short v4s __attribute__((ext_vector_type(4)));

template <int OP>
__global__ __launch_bounds__(1024) void lds_probe_kernel(const int *offs, int iters, long long *cyc, unsigned *sink) {
    __shared__ __align__(16) unsigned char lds[65536];
    const int lane = threadIdx.x & 63;
    for (int k = threadIdx.x; k < 16384; k += 1024) ((unsigned *)lds)[k] = k;
    __syncthreads();
    const int off0 = offs[lane];
    unsigned acc = 0;
    const long long t0 = clock64();
    for (int it = 0; it < iters; ++it) {
        int off = off0;
        asm volatile("" : "+v"(off));
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            unsigned char *p = lds + off + 8192 * r;
            if constexpr (OP == 0) acc ^= *(unsigned *)p;
            if constexpr (OP == 1) { u32x2 v = *(u32x2 *)p; acc ^= v.x ^ v.y; }
            if constexpr (OP == 2) { u32x4 v = *(u32x4 *)p; acc ^= v.x ^ v.y ^ v.z ^ v.w; }
            if constexpr (OP == 3) *(unsigned *)p = acc + r;
            if constexpr (OP == 4) *(u32x2 *)p = u32x2{acc + r, acc};
            if constexpr (OP == 5) *(u32x4 *)p = u32x4{acc + r, acc, acc, acc};
            if constexpr (OP == 6) {  // pi-order operand: 8 bytes at p and at p + 32
                const u32x2 a = *(u32x2 *)p, b = *(u32x2 *)(p + 32);
                acc ^= a.x ^ a.y ^ b.x ^ b.y;
            }
            if constexpr (OP == 7) {  // transpose load of 16-bit elements: 8 bytes at p
                const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s *)p);
                acc ^= (unsigned)(unsigned short)v.x ^ ((unsigned)(unsigned short)v.w << 16);
            }
        }
        asm volatile("" ::: "memory");
    }
    __builtin_amdgcn_s_waitcnt(0);
    const long long t1 = clock64();
    if (threadIdx.x == 0) cyc[blockIdx.x] = t1 - t0;
    sink[blockIdx.x * 1024 + threadIdx.x] = acc + lds[threadIdx.x];
}

// op: 0 r32, 1 r64, 2 r128, 3 w32, 4 w64, 5 w128, 6 pi-order pair read, 7 ds_read_tr16_b64
extern "C" int lds_probe(int op, const int *offs_dev, int iters, long long *cyc_dev, unsigned *sink_dev) {
    switch (op) {
    case 0: lds_probe_kernel<0><<<1, 1024>>>(offs_dev, iters, cyc_dev, sink_dev); break;
    case 1: lds_probe_kernel<1><<<1, 1024>>>(offs_dev, iters, cyc_dev, sink_dev); break;
    case 2: lds_probe_kernel<2><<<1, 1024>>>(offs_dev, iters, cyc_dev, sink_dev); break;
    case 3: lds_probe_kernel<3><<<1, 1024>>>(offs_dev, iters, cyc_dev, sink_dev); break;
    case 4: lds_probe_kernel<4><<<1, 1024>>>(offs_dev, iters, cyc_dev, sink_dev); break;
    case 5: lds_probe_kernel<5><<<1, 1024>>>(offs_dev, iters, cyc_dev, sink_dev); break;
    case 6: lds_probe_kernel<6><<<1, 1024>>>(offs_dev, iters, cyc_dev, sink_dev); break;
    case 7: lds_probe_kernel<7><<<1, 1024>>>(offs_dev, iters, cyc_dev, sink_dev); break;
    default: return -1;
    }
    return hipDeviceSynchronize() == hipSuccess ? 0 : -2;
}
