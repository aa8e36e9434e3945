// race_device.h -- device building blocks for the gfx950 RACE kernels.
//
// Matrix products use the CDNA4 16x16 MFMA tiles with 64-wide waves:
//   bf16: v_mfma_f32_16x16x32_bf16 (one instruction per 32-deep k step)
//   fp32: v_mfma_f32_16x16x4_f32   (eight instructions per 32-deep k step)
// Operand fragments: lane l = 16*g + i (g = l/16, i = l%16) holds row i of
// the 16-row A tile (or column i of the B tile) and the 8 consecutive k values
// 8g..8g+7 of the current 32-deep k step.  A and B use the same k mapping, so
// the contraction covers all 32 k values whatever order the instruction uses
// inside a step.  The fp32 accumulator of a 16x16 tile: lane l holds
// D[4g + e][i] in element e (e = 0..3).
//
// Operands are staged in LDS with k contiguous ("A as [m][k], B as [n][k]"),
// rows padded by 16 bytes so the 16 rows of a fragment fall in distinct banks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace race {

typedef __bf16 bf16;
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int D = 64;       // head dimension handled by this build
constexpr int TT = 32;      // tokens per tile
constexpr int NCOL = 32;    // projection columns (L*K <= 32)

// padded leading dimension (elements) of an LDS array with n logical columns
template <typename T> __host__ __device__ constexpr int ld_of(int n) { return n + 16 / (int)sizeof(T); }
// Leading dimension of rows that are read only as pi-order operand pairs
// (8 bytes at k = 4g and at k = 16 + 4g for bf16, ds_read2_b64) and written in
// 4- or 8-byte pieces.  ds_read_b64 serves 16 consecutive lanes per pass over
// 32 four-byte banks, so the 16 rows of one read are conflict-free when the
// row pitch is 8 (mod 16) bytes: a 4-element pad, 72-byte bf16 rows of 32.
template <typename T> __host__ __device__ constexpr int ldp_of(int n) { return n + 4; }

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
// wave index, uniform: read from the wave's first lane so that values derived
// from it (bucket ranges, task indices) live in scalar registers
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// ------------------------------------------------------------ conversions
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }

// ------------------------------------------------------------ fragments
template <typename T> struct Frag;
template <> struct Frag<bf16> { bf16x8 v; };
template <> struct Frag<float> { f32x4 lo, hi; };

__device__ __forceinline__ Frag<bf16> ld_frag(const bf16 *p) {
    Frag<bf16> f;
    f.v = *reinterpret_cast<const bf16x8 *>(p);
    return f;
}
__device__ __forceinline__ Frag<float> ld_frag(const float *p) {
    Frag<float> f;
    f.lo = *reinterpret_cast<const f32x4 *>(p);
    f.hi = *reinterpret_cast<const f32x4 *>(p + 4);
    return f;
}
// 8 k values spaced by `stride` elements (operand read across rows)
__device__ __forceinline__ Frag<bf16> ld_frag_strided(const bf16 *p, int stride) {
    Frag<bf16> f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f.v[e] = p[e * stride];
    return f;
}
__device__ __forceinline__ Frag<float> ld_frag_strided(const float *p, int stride) {
    Frag<float> f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        f.lo[e] = p[e * stride];
        f.hi[e] = p[(e + 4) * stride];
    }
    return f;
}

__device__ __forceinline__ void mma(f32x4 &c, const Frag<bf16> &a, const Frag<bf16> &b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, c, 0, 0, 0);
}
__device__ __forceinline__ void mma(f32x4 &c, const Frag<float> &a, const Frag<float> &b) {
#pragma unroll
    for (int e = 0; e < 4; ++e) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[e], b.lo[e], c, 0, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[e], b.hi[e], c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// acc += A[0:16, 0:32*ks] * B[0:16, 0:32*ks]^T, A/B pointers at the tile
// origin, stored k-contiguous with leading dimensions lda/ldb.
template <typename T>
__device__ __forceinline__ void tile_mma(f32x4 &acc, const T *A, int lda, const T *B, int ldb, int ksteps) {
    const int i = lane_id() & 15, g = lane_id() >> 4;
    const T *pa = A + i * lda + 8 * g;
    const T *pb = B + i * ldb + 8 * g;
    for (int ks = 0; ks < ksteps; ++ks) mma(acc, ld_frag(pa + 32 * ks), ld_frag(pb + 32 * ks));
}

// Same, with B read from a [k][n] (n contiguous) array: lane reads 8 k rows.
template <typename T>
__device__ __forceinline__ void tile_mma_bT(f32x4 &acc, const T *A, int lda, const T *Bkn, int ldb, int ksteps) {
    const int i = lane_id() & 15, g = lane_id() >> 4;
    const T *pa = A + i * lda + 8 * g;
    const T *pb = Bkn + (8 * g) * ldb + i;
    for (int ks = 0; ks < ksteps; ++ks)
        mma(acc, ld_frag(pa + 32 * ks), ld_frag_strided(pb + 32 * ks * ldb, ldb));
}

// store accumulator tile (origin row r0, col c0) to a [row][col] array
template <typename T>
__device__ __forceinline__ void st_tile(T *dst, int ld, const f32x4 &acc) {
    const int i = lane_id() & 15, g = lane_id() >> 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[(4 * g + e) * ld + i] = from_f32<T>(acc[e]);
}
// store accumulator tile transposed: dst[col][row]
template <typename T>
__device__ __forceinline__ void st_tile_T(T *dst, int ld, const f32x4 &acc) {
    const int i = lane_id() & 15, g = lane_id() >> 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[i * ld + 4 * g + e] = from_f32<T>(acc[e]);
}

// Operand fragment from a pair of accumulator tiles X0 (rows 0..15) and X1
// (rows 16..31) of a 32-row matrix: element j of lane (g, i) is row
// pi(g, j) = (j < 4 ? 4g + j : 16 + 4g + j - 4), column i.  Used as a B
// operand (k = row, n = i) or an A operand (m = i, k = row); the partner
// operand must be read with ld_frag_pi, which uses the same k order.
__device__ __forceinline__ Frag<bf16> frag_acc_bf16(const f32x4 &x0, const f32x4 &x1) {
    Frag<bf16> f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f.v[j] = (bf16)x0[j];
        f.v[j + 4] = (bf16)x1[j];
    }
    return f;
}
template <typename T> __device__ __forceinline__ Frag<T> frag_acc(const f32x4 &x0, const f32x4 &x1);
template <> __device__ __forceinline__ Frag<bf16> frag_acc<bf16>(const f32x4 &x0, const f32x4 &x1) {
    return frag_acc_bf16(x0, x1);
}
template <> __device__ __forceinline__ Frag<float> frag_acc<float>(const f32x4 &x0, const f32x4 &x1) {
    Frag<float> f;
    f.lo = x0;
    f.hi = x1;
    return f;
}
// 8 k values of one row in the pi order: p[4g..4g+3] then p[16+4g..16+4g+3]
__device__ __forceinline__ Frag<bf16> ld_frag_pi(const bf16 *p) {
    const int g = lane_id() >> 4;
    typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
    const bf16x4 a = *reinterpret_cast<const bf16x4 *>(p + 4 * g);
    const bf16x4 b = *reinterpret_cast<const bf16x4 *>(p + 16 + 4 * g);
    Frag<bf16> f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f.v[j] = a[j];
        f.v[j + 4] = b[j];
    }
    return f;
}
__device__ __forceinline__ Frag<float> ld_frag_pi(const float *p) {
    const int g = lane_id() >> 4;
    Frag<float> f;
    f.lo = *reinterpret_cast<const f32x4 *>(p + 4 * g);
    f.hi = *reinterpret_cast<const f32x4 *>(p + 16 + 4 * g);
    return f;
}

// 16-deep k step: lane (g, i) holds k = 4g..4g+3 of row/column i, so one
// accumulator tile (lane holds X[4g + e][i]) is directly such an operand over
// its 16 rows.  bf16 runs it as a 16x16x32 product whose k slots 4..7 of each
// lane are zero (the same instruction as every other bf16 product, so partial
// sums of both depths chain in one accumulator); fp32 runs four 16x16x4 steps.
template <typename T> struct Frag4;
template <> struct Frag4<bf16> { bf16x8 v; };
template <> struct Frag4<float> { f32x4 v; };

template <typename T> __device__ __forceinline__ Frag4<T> frag16_acc(const f32x4 &x);
template <> __device__ __forceinline__ Frag4<bf16> frag16_acc<bf16>(const f32x4 &x) {
    Frag4<bf16> f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f.v[j] = (bf16)x[j];
        f.v[j + 4] = (bf16)0.f;
    }
    return f;
}
template <> __device__ __forceinline__ Frag4<float> frag16_acc<float>(const f32x4 &x) {
    Frag4<float> f;
    f.v = x;
    return f;
}
// p[4g..4g+3]
__device__ __forceinline__ Frag4<bf16> ld_frag16(const bf16 *p) {
    typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
    const bf16x4 a = *reinterpret_cast<const bf16x4 *>(p + 4 * (lane_id() >> 4));
    Frag4<bf16> f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f.v[j] = a[j];
        f.v[j + 4] = (bf16)0.f;
    }
    return f;
}
__device__ __forceinline__ Frag4<float> ld_frag16(const float *p) {
    Frag4<float> f;
    f.v = *reinterpret_cast<const f32x4 *>(p + 4 * (lane_id() >> 4));
    return f;
}
// v_mfma_f32_16x16x16_bf16 is not used: the compiler may issue it and a
// following 16x16x32 product that reads its accumulator as SrcC back to back
// with no wait states, and on gfx950 the second product then reads a stale
// accumulator.
__device__ __forceinline__ void mma16(f32x4 &c, const Frag4<bf16> &a, const Frag4<bf16> &b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, c, 0, 0, 0);
}
__device__ __forceinline__ void mma16(f32x4 &c, const Frag4<float> &a, const Frag4<float> &b) {
#pragma unroll
    for (int e = 0; e < 4; ++e) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v[e], b.v[e], c, 0, 0, 0);
}

// -f (sign bits of the 8 bf16 values flipped): a product C + A (-B) subtracts
__device__ __forceinline__ Frag<bf16> neg_frag(const Frag<bf16> &f) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 u = __builtin_bit_cast(u32x4, f.v);
    u ^= 0x80008000u;
    Frag<bf16> r;
    r.v = __builtin_bit_cast(bf16x8, u);
    return r;
}

// fp64 -> fp32 as its own rounding step (kept from being fused with a
// following fp32 -> bf16 conversion into a double -> bf16 one, which the
// compiler expands into a multi-instruction round-to-odd sequence)
__device__ __forceinline__ float narrow(double x) {
    float f = (float)x;
    asm volatile("" : "+v"(f));
    return f;
}

// ------------------------------------------------------------ cross-row sums
// x + x[lane ^ 16] and x + x[lane ^ 32] with the gfx950 row/half swaps
__device__ __forceinline__ float xor16_sum(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ------------------------------------------------------------ row (16-lane) ops
// DPP moves inside each 16-lane row; lanes whose source is outside the row read 0.
template <int CTRL> __device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}
// inclusive prefix over the lanes of a row (row_shr 1,2,4,8)
__device__ __forceinline__ float row_prefix(float x) {
    x += dpp_f<0x111>(x);
    x += dpp_f<0x112>(x);
    x += dpp_f<0x114>(x);
    x += dpp_f<0x118>(x);
    return x;
}
// inclusive suffix over the lanes of a row (row_shl 1,2,4,8)
__device__ __forceinline__ float row_suffix(float x) {
    x += dpp_f<0x101>(x);
    x += dpp_f<0x102>(x);
    x += dpp_f<0x104>(x);
    x += dpp_f<0x108>(x);
    return x;
}
// lane 0 of each row in every lane of that row (row_newbcast:0, gfx90a and later)
__device__ __forceinline__ float row_bcast0(float x) { return dpp_f<0x150>(x); }
// total of a row in every lane of it (quad swaps, half-row mirror, row mirror)
__device__ __forceinline__ float row_sum(float x) {
    x += dpp_f<0xB1>(x);  // quad_perm [1,0,3,2]
    x += dpp_f<0x4E>(x);  // quad_perm [2,3,0,1]
    x += dpp_f<0x141>(x); // row_half_mirror
    x += dpp_f<0x140>(x); // row_mirror
    return x;
}

// row_sum of an fp64 value (both 32-bit halves move with the same pattern)
template <int CTRL> __device__ __forceinline__ double dpp_d(double x) {
    const long long b = __double_as_longlong(x);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(b & 0xffffffffll), CTRL, 0xF, 0xF, true);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), CTRL, 0xF, 0xF, true);
    return __longlong_as_double(((long long)hi << 32) | (long long)(unsigned)lo);
}
__device__ __forceinline__ double row_sum_f64(double x) {
    x += dpp_d<0xB1>(x);
    x += dpp_d<0x4E>(x);
    x += dpp_d<0x141>(x);
    x += dpp_d<0x140>(x);
    return x;
}

// ------------------------------------------------------------ sigmoids
__device__ __forceinline__ float rcp_f(float x) { return __builtin_amdgcn_rcpf(x); }
// (sigmoid(y), sigmoid(-y)) from z = -y log2(e): e = 2^z, sigmoid(y) = 1/(1+e),
// sigmoid(-y) = e/(1+e).  z is capped at 64, so e, 1+e and the reciprocal stay
// normal: for y < -44.36 sigmoid(y) reads 1/(1 + 2^64) instead of something
// smaller (absolute error < 6e-20) and sigmoid(-y) reads 1.  No branch or
// select on the sign of y.
__device__ __forceinline__ void sigmoid_pair_l2(float z, float &sp, float &sm) {
    const float e = __builtin_amdgcn_exp2f(fminf(z, 64.f));
    sp = rcp_f(1.0f + e);
    sm = e * sp;
}
// tanh(x) = 1 - 2 / (1 + e^{2x}): e^{2x} overflowing to +inf gives 1 and
// underflowing to 0 gives -1; absolute error ~1e-7
__device__ __forceinline__ float tanh_fast(float x) {
    const float e = __builtin_amdgcn_exp2f(x * 2.8853900817779268f);  // 2 log2(e)
    return fmaf(-2.f, rcp_f(1.f + e), 1.f);
}

} // namespace race
