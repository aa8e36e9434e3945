// race_kernels.hip -- gfx950 kernels of the RACE attention operator.
//
// Work decomposition.  A stream n = (m, b, h) is a sequence of T tokens cut
// into 32-token tiles; consecutive tiles form segments and one workgroup walks
// one (segment, stream) pair.  Across tiles the per-bucket state (A_s, B_s) =
// (sum P_K, sum P_K v) is carried in MFMA accumulators; across segments by a
// three-phase scan:
//   forward   k_fwd_reduce  per-segment sums of (A, B)       reads K, V
//             k_fwd_scan    exclusive segment prefixes (fp64, kept as state)
//             k_fwd_out     outputs                         reads Q, K, V, writes O
//   backward  k_bwd_reduce  forward walk: dQ and per-segment sums of
//                           alpha = sum dA, U = sum W^T g    reads Q, K, V, dO
//             k_bwd_scan    exclusive segment suffixes
//             k_bwd_out     reverse walk: dK, dV            reads Q, K, V, dO
// The reverse walk needs the forward state at every tile start: it subtracts
// each tile's (A, B) sums from the segment's end state -- A in fp64, B in
// fp64 (recomputed with exactly the code of k_fwd_reduce: bit-identical tile
// sums), except in the whole-tile bf16 instantiations, which keep B in fp32
// MFMA accumulators (see walk_f64).  The non-causal operator runs the same
// kernels with full-sequence sums and no triangles.
//
// Inside a workgroup wave w owns buckets [16w, 16w+16): the workgroup has
// SP/16 waves.  Per-bucket elementwise work (probabilities, W = P_Q/(A+eps),
// dA, the softmax backward) runs in the "bucket-row" accumulator layout: lane
// (g,i) holds bucket s = 16w + 4g + e and token t = 16nt + i.  Contractions
// over the wave's 16 buckets take such tiles directly as 16-deep MFMA
// operands.  Contractions over tokens need the token index in k: each tile is
// transposed on the matrix core (identity product) and a tile pair forms a
// 32-deep operand (frag_acc, pi order); token prefix sums and totals are the
// same operand against constant triangular / all-ones operands.  Sums over
// ALL buckets (the outputs O and dV) are computed as output tiles, one per
// wave, from [.][s] LDS arrays to which every wave writes its buckets' W,
// P_K and carry rows; the v.g triangle of the tile is built once per
// workgroup.  Within a tile the causal triangle is a masked 32x32 product:
// O = W B_start + tril(W P_K^T) V.
//
// Bucket probabilities are recomputed in every kernel: projection on MFMA,
// tanh, then P[t, l, r] = prod_k sigmoid(+-2 u_k), which equals the
// reference's softmax over the 2^K corner logits.
#include <type_traits>

#include "race_device.h"
#include "race_layout.h"

namespace race {

struct Strides {
    int64_t m, b, t, h;
};

struct Args {
    const void *q, *k, *v, *dout;
    void *out, *dq, *dk, *dv;
    Strides sq, sk, sv, sdo, so, sg;
    const float *planes;
    int64_t planes_m_stride;
    int M, B, H, L, K, R, S;
    int64_t T;
    float eps, inv_temp;
    const float *inv_temp_ptr;  // nullable device scalar replacing inv_temp (read at kernel start)
    int nseg, tps;   // segments per stream, tiles per segment
    // forward segments (fstate rows per stream - 1) and forward segments per
    // segment: the backward's segment s starts at forward boundary s * fmul
    int fnseg, fmul;
    int nslice, Spad;  // bucket slices (grid z) of SP buckets each; Spad = nslice * SP
    double *fstate;  // [N][fnseg+1][Spad][D+1] exclusive forward-segment prefixes; [fnseg] = totals
    double *fdelta;  // [N][nseg][Spad][D+1]
    float *rdelta;   // [N][nseg][Spad][D+1]  per-segment (U, alpha) sums
    float *rstate;   // [N][nseg][Spad][D+1]  exclusive suffixes (non-causal: totals)
    double *tpart;   // [2][N][nseg][nslice] partial sums of dU*th
    // sliced() instantiations: per-slice partial outputs [nslice][N][T][D] in the element type (bf16 or
    // fp32), summed in fp32 by k_slice_sum
    void *opart, *dvpart;
    // sliced dX outputs (dQ, dK; the probability backward's dx): each slice's
    // dproj columns, [nslice][N][T][xcols] in the element type (fp32 where
    // xpart_f32), multiplied by planes^T and summed over slices by k_dx_finish
    void *dqpart, *dkpart;
    // global normalisation (GN instantiations; eps is the floor of den):
    // den [N][T] output (sliced: per-slice partials denpart [nslice][N][T]);
    // backward: den and dden (dL/d den, nullable) in, and per-token
    // rden = 1/max(den, eps), gden = dL/d den + d(out)/d den terms [N][T],
    // written by k_bwd_reduce and read by k_bwd_out
    float *den, *denpart;
    const float *dden;
    float *rden, *gden;
    // bucket slices: each slice's share of sum_s P_Q G per token [nslice][N][T]
    // (the k_bwd_reduce pre-pass), summed by k_gn_terms into rden / gden
    float *gsum;
    // per-token key weights [B][T] on P_K (non-causal padding mask; nullable).
    // Non-causal F1 also writes den [N][T] when den is set and reads dden.
    const float *kw;
    // bucket probabilities as an output: probs [N][T][S] fp32 (k_probs) and
    // their upstream gradient dprobs (k_probs_bwd; x in q, dx in dq)
    float *probs;
    const float *dprobs;
};

constexpr int SROW = D + 1;  // state row: D values of B (or U) then A (or alpha)
constexpr int WB = 16;       // buckets per wave
__host__ __device__ constexpr int threads_of(int SP) { return 64 * (SP / WB); }

// Instantiations that may run several bucket slices (fp32, and bf16 with more
// than 4 hash bits) write partial outputs in the element type, summed in fp32
// by k_slice_sum; the others write the outputs directly and run one slice.
template <typename T, int KB> __host__ __device__ constexpr bool sliced() {
    return !std::is_same<T, bf16>::value || KB > 4;
}

// Row width (elements, a power of 2) of the sliced dX partials: the
// projection columns one slice's tables span -- SP / 2^KB tables of KB
// columns, or KB columns of a table wider than the slice -- rounded up.
__host__ __device__ constexpr int xcols_of(int SP, int KB) {
    const int c = (1 << KB) <= SP ? (SP >> KB) * KB : KB;
    const int m = c < NCOL ? c : NCOL;
    return m <= 8 ? 8 : (m <= 16 ? 16 : 32);
}

// bf16 tables wider than a slice (8-bit hashes in 128-bucket slices: two
// slices per table) split each (token, bit)'s du between two slices, whose
// partial sums can cancel.  Those slices keep their d(projection) partials in
// fp32 (8 columns, 32 bytes a token) and k_dx_finish8 adds a table's two
// slices before any rounding.
__host__ __device__ constexpr bool xpart_f32(bool bf, int SP, int KB) { return bf && (1 << KB) > SP; }

__device__ __forceinline__ int64_t stream_off(const Strides &s, int n, int B, int H) {
    const int h = n % H, b = (n / H) % B, m = n / (H * B);
    return (int64_t)m * s.m + (int64_t)b * s.b + (int64_t)h * s.h;
}

// Workgroup coordinates (segment, stream, bucket slice).  Unsliced launches
// are (nseg, N).  The bucket slices of one (segment, stream) read the same
// token tiles, so sliced launches are 1-D with a group's slices 8 workgroups
// apart: gfx950 hands workgroups to its 8 XCDs round-robin, so the slices of
// a group share one XCD's L2 and start together.  Groups past nseg * N (the
// blocks of 8 groups are whole) exit at once.
struct WgPos {
    int seg, n, z;
    bool live;
};
__device__ __forceinline__ WgPos wg_pos(int nseg, int N, int nslice, bool sl) {
    if (!sl) return WgPos{(int)blockIdx.x, (int)blockIdx.y, 0, true};
    const int L = (int)blockIdx.x, per = 8 * nslice, r = L % per;
    const int grp = (L / per) * 8 + (r & 7);
    return WgPos{grp % nseg, grp / nseg, r >> 3, (int64_t)grp < (int64_t)nseg * N};
}

__host__ __device__ constexpr size_t align16(size_t x) { return (x + 15) & ~(size_t)15; }
__host__ __device__ constexpr size_t cmax(size_t a, size_t b) { return a > b ? a : b; }

template <typename T> constexpr bool is_bf16() { return sizeof(T) == 2; }

// (slice z, stream n)'s [T][xcols] block of a sliced dX partial buffer
template <typename T, int SP, int KB> __device__ __forceinline__ void *xpart_at(void *base, int z, int64_t n, const Args &a) {
    const int64_t off = ((int64_t)z * a.M * a.B * a.H + n) * a.T * xcols_of(SP, KB);
    if constexpr (xpart_f32(is_bf16<T>(), SP, KB))
        return (float *)base + off;
    else
        return (T *)base + off;
}

// Register type of A (the per-bucket sum of P_K) walked forward through a
// segment from its fp64 start value, one fp32 tile total at a time: fp32 for
// bf16 inputs, fp64 for fp32 inputs.  Each addition of a positive total
// rounds once, so n tiles bound the relative error by n 2^-24 (1.5e-5 for
// the host's longest segment, 256 tiles, at any T; the rounding errors of a
// sum of positive terms grow as sqrt(n) in practice), below the 2^-9 of the
// bf16 operands that the quotients P/(A + eps) feed.  The reverse walk of
// k_bwd_out subtracts from a segment-end value and stays fp64 for both.
template <typename T> using CarryA = std::conditional_t<is_bf16<T>(), float, double>;

__device__ __forceinline__ int lg() { return (threadIdx.x & 63) >> 4; }
__device__ __forceinline__ int li() { return threadIdx.x & 15; }

// value as the MFMA will see it (bf16 rounding for the bf16 path)
template <typename T> __device__ __forceinline__ float as_operand(float x) { return to_f32(from_f32<T>(x)); }

__device__ __forceinline__ float rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// 4 consecutive elements (one lane's accumulator column) to global memory
template <typename T> __device__ __forceinline__ void store4(T *p, const f32x4 &v);
// 4 consecutive elements (8- or 16-byte aligned) as fp32
template <typename T> __device__ __forceinline__ f32x4 load4(const T *p);
template <> __device__ __forceinline__ f32x4 load4<float>(const float *p) { return *reinterpret_cast<const f32x4 *>(p); }
template <> __device__ __forceinline__ f32x4 load4<bf16>(const bf16 *p) {
    const uint2 u = *reinterpret_cast<const uint2 *>(p);
    return f32x4{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xFFFF0000u), __uint_as_float(u.y << 16),
                 __uint_as_float(u.y & 0xFFFF0000u)};
}
template <> __device__ __forceinline__ void store4<float>(float *p, const f32x4 &v) {
    *reinterpret_cast<f32x4 *>(p) = v;
}
template <> __device__ __forceinline__ void store4<bf16>(bf16 *p, const f32x4 &v) {
    typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
    bf16x4 o;
    for (int e = 0; e < 4; ++e) o[e] = (bf16)v[e];
    *reinterpret_cast<bf16x4 *>(p) = o;
}

// Wait for every load issued so far.  Placed after a kernel's state loads
// and before its first prefetch: otherwise the compiler keeps waits for the
// state registers inside the tile loop, where they would also wait for the
// prefetch of the next tile.
__device__ __forceinline__ void wait_state_loads() { __builtin_amdgcn_s_waitcnt(0); }
// Wait for vector memory operations only (s_waitcnt vmcnt(0); expcnt and
// lgkmcnt at their maxima).  Placed unconditionally ahead of a commit whose
// LDS stores sit under lane conditions, it retires the prefetch loads on every
// path, so no wait is needed before the registers are reused for the next
// tile's loads -- a wait there would also wait for the stores just issued.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// --------------------------------------------------------------- tile I/O
// Register-staged tile load: issue() starts the global loads of one tile
// into registers, commit() writes them to LDS (natural and/or transposed), so
// the next tile's loads overlap the current tile's compute.
// Token-tile global access: a uniform tile base and a 32-bit per-lane byte
// offset (the host bounds the token stride below 2^26 elements).
template <typename V, typename T> __device__ __forceinline__ V ld_at(const T *base, uint32_t off_bytes) {
    return *reinterpret_cast<const V *>(reinterpret_cast<const char *>(base) + off_bytes);
}
template <typename T> __device__ __forceinline__ T *at_bytes(T *base, uint32_t off_bytes) {
    return reinterpret_cast<T *>(reinterpret_cast<char *>(base) + off_bytes);
}
// The output tiles of k_fwd_out are written with buffer stores (measured
// faster there): a resource over the valid bytes from the tile's first row
// (word 3 = 0x00020000, the gfx9 raw-buffer format); every store is still
// guarded by t0 + t < T, the record count is only a second bound.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <typename T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const T *base, int64_t st, int64_t rows) {
    int64_t bytes = rows > 0 ? ((rows - 1) * st + D) * (int64_t)sizeof(T) : 0;
    if (bytes > 0x7FFFFFFFll) bytes = 0x7FFFFFFFll;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<T *>(base), 0, (int)bytes, 0x00020000);
}
// 4 consecutive elements (one accumulator column) at byte offset off
template <typename T> __device__ __forceinline__ void buf_st4(__amdgpu_buffer_rsrc_t r, uint32_t off, const f32x4 &v);
template <> __device__ __forceinline__ void buf_st4<float>(__amdgpu_buffer_rsrc_t r, uint32_t off, const f32x4 &v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, (int)off, 0, 0);
}
template <> __device__ __forceinline__ void buf_st4<bf16>(__amdgpu_buffer_rsrc_t r, uint32_t off, const f32x4 &v) {
    typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
    bf16x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (bf16)v[e];
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, o), r, (int)off, 0, 0);
}
// Base of the token tile that starts at t0 (a multiple of TT) of a tensor with
// token stride st.  The host bounds TT * st * sizeof(T) below 2^32 and T by
// 2^35, so the offset is one 32 x 32-bit product of the tile index and the
// tile's byte stride: two scalar multiplies per tile where a 64-bit
// t0 * st * sizeof(T) takes a dozen scalar instructions.
template <typename T> __device__ __forceinline__ T *tile_ptr(T *src, int64_t st, int64_t t0) {
    const uint32_t tb = (uint32_t)st * (uint32_t)(TT * sizeof(T));
    const uint64_t off = (uint64_t)(uint32_t)((uint64_t)t0 / TT) * tb;
    using C = std::conditional_t<std::is_const<T>::value, const char, char>;  // pointer arithmetic keeps the global loads
    return reinterpret_cast<T *>(reinterpret_cast<C *>(src) + off);
}
// byte offset of element (t, d) of a token tile
__device__ __forceinline__ uint32_t tile_off(int t, int64_t st, int d, int esize) {
    return ((uint32_t)t * (uint32_t)st + (uint32_t)d) * (uint32_t)esize;
}

// Element (t, d) of the tile at t0 of a [T][D] partial block (bucket
// slices): a uniform tile base and a 32-bit lane offset that stays the same
// on every tile.
template <typename P> __device__ __forceinline__ P *part_at(P *part, int64_t t0, int t, int d) {
    return at_bytes(part + t0 * D, (uint32_t)(t * D + d) * (uint32_t)sizeof(P));
}

template <int B> struct ChunkOf;
template <> struct ChunkOf<16> { typedef uint4 type; };
template <> struct ChunkOf<8> { typedef uint2 type; };

// ---- swizzled LDS rows (bf16; race_layout.h): arrays read as 16-byte
// operand pieces of 16 rows and written in 8-byte pieces.  fp32 keeps padded
// rows.  The swizzle stays inside each 32-element chunk, so a lane's k slots
// hold the same logical k in every row: products of two such operands pair
// equal k.
// row pitch (elements) of such an array
template <typename T, int N> __host__ __device__ constexpr int sw_ld() {
    return is_bf16<T>() ? layout::sw_pitch(N) : ld_of<T>(N);
}
// element offset of logical element e of row r of a [rows][N] array
template <typename T, int N> __device__ __forceinline__ int sw_off(int r, int e) {
    if constexpr (is_bf16<T>())
        return layout::sw_elem(N, r, e);
    else
        return r * sw_ld<T, N>() + e;
}
// gswz depends on r & 15 only, so rows 16 apart share it: a lane keeps one
// pointer for rows r, r + 16, ... (steps of 16 * sw_ld).
// Operand pointer of lane (g, i) into row r for 16-byte reads of logical
// elements 32 kp + 8g .. + 7 at ld_frag(p + 32 * kp).
template <typename T, int N> __device__ __forceinline__ const T *sw_frag_ptr(const T *base, int r) {
    return base + sw_off<T, N>(r, 8 * lg());
}

// ---- natural token tiles and planes ([rows][D], k = d).  With SW (bf16), k
// is stored in pi order inside each 32-element chunk (k = 16h + 4g + j at
// 8g + 4h + j) in the swizzled rows above, so a pi-order operand (k = 4g..,
// 16 + 4g..) is one contiguous 16-byte read like the operand of a [rows][k]
// product, and every operand read of 16 rows is conflict-free.  Runs of 4
// k aligned to 4 stay contiguous.  Without SW: padded natural rows.
template <typename T, bool SW> struct NatL {
    static constexpr bool P = SW && is_bf16<T>();
    static constexpr int LD = P ? sw_ld<T, D>() : ld_of<T>(D);
    __device__ __forceinline__ static int pos(int k) { return layout::pi_pos(k); }
    // element offset of logical (r, k)
    __device__ __forceinline__ static int off(int r, int k) {
        if constexpr (P)
            return sw_off<T, D>(r, pos(k));
        else
            return r * LD + k;
    }
    // operand of a [rows][k] product: row r, k chunk kp (both operands of
    // such a product read with this, so their k slots agree)
    __device__ __forceinline__ static Frag<T> frag(const T *base, int r, int kp) {
        if constexpr (P)
            return ld_frag(sw_frag_ptr<T, D>(base, r) + 32 * kp);
        else
            return ld_frag(base + r * LD + 8 * lg() + 32 * kp);
    }
    // pi-order operand of row r over k = 32h .. 32h + 31
    __device__ __forceinline__ static Frag<T> frag_pi(const T *base, int r, int h) {
        if constexpr (P)
            return ld_frag(sw_frag_ptr<T, D>(base, r) + 32 * h);
        else
            return ld_frag_pi(base + r * LD + 32 * h);
    }
};
// Plain token rows for tiles read only by LDS transpose loads (col_operand,
// bf16): row r at r * LD, k in natural order.  LD = D + 16 puts the rows of a
// 4-row group 8 dwords apart modulo the 32 banks of 8-byte accesses, so the 4
// rows x 4 runs of 8 bytes that one 16-lane pass of a transpose load reads
// fall on 32 distinct banks (the swizzled pi-order rows put them on 16).
template <typename T> struct TrL {
    static constexpr bool P = false;
    static constexpr int LD = D + 16;
    __device__ __forceinline__ static int off(int r, int k) { return r * LD + k; }
};

// acc += A[rA .. rA+15][:] * B[rB .. rB+15][:]^T over all D of two natural arrays
template <class NL, typename T>
__device__ __forceinline__ void nat_mma(f32x4 &acc, const T *A, int rA, const T *B, int rB) {
#pragma unroll
    for (int kp = 0; kp < D / 32; ++kp) mma(acc, NL::frag(A, rA + li(), kp), NL::frag(B, rB + li(), kp));
}

// Chunks of 16 bytes, or of 8 bytes when 16-byte chunks would leave some of
// the workgroup's threads without one (every wave shares the staging work).
// rows of the tile at t0 that exist (0 .. TT), as a wave-uniform 32-bit count
// (32-bit compares on the two halves of Tn - t0: the scalar unit has no
// 64-bit ordered compare, and a vector one would cost VALU work per tile)
__device__ __forceinline__ int tile_rows(int64_t t0, int64_t Tn) {
    const uint64_t r = (uint64_t)(Tn - t0);
    const int32_t hi = (int32_t)(r >> 32);
    const uint32_t lo = (uint32_t)r;
    return hi < 0 ? 0 : ((hi > 0 || lo >= (uint32_t)TT) ? TT : (int)lo);
}

// AL (whole tiles): the launch guarantees that every tile issued holds TT
// rows, so the loads need no row guards.
template <typename T, int NTH, bool AL = false> struct Prefetch {
    static constexpr int CB = (TT * D * (int)sizeof(T) / 16 >= NTH) ? 16 : 8;
    typedef typename ChunkOf<CB>::type chunk_t;
    static constexpr int EPC = CB / sizeof(T), CPR = D / EPC, CHUNKS = TT * CPR;
    static constexpr int PER = (CHUNKS + NTH - 1) / NTH;
    // whole tiles whose chunks every thread shares evenly
    static constexpr bool WHOLE = AL && CHUNKS % NTH == 0;
    chunk_t v[PER];
    // tile base src + t0 * st is uniform; the lane offset t * st + c * EPC is
    // 32-bit (the host bounds 32 * token stride below 2^31)
    __device__ __forceinline__ void issue(const T *__restrict__ src, int64_t st, int64_t t0, int64_t Tn) {
        const T *base = tile_ptr(src, st, t0);
        const int rem = AL ? TT : tile_rows(t0, Tn);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int idx = threadIdx.x + j * NTH, t = idx / CPR, c = idx % CPR;
            if constexpr (WHOLE) {  // every lane loads: no branch, counted waits stay exact
                v[j] = ld_at<chunk_t>(base, tile_off(t, st, c * EPC, sizeof(T)));
                continue;
            }
            v[j] = chunk_t{};
            if (idx < CHUNKS && t < rem) v[j] = ld_at<chunk_t>(base, tile_off(t, st, c * EPC, sizeof(T)));
        }
    }
    template <class NL = NatL<T, false>> __device__ __forceinline__ void commit(T *nat, T *trn) const {
        constexpr int LDT = ldp_of<T>(TT);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int idx = threadIdx.x + j * NTH, t = idx / CPR, c = idx % CPR;
            if (!WHOLE && idx >= CHUNKS) continue;
            if (nat) {
                if constexpr (NL::P && CB == 16) {  // two runs of 4 elements
                    *reinterpret_cast<uint2 *>(nat + NL::off(t, c * EPC)) = uint2{v[j].x, v[j].y};
                    *reinterpret_cast<uint2 *>(nat + NL::off(t, c * EPC + 4)) = uint2{v[j].z, v[j].w};
                } else {
                    *reinterpret_cast<chunk_t *>(nat + NL::off(t, c * EPC)) = v[j];
                }
            }
            if (trn) {
                const T *e = reinterpret_cast<const T *>(&v[j]);
#pragma unroll
                for (int q = 0; q < EPC; ++q) trn[(c * EPC + q) * LDT + t] = e[q];
            }
        }
    }
};

// Staging of a tile that is also needed transposed ([D][TT], t contiguous):
// each task is a pair of tokens (2tp, 2tp+1) times one 8-byte chunk of d.
// Lanes of a wave cover 16 token pairs x 4 chunks, so the transposed rows are
// written as packed token pairs to consecutive LDS words (few bank conflicts)
// while each token row is still read in 32-byte runs.  NPART tensors share
// the workgroup: this one uses threads [part*NTH/NPART, (part+1)*NTH/NPART).
// TRN = false: natural rows only (bf16 reads the token operands from them
// with LDS transpose loads, col_operand).
template <typename T, int NTH, int NPART, bool AL = false, bool TRN = true> struct PrefetchT {
    static constexpr int NT = NTH / NPART;
    static constexpr int EPC = 8 / sizeof(T), CPR = D / EPC, TASKS = (TT / 2) * CPR;
    static constexpr int PER = (TASKS + NT - 1) / NT;
    uint2 v[PER][2];
    __device__ __forceinline__ static bool task_of(int part, int j, int &tp, int &c) {
        const int local = (int)threadIdx.x - part * NT, task = local + j * NT;
        tp = (task >> 2) & 15;
        c = (task & 3) + 4 * (task >> 6);
        return local >= 0 && local < NT && task < TASKS;
    }
    __device__ __forceinline__ void issue(int part, const T *__restrict__ src, int64_t st, int64_t t0, int64_t Tn) {
        const T *base = tile_ptr(src, st, t0);
        const int rem = AL ? TT : tile_rows(t0, Tn);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            int tp, c;
            const bool ok = task_of(part, j, tp, c);
            const uint32_t off = tile_off(2 * tp, st, c * EPC, sizeof(T));
            v[j][0] = uint2{0, 0};
            v[j][1] = uint2{0, 0};
            if (ok && 2 * tp < rem) v[j][0] = ld_at<uint2>(base, off);
            if (ok && 2 * tp + 1 < rem) v[j][1] = ld_at<uint2>(base, off + (uint32_t)st * (uint32_t)sizeof(T));
        }
    }
    template <class NL = NatL<T, false>> __device__ __forceinline__ void commit(int part, T *nat, T *trn) const {
        constexpr int LDT = ldp_of<T>(TT);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            int tp, c;
            if (!task_of(part, j, tp, c)) continue;
            if (nat) {
                *reinterpret_cast<uint2 *>(nat + NL::off(2 * tp, c * EPC)) = v[j][0];
                *reinterpret_cast<uint2 *>(nat + NL::off(2 * tp + 1, c * EPC)) = v[j][1];
            }
            if constexpr (!TRN) continue;
            // element q of a chunk: bf16 -> 16-bit half q of the 64-bit chunk; fp32 -> word q
            const uint2 a = v[j][0], b = v[j][1];
            uint32_t *row = reinterpret_cast<uint32_t *>(trn + (c * EPC) * LDT + 2 * tp);
            constexpr int RW = LDT * (int)sizeof(T) / 4;  // words per transposed row
            if constexpr (sizeof(T) == 2) {
                row[0 * RW] = (a.x & 0xFFFFu) | (b.x << 16);
                row[1 * RW] = (a.x >> 16) | (b.x & 0xFFFF0000u);
                row[2 * RW] = (a.y & 0xFFFFu) | (b.y << 16);
                row[3 * RW] = (a.y >> 16) | (b.y & 0xFFFF0000u);
            } else {
                *reinterpret_cast<uint2 *>(row) = uint2{a.x, b.x};
                *reinterpret_cast<uint2 *>(row + RW) = uint2{a.y, b.y};
            }
        }
    }
};

// Two token tiles staged like PrefetchT (natural and/or transposed), the
// first by the workgroup's first half of waves and the second by the other
// half.  The tensor is chosen per wave (scalar selects of the source and
// destinations), so every lane takes part and no lane mask is needed.
// TRN: also write the transposed rows (fp32; bf16 reads its token operands
// from the natural rows with LDS transpose loads, col_operand).
template <typename T, int NTH, bool AL = false, bool TRN = true> struct PrefetchT2 {
    static constexpr int NT = NTH / 2;
    static constexpr int EPC = 8 / sizeof(T), CPR = D / EPC, TASKS = (TT / 2) * CPR;
    static_assert(NT % 64 == 0 && TASKS % NT == 0, "whole waves per tensor, whole tasks per lane");
    static constexpr int PER = TASKS / NT;
    uint2 v[PER][2];
    __device__ __forceinline__ static bool second() { return wave_id() >= NT / 64; }
    __device__ __forceinline__ static void task_of(int j, int &tp, int &c) {
        const int task = ((int)threadIdx.x & (NT - 1)) + j * NT;
        tp = (task >> 2) & 15;
        c = (task & 3) + 4 * (task >> 6);
    }
    __device__ __forceinline__ void issue(const T *__restrict__ src0, int64_t st0, const T *__restrict__ src1,
                                          int64_t st1, int64_t t0, int64_t Tn) {
        const bool sc = second();
        const int64_t st = sc ? st1 : st0;
        const T *base = tile_ptr(sc ? src1 : src0, st, t0);
        const int rem = AL ? TT : tile_rows(t0, Tn);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            int tp, c;
            task_of(j, tp, c);
            const uint32_t off = tile_off(2 * tp, st, c * EPC, sizeof(T));
            if constexpr (AL) {
                v[j][0] = ld_at<uint2>(base, off);
                v[j][1] = ld_at<uint2>(base, off + (uint32_t)st * (uint32_t)sizeof(T));
            } else {
                v[j][0] = uint2{0, 0};
                v[j][1] = uint2{0, 0};
                if (2 * tp < rem) v[j][0] = ld_at<uint2>(base, off);
                if (2 * tp + 1 < rem) v[j][1] = ld_at<uint2>(base, off + (uint32_t)st * (uint32_t)sizeof(T));
            }
        }
    }
    template <class NL = NatL<T, false>>
    __device__ __forceinline__ void commit(T *nat0, T *trn0, T *nat1, T *trn1) const {
        constexpr int LDT = ldp_of<T>(TT);
        const bool sc = second();
        T *nat = sc ? nat1 : nat0, *trn = sc ? trn1 : trn0;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            int tp, c;
            task_of(j, tp, c);
            *reinterpret_cast<uint2 *>(nat + NL::off(2 * tp, c * EPC)) = v[j][0];
            *reinterpret_cast<uint2 *>(nat + NL::off(2 * tp + 1, c * EPC)) = v[j][1];
            if constexpr (!TRN) continue;
            const uint2 a = v[j][0], b = v[j][1];
            uint32_t *row = reinterpret_cast<uint32_t *>(trn + (c * EPC) * LDT + 2 * tp);
            constexpr int RW = LDT * (int)sizeof(T) / 4;
            if constexpr (sizeof(T) == 2) {
                row[0 * RW] = (a.x & 0xFFFFu) | (b.x << 16);
                row[1 * RW] = (a.x >> 16) | (b.x & 0xFFFF0000u);
                row[2 * RW] = (a.y & 0xFFFFu) | (b.y << 16);
                row[3 * RW] = (a.y >> 16) | (b.y & 0xFFFF0000u);
            } else {
                *reinterpret_cast<uint2 *>(row) = uint2{a.x, b.x};
                *reinterpret_cast<uint2 *>(row + RW) = uint2{a.y, b.y};
            }
        }
    }
};

// Per-token fp32 pair (a[t], b[t]) of a 32-token tile (the GN backward's
// den and dden, or rden and gden), loaded by wave 0 with the token tiles and
// committed to LDS as [2][TT] with them; zero past the sequence end and for
// a null b.
struct TokPre {
    float v;
    __device__ __forceinline__ void issue(const float *__restrict__ a, const float *__restrict__ b, int64_t t0,
                                          int64_t Tn) {
        v = 0.f;
        if (threadIdx.x < 64) {
            const int t = threadIdx.x & 31;
            const float *src = threadIdx.x < 32 ? a : b;  // b may be null: zeros
            if (src && t < tile_rows(t0, Tn)) v = src[t0 + t];
        }
    }
    __device__ __forceinline__ void commit(float *dst) const {
        if (threadIdx.x < 64) dst[threadIdx.x] = v;
    }
};

// Planes [L*K][D] fp32 -> LDS.  pl/pllo: [NCOL][ld_of<T>(D)] (bf16 keeps a
// hi/lo split so the projection is close to fp32), plt: [D][ld_of<T>(NCOL)].
template <typename T, int NTH, class NL = NatL<T, false>>
__device__ void load_planes(const float *__restrict__ planes, int LK, T *pl, T *pllo, T *plt) {
    for (int idx = threadIdx.x; idx < NCOL * D; idx += NTH) {
        const int c = idx / D, d = idx % D;
        const float w = c < LK ? planes[c * D + d] : 0.f;
        const T hi = from_f32<T>(w);
        if (pl) pl[NL::off(c, d)] = hi;
        if (pllo) pllo[NL::off(c, d)] = from_f32<T>(w - to_f32(hi));
        if (plt) plt[sw_off<T, NCOL>(d, c)] = hi;
    }
}

// One 16x16 tile (rows c = 16mc.., columns t = 16nt..) of planes . X^T, then
// th = tanh and the sigmoid pair of 2*th*inv_temp, stored as sp/sm/sth
// [TT][ld_of<float>(NCOL)] (lane writes its 4 consecutive c of token t).
// The planes operands of one 16-column block (rows 16 mc.. of pl / pllo),
// held in registers by a wave whose projection task keeps that block on
// every tile.
template <typename T> struct PlaneOps {
    Frag<T> hi[D / 32], lo[D / 32];
    template <class NL> __device__ __forceinline__ void load(const T *pl, const T *pllo, int mc) {
#pragma unroll
        for (int kp = 0; kp < D / 32; ++kp) {
            hi[kp] = NL::frag(pl, 16 * mc + li(), kp);
            if constexpr (is_bf16<T>()) lo[kp] = NL::frag(pllo, 16 * mc + li(), kp);
        }
    }
};

// pc: the block's operands in registers (mc is then that block), or null.
// PAIR: instead of the corner pair of each column, write the products of
// corner pairs of the lane's 4 columns (a nibble: columns c0 .. c0+3, c0 = 4q;
// 8- and 4-bit tables are whole nibbles), the index's high bit choosing the
// first column's factor (1: sigmoid(2u)):
//   sp[c0 + j] = f(c0, j >> 1) f(c0 + 1, j & 1),  sm[c0 + j] = f(c0 + 2, j >> 1) f(c0 + 3, j & 1),
// so probs_st_ forms a bucket probability from two or four products.
template <typename T, class NL = NatL<T, false>, bool PAIR = false>
__device__ void project_tile(const T *sx, const T *pl, const T *pllo, int mc, int nt, float inv_temp, float *sp,
                             float *sm, float *sth, const PlaneOps<T> *pc = nullptr) {
    constexpr int LDC = ld_of<float>(NCOL);
    f32x4 acc = zero4();
#pragma unroll
    for (int kp = 0; kp < D / 32; ++kp) {
        const Frag<T> x = NL::frag(sx, 16 * nt + li(), kp);
        mma(acc, pc ? pc->hi[kp] : NL::frag(pl, 16 * mc + li(), kp), x);
        if constexpr (is_bf16<T>()) mma(acc, pc ? pc->lo[kp] : NL::frag(pllo, 16 * mc + li(), kp), x);
    }
    const int t = 16 * nt + li(), c0 = 16 * mc + 4 * lg();
    // the corner pair (sigmoid(2u), sigmoid(-2u)), u = th inv_temp, from
    // z = -2u log2(e) = th * zc
    const float zc = -2.8853900817779268f * inv_temp;
    f32x4 a, b, th;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        th[e] = tanh_fast(acc[e]);
        float x, y;
        sigmoid_pair_l2(th[e] * zc, x, y);
        a[e] = x;
        b[e] = y;
    }
    if constexpr (PAIR) {
        f32x4 hp, lp;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            hp[j] = ((j & 2) ? a[0] : b[0]) * ((j & 1) ? a[1] : b[1]);
            lp[j] = ((j & 2) ? a[2] : b[2]) * ((j & 1) ? a[3] : b[3]);
        }
        a = hp;
        b = lp;
    }
    *reinterpret_cast<f32x4 *>(sp + t * LDC + c0) = a;
    *reinterpret_cast<f32x4 *>(sm + t * LDC + c0) = b;
    if (sth) *reinterpret_cast<f32x4 *>(sth + t * LDC + c0) = th;
}

// Tables whose corner probabilities can be formed from nibble pair products
// (project_tile's PAIR rows): 4 and 8 bits.
template <int KB> constexpr bool pair_tables() { return KB == 4 || KB == 8; }

// tanh(u) = sigmoid(2u) - sigmoid(-2u) of column c of token row t: from the
// corner pair (sp - sm), or (PAIR) from the nibble's pair products, whose
// halves sum to one column's factor times (sigmoid(2u') + sigmoid(-2u')) = 1
// of the other column in the pair.
template <bool PAIR>
__device__ __forceinline__ float corner_tanh(const float *sp, const float *sm, int t, int c) {
    constexpr int LDC = ld_of<float>(NCOL);
    if constexpr (PAIR) {
        const int m = c & 3;
        const f32x4 h = *reinterpret_cast<const f32x4 *>((m < 2 ? sp : sm) + t * LDC + (c & ~3));
        return (m & 1) ? (h[1] + h[3]) - (h[0] + h[2]) : (h[2] + h[3]) - (h[0] + h[1]);
    } else {
        return sp[t * LDC + c] - sm[t * LDC + c];
    }
}

// Projection columns a workgroup needs: the K columns of every table its
// bucket slice [z SP, (z+1) SP) touches, as 16-column blocks pb0 .. pb0+nb-1
// (one task per block and 16-token half).  A slice of part of a table (bf16
// with K >= 5) or of a few tables (fp32) projects one block instead of all
// of them; C4's single slice of 8 tables of 4 bits needs both.
struct PlaneBlocks {
    int pb0, lg;  // first block; log2 of the tasks per projected tensor (1: one block, 2: both)
    // full: every column block (compile-time constants; the unsliced
    // instantiations, whose task loops then specialise per iteration)
    __device__ __forceinline__ PlaneBlocks(int z, int SP, int KB, int L, bool full) {
        if (full) {
            pb0 = 0;
            lg = 2;
            return;
        }
        const int l0 = (z * SP) >> KB;
        const int l1 = (min((z + 1) * SP, L << KB) - 1) >> KB;
        pb0 = __builtin_amdgcn_readfirstlane((l0 * KB) >> 4);
        lg = __builtin_amdgcn_readfirstlane(((((l1 + 1) * KB) - 1) >> 4) - pb0 + 1);  // blocks: 1 or 2
    }
    __device__ __forceinline__ int tasks() const { return 2 << (lg - 1); }  // per projected tensor
    __device__ __forceinline__ int task(int q) const { return q & (tasks() - 1); }   // task within its tensor
    __device__ __forceinline__ int tensor(int q) const { return q >> lg; }          // which tensor
    // column block of task r < tasks() (token half r & 1)
    __device__ __forceinline__ int mc(int r) const { return pb0 + (r >> 1); }
};

// Bucket probabilities of the wave's 16 buckets in bucket-row layout:
// P[nt][e] = P[t = 16nt + i][s = sw + 4g + e]; zero for s >= S or t >= nv (nv:
// the tile's rows that exist, tile_rows).
// For K >= 2 the 4 buckets of a lane share one table and differ in the two
// lowest corner bits: P = hi * (bit1 ? s+ : s-) * (bit0 ? s+ : s-).
// FULL: every token of the tile exists and every bucket of the wave is below
// S (no validity masks; the whole-tile instantiations, AL).
// PAIR: sp/sm hold project_tile's PAIR rows (4 or 8 bits).  The lane's 4
// buckets r0 .. r0+3 (r0 = 4g in a 16-bucket run) differ in the last
// nibble's two low bits: P = sp[n + (r >> 2 & 3)] sm[n + (r & 3)] over the
// table's last nibble n, times (8 bits) the first nibble's two products,
// which the wave's buckets share.
template <int KB, bool FULL, bool PAIR = false>
__device__ __forceinline__ void probs_st_(const float *sp, const float *sm, int sw, int S, int nv, f32x4 (&P)[2]) {
    constexpr int LDC = ld_of<float>(NCOL);
    constexpr int R = 1 << KB;
    const int g = lg(), i = li();
    const int s0 = sw + 4 * g;
    static_assert(!PAIR || pair_tables<KB>(), "pair rows of 4- and 8-bit tables");
    // Padding buckets (s >= S) read the last table's rows, which every slice
    // holding padding projects (a slice's columns hold only its own tables:
    // other rows of its LDS are left over from earlier work), and padding
    // buckets and tokens are cleared by a select: a product with zero would
    // keep a NaN or infinity of those rows.
    const int lpad = (S >> KB) - 1;
    if constexpr (PAIR) {
        const bool sv = FULL || s0 < S;
        const int l = sv ? s0 >> KB : lpad, r0 = s0 & (R - 1);
        const int n1 = l * KB + KB - 4;  // the table's last nibble
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int t = 16 * nt + i;
            const bool v = sv && (FULL || t < nv);
            float hi = sp[t * LDC + n1 + ((r0 >> 2) & 3)];
            if constexpr (KB == 8) hi *= sp[t * LDC + l * KB + (r0 >> 6)] * sm[t * LDC + l * KB + ((r0 >> 4) & 3)];
            const f32x4 lo = *reinterpret_cast<const f32x4 *>(sm + t * LDC + n1);
#pragma unroll
            for (int e = 0; e < 4; ++e) P[nt][e] = (FULL || v) ? hi * lo[e] : 0.f;
        }
        return;
    }
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int t = 16 * nt + i;
        const bool tv = FULL || t < nv;
        if constexpr (KB == 1) {
            // tables s0/2 and s0/2 + 1; corner r = 1 is sigmoid(+2u)
            const bool v01 = FULL || (tv && s0 < S), v23 = FULL || (tv && s0 + 2 < S);
            const int l0 = v01 ? s0 >> 1 : lpad, l1 = v23 ? (s0 >> 1) + 1 : lpad;
            P[nt][0] = v01 ? sm[t * LDC + l0] : 0.f;
            P[nt][1] = v01 ? sp[t * LDC + l0] : 0.f;
            P[nt][2] = v23 ? sm[t * LDC + l1] : 0.f;
            P[nt][3] = v23 ? sp[t * LDC + l1] : 0.f;
        } else {
            const bool v = FULL || (tv && s0 < S);
            const int l = (FULL || s0 < S) ? s0 >> KB : lpad;
            const int r0 = s0 & (R - 1);
            const float *pp = sp + t * LDC + l * KB, *pm = sm + t * LDC + l * KB;
            float fp[KB], fm[KB];
#pragma unroll
            for (int k = 0; k < KB; ++k) {
                fp[k] = pp[k];
                fm[k] = pm[k];
            }
            float hi = 1.f;
            if constexpr (KB > 2) {
                hi = ((r0 >> (KB - 1)) & 1) ? fp[0] : fm[0];
#pragma unroll
                for (int k = 1; k < KB - 2; ++k) hi *= ((r0 >> (KB - 1 - k)) & 1) ? fp[k] : fm[k];
            }
            const float h0 = hi * fm[KB - 2], h1 = hi * fp[KB - 2];
            P[nt][0] = v ? h0 * fm[KB - 1] : 0.f;
            P[nt][1] = v ? h0 * fp[KB - 1] : 0.f;
            P[nt][2] = v ? h1 * fm[KB - 1] : 0.f;
            P[nt][3] = v ? h1 * fp[KB - 1] : 0.f;
        }
    }
}
template <int KB, bool AL = false, bool PAIR = false>
__device__ __forceinline__ void probs_st(const float *sp, const float *sm, int sw, int S, int nv, f32x4 (&P)[2]) {
    probs_st_<KB, AL, PAIR>(sp, sm, sw, S, nv, P);
}

// Operand of 8 consecutive k values (k = 8g .. 8g+7 of lane (g, i)), the
// layout ld_frag reads from k-contiguous rows, from registers.
template <typename T> __device__ __forceinline__ Frag<T> frag_seq(const float (&v)[8]);
template <> __device__ __forceinline__ Frag<bf16> frag_seq<bf16>(const float (&v)[8]) {
    Frag<bf16> f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f.v[j] = (bf16)v[j];
    return f;
}
template <> __device__ __forceinline__ Frag<float> frag_seq<float>(const float (&v)[8]) {
    Frag<float> f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f.lo[j] = v[j];
        f.hi[j] = v[4 + j];
    }
    return f;
}

// ------------------------------------------------------------ constant operands
// Operand slots in the pi order of frag_acc: slot j < 4 is row 4g + j, slot
// 4 + j is row 16 + 4g + j of a 32-row operand.
template <typename T> __device__ __forceinline__ Frag<T> frag_pi_from(const float (&v)[8]);
template <> __device__ __forceinline__ Frag<bf16> frag_pi_from<bf16>(const float (&v)[8]) {
    Frag<bf16> f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f.v[j] = (bf16)v[j];
    return f;
}
template <> __device__ __forceinline__ Frag<float> frag_pi_from<float>(const float (&v)[8]) {
    Frag<float> f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f.lo[j] = v[j];
        f.hi[j] = v[4 + j];
    }
    return f;
}

// B operands that turn token contractions into prefix sums, totals and
// transposes on the matrix cores, read from small LDS tables:
//   tri[t][tau] = (tau <= t): column t = 16nt + i of the prefix (row 31 is
//                 all ones: token totals, replicated over the columns)
//   id[s][s']   = (s == s'): 16-deep identity for transposes
template <typename T> struct Consts {
    static constexpr int LDT = ldp_of<T>(TT), LDI = ldp_of<T>(16);
    static constexpr size_t bytes = sizeof(T) * (TT * LDT + 16 * LDI);
    const T *tri, *id;
    // bf16: the prefix and total operands in registers (cache(), once the
    // table is visible), so the tile loops do not read them from LDS
    Frag<T> tri0_, tri1_, ones_;
    __device__ __forceinline__ void init(T *buf, int nth) {
        T *t = buf, *d = buf + TT * LDT;
        for (int idx = threadIdx.x; idx < TT * LDT; idx += nth)
            t[idx] = from_f32<T>(idx % LDT <= idx / LDT ? 1.f : 0.f);
        for (int idx = threadIdx.x; idx < 16 * LDI; idx += nth)
            d[idx] = from_f32<T>(idx % LDI == idx / LDI ? 1.f : 0.f);
        tri = t;
        id = d;
    }
    __device__ __forceinline__ void cache() {
        if constexpr (is_bf16<T>()) {
            tri0_ = ld_frag_pi(tri + li() * LDT);
            tri1_ = ld_frag_pi(tri + (16 + li()) * LDT);
            ones_ = ld_frag_pi(tri + (TT - 1) * LDT);
        }
    }
    __device__ __forceinline__ Frag<T> tri_op(int nt) const {
        if constexpr (is_bf16<T>())
            return nt ? tri1_ : tri0_;
        else
            return ld_frag_pi(tri + (16 * nt + li()) * LDT);
    }
    __device__ __forceinline__ Frag<T> ones() const {
        if constexpr (is_bf16<T>())
            return ones_;
        else
            return ld_frag_pi(tri + (TT - 1) * LDT);
    }
    __device__ __forceinline__ Frag4<T> ident() const { return ld_frag16(id + li() * LDI); }
};
// bf16 pairwise transposes: id[n][k] = (k == n), 32 x 32.  With the pair
// operand A = frag_acc(X0, X1) of two bucket-row tiles, A . lo() = X0^T and
// A . hi() = X1^T: every k slot holds data, none is zero padding.
template <typename T> struct PairOps {
    static constexpr int LDT = ldp_of<T>(TT);
    static constexpr size_t bytes = is_bf16<T>() ? sizeof(T) * TT * LDT : 0;
    const T *id = nullptr;
    Frag<T> lo_, hi_;  // in registers after cache()
    __device__ __forceinline__ void init(T *buf, int nth) {
        if constexpr (is_bf16<T>()) {
            for (int idx = threadIdx.x; idx < TT * LDT; idx += nth)
                buf[idx] = from_f32<T>(idx % LDT == idx / LDT ? 1.f : 0.f);
            id = buf;
        }
    }
    __device__ __forceinline__ void cache() {
        if constexpr (is_bf16<T>()) {
            lo_ = ld_frag_pi(id + li() * LDT);
            hi_ = ld_frag_pi(id + (16 + li()) * LDT);
        }
    }
    __device__ __forceinline__ Frag<T> lo() const { return lo_; }
    __device__ __forceinline__ Frag<T> hi() const { return hi_; }
};

// 16-deep constant A operand of mma16_x: bf16 holds the row's 16 k values
// twice (slots j and 4 + j) so that one 16x16x32 product takes B = (hi, lo);
// fp32 holds them once.
template <typename T> struct OpX;
template <> struct OpX<bf16> { Frag<bf16> f; };
template <> struct OpX<float> { Frag4<float> f; };

// Softmax / corner backward over the wave's 16 buckets (tables of 2^KB
// buckets, R-aligned): one 16-deep A operand (row r, k = local bucket s) whose
// product with pd = P dP gives, per local table tl, the corner sums
// sum_s pd c_{s,k} (c = +-1, corner bit) and the table sum sum_s pd, with
// each corner row and its table's sum row in the same lane group (rows
// 4g..4g+3), so no value crosses lanes:
//   KB=4: g0 = c0 c1 c2 sum, g1 = c3 sum;  KB=3: g = table g: c0 c1 c2 sum;
//   KB=2: g = table g: c0 c1 sum;          KB=1: g = tables 2g, 2g+1: (c0 sum) x 2.
template <typename T, int KB> struct HashOps {
    static constexpr int W_ = is_bf16<T>() ? TT : 16;  // bf16: 16 k values, then the same 16 again
    static constexpr int LDI = ldp_of<T>(W_);
    static constexpr size_t bytes = sizeof(T) * 16 * LDI;
    const T *a;
    // row r = 4g + e (lane group g, slot e of the product's accumulator):
    // 1 = corner k of local table tl, 2 = sum of tl, 0 = unused; de = slot of
    // tl's sum row in the row's lane group.  The corners are spread over the
    // lane groups so that every lane has at most one corner per pair of
    // slots: K = 4 puts corner k = g in slot 0 (one pass over the slots),
    // K = 3 corner k = g (g < 3) of tables 0 and 1 in slots 0 and 2.
    __host__ __device__ static constexpr int kind_of(int r, int &k, int &tl, int &de) {
        const int g = r >> 2, e = r & 3;
        k = 0;
        if constexpr (KB == 4) {
            tl = 0;
            de = 1;
            k = g;
            return e == 0 ? 1 : (e == 1 ? 2 : 0);
        } else if constexpr (KB == 3) {
            tl = e >> 1;
            de = (e & 2) | 1;
            k = g;
            if (g == 3) return 0;
            return (e & 1) ? 2 : 1;
        } else if constexpr (KB == 2) {
            tl = g;
            de = 2;
            return e < 2 ? (k = e, 1) : (e == 2 ? 2 : 0);
        } else {
            tl = 2 * g + (e >> 1);
            de = (e & 2) | 1;
            return (e & 1) ? 2 : 1;
        }
    }
    __device__ __forceinline__ void init(T *buf, int nth) {
        for (int idx = threadIdx.x; idx < 16 * LDI; idx += nth) {
            const int r = idx / LDI, kk = idx % LDI, sb = kk & 15;
            int k = 0, tl = 0, de = 0;
            const int kind = kind_of(r, k, tl, de);
            float v = 0.f;
            if (kk < W_ && (sb >> KB) == tl) v = kind == 2 ? 1.f : (kind == 1 ? (((sb >> (KB - 1 - k)) & 1) ? 1.f : -1.f) : 0.f);
            buf[idx] = from_f32<T>(v);
        }
        a = buf;
    }
    OpX<T> op_;  // in registers after cache()
    __device__ __forceinline__ void cache() {
        if constexpr (is_bf16<T>())
            op_.f = ld_frag_pi(a + li() * LDI);
        else
            op_.f = ld_frag16(a + li() * LDI);
    }
    __device__ __forceinline__ OpX<T> op() const { return op_; }
};

// Every (table, corner) pair of the wave's 16 buckets has exactly one corner
// row, whose sum slot de (same lane group) holds the sum row of its table.
template <int KB> constexpr bool hash_rows_valid() {
    constexpr int NTAB = 16 >> KB > 0 ? 16 >> KB : 1;
    for (int tl = 0; tl < NTAB; ++tl)
        for (int kk = 0; kk < KB; ++kk) {
            int found = 0;
            for (int r = 0; r < 16; ++r) {
                int k = 0, t = 0, de = 0;
                if (HashOps<float, KB>::kind_of(r, k, t, de) == 1 && t == tl && k == kk) {
                    ++found;
                    int k2 = 0, t2 = 0, de2 = 0;
                    if (HashOps<float, KB>::kind_of((r & ~3) | de, k2, t2, de2) != 2 || t2 != tl) return false;
                }
            }
            if (found != 1) return false;
        }
    return true;
}
static_assert(hash_rows_valid<1>() && hash_rows_valid<2>() && hash_rows_valid<3>() && hash_rows_valid<4>(),
              "softmax-backward row layout");

// Token-direction operand of the wave's bucket-row tiles X[2] (lane holds
// X[s = 4g + e][t = 16nt + i]): each tile is transposed on the matrix core
// (identity product; exact for operand-rounded values) into token-row
// layout, and the pair forms the operand with row s and k = t (pi order).
template <typename T> __device__ __forceinline__ Frag<T> token_operand(const f32x4 (&X)[2], const Consts<T> &cst) {
    const Frag4<T> ident = cst.ident();
    f32x4 r0 = zero4(), r1 = zero4();
    mma16(r0, frag16_acc<T>(X[0]), ident);
    mma16(r1, frag16_acc<T>(X[1]), ident);
    return frag_acc<T>(r0, r1);
}

// bf16: the exact transposes of a pair operand A = (X0, X1), as the operand
// with row s and k = t (pi order) -- two products, no padded k slots
__device__ __forceinline__ Frag<bf16> transpose_pair(const Frag<bf16> &A, const PairOps<bf16> &po) {
    f32x4 r0 = zero4(), r1 = zero4();
    mma(r0, A, po.lo());
    mma(r1, A, po.hi());
    return frag_acc<bf16>(r0, r1);
}
template <typename T>
__device__ __forceinline__ Frag<T> token_operand(const f32x4 (&X)[2], const Consts<T> &cst, const PairOps<T> &po) {
    if constexpr (is_bf16<T>())
        return transpose_pair(frag_acc<T>(X[0], X[1]), po);
    else
        return token_operand<T>(X, cst);
}

// fp32-accurate bf16 pair operand of two accumulator tiles (the pi-order pair
// of frag_acc): hi = each value truncated to its upper 16 bits (exact as
// bf16, no rounding step), lo = the exact remainder rounded to bf16, so that
// hi + lo is within 2^-16 of the value.
__device__ __forceinline__ void frag_acc_hilo(const f32x4 &x0, const f32x4 &x1, Frag<bf16> &hi, Frag<bf16> &lo) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float x = j < 4 ? x0[j] : x1[j - 4];
        const uint32_t u = __float_as_uint(x) & 0xFFFF0000u;
        hi.v[j] = __builtin_bit_cast(bf16, (unsigned short)(u >> 16));
        lo.v[j] = (bf16)(x - __uint_as_float(u));
    }
}

// Small tables -- bf16 with at most 3 hash bits, or 4 bits in at most 64
// buckets: P_K, W and the carried U enter the products that sum them as
// fp32-accurate pairs (the operand hi plus a second product with lo = the
// remainder).  A table of few wide buckets at a low temperature has nearly
// flat probabilities (P_s = 2^-K + a small variation); the softmax backward
// of dQ and dK cancels what is common to a table's buckets, so a bf16 operand
// alone would leave 2^-9 of P itself, not of its variation, in the gradients:
// through A's prefix sums and totals, the in-tile G term and the B sums (P_K),
// dP_K's in-tile term and the U sums (W), and dP_K's v . U term (U).  The
// 4-bit, 128-bucket and wider instantiations average over more tables and
// keep the single operands.
template <typename T, int SP, int KB> __host__ __device__ constexpr bool hl_ops() {
    return is_bf16<T>() && (KB <= 3 || (KB == 4 && SP <= 64));
}
// bf16 B state in fp64: k_fwd_reduce's segment sums and k_bwd_out's
// reverse walk add the tiles' fp32 sums to fp64 totals instead of
// accumulating them on the matrix core.  The walk derives B at a tile start
// as the state at the segment end minus the later tiles' sums, so an fp32
// walk carries an error relative to the segment-end state; with a sharp
// softmax a bucket's B can grow by orders of magnitude within a segment, and
// dA, whose factor W / (A + eps) is largest where A (hence B) is smallest,
// takes that error as it is.  Both sides change together: fp32 sums and an
// fp32 walk round the same tile sums the same way, and their errors partly
// cancel.  Every bf16 instantiation but the whole-tile ones (4- and 8-bit,
// 128 buckets), whose fp32 accumulators keep the registers of k_bwd_out's
// two-wave and k_fwd_reduce's four-wave occupancy.  Where the bucket
// probabilities can span a wide range, the host runs whole tiles through the
// generic k_fwd_reduce and the whole-tile k_bwd_out with XW (race_capi.hip
// exact_walk): their tile sums come from the same P_K and V operands in the
// same order, so the fp64 walk subtracts exactly what the sums added.
template <typename T, bool AL> __host__ __device__ constexpr bool walk_f64() { return is_bf16<T>() && !AL; }
// R = X - bf16(X) (exact in fp32): the lo part of a tile pair whose hi part is
// the round-to-nearest operand the kernels take from X
__device__ __forceinline__ void lo_rem(const f32x4 (&X)[2], f32x4 (&R)[2]) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) R[nt][e] = X[nt][e] - as_operand<bf16>(X[nt][e]);
}

// c += A . X^T over the wave's 16 buckets, X a bucket-row tile taken as the B
// operand (column t, k = s); bf16 runs A . hi + A . lo as one 32-deep product
// (A duplicated in OpX, X split into its two bf16 parts, hi + lo within
// 2^-16 of x), fp32 accuracy.
template <typename T> __device__ __forceinline__ void mma16_x(f32x4 &c, const OpX<T> &A, const f32x4 &x) {
    if constexpr (is_bf16<T>()) {
        // hi: x truncated to its upper 16 bits (exact as bf16, no rounding
        // step); lo: the exact remainder x - hi, rounded to bf16
        Frag<bf16> hl;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t u = __float_as_uint(x[j]) & 0xFFFF0000u;
            hl.v[j] = __builtin_bit_cast(bf16, (unsigned short)(u >> 16));
            hl.v[j + 4] = (bf16)(x[j] - __uint_as_float(u));
        }
        mma(c, A.f, hl);
    } else {
        mma16(c, A.f, frag16_acc<T>(x));
    }
}

// Tables of 2^KB >= 32 buckets span several waves (and, when 2^KB > SP,
// several bucket slices).  The corner backward is linear in the buckets:
//   du_k = sum_r P_r dP_r c_rk - (sum_r P_r dP_r) tanh(u_k),
// since sum_r P_r c_rk = sigmoid(2u_k) - sigmoid(-2u_k) = tanh(u_k) over a
// whole table.  Each wave writes its buckets' sums (sum P dP c_k, sum P dP)
// per token (softhash_share); the waves of a table are then summed in a fixed
// order (softhash_combine), and slices of a table add up through the partial
// dQ / dK outputs.
template <typename T, int KB> struct WideHash {
    static constexpr size_t bytes(int nw) { return sizeof(float) * nw * TT * (KB + 1); }
    OpX<T> cs, ones;  // A operands over the wave's 16 buckets: rows k < KB: c_{s,k}; all ones
    __device__ __forceinline__ void init(int sg) {
        const int g = lg(), i = li();
        f32x4 c, o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = (sg + 4 * g + j) & ((1 << KB) - 1);
            c[j] = i < KB ? (((r >> (KB - 1 - i)) & 1) ? 1.f : -1.f) : 0.f;
            o[j] = 1.f;
        }
        if constexpr (is_bf16<T>()) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                cs.f.v[j] = cs.f.v[j + 4] = (bf16)c[j];
                ones.f.v[j] = ones.f.v[j + 4] = (bf16)o[j];
            }
        } else {
            cs.f = frag16_acc<T>(c);
            ones.f = frag16_acc<T>(o);
        }
    }
};

template <int KB, typename T>
__device__ void softhash_share(const f32x4 (&P)[2], const f32x4 (&dP)[2], const WideHash<T, KB> &wh, float *share) {
    const int g = lg(), i = li();
    float *mine = share + wave_id() * TT * (KB + 1);
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        f32x4 pd, X = zero4(), Sd = zero4();
#pragma unroll
        for (int e = 0; e < 4; ++e) pd[e] = P[nt][e] * dP[nt][e];
        mma16_x<T>(X, wh.cs, pd);    // rows k: sum_s c_{s,k} P dP
        mma16_x<T>(Sd, wh.ones, pd); // every row: sum_s P dP
        const int t = 16 * nt + i;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (4 * g + e < KB) mine[t * (KB + 1) + 4 * g + e] = X[e];
        if (g == 0) mine[t * (KB + 1) + KB] = Sd[0];
    }
}

// after the shares are visible: du -> dproj for the slice's tables; returns
// this thread's part of sum du * th.  Each (token, table, bit) item's sum over
// the table's waves is split between two neighbouring lanes (half the waves
// each, in order) and joined with a DPP swap, so every wave of the workgroup
// takes part and the dependent chain of LDS reads is half as long.
template <int KB, typename T, int SP, int NTH, bool PAIR = false>
__device__ float softhash_combine(const float *share, const float *sp, const float *sm, const float *sth, int z, int L,
                                  float inv_temp, T *dproj) {
    constexpr int LDC = ld_of<float>(NCOL), R = 1 << KB, NW_ = SP / WB;
    constexpr int NTAB = SP >= R ? SP / R : 1;          // tables (or one table part) in the slice
    constexpr int WPT = (R / WB) < NW_ ? R / WB : NW_;  // waves per table in the slice
    constexpr int SPLIT = WPT % 2 == 0 ? 2 : 1, WPL = WPT / SPLIT, ITEMS = TT * NTAB * KB;
    const int l0 = (z * SP) >> KB;
    float tsum = 0.f;
    for (int base = 0; base < ITEMS * SPLIT; base += NTH) {  // the same trip count in every lane
        const int idx = base + (int)threadIdx.x, item = idx / SPLIT, half = idx % SPLIT;
        const int t = item / (NTAB * KB), r = item % (NTAB * KB), tl = r / KB, k = r % KB;
        const bool live = item < ITEMS && l0 + tl < L;
        float sx = 0.f, sd = 0.f;
        if (live)
            for (int u = 0; u < WPL; ++u) {
                const int ww = tl * WPT + half * WPL + u;
                sx += share[(ww * TT + t) * (KB + 1) + k];
                sd += share[(ww * TT + t) * (KB + 1) + KB];
            }
        if constexpr (SPLIT == 2) {  // lanes 2m and 2m + 1 hold one item
            sx += dpp_f<0xB1>(sx);
            sd += dpp_f<0xB1>(sd);
        }
        if (live && half == 0) {
            const int col = (l0 + tl) * KB + k;
            const float th = sth[t * LDC + col];
            const float du = sx - sd * corner_tanh<PAIR>(sp, sm, t, col);
            tsum += du * th;
            const float dp = du * inv_temp * (1.f - th * th);
            if constexpr (xpart_f32(is_bf16<T>(), SP, KB))
                reinterpret_cast<float *>(dproj)[t * 8 + k] = dp;  // the slice's one table: [TT][8] fp32
            else
                dproj[sw_off<T, NCOL>(t, col)] = from_f32<T>(dp);
        }
    }
    return tsum;
}

// Inclusive token suffix Y (plus y0, the lane's per-bucket carry) and token
// totals of a bucket-row tile pair (lane holds X[s = 4g + e][t = 16nt + i]):
// fp32 suffix scans over the 16 lanes of each row (DPP), tile 1 first; a
// row's total is its suffix at lane 0, broadcast to the row.
__device__ __forceinline__ void suffix_totals(const f32x4 (&X)[2], const f32x4 &y0, f32x4 (&Y)[2], f32x4 &tot) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float s1 = row_suffix(X[1][e]), t1 = row_bcast0(s1);
        const float s0 = row_suffix(X[0][e]);
        Y[1][e] = y0[e] + s1;
        Y[0][e] = (y0[e] + t1) + s0;
        tot[e] = row_bcast0(s0) + t1;
    }
}
// token totals only (lane: bucket 4g + e), fp32 row sums over the 16 lanes
// of each row
__device__ __forceinline__ void totals_of(const f32x4 (&X)[2], f32x4 &tot) {
#pragma unroll
    for (int e = 0; e < 4; ++e) tot[e] = row_sum(X[0][e] + X[1][e]);
}

// Softmax / corner / tanh backward for the wave's buckets on the matrix
// cores: dP (and P, fp32, bucket-row) -> dproj [TT][NCOL] columns l*K + k of
// the wave's tables; returns this lane's share of sum du * th.
//   du_k = sum_table P (dP - sum_table P dP) c_k
//        = sum_table pd c_k - (sum_table pd) tanh(u_k),  pd = P dP,
// since sum_table P c_k = sigmoid(2u_k) - sigmoid(-2u_k) = tanh(u_k) (= sp - sm);
//   dproj = du * inv_temp * (1 - th^2).
template <int KB, typename T, bool PAIR = false>
__device__ float softhash_bwd(const f32x4 (&P)[2], const f32x4 (&dP)[2], const float *sp, const float *sm,
                              const float *sth, int sw, int L, float inv_temp, T *dproj, const HashOps<T, KB> &ho) {
    constexpr int LDC = ld_of<float>(NCOL);
    const int g = lg(), i = li(), l0 = sw >> KB;
    const OpX<T> A = ho.op();
    // the corner rows' tanh(u) = sp - sm and th, read ahead of the products
    // (column 0 stands in for tables past L, whose results are dropped)
    float tu[2][4], th[2][4];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            int k = 0, tl = 0, de = 0;
            const int kind = HashOps<T, KB>::kind_of(4 * g + e, k, tl, de);
            const int l = l0 + tl, c = l < L ? l * KB + k : 0, t = 16 * nt + i;
            tu[nt][e] = th[nt][e] = 0.f;
            if (kind == 1) {
                tu[nt][e] = corner_tanh<PAIR>(sp, sm, t, c);
                th[nt][e] = sth[t * LDC + c];
            }
        }
    float tsum = 0.f;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        f32x4 pd, X = zero4();
#pragma unroll
        for (int e = 0; e < 4; ++e) pd[e] = P[nt][e] * dP[nt][e];
        mma16_x<T>(X, A, pd);
        const int t = 16 * nt + i;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            int k = 0, tl = 0, de = 0;
            const int kind = HashOps<T, KB>::kind_of(4 * g + e, k, tl, de);
            const int l = l0 + tl, col = l * KB + k;
            if (kind == 1 && l < L) {
                float sum;
                if constexpr (KB == 4)
                    sum = X[1];
                else if constexpr (KB == 2)
                    sum = X[2];
                else
                    sum = X[(e & 2) | 1];
                const float du = X[e] - sum * tu[nt][e];
                tsum += du * th[nt][e];
                dproj[sw_off<T, NCOL>(t, col)] = from_f32<T>(du * inv_temp * (1.f - th[nt][e] * th[nt][e]));
            }
        }
    }
    return tsum;
}

// bucket-row tiles -> [t][s] LDS array (s contiguous, leading dimension ld):
// each lane writes its 4 consecutive buckets of one token
template <typename T, int N> __device__ __forceinline__ void store_ts(T *dst, int sw, const f32x4 (&X)[2]) {
    T *p = dst + sw_off<T, N>(li(), sw + 4 * lg());
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) store4<T>(p + 16 * sw_ld<T, N>() * nt, X[nt]);
}
// The wave's token operand of what store_ts wrote (bucket s = sw + i, k =
// token t in pi order: 4g + j, then 16 + 4g + j), read back with two LDS
// transpose loads (ds_read_b64_tr_b16: in each 16-lane group, lane 4e + q
// reads 4 elements and lane 4q' + c receives element c of lanes q' + 4e,
// e = 0..3).  bf16 only; the values are the ones store_ts rounded.
template <int N> __device__ __forceinline__ Frag<bf16> ts_operand_tr(const bf16 *base, int sw) {
    typedef short v4s __attribute__((ext_vector_type(4)));
    typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
    const int g = lg(), p = li();
    const int c = sw + 4 * (p & 3);
    const bf16 *a = base + sw_off<bf16, N>(4 * g + (p >> 2), c);
    const bf16 *b = base + sw_off<bf16, N>(16 + 4 * g + (p >> 2), c);
    const v4s ra = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s *)a);
    const v4s rb = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s *)b);
    const bf16x4 x = __builtin_bit_cast(bf16x4, ra), y = __builtin_bit_cast(bf16x4, rb);
    Frag<bf16> f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f.v[j] = x[j];
        f.v[j + 4] = y[j];
    }
    return f;
}
// The pi-order token operand of column d = 16 md + i of a staged token tile
// (k = token t: 4g + j, then 16 + 4g + j), the operand ld_frag_pi reads from a
// transposed [D][TT] tile's row d.  bf16 reads it from the natural rows with
// two LDS transpose loads: lane (g, p) reads columns 16 md + 4(p & 3) .. +3 of
// row 4g + (p >> 2) (and row 16 + ...), runs of 4 columns that the natural
// layout keeps contiguous; fp32 reads the transposed rows trn.
template <typename T, class NL, bool NAT = is_bf16<T>()>
__device__ __forceinline__ Frag<T> col_operand(const T *nat, const T *trn, int md) {
    if constexpr (NAT) {
        static_assert(is_bf16<T>(), "transpose loads of 16-bit elements");
        typedef short v4s __attribute__((ext_vector_type(4)));
        typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
        const int g = lg(), p = li(), d0 = 16 * md + 4 * (p & 3);
        const bf16 *a = nat + NL::off(4 * g + (p >> 2), d0);
        const bf16 *b = nat + NL::off(16 + 4 * g + (p >> 2), d0);
        const v4s ra = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s *)a);
        const v4s rb = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s *)b);
        const bf16x4 x = __builtin_bit_cast(bf16x4, ra), y = __builtin_bit_cast(bf16x4, rb);
        Frag<bf16> f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f.v[j] = x[j];
            f.v[j + 4] = y[j];
        }
        return f;
    } else {
        return ld_frag_pi(trn + (16 * md + li()) * ldp_of<T>(TT));
    }
}
// token operand of a bucket-row tile pair X that the wave also stores to its
// [t][s] rows: bf16 stores first and reads the operand back transposed
template <typename T, int N>
__device__ __forceinline__ Frag<T> store_ts_operand(T *dst, int sw, const f32x4 (&X)[2], const Consts<T> &cst) {
    if constexpr (is_bf16<T>()) {
        store_ts<T, N>(dst, sw, X);
        return ts_operand_tr<N>(dst, sw);
    } else {
        const Frag<T> f = token_operand<T>(X, cst);
        store_ts<T, N>(dst, sw, X);
        return f;
    }
}
// bucket-row [s][d] carry (lane holds [s = sw + 4g + e][d = 16md + i]) ->
// [d][s] LDS array (s contiguous)
template <typename T, int N> __device__ __forceinline__ void store_ds(T *dst, int sw, const f32x4 (&X)[4]) {
    T *p = dst + sw_off<T, N>(li(), sw + 4 * lg());
#pragma unroll
    for (int md = 0; md < 4; ++md) store4<T>(p + 16 * sw_ld<T, N>() * md, X[md]);
}

// d-row U^T (lane holds U^T[d = 16md + 4g + e][s = sw + i]) -> [d][s] LDS
// array, each 16x16 block transposed on the matrix core into bucket-row
// layout (lane: [s = sw + 4g + e][d = 16md + i]) for 4-bucket stores
template <typename T, int N>
__device__ __forceinline__ void store_ut(T *dst, int sw, const f32x4 (&Ut)[4], const Consts<T> &cst,
                                         const PairOps<T> &po) {
    f32x4 Us[4];
    if constexpr (is_bf16<T>()) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const Frag<bf16> A = frag_acc<bf16>(Ut[2 * p], Ut[2 * p + 1]);
            Us[2 * p] = zero4();
            Us[2 * p + 1] = zero4();
            mma(Us[2 * p], A, po.lo());
            mma(Us[2 * p + 1], A, po.hi());
        }
    } else {
        const Frag4<T> ident = cst.ident();
#pragma unroll
        for (int md = 0; md < 4; ++md) {
            Us[md] = zero4();
            mma16(Us[md], frag16_acc<T>(Ut[md]), ident);
        }
    }
    store_ds<T, N>(dst, sw, Us);
}

// M[tau][t] = v_tau . g_t for tau <= t, 0 above the diagonal, for the tile's
// causal triangle.  Task q < 3 writes tile q of X[t][tau] (rows t, the G
// term's operand), q >= 3 tile q - 3 of Y[tau][t] (rows tau, the dP_K term's);
// tiles (mt, nt) = (0,0), (0,1), (1,1); the all-zero tile (1,0) is cleared
// once at kernel start.
template <typename T, class NL = NatL<T, false>> __device__ void m_tile(int q, const T *sV, const T *sG, T *X, T *Y) {
    constexpr int LDT = ldp_of<T>(TT);
    const int g = lg(), i = li();
    const int r = q % 3, mt = r == 2 ? 1 : 0, nt = r == 0 ? 0 : 1;
    f32x4 acc = zero4();
    if (q < 3) {
        nat_mma<NL>(acc, sV, 16 * mt, sG, 16 * nt);  // [tau = 16mt+4g+e][t = 16nt+i]
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (16 * mt + 4 * g + e > 16 * nt + i) acc[e] = 0.f;
        store4<T>(X + (16 * nt + i) * LDT + 16 * mt + 4 * g, acc);
    } else {
        nat_mma<NL>(acc, sG, 16 * nt, sV, 16 * mt);  // [t = 16nt+4g+e][tau = 16mt+i]
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (16 * mt + i > 16 * nt + 4 * g + e) acc[e] = 0.f;
        store4<T>(Y + (16 * mt + i) * LDT + 16 * nt + 4 * g, acc);
    }
}

// Block r of X (as m_tile) and, from the same product, its transposed copy
// Y[tau][t] (one 2-byte store per element): no second product.
template <typename T, class NL = NatL<T, false>>
__device__ void m_tile_xy(int r, const T *sV, const T *sG, T *X, T *Y) {
    constexpr int LDT = ldp_of<T>(TT);
    const int g = lg(), i = li();
    const int mt = r == 2 ? 1 : 0, nt = r == 0 ? 0 : 1;
    f32x4 acc = zero4();
    nat_mma<NL>(acc, sV, 16 * mt, sG, 16 * nt);  // [tau = 16mt+4g+e][t = 16nt+i]
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (16 * mt + 4 * g + e > 16 * nt + i) acc[e] = 0.f;
    store4<T>(X + (16 * nt + i) * LDT + 16 * mt + 4 * g, acc);
#pragma unroll
    for (int e = 0; e < 4; ++e) Y[(16 * mt + 4 * g + e) * LDT + 16 * nt + i] = from_f32<T>(acc[e]);
}

// The G term's in-tile operand, built by each wave in registers: blocks
// C[tau][t] = v_tau . g_t (tau <= t) of the tile as the B operand with k = tau
// (pi order) and n = t for token half nt -- the values m_tile stores, without
// the shared task, its barrier phase or LDS round trip.
template <typename T, class NL>
__device__ __forceinline__ void x_operands(const T *sV, const T *sG, Frag<T> (&X)[2]) {
    const int g = lg(), i = li();
    f32x4 c00 = zero4(), c01 = zero4(), c11 = zero4();
    nat_mma<NL>(c00, sV, 0, sG, 0);    // [tau = 4g + e][t = i]
    nat_mma<NL>(c01, sV, 0, sG, 16);   // [tau = 4g + e][t = 16 + i]: all tau <= t
    nat_mma<NL>(c11, sV, 16, sG, 16);  // [tau = 16 + 4g + e][t = 16 + i]
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (4 * g + e > i) {
            c00[e] = 0.f;
            c11[e] = 0.f;
        }
    X[0] = frag_acc<T>(c00, zero4());
    X[1] = frag_acc<T>(c01, c11);
}

template <typename T> __device__ void zero_lds(T *p, int n, int nth) {
    for (int idx = threadIdx.x; idx < n; idx += nth) p[idx] = from_f32<T>(0.f);
}

// dX for the tile: dX^T = planes^T dproj^T, 8 tiles over the workgroup's waves,
// stored straight to rows t0.. (< T) of dst.
// part != nullptr (bucket slices): this slice's dproj columns c0 .. c0 + XC - 1
// instead, rows t0.. of a [T][XC] block -- the product with planes^T and the
// sum over slices happen in k_dx_finish, on the same operand values.  XF: the
// rows are fp32 ([TT][8] at dproj's start, softhash_combine), copied as they are.
template <typename T, int NW_, int XC = 8, bool AL = false, bool XF = false>
__device__ void dx_store(const T *dproj, const T *plt, T *dst, int64_t st, int64_t t0, int64_t Tn, void *vpart,
                         int c0 = 0) {
    if constexpr (XF) {
        static_assert(XC == 8, "fp32 dproj partials are 8-column rows");
        // two lanes a token, 16 bytes each: the tile's rows are 1 KB of contiguous partials
        const int l = threadIdx.x, t = l >> 1;
        if (l < 2 * TT && (AL || t < tile_rows(t0, Tn)))
            *reinterpret_cast<f32x4 *>(at_bytes((float *)vpart + t0 * 8, (uint32_t)l * 16u)) =
                *reinterpret_cast<const f32x4 *>(reinterpret_cast<const float *>(dproj) + 4 * l);
        return;
    }
    T *part = (T *)vpart;
    if (part) {
        if constexpr (is_bf16<T>() && XC == 8) {
            if ((c0 & 7) == 0) {
                // the 8 columns are one 16-byte granule of each swizzled dproj
                // row (c0 + 8 <= NCOL): one 16-byte copy per token
                const int t = threadIdx.x;
                if (t < TT && (AL || t < tile_rows(t0, Tn)))
                    *reinterpret_cast<uint4 *>(at_bytes(part + t0 * XC, (uint32_t)(t * XC) * (uint32_t)sizeof(T))) =
                        *reinterpret_cast<const uint4 *>(dproj + sw_off<T, NCOL>(t, c0));
                return;
            }
        }
        for (int idx = threadIdx.x; idx < TT * XC; idx += 64 * NW_) {
            const int t = idx / XC, c = idx % XC;
            if (AL || t < tile_rows(t0, Tn)) part[(t0 + t) * XC + c] = c0 + c < NCOL ? dproj[sw_off<T, NCOL>(t, c0 + c)] : from_f32<T>(0.f);
        }
        return;
    }
    const int g = lg(), i = li(), w = wave_id();
    T *base = tile_ptr(dst, st, t0);
    for (int q = w; q < 8; q += NW_) {
        const int md = q >> 1, nt = q & 1;
        f32x4 acc = zero4();
        mma(acc, ld_frag(sw_frag_ptr<T, NCOL>(plt, 16 * md + i)), ld_frag(sw_frag_ptr<T, NCOL>(dproj, 16 * nt + i)));
        const int t = 16 * nt + i;
        if (AL || t < tile_rows(t0, Tn)) store4<T>(at_bytes(base, tile_off(t, st, 16 * md + 4 * g, sizeof(T))), acc);
    }
}

// Workgroups per CU of a backward tile kernel with nw waves and `bytes` of
// LDS: the kernels need more than 128 VGPRs, so at most 2 waves per SIMD
// (8 per CU) run, whatever the LDS allows.
__host__ __device__ constexpr size_t bwd_wgs_per_cu(int nw, size_t bytes) {
    return (160 * 1024 / bytes) < (size_t)(8 / nw) ? 160 * 1024 / bytes : (size_t)(8 / nw);
}

// Sum of a per-thread value over the workgroup in a fixed order, in fp64 (the
// temperature and beta gradients: one sum over every token, whose terms can
// cancel by orders of magnitude): a butterfly within each wave (every lane
// ends with the same value), then the waves in order.
template <int NTH> __device__ double block_sum_f64(double v, float *scratch) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    double *red = reinterpret_cast<double *>(scratch);
    if (lane_id() == 0) red[wave_id()] = v;
    __syncthreads();
    double r = 0.0;
    for (int j = 0; j < NTH / 64; ++j) r += red[j];
    __syncthreads();
    return r;
}

// state row index of (bucket s, column d)
__device__ __forceinline__ int64_t sidx(int s, int d) { return (int64_t)s * SROW + d; }

// =====================================================================
// k_fwd_reduce: per-segment (A, B) sums (fp64 over fp32 tile sums).
// =====================================================================
// Tiles are processed in groups of GT: one barrier after the group's rows are
// committed (the 4 GT projection tasks then spread over the waves) and one
// after the projections; V^T and the key weights alternate between two
// buffers so the next group's commit can start while waves still read them.
template <typename T, int SP> struct FwdReduceL {
    static constexpr int NW_ = SP / WB;
    static constexpr int GT = 2;  // tiles per barrier group
    static constexpr int LDN = NatL<T, true>::LD, LDT = ldp_of<T>(TT), LDC = ld_of<float>(NCOL);
    static constexpr size_t oK = 0;                                          // [GT][TT][LDN]
    // V tiles [2][GT]: bf16 natural rows (token operands by transpose loads,
    // col_operand), fp32 transposed [D][LDT]
    static constexpr int VTE = is_bf16<T>() ? TT * LDN : D * LDT;  // elements per tile
    static constexpr size_t oVt = align16(oK + sizeof(T) * GT * TT * LDN);
    static constexpr size_t oPl = align16(oVt + sizeof(T) * 2 * GT * VTE);
    static constexpr size_t oPlLo = align16(oPl + sizeof(T) * NCOL * LDN);
    static constexpr size_t oSig = align16(oPlLo + sizeof(T) * NCOL * LDN);  // [GT][sp, sm][TT][LDC]
    static constexpr size_t oCst = align16(oSig + sizeof(float) * GT * 2 * TT * LDC);
    static constexpr size_t oTok = align16(oCst + Consts<T>::bytes);  // key weights [2][GT][2 * TT]
    static constexpr size_t bytes = align16(oTok + sizeof(float) * 2 * GT * 2 * TT);
};

// The tile's (A, B) sums -- tot (lane: bucket 4g + e) and dB^T (d-row) --
// from the wave's token operand Pf.  In the fp32 instantiations k_bwd_out
// subtracts exactly these values (same operands, same instructions) from the
// fp64 state to walk it backwards; bf16 accumulates B in fp32 MFMA
// accumulators instead (k_fwd_reduce adds, k_bwd_out subtracts).
template <typename T>
__device__ __forceinline__ void tile_sums(const Frag<T> &Pf, const Consts<T> &cst, const T *sVt, f32x4 &tot,
                                          f32x4 (&dB)[4]) {
    constexpr int LDT = ldp_of<T>(TT);
    tot = zero4();
    mma(tot, Pf, cst.ones());
#pragma unroll
    for (int md = 0; md < 4; ++md) {
        dB[md] = zero4();
        mma(dB[md], ld_frag_pi(sVt + (16 * md + li()) * LDT), Pf);
    }
}
// bf16: the same sums from a V tile that col_operand reads (natural rows nat
// or transposed rows trn, per VL), with HL the lo part Pl of P_K added
template <class VL, bool HL>
__device__ __forceinline__ void tile_sums_bf(const Frag<bf16> &Pf, const Frag<bf16> &Pl, const Consts<bf16> &cst,
                                             const bf16 *nat, const bf16 *trn, f32x4 &tot, f32x4 (&dB)[4]) {
    tot = zero4();
    mma(tot, Pf, cst.ones());
    if constexpr (HL) mma(tot, Pl, cst.ones());
#pragma unroll
    for (int md = 0; md < 4; ++md) {
        const Frag<bf16> vo = col_operand<bf16, VL>(nat, trn, md);
        dB[md] = zero4();
        mma(dB[md], vo, Pf);
        if constexpr (HL) mma(dB[md], vo, Pl);
    }
}

template <typename T, int SP, int KB, bool AL = false>
__global__ __launch_bounds__(threads_of(SP)) void k_fwd_reduce(Args a) {
    if (a.inv_temp_ptr) a.inv_temp = *a.inv_temp_ptr;  // uniform scalar load
    using Ly = FwdReduceL<T, SP>;
    using NL = NatL<T, true>;
    constexpr bool PR = pair_tables<KB>();  // K's sigmoid rows as pair products
    using VL = TrL<T>;                      // V rows: read only by transpose loads
    static_assert(!is_bf16<T>() || TrL<T>::LD <= NatL<T, true>::LD, "V rows within the tile buffer");
    constexpr int NW_ = Ly::NW_, NTH = 64 * NW_, LDC = Ly::LDC, LDT = ldp_of<T>(TT), LDN = Ly::LDN, GT = Ly::GT;
    __shared__ __align__(16) unsigned char smem[Ly::bytes];
    T *sK = (T *)(smem + Ly::oK), *sVt0 = (T *)(smem + Ly::oVt);
    T *sPl = (T *)(smem + Ly::oPl), *sPlLo = (T *)(smem + Ly::oPlLo);
    float *sSig = (float *)(smem + Ly::oSig), *sTok0 = (float *)(smem + Ly::oTok);
    const WgPos wp = wg_pos(a.nseg, a.M * a.B * a.H, a.nslice, sliced<T, KB>());
    if (!wp.live) return;
    const int w = wave_id(), i = li(), g = lg(), sw = WB * w, z = wp.z,
              sg = z * SP + sw;
    const PlaneBlocks pbk(z, SP, KB, a.L, !sliced<T, KB>());  // projection columns of this slice

    const int n = wp.n, seg = wp.seg;
    const int m = n / (a.B * a.H);
    const int ntiles = (int)((a.T + TT - 1) / TT);  // the host bounds T by 2^35
    const int j0 = seg * a.tps, j1 = min(ntiles, j0 + a.tps);
    const int64_t send = min(a.T, (int64_t)j1 * TT);  // the segment's tokens end here (tiles past it load nothing)
    const T *kp = (const T *)a.k + stream_off(a.sk, n, a.B, a.H);
    const T *vp = (const T *)a.v + stream_off(a.sv, n, a.B, a.H);
    const float *kwp = a.kw ? a.kw + (int64_t)((n / a.H) % a.B) * a.T : nullptr;  // batch row's key weights

    Consts<T> cst;
    cst.init((T *)(smem + Ly::oCst), NTH);
    load_planes<T, NTH, NL>(a.planes + m * a.planes_m_stride, a.L * a.K, sPl, is_bf16<T>() ? sPlLo : nullptr, nullptr);
    __syncthreads();  // the constant tables in LDS; their operands to registers
    cst.cache();
    // whole-tile instantiations: each wave has at most one projection task,
    // the same column block on every tile, whose planes stay in registers
    PlaneOps<T> pcw;
    if constexpr (AL) pcw.template load<NL>(sPl, sPlLo, pbk.mc(pbk.task(w)));
    // segment sums: A in fp64; B in fp64, except in the whole-tile bf16
    // instantiations' fp32 MFMA accumulators (walk_f64).  Tile sums are added
    // tile by tile in token order.
    constexpr bool HL = hl_ops<T, SP, KB>();  // P_K as a hi + lo pair
    constexpr bool BM = is_bf16<T>() && !walk_f64<T, AL>();
    double accB[4][4], accA[4];
    f32x4 accBm[4];
    for (int e = 0; e < 4; ++e) {
        accA[e] = 0.0;
        for (int md = 0; md < 4; ++md) accB[md][e] = 0.0;
    }
    for (int md = 0; md < 4; ++md) accBm[md] = zero4();

    wait_state_loads();
    // The group's work once its rows are in LDS (K tiles; V tiles and key
    // weights in buffer b): projections, then each tile's probabilities and
    // sums.
    auto work = [&](int jg, int b) {
        const T *sVt = sVt0 + b * GT * Ly::VTE;
        const float *sTok = sTok0 + b * GT * 2 * TT;
        __syncthreads();  // the group's rows in LDS; the last group's sigmoid rows are read
        for (int q = w; q < pbk.tasks() * GT; q += NW_) {
            const int u = pbk.tensor(q), r = pbk.task(q);
            float *sp = sSig + u * 2 * TT * LDC;
            project_tile<T, NL, PR>(sK + u * TT * LDN, sPl, sPlLo, pbk.mc(r), r & 1, a.inv_temp, sp, sp + TT * LDC,
                                nullptr, (AL && q == w) ? &pcw : nullptr);
        }
        __syncthreads();  // sigmoid rows in LDS
#pragma unroll
        for (int u = 0; u < GT; ++u) {
            const int jt = jg + u;
            if (jt >= j1) break;
            const float *sp = sSig + u * 2 * TT * LDC;
            const T *vt = sVt + u * Ly::VTE;
            f32x4 PK[2];
            probs_st<KB, AL, PR>(sp, sp + TT * LDC, sg, a.S, tile_rows((int64_t)jt * TT, a.T), PK);
            if (kwp)  // P_K' = w_t P_K
                for (int nt = 0; nt < 2; ++nt) {
                    const float wt = sTok[u * 2 * TT + 16 * nt + i];
                    for (int e = 0; e < 4; ++e) PK[nt][e] *= wt;
                }
            const Frag<T> Pf = token_operand<T>(PK, cst);
            Frag<T> Pl;  // the lo part of P_K (HL)
            if constexpr (HL) {
                f32x4 R[2];
                lo_rem(PK, R);
                Pl = token_operand<T>(R, cst);
            }
            if constexpr (BM) {
                f32x4 tot = zero4();
                mma(tot, Pf, cst.ones());
                if constexpr (HL) mma(tot, Pl, cst.ones());
                for (int md = 0; md < 4; ++md) {
                    const Frag<T> vo = col_operand<T, VL>(vt, vt, md);
                    mma(accBm[md], vo, Pf);
                    if constexpr (HL) mma(accBm[md], vo, Pl);
                }
                for (int e = 0; e < 4; ++e) accA[e] += (double)tot[e];
            } else {
                f32x4 tot, dB[4];
                if constexpr (is_bf16<T>())
                    tile_sums_bf<VL, HL>(Pf, Pl, cst, vt, vt, tot, dB);
                else
                    tile_sums<T>(Pf, cst, vt, tot, dB);
                for (int e = 0; e < 4; ++e) {
                    accA[e] += (double)tot[e];
                    for (int md = 0; md < 4; ++md) accB[md][e] += (double)dB[md][e];
                }
            }
        }
    };
    constexpr bool TWO = AL && is_bf16<T>();
    if (TWO && !kwp) {
        // Whole tiles, bf16 (natural V rows), no key weights: two groups'
        // loads in flight.  Register sets A and B alternate; a set is
        // committed and at once reloaded with the group two ahead, so each
        // group's loads have two groups of work to arrive.  Every lane issues
        // the same loads each time (tiles past the segment reload its last
        // one), so the compiler's counted waits at a commit cover only the
        // older set.
        using PF = Prefetch<T, NTH, true>;
        PF ka[GT], va[GT], kb[GT], vb[GT];
        auto issue2 = [&](PF (&pk)[GT], PF (&pv)[GT], int jg) {
#pragma unroll
            for (int u = 0; u < GT; ++u) {
                const int64_t t0 = (int64_t)min(jg + u, j1 - 1) * TT;
                pk[u].issue(kp, a.sk.t, t0, send);
                pv[u].issue(vp, a.sv.t, t0, send);
            }
        };
        // K tiles are read only by the projections, which every wave has
        // finished at the previous group's second barrier; V buffer b was
        // last read by the group before last.
        auto commit2 = [&](const PF (&pk)[GT], const PF (&pv)[GT], int b) {
            T *sVt = sVt0 + b * GT * Ly::VTE;
#pragma unroll
            for (int u = 0; u < GT; ++u) {
                pk[u].template commit<NL>(sK + u * TT * LDN, nullptr);
                pv[u].template commit<VL>(sVt + u * Ly::VTE, nullptr);
            }
        };
        if (j0 < j1) {
            issue2(ka, va, j0);
            issue2(kb, vb, j0 + GT);
        }
        for (int jg = j0; jg < j1; jg += 2 * GT) {
            commit2(ka, va, 0);
            issue2(ka, va, jg + 2 * GT);
            work(jg, 0);
            commit2(kb, vb, 1);  // unconditional: the same pending sets at the loop head on every path
            issue2(kb, vb, jg + 3 * GT);
            if (jg + GT < j1) work(jg + GT, 1);
        }
    } else {
        Prefetch<T, NTH, AL> pk_[GT];
        PrefetchT<T, NTH, 1, AL, !is_bf16<T>()> pv_[GT];
        TokPre pt_[GT];
        auto issue = [&](int jg) {
#pragma unroll
            for (int u = 0; u < GT; ++u) {
                // AL loads whole tiles without row guards: a group's tile past
                // the segment reloads the segment's last tile (unused)
                const int64_t t0 = (int64_t)(AL ? min(jg + u, j1 - 1) : jg + u) * TT;
                pk_[u].issue(kp, a.sk.t, t0, send);
                pv_[u].issue(0, vp, a.sv.t, t0, send);
                if (kwp) pt_[u].issue(kwp, nullptr, t0, send);
            }
        };
        if (j0 < j1) issue(j0);
        int b = 0;
        for (int jg = j0; jg < j1; jg += GT, b ^= 1) {
            // commit the group's rows (V^T and key weights to buffer b: the
            // group before last read the other one, and its readers passed the
            // last barrier), then start the next group's loads
            T *sVt = sVt0 + b * GT * Ly::VTE;
            float *sTok = sTok0 + b * GT * 2 * TT;
            wait_vmem();
#pragma unroll
            for (int u = 0; u < GT; ++u) {
                pk_[u].template commit<NL>(sK + u * TT * LDN, nullptr);
                pv_[u].template commit<VL>(0, is_bf16<T>() ? sVt + u * Ly::VTE : nullptr,
                                           is_bf16<T>() ? nullptr : sVt + u * Ly::VTE);
                if (kwp) pt_[u].commit(sTok + u * 2 * TT);
            }
            if (jg + GT < j1) issue(jg + GT);
            work(jg, b);
        }
    }
    double *out = a.fdelta + ((int64_t)n * a.nseg + seg) * a.Spad * SROW;
    for (int md = 0; md < 4; ++md)
        for (int e = 0; e < 4; ++e)
            out[sidx(sg + i, 16 * md + 4 * g + e)] = BM ? (double)accBm[md][e] : accB[md][e];
    if (i == 0)
        for (int e = 0; e < 4; ++e) out[sidx(sg + 4 * g + e, D)] = accA[e];
}

// exclusive prefix over segments; [nseg] receives the total
// (one thread per state element of one stream, segments in order; the loads
// of SCAN_BATCH segments are issued together so that many are in flight)
constexpr int SCAN_BATCH = 16;
constexpr int SCAN_THREADS = 64;
__global__ __launch_bounds__(SCAN_THREADS) void k_fwd_scan(double *fstate, const double *fdelta, int nseg,
                                                           int elems) {
    const int n = blockIdx.y, e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= elems) return;
    const double *src = fdelta + (int64_t)n * nseg * elems + e;
    double *dst = fstate + (int64_t)n * (nseg + 1) * elems + e;
    double acc = 0.0;
    int s = 0;
    for (; s + SCAN_BATCH <= nseg; s += SCAN_BATCH) {
        double v[SCAN_BATCH];
#pragma unroll
        for (int j = 0; j < SCAN_BATCH; ++j) v[j] = src[(int64_t)(s + j) * elems];
#pragma unroll
        for (int j = 0; j < SCAN_BATCH; ++j) {
            dst[(int64_t)(s + j) * elems] = acc;
            acc += v[j];
        }
    }
    for (; s < nseg; ++s) {
        const double v = src[(int64_t)s * elems];
        dst[(int64_t)s * elems] = acc;
        acc += v;
    }
    dst[(int64_t)nseg * elems] = acc;
}

// =====================================================================
// k_fwd_out: O^T[d][t] = sum_s B[s][d] W[t][s] + sum_{t' <= t} V[t'][d] Sc[t'][t],
// Sc[t'][t] = sum_s P_K[t'][s] W[t][s].  Each wave writes its buckets' W,
// P_K and B (tile start) to LDS as [.][s] arrays, then computes output tiles
// over all buckets; the B carry of its buckets stays in registers.
// =====================================================================
template <typename T, int SP, bool CAUSAL, bool GN> struct FwdOutL {
    static constexpr int NW_ = SP / WB;
    // The Q and K tiles live inside the P_K / W region when they fit: they
    // are dead from the projection until the next tile's commit, P_K and W
    // are written after the projection and read before that commit (barriers
    // separate all four steps).  Then they also take the swizzled layout.
    static constexpr bool ALIAS = sw_ld<T, SP>() >= NatL<T, true>::LD;
    using NL = NatL<T, ALIAS>;
    static constexpr int LDN = NL::LD, LDT = ldp_of<T>(TT), LDC = ld_of<float>(NCOL), LDS_ = sw_ld<T, SP>();
    // the V tile: natural rows, its token operands read with transpose loads
    // (bf16 F1), or transposed (fp32, and the global normalisation, whose
    // registers are at the 4-waves-per-SIMD limit)
    static constexpr bool VNAT = is_bf16<T>() && !GN;
    static constexpr size_t VTB = VNAT ? sizeof(T) * TT * TrL<T>::LD : sizeof(T) * D * LDT;
    static constexpr size_t oVt = 0;
    static constexpr size_t oSig = align16(oVt + (CAUSAL ? VTB : 0));  // Q sp, Q sm, K sp, K sm
    static constexpr size_t oPts = align16(oSig + sizeof(float) * (CAUSAL ? 4 : 2) * TT * LDC);
    static constexpr size_t oWts = align16(oPts + (CAUSAL ? sizeof(T) * TT * LDS_ : 0));
    static constexpr size_t oBT = align16(oWts + sizeof(T) * TT * LDS_);
    static constexpr size_t oEnd = align16(oBT + sizeof(T) * D * LDS_);
    static constexpr size_t oQ = ALIAS ? oPts : oEnd;
    static constexpr size_t oK = align16(oQ + sizeof(T) * TT * LDN);
    static constexpr size_t oKEnd = align16(oK + (CAUSAL ? sizeof(T) * TT * LDN : 0));
    static_assert(!ALIAS || oKEnd <= oBT, "Q/K tiles must fit in the P_K / W region");
    static constexpr size_t oPl = ALIAS ? oEnd : oKEnd;
    static constexpr size_t oPlLo = align16(oPl + sizeof(T) * NCOL * LDN);
    static constexpr size_t oCst = align16(oPlLo + sizeof(T) * NCOL * LDN);
    // [NW_][TT] per-wave den shares (GN; non-causal F1 when den is requested)
    static constexpr size_t oDen = align16(oCst + Consts<T>::bytes);
    static constexpr size_t bytes1 = align16(oDen + (GN || !CAUSAL ? sizeof(float) * NW_ * TT : 0));
    // causal, when it costs no workgroup per CU (160 KiB of LDS): a second
    // transposed V tile and the tile's Sc^T [t][t'] blocks, computed once
    static constexpr size_t oVt2 = bytes1;
    static constexpr size_t oSc = align16(oVt2 + VTB);
    static constexpr size_t bytes2 = align16(oSc + sizeof(T) * TT * LDT);
    static constexpr size_t LDS_CU = 160 * 1024;
    static constexpr bool SCN = CAUSAL && LDS_CU / bytes2 >= LDS_CU / bytes1;
    static constexpr size_t bytes = SCN ? bytes2 : bytes1;
};

// Output tile (d = 16md.., t = 16nt..).  With sDen set, den is summed from
// the waves' shares (sDen [NW_][TT]) and the md == 0 tiles write it (sliced
// instantiations: this slice's den share, a partial).  GN also divides the
// tile's numerator by max(den, eps) (sliced: the numerator is the partial).
template <typename T, int SP, bool CAUSAL, bool GN = false, bool AL = false, class NL = NatL<T, true>,
          bool VNAT = is_bf16<T>()>
__device__ void fwd_out_tile(int md, int nt, const T *sBT, const T *Pts, const T *Wts, const T *sVt, T *op,
                             int64_t st, int64_t t0, int64_t Tn, T *part, const float *sDen = nullptr,
                             float *den = nullptr, float eps = 0.f) {
    constexpr int LDT = ldp_of<T>(TT);
    const int g = lg(), i = li();
    const T *pb = sw_frag_ptr<T, SP>(sBT, 16 * md + i), *pw = sw_frag_ptr<T, SP>(Wts, 16 * nt + i);
    f32x4 O = zero4();
#pragma unroll
    for (int kp = 0; kp < SP / 32; ++kp) mma(O, ld_frag(pb + 32 * kp), ld_frag(pw + 32 * kp));
    if constexpr (CAUSAL) {
        f32x4 Sc[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            Sc[mt] = zero4();
            if (mt <= nt) {
                const T *pp = sw_frag_ptr<T, SP>(Pts, 16 * mt + i);
#pragma unroll
                for (int kp = 0; kp < SP / 32; ++kp) mma(Sc[mt], ld_frag(pp + 32 * kp), ld_frag(pw + 32 * kp));
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (16 * mt + 4 * g + e > 16 * nt + i) Sc[mt][e] = 0.f;  // keep t' <= t
            }
        }
        mma(O, col_operand<T, NL, VNAT>(sVt, sVt, md), frag_acc<T>(Sc[0], Sc[1]));
    }
    const int t = 16 * nt + i;
    if (GN || !CAUSAL ? sDen != nullptr : false) {
        constexpr int NW_ = SP / WB;
        float dn = 0.f;
#pragma unroll
        for (int w = 0; w < NW_; ++w) dn += sDen[w * TT + t];
        if (GN && !part) {
            const float r = 1.0f / fmaxf(dn, eps);
#pragma unroll
            for (int e = 0; e < 4; ++e) O[e] *= r;
        }
        if (md == 0 && g == 0 && (AL || t < tile_rows(t0, Tn))) den[t0 + t] = dn;
    }
    if ((AL || t < tile_rows(t0, Tn))) {
        if (part)
            store4<T>(part_at(part, t0, t, 16 * md + 4 * g), O);
        else
            buf_st4<T>(tile_rsrc(tile_ptr(op, st, t0), st, AL ? (int64_t)TT : Tn - t0), tile_off(t, st, 16 * md + 4 * g, sizeof(T)), O);
    }
}

// Sc block r = (mt, nt) in {(0,0), (0,1), (1,1)} of Sc[t'][t] = sum_s P_K[t'][s]
// W[t][s] (the (1,0) block is zero), masked to t' <= t, stored as
// sc[t][t'] (row t, t' contiguous).
template <typename T, int SP> __device__ void sc_fwd_tile(int r, const T *Pts, const T *Wts, T *sc) {
    constexpr int LDT = ldp_of<T>(TT);
    const int g = lg(), i = li(), mt = r == 2 ? 1 : 0, nt = r == 0 ? 0 : 1;
    const T *pp = sw_frag_ptr<T, SP>(Pts, 16 * mt + i), *pw = sw_frag_ptr<T, SP>(Wts, 16 * nt + i);
    f32x4 acc = zero4();
#pragma unroll
    for (int kp = 0; kp < SP / 32; ++kp) mma(acc, ld_frag(pp + 32 * kp), ld_frag(pw + 32 * kp));
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (16 * mt + 4 * g + e > 16 * nt + i) acc[e] = 0.f;  // keep t' <= t
    store4<T>(sc + (16 * nt + i) * LDT + 16 * mt + 4 * g, acc);
}
// Output tile (md, nt) in two steps: the carried-state part W B_start, then
// the in-tile part V^T Sc from the Sc rows, the den terms and the store (as
// fwd_out_tile).
template <typename T, int SP> __device__ f32x4 fwd_out_partial(int md, int nt, const T *sBT, const T *Wts) {
    const int i = li();
    const T *pb = sw_frag_ptr<T, SP>(sBT, 16 * md + i), *pw = sw_frag_ptr<T, SP>(Wts, 16 * nt + i);
    f32x4 O = zero4();
#pragma unroll
    for (int kp = 0; kp < SP / 32; ++kp) mma(O, ld_frag(pb + 32 * kp), ld_frag(pw + 32 * kp));
    return O;
}
// Output tiles (md, 0) and (md, 1): their carried-state parts from one read
// of the B^T operand.
template <typename T, int SP> __device__ void fwd_out_partial2(int md, const T *sBT, const T *Wts, f32x4 (&O)[2]) {
    const int i = li();
    const T *pb = sw_frag_ptr<T, SP>(sBT, 16 * md + i), *pw0 = sw_frag_ptr<T, SP>(Wts, i),
            *pw1 = sw_frag_ptr<T, SP>(Wts, 16 + i);
    O[0] = zero4();
    O[1] = zero4();
#pragma unroll
    for (int kp = 0; kp < SP / 32; ++kp) {
        const Frag<T> b = ld_frag(pb + 32 * kp);
        mma(O[0], b, ld_frag(pw0 + 32 * kp));
        mma(O[1], b, ld_frag(pw1 + 32 * kp));
    }
}
template <typename T, int SP, bool GN, bool AL = false, class NL = NatL<T, true>, bool VNAT = is_bf16<T>()>
__device__ void fwd_out_final(int md, int nt, f32x4 O, const T *sVt, const T *sc, T *op, int64_t st, int64_t t0,
                              int64_t Tn, T *part, const float *sDen, float *den, float eps) {
    constexpr int LDT = ldp_of<T>(TT);
    const int g = lg(), i = li();
    mma(O, col_operand<T, NL, VNAT>(sVt, sVt, md), ld_frag_pi(sc + (16 * nt + i) * LDT));
    const int t = 16 * nt + i;
    if (GN && sDen != nullptr) {
        constexpr int NW_ = SP / WB;
        float dn = 0.f;
#pragma unroll
        for (int w = 0; w < NW_; ++w) dn += sDen[w * TT + t];
        if (!part) {
            const float r = 1.0f / fmaxf(dn, eps);
#pragma unroll
            for (int e = 0; e < 4; ++e) O[e] *= r;
        }
        if (md == 0 && g == 0 && (AL || t < tile_rows(t0, Tn))) den[t0 + t] = dn;
    }
    if ((AL || t < tile_rows(t0, Tn))) {
        if (part)
            store4<T>(part_at(part, t0, t, 16 * md + 4 * g), O);
        else
            buf_st4<T>(tile_rsrc(tile_ptr(op, st, t0), st, AL ? (int64_t)TT : Tn - t0), tile_off(t, st, 16 * md + 4 * g, sizeof(T)), O);
    }
}

// GN: global normalisation (causal only) -- W = P_Q, and the output is
// divided by den(t) = sum over all buckets of P_Q A_s(t), clamped below at eps.
template <typename T, int SP, bool CAUSAL, int KB, bool GN, bool AL = false>
__global__ __launch_bounds__(threads_of(SP), SP == 128 ? 4 : 1) void k_fwd_out(Args a) {
    if (a.inv_temp_ptr) a.inv_temp = *a.inv_temp_ptr;  // uniform scalar load
    static_assert(CAUSAL || !GN, "global normalisation is causal only");
    using Ly = FwdOutL<T, SP, CAUSAL, GN>;
    using NL = typename Ly::NL;
    constexpr bool VNAT = Ly::VNAT;
    constexpr bool PR = pair_tables<KB>();  // Q's and K's sigmoid rows as pair products
    constexpr bool HL = hl_ops<T, SP, KB>();  // P_K as a hi + lo pair
    using VL = TrL<T>;                      // V rows (VNAT): read only by transpose loads
    constexpr int NW_ = Ly::NW_, NTH = 64 * NW_, LDT = Ly::LDT, LDC = Ly::LDC, LDS_ = Ly::LDS_;
    __shared__ __align__(16) unsigned char smem[Ly::bytes];
    T *sQ = (T *)(smem + Ly::oQ), *sK = (T *)(smem + Ly::oK), *sVt = (T *)(smem + Ly::oVt);
    T *sPts = (T *)(smem + Ly::oPts), *sWts = (T *)(smem + Ly::oWts), *sBT = (T *)(smem + Ly::oBT);
    T *sPl = (T *)(smem + Ly::oPl), *sPlLo = (T *)(smem + Ly::oPlLo);
    float *sSig = (float *)(smem + Ly::oSig);
    float *sSpQ = sSig, *sSmQ = sSig + TT * LDC, *sSpK = sSig + 2 * TT * LDC, *sSmK = sSig + 3 * TT * LDC;
    const WgPos wp = wg_pos(a.nseg, a.M * a.B * a.H, a.nslice, sliced<T, KB>());
    if (!wp.live) return;
    const int w = wave_id(), g = lg(), i = li(), sw = WB * w, z = wp.z,
              sg = z * SP + sw;
    const PlaneBlocks pbk(z, SP, KB, a.L, !sliced<T, KB>());  // projection columns of this slice

    const int n = wp.n, seg = wp.seg;
    const int m = n / (a.B * a.H);
    const int ntiles = (int)((a.T + TT - 1) / TT);  // the host bounds T by 2^35
    const int lastv = (int)(a.T - (int64_t)(ntiles - 1) * TT);  // rows of the last tile
    const int j0 = seg * a.tps, j1 = min(ntiles, j0 + a.tps);
    const T *qp = (const T *)a.q + stream_off(a.sq, n, a.B, a.H);
    const T *kp = (const T *)a.k + stream_off(a.sk, n, a.B, a.H);
    const T *vp = (const T *)a.v + stream_off(a.sv, n, a.B, a.H);
    T *op = (T *)a.out + stream_off(a.so, n, a.B, a.H);
    T *opart = sliced<T, KB>() ? (T *)a.opart + ((int64_t)z * a.M * a.B * a.H + n) * a.T * D : nullptr;
    const bool want_den = GN || (!CAUSAL && a.den);
    float *sDen = want_den ? (float *)(smem + Ly::oDen) : nullptr;
    float *denp = !want_den       ? nullptr
                  : sliced<T, KB>() ? a.denpart + ((int64_t)z * a.M * a.B * a.H + n) * a.T
                                    : a.den + (int64_t)n * a.T;

    Consts<T> cst;
    cst.init((T *)(smem + Ly::oCst), NTH);
    load_planes<T, NTH, NL>(a.planes + m * a.planes_m_stride, a.L * a.K, sPl, is_bf16<T>() ? sPlLo : nullptr, nullptr);
    __syncthreads();  // the constant tables in LDS; their operands to registers
    cst.cache();
    // whole-tile instantiations: each wave has at most one projection task,
    // the same column block on every tile, whose planes stay in registers
    PlaneOps<T> pcw;
    if constexpr (AL) pcw.template load<NL>(sPl, sPlLo, pbk.mc(pbk.task(w)));
    // carried state: causal = prefix at the segment start, non-causal = totals.
    // B in bucket-row layout: lane holds B[s = sw + 4g + e][d = 16md + i]
    const double *st = a.fstate + ((int64_t)n * (a.fnseg + 1) + (CAUSAL ? seg * a.fmul : a.fnseg)) * a.Spad * SROW;
    f32x4 Bc[4];
    CarryA<T> a0[4];  // A at the tile start
    for (int e = 0; e < 4; ++e) {
        for (int md = 0; md < 4; ++md) Bc[md][e] = (float)st[sidx(sg + 4 * g + e, 16 * md + i)];
        a0[e] = (CarryA<T>)st[sidx(sg + 4 * g + e, D)];
    }
    if constexpr (!CAUSAL) store_ds<T, SP>(sBT, sw, Bc);  // constant totals

    wait_state_loads();
    Prefetch<T, NTH, AL> pq_, pk_;
    // V: plain rows read by transpose loads (VNAT; staged row by row, 16
    // lanes per row, conflict-free) or transposed rows
    std::conditional_t<VNAT, Prefetch<T, NTH, AL>, PrefetchT<T, NTH, 1, AL, true>> pv_;
    auto v_issue = [&](int64_t t0) {
        if constexpr (VNAT)
            pv_.issue(vp, a.sv.t, t0, a.T);
        else
            pv_.issue(0, vp, a.sv.t, t0, a.T);
    };
    auto v_commit = [&](T *buf) {
        if constexpr (VNAT)
            pv_.template commit<VL>(buf, nullptr);
        else
            pv_.template commit<NL>(0, nullptr, buf);
    };
    if (j0 < j1) {
        pq_.issue(qp, a.sq.t, (int64_t)j0 * TT, a.T);
        if constexpr (CAUSAL) {
            pk_.issue(kp, a.sk.t, (int64_t)j0 * TT, a.T);
            v_issue((int64_t)j0 * TT);
        }
    }
    if constexpr (Ly::SCN) {
        // Per tile: commit barrier, projections, barrier, probabilities and
        // rows, barrier, Sc blocks and the carried-state part of O, barrier,
        // then the next tile's rows (Q/K alias the P_K / W rows, now read;
        // V^T goes to the other buffer) and the rest of O.
        // Whole 4-bit tiles (QKP; F1 and the global normalisation): every
        // wave's planes are in registers, so Q and K take the planes' rows
        // instead (same layout and size: NCOL = TT rows).  The next tile's rows are then committed in the third
        // phase (this tile's projections are done by then), and the next
        // tile's projections run at the end of the last phase, after the
        // output tiles: three barriers per tile (probabilities and rows,
        // barrier, Sc blocks, carried-state part of O and the next rows'
        // commit, barrier, the rest of O and the next projections, barrier).
        constexpr bool QKP = AL && KB == 4;
        static_assert(NCOL == TT, "Q and K rows in the planes' rows");
        if constexpr (QKP) {
            sQ = sPl;
            sK = sPlLo;
            __syncthreads();  // every wave has read its planes
        }
        T *sSc = (T *)(smem + Ly::oSc);
        zero_lds<T>(sSc, TT * LDT, NTH);  // its (t < 16 <= t') block stays zero
        auto vt_of = [&](int j) { return (T *)(smem + ((j & 1) ? Ly::oVt2 : Ly::oVt)); };
        auto commit = [&](int j) {  // the prefetched rows, V^T to the buffer of tile j
            wait_vmem();
            pq_.template commit<NL>(sQ, nullptr);
            pk_.template commit<NL>(sK, nullptr);
            v_commit(vt_of(j));
        };
        // The rows of tile j + 1 are loaded from the commit of tile j on
        // (the registers are free then), a tile and a phase ahead of their
        // own commit.  The last tile's commit writes rows nobody reads.
        auto issue = [&](int j) {
            const int64_t tn = (int64_t)min(j, j1 - 1) * TT;
            pq_.issue(qp, a.sq.t, tn, a.T);
            pk_.issue(kp, a.sk.t, tn, a.T);
            v_issue(tn);
        };
        if (j0 < j1) {
            commit(j0);
            issue(j0 + 1);
        }
        // whole tiles: at most one projection task per wave (Q first), one code path
        auto project_al = [&]() {
            if (2 * pbk.tasks() >= NW_ || w < 2 * pbk.tasks()) {
                const bool isq = w < pbk.tasks();
                const int r = pbk.task(w);
                project_tile<T, NL, PR>(isq ? sQ : sK, sPl, sPlLo, pbk.mc(r), r & 1, a.inv_temp, isq ? sSpQ : sSpK,
                                        isq ? sSmQ : sSmK, nullptr, &pcw);
            }
        };
        if constexpr (QKP) {
            __syncthreads();  // the first tile's rows in LDS
            project_al();
        }
        constexpr int NQ = (8 + NW_ - 1) / NW_;  // output tiles per wave
        // 8 waves: half of them take two output tiles each (fewer LDS operand
        // reads), for the output and for the slices' partials alike
        constexpr bool OPAIR = NW_ == 8;
        for (int jt = j0; jt < j1; ++jt) {
            const int64_t t0 = (int64_t)jt * TT;
            sVt = vt_of(jt);
            if constexpr (QKP) {
                // this tile's projections ran at the end of the last tile (or before the loop)
            } else if constexpr (AL) {
                __syncthreads();  // this tile's rows in LDS; the previous tile's O rows are done
                project_al();
            } else {
                __syncthreads();
                for (int q = w; q < 2 * pbk.tasks(); q += NW_) {
                    const int r = pbk.task(q);
                    if (q < pbk.tasks())
                        project_tile<T, NL, PR>(sQ, sPl, sPlLo, pbk.mc(r), r & 1, a.inv_temp, sSpQ, sSmQ, nullptr,
                                                (AL && q == w) ? &pcw : nullptr);
                    else
                        project_tile<T, NL, PR>(sK, sPl, sPlLo, pbk.mc(r), r & 1, a.inv_temp, sSpK, sSmK, nullptr,
                                                (AL && q == w) ? &pcw : nullptr);
                }
            }
            __syncthreads();
            f32x4 PQ[2], PK[2], Acum[2], W[2], tot;
            Frag<T> Pf, Pl;  // Pl: the lo part of P_K (HL)
            probs_st<KB, AL, PR>(sSpQ, sSmQ, sg, a.S, jt + 1 < ntiles ? TT : lastv, PQ);
            if constexpr (CAUSAL) {
                probs_st<KB, AL, PR>(sSpK, sSmK, sg, a.S, jt + 1 < ntiles ? TT : lastv, PK);
                Pf = store_ts_operand<T, SP>(sPts, sw, PK, cst);
                if constexpr (HL) {
                    f32x4 R[2];
                    lo_rem(PK, R);
                    Pl = token_operand<T>(R, cst);
                }
                for (int nt = 0; nt < 2; ++nt) {
                    Acum[nt] = zero4();
                    mma(Acum[nt], Pf, cst.tri_op(nt));
                    if constexpr (HL) mma(Acum[nt], Pl, cst.tri_op(nt));
                }
                tot = zero4();
                mma(tot, Pf, cst.ones());
                if constexpr (HL) mma(tot, Pl, cst.ones());
            }
            if constexpr (GN) {
                // W = P_Q; this wave's share of den(t) = sum_s P_Q A_s(t)
                for (int nt = 0; nt < 2; ++nt) {
                    float dp = 0.f;
                    for (int e = 0; e < 4; ++e) {
                        dp += PQ[nt][e] * ((float)a0[e] + Acum[nt][e]);
                        W[nt][e] = PQ[nt][e];
                    }
                    dp = xor32_sum(xor16_sum(dp));
                    if (g == 0) sDen[w * TT + 16 * nt + i] = dp;
                }
            } else {
                // W = P_Q / (A(t) + eps)
                float ae[4];
                for (int e = 0; e < 4; ++e) ae[e] = (float)a0[e] + a.eps;
                for (int nt = 0; nt < 2; ++nt)
                    for (int e = 0; e < 4; ++e) W[nt][e] = PQ[nt][e] * rcp(CAUSAL ? ae[e] + Acum[nt][e] : ae[e]);
                if constexpr (!CAUSAL) {
                    if (want_den)  // this wave's share of den(t) = sum_s P_Q A_s
                        for (int nt = 0; nt < 2; ++nt) {
                            float dp = 0.f;
                            for (int e = 0; e < 4; ++e) dp += PQ[nt][e] * (float)a0[e];
                            dp = xor32_sum(xor16_sum(dp));
                            if (g == 0) sDen[w * TT + 16 * nt + i] = dp;
                        }
                }
            }
            store_ts<T, SP>(sWts, sw, W);
            store_ds<T, SP>(sBT, sw, Bc);
            __syncthreads();
            f32x4 Op[NQ > 2 ? NQ : 2];
            if constexpr (OPAIR) {
                // waves 0-3: the output tiles (md = w, nt = 0, 1), one B^T
                // operand for both; waves 4-6: the Sc blocks
                if (w < 4) fwd_out_partial2<T, SP>(w, sBT, sWts, Op);
                else if (w < 7) sc_fwd_tile<T, SP>(w - 4, sPts, sWts, sSc);
            } else {
                for (int r = w; r < 3; r += NW_) sc_fwd_tile<T, SP>(r, sPts, sWts, sSc);
#pragma unroll
                for (int k = 0; k < NQ; ++k)
                    if (w + k * NW_ < 8) Op[k] = fwd_out_partial<T, SP>((w + k * NW_) >> 1, (w + k * NW_) & 1, sBT, sWts);
            }
            // carry: B[s][d] += sum_t P_K[t][s] V[t][d]
            for (int md = 0; md < 4; ++md) {
                const Frag<T> vo = col_operand<T, VL, VNAT>(sVt, sVt, md);
                mma(Bc[md], Pf, vo);
                if constexpr (HL) mma(Bc[md], Pl, vo);
            }
            for (int e = 0; e < 4; ++e) a0[e] += (CarryA<T>)tot[e];
            if constexpr (QKP) commit(jt + 1);  // Q/K rows read by this tile's projections before the second barrier
            __syncthreads();  // Sc rows in LDS; the P_K / W / B rows are read
            if constexpr (!QKP) commit(jt + 1);
            if (jt + 2 < j1) issue(jt + 2);
            if constexpr (OPAIR) {
                if (w < 4)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt)
                        fwd_out_final<T, SP, GN, AL, VL, VNAT>(w, nt, Op[nt], sVt, sSc, op, a.so.t, t0, a.T, opart, sDen,
                                                               denp, a.eps);
                if constexpr (QKP)
                    if (jt + 1 < j1) project_al();  // the next tile's rows, committed before the last barrier
            } else {
#pragma unroll
                for (int k = 0; k < NQ; ++k) {
                    const int q = w + k * NW_;
                    if (q < 8)
                        fwd_out_final<T, SP, GN, AL, VL, VNAT>(q >> 1, q & 1, Op[k], sVt, sSc, op, a.so.t, t0, a.T, opart,
                                                               sDen, denp, a.eps);
                }
            }
        }
        return;
    }
    for (int jt = j0; jt < j1; ++jt) {
        const int64_t t0 = (int64_t)jt * TT;
        __syncthreads();  // previous tile's readers of sVt / sPts / sWts / sBT are done
        pq_.template commit<NL>(sQ, nullptr);
        if constexpr (CAUSAL) {
            pk_.template commit<NL>(sK, nullptr);
            v_commit(sVt);
        }
        if (jt + 1 < j1) {
            pq_.issue(qp, a.sq.t, t0 + TT, a.T);
            if constexpr (CAUSAL) {
                pk_.issue(kp, a.sk.t, t0 + TT, a.T);
                v_issue(t0 + TT);
            }
        }
        __syncthreads();
        for (int q = w; q < (CAUSAL ? 2 : 1) * pbk.tasks(); q += NW_) {
            const int r = pbk.task(q);
            if (q < pbk.tasks())
                project_tile<T, NL, PR>(sQ, sPl, sPlLo, pbk.mc(r), r & 1, a.inv_temp, sSpQ, sSmQ, nullptr,
                                    (AL && q == w) ? &pcw : nullptr);
            else
                project_tile<T, NL, PR>(sK, sPl, sPlLo, pbk.mc(r), r & 1, a.inv_temp, sSpK, sSmK, nullptr,
                                    (AL && q == w) ? &pcw : nullptr);
        }
        __syncthreads();
        f32x4 PQ[2], PK[2], Acum[2], W[2], tot;
        Frag<T> Pf, Pl;  // Pl: the lo part of P_K (HL)
        probs_st<KB, AL, PR>(sSpQ, sSmQ, sg, a.S, jt + 1 < ntiles ? TT : lastv, PQ);
        if constexpr (CAUSAL) {
            probs_st<KB, AL, PR>(sSpK, sSmK, sg, a.S, jt + 1 < ntiles ? TT : lastv, PK);
            if constexpr (HL) {
                f32x4 R[2];
                lo_rem(PK, R);
                Pl = token_operand<T>(R, cst);
            }
            for (int nt = 0; nt < 2; ++nt)
                for (int e = 0; e < 4; ++e) PK[nt][e] = as_operand<T>(PK[nt][e]);
            Pf = token_operand<T>(PK, cst);
            for (int nt = 0; nt < 2; ++nt) {
                Acum[nt] = zero4();
                mma(Acum[nt], Pf, cst.tri_op(nt));
                if constexpr (HL) mma(Acum[nt], Pl, cst.tri_op(nt));
            }
            tot = zero4();
            mma(tot, Pf, cst.ones());
            if constexpr (HL) mma(tot, Pl, cst.ones());
        }
        if constexpr (GN) {
            // W = P_Q; this wave's share of den(t) = sum_s P_Q A_s(t)
            for (int nt = 0; nt < 2; ++nt) {
                float dp = 0.f;
                for (int e = 0; e < 4; ++e) {
                    dp += PQ[nt][e] * ((float)a0[e] + Acum[nt][e]);
                    W[nt][e] = PQ[nt][e];
                }
                dp = xor32_sum(xor16_sum(dp));
                if (g == 0) sDen[w * TT + 16 * nt + i] = dp;
            }
        } else {
            // W = P_Q / (A(t) + eps)
            float ae[4];
            for (int e = 0; e < 4; ++e) ae[e] = (float)a0[e] + a.eps;
            for (int nt = 0; nt < 2; ++nt)
                for (int e = 0; e < 4; ++e) W[nt][e] = PQ[nt][e] * rcp(CAUSAL ? ae[e] + Acum[nt][e] : ae[e]);
            if constexpr (!CAUSAL) {
                if (want_den)  // this wave's share of den(t) = sum_s P_Q A_s
                    for (int nt = 0; nt < 2; ++nt) {
                        float dp = 0.f;
                        for (int e = 0; e < 4; ++e) dp += PQ[nt][e] * (float)a0[e];
                        dp = xor32_sum(xor16_sum(dp));
                        if (g == 0) sDen[w * TT + 16 * nt + i] = dp;
                    }
            }
        }
        store_ts<T, SP>(sWts, sw, W);
        if constexpr (CAUSAL) {
            store_ts<T, SP>(sPts, sw, PK);
            store_ds<T, SP>(sBT, sw, Bc);
        }
        __syncthreads();
        for (int q = w; q < 8; q += NW_)
            fwd_out_tile<T, SP, CAUSAL, GN, AL, VL, VNAT>(q >> 1, q & 1, sBT, sPts, sWts, sVt, op, a.so.t, t0, a.T, opart, sDen,
                                            denp, a.eps);
        if constexpr (CAUSAL) {
            // carry: B[s][d] += sum_t P_K[t][s] V[t][d]
            for (int md = 0; md < 4; ++md) {
                const Frag<T> vo = col_operand<T, VL, VNAT>(sVt, sVt, md);
                mma(Bc[md], Pf, vo);
                if constexpr (HL) mma(Bc[md], Pl, vo);
            }
            for (int e = 0; e < 4; ++e) a0[e] += (CarryA<T>)tot[e];
        }
    }
}

// =====================================================================
// k_bwd_reduce: forward walk.  dQ, and per-segment sums of
// alpha = sum_t dA and U = sum_t W^T g.
// =====================================================================
// GN: gd = dL/d den per token is formed from the kernels' own sums,
//   gd = dden - [den >= eps] rd^2 S_t,   S_t = sum_s P_Q[t][s] G[s][t]
// (S_t = dO . num in exact arithmetic; the stored output is not read).
// dP_Q = G rd + gd A then has sum_s P_Q dP_Q = dden den to fp32 rounding, as
// the exact gradient has, so a token whose keys all carry one value (t = 0:
// out = v_0, exact dq = 0 without dden) gets no gradient from the roundings
// of O, of P_K or of the in-tile v.g products -- which do not cancel where
// den is small, and there outweigh the true gradient.  The in-tile products
// enter G rounded to bf16 exactly as k_bwd_out's in-tile dP_K term takes
// them (the same MFMA, the same rounding), so its t = tau terms, alpha's
// gd P_Q against W v.g, cancel as well.
// With every bucket of the stream in one workgroup (bf16, K <= 4: GC) the
// kernel sums S_t itself, over its waves, after the tile's G.  Bucket slices
// (GS) take it from a pre-pass: the same kernel with GP set walks the tiles
// as far as G and writes its slice's share of S_t; k_gn_terms adds the
// shares and writes rd and gd per token for the second pass and k_bwd_out.
template <typename T, int KB> __host__ __device__ constexpr bool gn_own_gd() { return !sliced<T, KB>(); }

template <typename T, int SP, bool CAUSAL, int KB, bool GN> struct BwdReduceL {
    static constexpr int NW_ = SP / WB;
    static constexpr int LDN = NatL<T, true>::LD, LDT = ldp_of<T>(TT), LDC = ld_of<float>(NCOL), LDDP = sw_ld<T, NCOL>();
    static constexpr bool GS = GN && !gn_own_gd<T, KB>();  // gd per token from k_gn_terms
    static constexpr bool GC = GN && gn_own_gd<T, KB>();   // gd from this kernel's own sums
    // token block: one tile's staged rows (Q, K, V, dO natural; V, dO
    // transposed; GN: (den, dden) [2][TT], GS (den, gd); non-causal: dden [TT])
    static constexpr size_t oQ = 0;
    static constexpr size_t oK = align16(oQ + sizeof(T) * TT * LDN);
    static constexpr size_t oV = align16(oK + (CAUSAL ? sizeof(T) * TT * LDN : 0));
    static constexpr size_t oG = align16(oV + (CAUSAL ? sizeof(T) * TT * LDN : 0));
    static constexpr size_t oVt = align16(oG + sizeof(T) * TT * LDN);
    static constexpr size_t oGt = align16(oVt + (CAUSAL ? sizeof(T) * D * LDT : 0));
    static constexpr size_t oTokIn = align16(oGt + sizeof(T) * D * LDT);
    static constexpr size_t TB = align16(oTokIn + (GN || !CAUSAL ? sizeof(float) * 2 * TT : 0));
    // the rest, relative to its start
    static constexpr size_t rX = 0;  // (the in-tile v.g^T blocks live in each wave's registers)
    static constexpr size_t rDproj = rX;
    static constexpr size_t rPl = align16(rDproj + sizeof(T) * TT * LDDP);
    static constexpr size_t rPlLo = align16(rPl + sizeof(T) * NCOL * LDN);
    static constexpr size_t rPlT = align16(rPlLo + sizeof(T) * NCOL * LDN);
    static constexpr size_t rSig = align16(rPlT + sizeof(T) * D * LDDP);  // Q sp, Q sm, Q th, K sp, K sm
    static constexpr size_t rRed = align16(rSig + sizeof(float) * 5 * TT * LDC);
    static constexpr size_t rCst = align16(rRed + sizeof(float) * 64 * NW_);
    static constexpr size_t rHash = align16(rCst + Consts<T>::bytes);
    static constexpr size_t rPair = align16(rHash + HashOps<T, 4>::bytes);
    static constexpr size_t rShare = align16(rPair + PairOps<T>::bytes);
    static constexpr size_t rTok = align16(rShare + (KB > 4 ? WideHash<T, KB>::bytes(NW_) : 0));
    // GN (GC, and GS's pre-pass): the waves' shares of sum_s P_Q G [NW_][TT]
    static constexpr size_t rGs = rTok;
    static constexpr size_t rEnd = align16(rGs + (GN ? sizeof(float) * NW_ * TT : 0));
    // two token blocks when they cost no workgroup per CU (160 KiB of LDS):
    // the next tile's rows then go to the other block while this tile still
    // reads its own, and the barrier ahead of that commit goes away
    static constexpr size_t LDS_CU = 160 * 1024;
    static constexpr int NB = bwd_wgs_per_cu(NW_, 2 * TB + rEnd) >= bwd_wgs_per_cu(NW_, TB + rEnd) ? 2 : 1;
    static constexpr size_t R0 = NB * TB;
    static constexpr size_t oX = R0 + rX, oDproj = R0 + rDproj, oPl = R0 + rPl, oPlLo = R0 + rPlLo, oPlT = R0 + rPlT,
                            oSig = R0 + rSig, oRed = R0 + rRed, oCst = R0 + rCst, oHash = R0 + rHash, oPair = R0 + rPair,
                            oShare = R0 + rShare, oGs = R0 + rGs;
    static constexpr size_t bytes = R0 + rEnd;
};

// GN (global normalisation, causal only): with rd = 1/max(den, eps) and
// gd = dL/d den per token (GC: from sum_s P_Q G after the tile's G; GS: read,
// as k_gn_terms wrote it from GP's shares), W = P_Q rd, dP_Q = G rd + gd A_s(t),
// dA = gd P_Q.  GP: the GS pre-pass, which writes this slice's share of
// sum_s P_Q G per token (gsum) and nothing else.
template <typename T, int SP, bool CAUSAL, int KB, bool GN, bool AL = false, bool GP = false>
__global__ __launch_bounds__(threads_of(SP), 2) void k_bwd_reduce(Args a) {
    if (a.inv_temp_ptr) a.inv_temp = *a.inv_temp_ptr;  // uniform scalar load
    static_assert(CAUSAL || !GN, "global normalisation is causal only");
    using Ly = BwdReduceL<T, SP, CAUSAL, KB, GN>;
    using NL = NatL<T, true>;
    // K's sigmoid rows as pair products, as in the forward kernels (the walk of
    // the forward state needs the same P_K); Q's stay corner pairs, which its
    // softmax backward reads directly
    constexpr bool PR = pair_tables<KB>();
    constexpr bool HL = hl_ops<T, SP, KB>();  // P_K and W as hi + lo pairs
    constexpr bool GS = Ly::GS, GC = Ly::GC;   // GN: gd read per token / from this kernel's sums
    static_assert(!GP || GS, "the pre-pass is the bucket-slice instantiations'");
    constexpr int NW_ = Ly::NW_, NTH = 64 * NW_, LDN = Ly::LDN, LDT = Ly::LDT, LDC = Ly::LDC, LDDP = Ly::LDDP;
    __shared__ __align__(16) unsigned char smem[Ly::bytes];
    // this tile's token block (block jt & 1 of two; block 0 of one)
    T *sQ, *sK, *sV, *sG, *sVt, *sGt;
    float *sTokIn;
    auto use_block = [&](int b) {
        unsigned char *tb = smem + b * Ly::TB;
        sQ = (T *)(tb + Ly::oQ);
        sK = (T *)(tb + Ly::oK);
        sV = (T *)(tb + Ly::oV);
        sG = (T *)(tb + Ly::oG);
        sVt = (T *)(tb + Ly::oVt);
        sGt = (T *)(tb + Ly::oGt);
        sTokIn = (float *)(tb + Ly::oTokIn);
    };
    T *sDproj = (T *)(smem + Ly::oDproj);
    T *sPl = (T *)(smem + Ly::oPl), *sPlLo = (T *)(smem + Ly::oPlLo), *sPlT = (T *)(smem + Ly::oPlT);
    float *sSig = (float *)(smem + Ly::oSig), *sRed = (float *)(smem + Ly::oRed);
    float *sSpQ = sSig, *sSmQ = sSig + TT * LDC, *sThQ = sSig + 2 * TT * LDC;
    float *sSpK = sSig + 3 * TT * LDC, *sSmK = sSig + 4 * TT * LDC;
    const WgPos wp = wg_pos(a.nseg, a.M * a.B * a.H, a.nslice, sliced<T, KB>());
    if (!wp.live) return;
    const int w = wave_id(), g = lg(), i = li(), sw = WB * w, z = wp.z,
              sg = z * SP + sw;
    const PlaneBlocks pbk(z, SP, KB, a.L, !sliced<T, KB>());  // projection columns of this slice

    const int n = wp.n, seg = wp.seg;
    const int m = n / (a.B * a.H);
    const int ntiles = (int)((a.T + TT - 1) / TT);  // the host bounds T by 2^35
    const int lastv = (int)(a.T - (int64_t)(ntiles - 1) * TT);  // rows of the last tile
    const int j0 = seg * a.tps, j1 = min(ntiles, j0 + a.tps);
    const T *qp = (const T *)a.q + stream_off(a.sq, n, a.B, a.H);
    const T *kp = (const T *)a.k + stream_off(a.sk, n, a.B, a.H);
    const T *vp = (const T *)a.v + stream_off(a.sv, n, a.B, a.H);
    const T *gp = (const T *)a.dout + stream_off(a.sdo, n, a.B, a.H);
    T *dqp = (T *)a.dq + stream_off(a.sg, n, a.B, a.H);
    constexpr int XC = xcols_of(SP, KB);
    constexpr bool XF = xpart_f32(is_bf16<T>(), SP, KB);
    void *xpart = sliced<T, KB>() ? xpart_at<T, SP, KB>(a.dqpart, z, n, a) : nullptr;
    const int xc0 = ((z * SP) >> KB) * KB;  // first projection column of the slice's tables
    float *sGs = (float *)(smem + Ly::oGs);
    const float *denp = GN ? a.den + (int64_t)n * a.T : nullptr;
    // the second token row: dden (GS: gd, from k_gn_terms)
    const float *ddp = GS && !GP       ? a.gden + (int64_t)n * a.T
                       : (GN || !CAUSAL) && a.dden ? a.dden + (int64_t)n * a.T
                                                   : nullptr;
    float *gsp = GP ? a.gsum + ((int64_t)z * a.M * a.B * a.H + n) * a.T : nullptr;
    // GC writes the per-token terms for k_bwd_out (GS: k_gn_terms does)
    float *rdw = GC ? a.rden + (int64_t)n * a.T : nullptr;
    float *gdw = GC ? a.gden + (int64_t)n * a.T : nullptr;

    Consts<T> cst;
    cst.init((T *)(smem + Ly::oCst), NTH);
    HashOps<T, KB> ho;
    WideHash<T, KB> wh;
    float *sShare = (float *)(smem + Ly::oShare);
    if constexpr (KB <= 4)
        ho.init((T *)(smem + Ly::oHash), NTH);
    else
        wh.init(sg);
    PairOps<T> po;
    po.init((T *)(smem + Ly::oPair), NTH);
    load_planes<T, NTH, NL>(a.planes + m * a.planes_m_stride, a.L * a.K, sPl, is_bf16<T>() ? sPlLo : nullptr, sPlT);
    zero_lds<T>(sDproj, TT * LDDP, NTH);
    __syncthreads();  // the constant tables in LDS; their operands to registers
    cst.cache();
    if constexpr (KB <= 4) ho.cache();
    po.cache();
    // whole-tile instantiations: each wave has at most one projection task,
    // the same column block on every tile, whose planes stay in registers
    PlaneOps<T> pcw;
    if constexpr (AL) pcw.template load<NL>(sPl, sPlLo, pbk.mc(pbk.task(w)));
    // forward state in d-row layout: lane holds B^T[d = 16md + 4g + e][s = sw + i]
    const double *st = a.fstate + ((int64_t)n * (a.fnseg + 1) + (CAUSAL ? seg * a.fmul : a.fnseg)) * a.Spad * SROW;
    f32x4 Bt[4], Ut[4];
    CarryA<T> a0[4];  // A at the tile start
    double al[4];
    for (int md = 0; md < 4; ++md) {
        Ut[md] = zero4();
        for (int e = 0; e < 4; ++e) Bt[md][e] = (float)st[sidx(sg + i, 16 * md + 4 * g + e)];
    }
    for (int e = 0; e < 4; ++e) {
        a0[e] = (CarryA<T>)st[sidx(sg + 4 * g + e, D)];
        al[e] = 0.0;
    }
    CarryA<T> tsum = 0;  // this thread's share of sum du * th

    wait_state_loads();
    constexpr int NP = CAUSAL ? 2 : 1;  // transposed tiles: dO (and V)
    Prefetch<T, NTH, AL> pq_, pk_;
    PrefetchT<T, NTH, NP, AL> pg_;  // non-causal dO
    PrefetchT2<T, NTH, AL, !is_bf16<T>()> pgv_;  // causal dO (first half of the waves) and V
    TokPre pt_;
    // Writes the prefetched rows to token block b.
    auto commit = [&](int b) {
        unsigned char *tb = smem + b * Ly::TB;
        float *tin = (float *)(tb + Ly::oTokIn);
        wait_vmem();
        pq_.template commit<NL>((T *)(tb + Ly::oQ), nullptr);
        if constexpr (CAUSAL) {
            pk_.template commit<NL>((T *)(tb + Ly::oK), nullptr);
            pgv_.template commit<NL>((T *)(tb + Ly::oG), (T *)(tb + Ly::oGt), (T *)(tb + Ly::oV), (T *)(tb + Ly::oVt));
        } else {
            pg_.template commit<NL>(0, (T *)(tb + Ly::oG), (T *)(tb + Ly::oGt));
        }
        if constexpr (GN) {
            pt_.commit(tin);
        } else if constexpr (!CAUSAL) {
            if (ddp) pt_.commit(tin);
        }
    };
    constexpr int NB = Ly::NB;
    if (j0 < j1) {
        pq_.issue(qp, a.sq.t, (int64_t)j0 * TT, a.T);
        if constexpr (CAUSAL) {
            pk_.issue(kp, a.sk.t, (int64_t)j0 * TT, a.T);
            pgv_.issue(gp, a.sdo.t, vp, a.sv.t, (int64_t)j0 * TT, a.T);
        } else {
            pg_.issue(0, gp, a.sdo.t, (int64_t)j0 * TT, a.T);
        }
        if constexpr (GN) {
            pt_.issue(denp, ddp, (int64_t)j0 * TT, a.T);
        } else if constexpr (!CAUSAL) {
            if (ddp) pt_.issue(ddp, nullptr, (int64_t)j0 * TT, a.T);
        }
        commit(NB == 2 ? (int)(j0 & 1) : 0);
    }
    for (int jt = j0; jt < j1; ++jt) {
        const int64_t t0 = (int64_t)jt * TT;
        use_block(NB == 2 ? (int)(jt & 1) : 0);
        // next tile's rows; the last tile reloads itself (loads stay in range).
        // Issue and commit run every iteration: a commit under a condition
        // leaves the prefetch registers possibly pending at the loop head, and
        // the wait placed there also waits for the previous tile's stores.
        const int64_t tn = (int64_t)(jt + 1 < j1 ? jt + 1 : jt) * TT;
        auto issue = [&]() {
            pq_.issue(qp, a.sq.t, tn, a.T);
            if constexpr (CAUSAL) {
                pk_.issue(kp, a.sk.t, tn, a.T);
                pgv_.issue(gp, a.sdo.t, vp, a.sv.t, tn, a.T);
            } else {
                pg_.issue(0, gp, a.sdo.t, tn, a.T);
            }
            if constexpr (GN) {
                pt_.issue(denp, ddp, tn, a.T);
            } else if constexpr (!CAUSAL) {
                if (ddp) pt_.issue(ddp, nullptr, tn, a.T);
            }
        };
        // one token block: loads issued ahead of the barrier; two: after it,
        // with the previous tile's dQ stores issued next, so that both have
        // the whole tile to complete before the commit's wait at its end
        if constexpr (NB == 1) issue();
        __syncthreads();
        if constexpr (NB == 2) {
            issue();
            if constexpr (!GP)
                if (jt > j0) dx_store<T, NW_, XC, AL, XF>(sDproj, sPlT, dqp, a.sg.t, t0 - TT, a.T, xpart, xc0);
        }
        for (int q = w; q < (CAUSAL ? 2 : 1) * pbk.tasks(); q += NW_) {
            const int r = pbk.task(q);
            if (q < pbk.tasks())
                project_tile<T, NL>(sQ, sPl, sPlLo, pbk.mc(r), r & 1, a.inv_temp, sSpQ, sSmQ, GP ? nullptr : sThQ,
                                    (AL && q == w) ? &pcw : nullptr);
            else
                project_tile<T, NL, PR>(sK, sPl, sPlLo, pbk.mc(r), r & 1, a.inv_temp, sSpK, sSmK, nullptr,
                                    (AL && q == w) ? &pcw : nullptr);
        }
        // one token block: dQ of the previous tile, from the dproj rows its
        // softmax backward left in LDS, after the projections (they overlap);
        // the next write of sDproj is a barrier away
        if constexpr (NB == 1 && !GP)
            if (jt > j0) dx_store<T, NW_, XC, AL, XF>(sDproj, sPlT, dqp, a.sg.t, t0 - TT, a.T, xpart, xc0);
        __syncthreads();
        f32x4 PQ[2], PK[2], Acum[2], W[2], inv[2], tot;
        Frag<T> Pf, Pl;  // Pl: the lo part of P_K (HL)
        probs_st<KB, AL>(sSpQ, sSmQ, sg, a.S, jt + 1 < ntiles ? TT : lastv, PQ);
        if constexpr (CAUSAL) {
            probs_st<KB, AL, PR>(sSpK, sSmK, sg, a.S, jt + 1 < ntiles ? TT : lastv, PK);
            Pf = token_operand<T>(PK, cst, po);
            if constexpr (HL) {
                f32x4 R[2];
                lo_rem(PK, R);
                Pl = token_operand<T>(R, cst, po);
            }
            for (int nt = 0; nt < 2; ++nt) {
                Acum[nt] = zero4();
                mma(Acum[nt], Pf, cst.tri_op(nt));
                if constexpr (HL) mma(Acum[nt], Pl, cst.tri_op(nt));
            }
            tot = zero4();
            mma(tot, Pf, cst.ones());
            if constexpr (HL) mma(tot, Pl, cst.ones());
        }
        f32x4 Ag[2];  // GN: A_s(t)
        float rd[2], gd[2], ae[4];  // ae: A at the tile start (+ eps unless GN)
        for (int e = 0; e < 4; ++e) ae[e] = GN ? (float)a0[e] : (float)a0[e] + a.eps;
        for (int nt = 0; nt < 2; ++nt) {
            if constexpr (GN) rd[nt] = 1.0f / fmaxf(sTokIn[16 * nt + i], a.eps);
            if constexpr (GS) gd[nt] = sTokIn[TT + 16 * nt + i];
            for (int e = 0; e < 4; ++e) {
                const float A = CAUSAL ? ae[e] + Acum[nt][e] : ae[e];
                if constexpr (GN) {
                    Ag[nt][e] = A;
                    inv[nt][e] = rd[nt];
                } else {
                    inv[nt][e] = rcp(A);
                }
                W[nt][e] = PQ[nt][e] * inv[nt][e];
            }
        }
        const Frag<T> Wf = token_operand<T>(W, cst, po);
        Frag<T> Wl;  // the lo part of W (HL)
        if constexpr (HL) {
            f32x4 R[2];
            lo_rem(W, R);
            Wl = token_operand<T>(R, cst, po);
        }
        // G[s][t] = g_t . B_s(t) = sum_d B[s][d] g[t][d] + sum_{tau<=t} P_K[tau][s] M[tau][t]
        f32x4 dPQ[2], dA[2], Gv[2];  // Gv: G, kept for GC's gd
        {
            // The carried B enters G as an fp32-accurate operand pair (hi + lo, for bf16): with values
            // of non-zero mean, B_s carries a component common to all buckets that the softmax
            // backward of dQ cancels, so a one-part bf16 B would put 2^-9 of that component into dQ.
            Frag<T> b0, b1, b0l, b1l;
            if constexpr (is_bf16<T>()) {
                frag_acc_hilo(Bt[0], Bt[1], b0, b0l);
                frag_acc_hilo(Bt[2], Bt[3], b1, b1l);
            } else {
                b0 = frag_acc<T>(Bt[0], Bt[1]);
                b1 = frag_acc<T>(Bt[2], Bt[3]);
            }
            Frag<T> Xop[2];
            if constexpr (CAUSAL) x_operands<T, NL>(sV, sG, Xop);
            for (int nt = 0; nt < 2; ++nt) {
                f32x4 G = zero4();
                const Frag<T> g0 = NL::frag_pi(sG, 16 * nt + i, 0), g1 = NL::frag_pi(sG, 16 * nt + i, 1);
                mma(G, b0, g0);
                mma(G, b1, g1);
                if constexpr (is_bf16<T>()) {
                    mma(G, b0l, g0);
                    mma(G, b1l, g1);
                }
                if constexpr (CAUSAL) mma(G, Pf, Xop[nt]);
                if constexpr (CAUSAL && HL) mma(G, Pl, Xop[nt]);
                if constexpr (GC || GP) {
                    // this wave's share of sum_s P_Q G (GC: dP_Q follows the barrier)
                    Gv[nt] = G;
                    float p = 0.f;
                    for (int e = 0; e < 4; ++e) p += PQ[nt][e] * G[e];
                    p = xor32_sum(xor16_sum(p));
                    if (g == 0) sGs[w * TT + 16 * nt + i] = p;
                    continue;
                }
                // dP_Q = G/(A+eps); dA = -W G/(A+eps).  GN: dP_Q = G rd + gd A; dA = gd P_Q
                for (int e = 0; e < 4; ++e) {
                    if constexpr (GN) {
                        dPQ[nt][e] = G[e] * inv[nt][e] + gd[nt] * Ag[nt][e];
                        dA[nt][e] = gd[nt] * PQ[nt][e];
                    } else {
                        dPQ[nt][e] = G[e] * inv[nt][e];
                        dA[nt][e] = -W[nt][e] * dPQ[nt][e];
                    }
                }
                if constexpr (!CAUSAL && !GN) {
                    if (ddp) {  // den = sum_s P_Q A_s: dP_Q += h A, dA += h P_Q
                        const float h = sTokIn[16 * nt + i];
                        for (int e = 0; e < 4; ++e) {
                            dA[nt][e] += h * PQ[nt][e];
                            dPQ[nt][e] += h * (float)a0[e];
                        }
                    }
                }
            }
        }
        // the lane's share of the segment's dA totals (summed over the row's
        // lanes after the walk)
        if constexpr (!GC && !GP)
            for (int e = 0; e < 4; ++e) al[e] += (double)(dA[0][e] + dA[1][e]);
        // U^T[d][s] += sum_t g[t][d] W[t][s]; carry B^T[d][s] += sum_t V[t][d] P_K[t][s]
        for (int md = 0; md < 4; ++md) {
            if constexpr (!GP) {
                const Frag<T> go = col_operand<T, NL>(sG, sGt, md);
                mma(Ut[md], go, Wf);
                if constexpr (HL) mma(Ut[md], go, Wl);
            }
            if constexpr (CAUSAL) {
                const Frag<T> vo = col_operand<T, NL>(sV, sVt, md);
                mma(Bt[md], vo, Pf);
                if constexpr (HL) mma(Bt[md], vo, Pl);
            }
        }
        if constexpr (CAUSAL)
            for (int e = 0; e < 4; ++e) a0[e] += (CarryA<T>)tot[e];
        if constexpr (GC) {
            __syncthreads();  // every wave's share of sum_s P_Q G
            for (int nt = 0; nt < 2; ++nt) {
                const int t = 16 * nt + i;
                float sq = 0.f;
#pragma unroll
                for (int v = 0; v < NW_; ++v) sq += sGs[v * TT + t];
                const float dn = sTokIn[t];
                gd[nt] = sTokIn[TT + t] - (dn >= a.eps ? rd[nt] * rd[nt] * sq : 0.f);
                if (rdw && w == 0 && g == 0 && t < tile_rows(t0, a.T)) {
                    rdw[t0 + t] = rd[nt];
                    gdw[t0 + t] = gd[nt];
                }
                for (int e = 0; e < 4; ++e) {
                    dPQ[nt][e] = Gv[nt][e] * inv[nt][e] + gd[nt] * Ag[nt][e];
                    dA[nt][e] = gd[nt] * PQ[nt][e];
                }
            }
            for (int e = 0; e < 4; ++e) al[e] += (double)(dA[0][e] + dA[1][e]);
        }
        if constexpr (GP) {
            __syncthreads();  // every wave's share of this slice's sum_s P_Q G
            if (w == 0 && g == 0)
                for (int nt = 0; nt < 2; ++nt) {
                    const int t = 16 * nt + i;
                    float sq = 0.f;
#pragma unroll
                    for (int v = 0; v < NW_; ++v) sq += sGs[v * TT + t];
                    if (t < tile_rows(t0, a.T)) gsp[t0 + t] = sq;
                }
        } else if constexpr (KB <= 4) {
            tsum += softhash_bwd<KB, T>(PQ, dPQ, sSpQ, sSmQ, sThQ, sg, a.L, a.inv_temp, sDproj, ho);
        } else {
            softhash_share<KB, T>(PQ, dPQ, wh, sShare);
            __syncthreads();
            tsum += softhash_combine<KB, T, SP, NTH>(sShare, sSpQ, sSmQ, sThQ, z, a.L, a.inv_temp, sDproj);
        }
        // The next tile's rows go to the other token block (its last readers
        // finished before this tile's first barrier), or with one block to it
        // after a barrier.  The tile's dQ is stored in the next iteration (or
        // after the loop).
        if constexpr (NB == 1) __syncthreads();
        commit(NB == 2 ? (int)((jt + 1) & 1) : 0);
    }
    if constexpr (GP) return;  // the pre-pass writes gsum only
    if (j0 < j1) {
        if constexpr (NB == 2) __syncthreads();  // every wave's dproj rows of the last tile
        dx_store<T, NW_, XC, AL, XF>(sDproj, sPlT, dqp, a.sg.t, (int64_t)(j1 - 1) * TT, a.T, xpart, xc0);
    }
    float *out = a.rdelta + ((int64_t)n * a.nseg + seg) * a.Spad * SROW;
    for (int md = 0; md < 4; ++md)
        for (int e = 0; e < 4; ++e) out[sidx(sg + i, 16 * md + 4 * g + e)] = Ut[md][e];
    for (int e = 0; e < 4; ++e) al[e] = row_sum_f64(al[e]);
    if (i == 0)
        for (int e = 0; e < 4; ++e) out[sidx(sg + 4 * g + e, D)] = (float)al[e];
    const double ts = block_sum_f64<NTH>((double)tsum, sRed);
    if (threadIdx.x == 0) a.tpart[((int64_t)n * a.nseg + seg) * a.nslice + z] = ts;
}

// exclusive suffix over segments (causal) or totals (non-causal)
__global__ __launch_bounds__(SCAN_THREADS) void k_bwd_scan(float *rstate, const float *rdelta, int nseg, int elems,
                                                           int causal) {
    const int n = blockIdx.y, e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= elems) return;
    const float *src = rdelta + (int64_t)n * nseg * elems + e;
    float *dst = rstate + (int64_t)n * nseg * elems + e;
    double acc = 0.0;
    if (causal) {  // segments in reverse order
        int s = nseg;
        for (; s >= SCAN_BATCH; s -= SCAN_BATCH) {
            float v[SCAN_BATCH];
#pragma unroll
            for (int j = 0; j < SCAN_BATCH; ++j) v[j] = src[(int64_t)(s - 1 - j) * elems];
#pragma unroll
            for (int j = 0; j < SCAN_BATCH; ++j) {
                dst[(int64_t)(s - 1 - j) * elems] = (float)acc;
                acc += v[j];
            }
        }
        for (; s > 0; --s) {
            const float v = src[(int64_t)(s - 1) * elems];
            dst[(int64_t)(s - 1) * elems] = (float)acc;
            acc += v;
        }
    } else {
        for (int s = 0; s < nseg; ++s) acc += src[(int64_t)s * elems];
        for (int s = 0; s < nseg; ++s) dst[(int64_t)s * elems] = (float)acc;
    }
}

// =====================================================================
// k_bwd_out: reverse walk.  dK, dV.
// dV^T[d][tau] = sum_s U[s][d] P_K[tau][s] + sum_{t >= tau} g[t][d] Sc2[t][tau],
// Sc2[t][tau] = sum_s W[t][s] P_K[tau][s], computed as output tiles over all
// buckets from the waves' [.][s] LDS arrays; dK through each wave's buckets.
// =====================================================================
template <typename T, int SP, bool CAUSAL, int KB, bool GN> struct BwdOutL {
    static constexpr int NW_ = SP / WB;
    // the configuration of the whole-tile 4-bit instantiation (bf16, 128-bucket
    // slices, causal F1): it projects a tile in the previous tile's last phase,
    // so K's sigmoid rows are double-buffered, and the transposed V / dO rows,
    // which bf16 never reads, take no LDS.  (8-bit slices measured faster with
    // the projections in a phase of their own: only half of their waves have a
    // projection task, and their last phase already ends at the wide-table
    // barrier.)
    static constexpr bool P2L = is_bf16<T>() && SP == 128 && CAUSAL && !GN && KB == 4;
    static constexpr int NSIG = P2L ? 8 : (CAUSAL ? 5 : 3);  // sigmoid row arrays
    static constexpr int LDN = NatL<T, true>::LD, LDT = ldp_of<T>(TT), LDC = ld_of<float>(NCOL), LDDP = sw_ld<T, NCOL>(),
                         LDS_ = sw_ld<T, SP>();
    // token block: one tile's staged rows (K, Q, V, dO natural; V, dO
    // transposed; GN: rden, gden [2][TT]; non-causal: key weights [TT])
    static constexpr size_t oK = 0;
    static constexpr size_t oQ = align16(oK + sizeof(T) * TT * LDN);
    static constexpr size_t oV = align16(oQ + (CAUSAL ? sizeof(T) * TT * LDN : 0));
    static constexpr size_t oG = align16(oV + sizeof(T) * TT * LDN);
    static constexpr size_t oVt = align16(oG + (CAUSAL ? sizeof(T) * TT * LDN : 0));
    static constexpr size_t oGt = align16(oVt + (CAUSAL && !P2L ? sizeof(T) * D * LDT : 0));
    static constexpr size_t oTok = align16(oGt + (CAUSAL && !P2L ? sizeof(T) * D * LDT : 0));
    static constexpr size_t TB = align16(oTok + (GN || !CAUSAL ? sizeof(float) * 2 * TT : 0));
    // the rest, relative to its start
    static constexpr size_t rX = 0;
    static constexpr size_t rY = align16(rX + (CAUSAL ? sizeof(T) * TT * LDT : 0));
    static constexpr size_t rPts = align16(rY + (CAUSAL ? sizeof(T) * TT * LDT : 0));
    static constexpr size_t rWts = align16(rPts + sizeof(T) * TT * LDS_);
    static constexpr size_t rUT = align16(rWts + (CAUSAL ? sizeof(T) * TT * LDS_ : 0));
    static constexpr size_t rDproj = align16(rUT + sizeof(T) * D * LDS_);
    static constexpr size_t rPl = align16(rDproj + sizeof(T) * TT * LDDP);
    static constexpr size_t rPlLo = align16(rPl + sizeof(T) * NCOL * LDN);
    static constexpr size_t rPlT = align16(rPlLo + sizeof(T) * NCOL * LDN);
    // K sp, K sm, K th, Q sp, Q sm (P2L: then K sp, K sm, K th of odd tiles)
    static constexpr size_t rSig = align16(rPlT + sizeof(T) * D * LDDP);
    // the end-of-kernel block sum's scratch [64 * NW_] reuses the sigmoid rows
    static_assert(64 * NW_ <= (CAUSAL ? 5 : 3) * TT * LDC, "block-sum scratch inside the sigmoid rows");
    static constexpr size_t rRed = rSig;
    static constexpr size_t rCst = align16(rSig + sizeof(float) * NSIG * TT * LDC);
    static constexpr size_t rHash = align16(rCst + Consts<T>::bytes);
    // causal: Sc2^T [tau][t] of the last tile, for the dV tiles of the next
    // iteration (with two token blocks)
    static constexpr size_t rSc2 = align16(rHash + HashOps<T, 4>::bytes);
    static constexpr size_t rPair = align16(rSc2 + (CAUSAL ? sizeof(T) * TT * LDT : 0));
    static constexpr size_t rShare = align16(rPair + PairOps<T>::bytes);
    static constexpr size_t rEnd = align16(rShare + (KB > 4 ? WideHash<T, KB>::bytes(NW_) : 0));
    // two token blocks when they cost no workgroup per CU (160 KiB of LDS):
    // the next tile's rows then go to the other block while this tile still
    // reads its own, and the barrier ahead of that commit goes away
    static constexpr size_t LDS_CU = 160 * 1024;
    static constexpr int NB = bwd_wgs_per_cu(NW_, 2 * TB + rEnd) >= bwd_wgs_per_cu(NW_, TB + rEnd) ? 2 : 1;
    static constexpr size_t R0 = NB * TB;
    static constexpr size_t oX = R0 + rX, oY = R0 + rY, oPts = R0 + rPts, oWts = R0 + rWts, oUT = R0 + rUT,
                            oDproj = R0 + rDproj, oPl = R0 + rPl, oPlLo = R0 + rPlLo, oPlT = R0 + rPlT,
                            oSig = R0 + rSig, oRed = R0 + rRed, oCst = R0 + rCst, oHash = R0 + rHash,
                            oPair = R0 + rPair, oShare = R0 + rShare, oSc2 = R0 + rSc2;
    static constexpr size_t bytes = R0 + rEnd;
};

// Sc2 output tile r = (mt, nt) in {(0,0), (1,0), (1,1)} (the (0,1) tile is
// zero), masked to t >= tau and stored transposed: sc2[tau][t].
template <typename T, int SP> __device__ void sc2_tile(int r, const T *Wts, const T *Pts, T *sc2) {
    constexpr int LDT = ldp_of<T>(TT);
    const int g = lg(), i = li(), mt = r == 0 ? 0 : 1, nt = r == 2 ? 1 : 0;
    const T *pw = sw_frag_ptr<T, SP>(Wts, 16 * mt + i), *pp = sw_frag_ptr<T, SP>(Pts, 16 * nt + i);
    f32x4 acc = zero4();
#pragma unroll
    for (int kp = 0; kp < SP / 32; ++kp) mma(acc, ld_frag(pw + 32 * kp), ld_frag(pp + 32 * kp));
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (16 * mt + 4 * g + e < 16 * nt + i) acc[e] = 0.f;  // keep t >= tau
    store4<T>(sc2 + (16 * nt + i) * LDT + 16 * mt + 4 * g, acc);
}

template <typename T, int SP, bool CAUSAL, bool AL = false, class NL = NatL<T, true>>
__device__ void dv_tile(int md, int nt, const T *sUT, const T *Pts, const T *Wts, const T *sG, const T *sGt, T *dvp,
                        int64_t st,
                        int64_t t0, int64_t Tn, T *part) {
    constexpr int LDT = ldp_of<T>(TT);
    const int g = lg(), i = li();
    const T *pu = sw_frag_ptr<T, SP>(sUT, 16 * md + i), *pp = sw_frag_ptr<T, SP>(Pts, 16 * nt + i);
    f32x4 acc = zero4();
#pragma unroll
    for (int kp = 0; kp < SP / 32; ++kp) mma(acc, ld_frag(pu + 32 * kp), ld_frag(pp + 32 * kp));
    if constexpr (CAUSAL) {
        f32x4 Sc2[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            Sc2[mt] = zero4();
            if (mt >= nt) {
                const T *pw = sw_frag_ptr<T, SP>(Wts, 16 * mt + i);
#pragma unroll
                for (int kp = 0; kp < SP / 32; ++kp) mma(Sc2[mt], ld_frag(pw + 32 * kp), ld_frag(pp + 32 * kp));
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (16 * mt + 4 * g + e < 16 * nt + i) Sc2[mt][e] = 0.f;  // keep t >= tau
            }
        }
        mma(acc, col_operand<T, NL>(sG, sGt, md), frag_acc<T>(Sc2[0], Sc2[1]));
    }
    const int t = 16 * nt + i;
    if ((AL || t < tile_rows(t0, Tn))) {
        if (part)
            store4<T>(part_at(part, t0, t, 16 * md + 4 * g), acc);
        else
            store4<T>(at_bytes(tile_ptr(dvp, st, t0), tile_off(t, st, 16 * md + 4 * g, sizeof(T))), acc);
    }
}

// dV tile (md, nt) in two steps: the carried part U P_K (over all buckets,
// from the U and P_K rows), then, once the tile's Sc2 rows exist (sc2_tile),
// the in-tile part g^T Sc2 and the store.
// The d-row carry U^T (lane: [d = 16md + 4g + e][s = sw + i]) as the operand
// of acc[s][tau] += sum_d U[s][d] v_tau[d]; with HL an fp32-accurate hi + lo
// pair
template <typename T, bool HL> struct UOps {
    Frag<T> u0, u1, u0l, u1l;
    __device__ __forceinline__ explicit UOps(const f32x4 (&Ut)[4]) {
        if constexpr (HL) {
            frag_acc_hilo(Ut[0], Ut[1], u0, u0l);
            frag_acc_hilo(Ut[2], Ut[3], u1, u1l);
        } else {
            u0 = frag_acc<T>(Ut[0], Ut[1]);
            u1 = frag_acc<T>(Ut[2], Ut[3]);
        }
    }
    // the tile's tokens tau = 16 nt + i
    template <class NL> __device__ __forceinline__ void apply(f32x4 &acc, const T *sV, int nt) const {
        const Frag<T> v0 = NL::frag_pi(sV, 16 * nt + li(), 0), v1 = NL::frag_pi(sV, 16 * nt + li(), 1);
        mma(acc, u0, v0);
        mma(acc, u1, v1);
        if constexpr (HL) {
            mma(acc, u0l, v0);
            mma(acc, u1l, v1);
        }
    }
};
template <typename T, int SP> __device__ f32x4 dv_part(int md, int nt, const T *sUT, const T *Pts) {
    const int i = li();
    const T *pu = sw_frag_ptr<T, SP>(sUT, 16 * md + i), *pp = sw_frag_ptr<T, SP>(Pts, 16 * nt + i);
    f32x4 acc = zero4();
#pragma unroll
    for (int kp = 0; kp < SP / 32; ++kp) mma(acc, ld_frag(pu + 32 * kp), ld_frag(pp + 32 * kp));
    return acc;
}
template <typename T, bool AL = false, class NL = NatL<T, true>>
__device__ void dv_finish(int md, int nt, f32x4 acc, const T *sG, const T *sGt, const T *sc2, T *dvp, int64_t st,
                          int64_t t0,
                          int64_t Tn, T *part) {
    constexpr int LDT = ldp_of<T>(TT);
    const int g = lg(), i = li();
    mma(acc, col_operand<T, NL>(sG, sGt, md), ld_frag_pi(sc2 + (16 * nt + i) * LDT));
    const int t = 16 * nt + i;
    if ((AL || t < tile_rows(t0, Tn))) {
        if (part)
            store4<T>(part_at(part, t0, t, 16 * md + 4 * g), acc);
        else
            store4<T>(at_bytes(tile_ptr(dvp, st, t0), tile_off(t, st, 16 * md + 4 * g, sizeof(T))), acc);
    }
}

// GN (global normalisation, causal only): W = P_Q rd and dA = gd P_Q per
// token (rd = 1/max(den, eps), gd = dL/d den), so the reverse walk needs
// neither the forward state nor G.
template <typename T, int SP, bool CAUSAL, int KB, bool GN, bool AL = false, bool XW = walk_f64<T, AL>()>
__global__ __launch_bounds__(threads_of(SP), 2) void k_bwd_out(Args a) {
    if (a.inv_temp_ptr) a.inv_temp = *a.inv_temp_ptr;  // uniform scalar load
    static_assert(CAUSAL || !GN, "global normalisation is causal only");
    using Ly = BwdOutL<T, SP, CAUSAL, KB, GN>;
    using NL = NatL<T, true>;
    // Q's and K's sigmoid rows as pair products (K's as in the forward kernels:
    // the walk back of the forward state subtracts the same P_K)
    constexpr bool PR = pair_tables<KB>();
    constexpr bool HL = hl_ops<T, SP, KB>();  // P_K, W and U as hi + lo pairs
    // bf16 tables of up to 7 bits: W as a hi + lo pair in dP_K's in-tile term
    // sum_{t >= tau} M[tau][t] W[t][s], the leading bf16 rounding of dK there
    // (with a value mean, v.g is large and the softmax backward cancels what a
    // table's buckets share of it).  An 8-bit table's 256 buckets spread W, and
    // the single operand costs it no more than the other roundings do.
    constexpr bool WM = is_bf16<T>() && KB < 8;
    constexpr int NW_ = Ly::NW_, NTH = 64 * NW_, LDN = Ly::LDN, LDT = Ly::LDT, LDC = Ly::LDC, LDDP = Ly::LDDP,
                  LDS_ = Ly::LDS_;
    __shared__ __align__(16) unsigned char smem[Ly::bytes];
    // this tile's token block (block jr & 1 of two; block 0 of one)
    T *sQ, *sK, *sV, *sG, *sVt, *sGt;
    float *sTok;
    auto use_block = [&](int b) {
        unsigned char *tb = smem + b * Ly::TB;
        sK = (T *)(tb + Ly::oK);
        sQ = (T *)(tb + Ly::oQ);
        sV = (T *)(tb + Ly::oV);
        sG = (T *)(tb + Ly::oG);
        sVt = (T *)(tb + Ly::oVt);
        sGt = (T *)(tb + Ly::oGt);
        sTok = (float *)(tb + Ly::oTok);
    };
    T *sX = (T *)(smem + Ly::oX), *sY = (T *)(smem + Ly::oY);
    T *sPts = (T *)(smem + Ly::oPts), *sWts = (T *)(smem + Ly::oWts), *sUT = (T *)(smem + Ly::oUT);
    T *sDproj = (T *)(smem + Ly::oDproj), *sSc2 = (T *)(smem + Ly::oSc2);
    T *sPl = (T *)(smem + Ly::oPl), *sPlLo = (T *)(smem + Ly::oPlLo), *sPlT = (T *)(smem + Ly::oPlT);
    float *sSig = (float *)(smem + Ly::oSig), *sRed = (float *)(smem + Ly::oRed);
    float *sSpK = sSig, *sSmK = sSig + TT * LDC, *sThK = sSig + 2 * TT * LDC;
    float *sSpQ = sSig + 3 * TT * LDC, *sSmQ = sSig + 4 * TT * LDC;
    const WgPos wp = wg_pos(a.nseg, a.M * a.B * a.H, a.nslice, sliced<T, KB>());
    if (!wp.live) return;
    const int w = wave_id(), g = lg(), i = li(), sw = WB * w, z = wp.z,
              sg = z * SP + sw;
    const PlaneBlocks pbk(z, SP, KB, a.L, !sliced<T, KB>());  // projection columns of this slice

    const int n = wp.n, seg = wp.seg;
    const int m = n / (a.B * a.H);
    const int ntiles = (int)((a.T + TT - 1) / TT);  // the host bounds T by 2^35
    const int lastv = (int)(a.T - (int64_t)(ntiles - 1) * TT);  // rows of the last tile
    const int j0 = seg * a.tps, j1 = min(ntiles, j0 + a.tps);
    const T *qp = (const T *)a.q + stream_off(a.sq, n, a.B, a.H);
    const T *kp = (const T *)a.k + stream_off(a.sk, n, a.B, a.H);
    const T *vp = (const T *)a.v + stream_off(a.sv, n, a.B, a.H);
    const T *gp = (const T *)a.dout + stream_off(a.sdo, n, a.B, a.H);
    T *dkp = (T *)a.dk + stream_off(a.sg, n, a.B, a.H);
    T *dvp = (T *)a.dv + stream_off(a.sg, n, a.B, a.H);
    constexpr int XC = xcols_of(SP, KB);
    constexpr bool XF = xpart_f32(is_bf16<T>(), SP, KB);
    void *xpart = sliced<T, KB>() ? xpart_at<T, SP, KB>(a.dkpart, z, n, a) : nullptr;
    const int xc0 = ((z * SP) >> KB) * KB;  // first projection column of the slice's tables
    T *vpart = sliced<T, KB>() ? (T *)a.dvpart + ((int64_t)z * a.M * a.B * a.H + n) * a.T * D : nullptr;
    const float *rdp = GN ? a.rden + (int64_t)n * a.T : nullptr, *gdp = GN ? a.gden + (int64_t)n * a.T : nullptr;
    const float *kwp = !CAUSAL && a.kw ? a.kw + (int64_t)((n / a.H) % a.B) * a.T : nullptr;

    Consts<T> cst;
    cst.init((T *)(smem + Ly::oCst), NTH);
    HashOps<T, KB> ho;
    WideHash<T, KB> wh;
    float *sShare = (float *)(smem + Ly::oShare);
    if constexpr (KB <= 4)
        ho.init((T *)(smem + Ly::oHash), NTH);
    else
        wh.init(sg);
    PairOps<T> po;
    po.init((T *)(smem + Ly::oPair), NTH);
    load_planes<T, NTH, NL>(a.planes + m * a.planes_m_stride, a.L * a.K, sPl, is_bf16<T>() ? sPlLo : nullptr, sPlT);
    zero_lds<T>(sDproj, TT * LDDP, NTH);
    if constexpr (CAUSAL) {
        zero_lds<T>(sX, TT * LDT, NTH);
        zero_lds<T>(sY, TT * LDT, NTH);
        zero_lds<T>(sSc2, TT * LDT, NTH);  // its (t < 16 <= tau) block stays zero
    }
    __syncthreads();  // the constant tables in LDS; their operands to registers
    cst.cache();
    if constexpr (KB <= 4) ho.cache();
    po.cache();
    // whole-tile instantiations: each wave has at most one projection task,
    // the same column block on every tile, whose planes stay in registers
    PlaneOps<T> pcw;
    if constexpr (AL) pcw.template load<NL>(sPl, sPlLo, pbk.mc(pbk.task(w)));
    // reverse carries (U, alpha) after the segment; forward state at the segment end
    const float *rs = a.rstate + ((int64_t)n * a.nseg + seg) * a.Spad * SROW;
    const double *fs =
        a.fstate + ((int64_t)n * (a.fnseg + 1) + min((seg + 1) * a.fmul, a.fnseg)) * a.Spad * SROW;
    f32x4 Ut[4];  // U^T[d = 16md + 4g + e][s = sw + i]
    // Forward state, walked back from the segment end.  B only feeds the
    // G product's operand: the whole-tile bf16 instantiations carry it in
    // fp32 MFMA accumulators and subtract the tile sums on the matrix core
    // (Bm); the others walk it in fp64 (Be, walk_f64).  A stays fp64: A(t)
    // is far below the segment-end value early in a sequence.
    constexpr bool BM = is_bf16<T>() && !XW;  // the walk of B in fp64 (walk_f64)
    double Be[4][4], Ae[4];
    f32x4 Bm[4];
    f32x4 al;
    constexpr bool FSTATE = CAUSAL && !GN;
    for (int md = 0; md < 4; ++md)
        for (int e = 0; e < 4; ++e) {
            const int64_t r = sidx(sg + i, 16 * md + 4 * g + e);
            Ut[md][e] = rs[r];
            if constexpr (BM)
                Bm[md][e] = FSTATE ? (float)fs[r] : 0.f;
            else
                Be[md][e] = FSTATE ? fs[r] : 0.0;
        }
    for (int e = 0; e < 4; ++e) {
        al[e] = rs[sidx(sg + 4 * g + e, D)];
        Ae[e] = FSTATE ? fs[sidx(sg + 4 * g + e, D)] : 0.0;
    }
    if constexpr (!CAUSAL) store_ut<T, SP>(sUT, sw, Ut, cst, po);  // constant totals
    CarryA<T> tsum = 0;  // this thread's share of sum du * th

    wait_state_loads();
    Prefetch<T, NTH, AL> pq_, pk_, pvn_;  // pvn_: non-causal V (natural only)
    PrefetchT2<T, NTH, AL, !is_bf16<T>()> pgv_;  // causal dO (first half of the waves) and V
    TokPre pt_;
    // Writes the prefetched rows to token block b.
    auto commit = [&](int b) {
        unsigned char *tb = smem + b * Ly::TB;
        float *tok = (float *)(tb + Ly::oTok);
        wait_vmem();
        pk_.template commit<NL>((T *)(tb + Ly::oK), nullptr);
        if constexpr (CAUSAL) {
            pq_.template commit<NL>((T *)(tb + Ly::oQ), nullptr);
            pgv_.template commit<NL>((T *)(tb + Ly::oG), (T *)(tb + Ly::oGt), (T *)(tb + Ly::oV), (T *)(tb + Ly::oVt));
        } else {
            pvn_.template commit<NL>((T *)(tb + Ly::oV), nullptr);
            if (kwp) pt_.commit(tok);
        }
        if constexpr (GN) pt_.commit(tok);
    };
    constexpr int NB = Ly::NB;
    // causal with two token blocks: a tile's dV is stored in the next
    // iteration, from Sc2 rows computed once in LDS
    constexpr bool SCN = CAUSAL && NB == 2;
    constexpr int NQD = (8 + NW_ - 1) / NW_;  // dV tiles per wave
    f32x4 dvacc[NQD];                          // SCN: carried part of the last tile's dV tiles
#pragma unroll
    for (int k = 0; k < NQD; ++k) dvacc[k] = zero4();
    // Whole 4-bit tiles (P2): two barriers per tile instead of three.  The Q and K
    // rows of tile j - 1 are committed in tile j's second phase and projected
    // at the end of its last phase, into the Q rows (read only in the second
    // phase) and K rows of the other parity (K's are also read by the
    // softmax backward of the last phase); V and dO are committed in the last
    // phase as before.  Each prefetch set is reloaded right after its commit,
    // a tile ahead, and its commit waits on it by count (every lane issues the
    // same branch-free loads), not on the stores issued since.
    constexpr bool P2 = AL && SCN && Ly::P2L;
    // the three masked v.g^T blocks: with the projections, or (two token
    // blocks, every projection task on a wave of its own) in the next phase,
    // whose bucket work leaves issue slots to fill
    constexpr bool MT2 = SCN;
    static_assert(!Ly::P2L || !AL || SCN, "the 4-bit whole-tile instantiation runs the two-barrier walk");
    auto commit_qk = [&](int b) {
        unsigned char *tb = smem + b * Ly::TB;
        pk_.template commit<NL>((T *)(tb + Ly::oK), nullptr);
        pq_.template commit<NL>((T *)(tb + Ly::oQ), nullptr);
    };
    auto commit_vg = [&](int b) {
        unsigned char *tb = smem + b * Ly::TB;
        pgv_.template commit<NL>((T *)(tb + Ly::oG), (T *)(tb + Ly::oGt), (T *)(tb + Ly::oV), (T *)(tb + Ly::oVt));
    };
    auto issue_qk = [&](int64_t tq) {
        pk_.issue(kp, a.sk.t, tq, a.T);
        pq_.issue(qp, a.sq.t, tq, a.T);
    };
    auto issue_vg = [&](int64_t tq) { pgv_.issue(gp, a.sdo.t, vp, a.sv.t, tq, a.T); };
    // the wave's projection task (at most one: K in the first half, Q) of the
    // tile in token block b, into the Q rows and the K rows of parity par
    auto project2 = [&](int b, int par) {
        unsigned char *tb = smem + b * Ly::TB;
        if (2 * pbk.tasks() >= NW_ || w < 2 * pbk.tasks()) {
            const bool isk = w < pbk.tasks();
            const int r = pbk.task(w);
            float *kr = sSig + (par ? 5 : 0) * TT * LDC;
            project_tile<T, NL, PR>(isk ? (const T *)(tb + Ly::oK) : (const T *)(tb + Ly::oQ), sPl, sPlLo, pbk.mc(r),
                                    r & 1, a.inv_temp, isk ? kr : sSpQ, isk ? kr + TT * LDC : sSmQ,
                                    isk ? kr + 2 * TT * LDC : nullptr, &pcw);
        }
    };
    if (P2 && j0 < j1) {
        const int64_t tl = (int64_t)(j1 - 1) * TT, tl2 = (int64_t)max(j1 - 2, j0) * TT;
        issue_qk(tl);
        issue_vg(tl);
        commit_qk((j1 - 1) & 1);
        commit_vg((j1 - 1) & 1);
        issue_qk(tl2);
        issue_vg(tl2);
        __syncthreads();
        project2((j1 - 1) & 1, (j1 - 1) & 1);
    } else if (j0 < j1) {
        const int64_t tl = (int64_t)(j1 - 1) * TT;
        pk_.issue(kp, a.sk.t, tl, a.T);
        if constexpr (CAUSAL) {
            pq_.issue(qp, a.sq.t, tl, a.T);
            pgv_.issue(gp, a.sdo.t, vp, a.sv.t, tl, a.T);
        } else {
            pvn_.issue(vp, a.sv.t, tl, a.T);
            if (kwp) pt_.issue(kwp, nullptr, tl, a.T);
        }
        if constexpr (GN) pt_.issue(rdp, gdp, tl, a.T);
        commit(NB == 2 ? (int)((j1 - 1) & 1) : 0);
    }
    for (int jr = j1 - 1; jr >= j0; --jr) {
        const int64_t t0 = (int64_t)jr * TT;
        use_block(NB == 2 ? (int)(jr & 1) : 0);
        // next tile's rows (walking down); the last tile reloads itself (loads
        // stay in range).  Issue and commit run every iteration: a commit under
        // a condition leaves the prefetch registers possibly pending at the
        // loop head, and the wait placed there also waits for the previous
        // tile's stores.
        const int64_t tn = (int64_t)(jr > j0 ? jr - 1 : jr) * TT;
        if constexpr (P2) {
            sSpK = sSig + ((jr & 1) ? 5 : 0) * TT * LDC;  // this tile's K rows
            sSmK = sSpK + TT * LDC;
            sThK = sSpK + 2 * TT * LDC;
        } else {
            __syncthreads();
            // issued after the barrier: the previous tile's dK stores have had
            // the barrier's time to drain from the memory pipeline
            pk_.issue(kp, a.sk.t, tn, a.T);
            if constexpr (CAUSAL) {
                pq_.issue(qp, a.sq.t, tn, a.T);
                pgv_.issue(gp, a.sdo.t, vp, a.sv.t, tn, a.T);
            } else {
                pvn_.issue(vp, a.sv.t, tn, a.T);
                if (kwp) pt_.issue(kwp, nullptr, tn, a.T);
            }
            if constexpr (GN) pt_.issue(rdp, gdp, tn, a.T);
            if constexpr (AL && MT2) {
                // whole tiles: at most one task per wave, K (first half) or Q --
                // one code path on scalar-selected rows, which the compiler can
                // interleave with the rest of the phase
                if (w < 2 * pbk.tasks()) {
                    const bool isk = w < pbk.tasks();
                    const int r = pbk.task(w);
                    project_tile<T, NL, PR>(isk ? sK : sQ, sPl, sPlLo, pbk.mc(r), r & 1, a.inv_temp,
                                            isk ? sSpK : sSpQ, isk ? sSmK : sSmQ, isk ? sThK : nullptr, &pcw);
                }
            } else {
                for (int q = w; q < (CAUSAL ? 2 * pbk.tasks() + (MT2 ? 0 : 3) : pbk.tasks()); q += NW_) {
                    const int r = pbk.task(q);
                    if (q < pbk.tasks())
                        project_tile<T, NL, PR>(sK, sPl, sPlLo, pbk.mc(r), r & 1, a.inv_temp, sSpK, sSmK, sThK,
                                                (AL && q == w) ? &pcw : nullptr);
                    else if (q < 2 * pbk.tasks())
                        project_tile<T, NL, PR>(sQ, sPl, sPlLo, pbk.mc(r), r & 1, a.inv_temp, sSpQ, sSmQ, nullptr,
                                                (AL && q == w) ? &pcw : nullptr);
                    else
                        m_tile_xy<T, NL>(q - 2 * pbk.tasks(), sV, sG, sX, sY);
                }
            }
            // dK of the tile after this one (walking down), from the dproj rows its
            // softmax backward left in LDS: with one token block beside the
            // projections, with two (below) beside the probabilities, after the
            // second barrier; the next write of sDproj is after the third
            if constexpr (!SCN)
                if (jr + 1 < j1) dx_store<T, NW_, XC, AL, XF>(sDproj, sPlT, dkp, a.sg.t, t0 + TT, a.T, xpart, xc0);
            // causal, two token blocks: dV of that tile too, its carried part
            // (computed last iteration) plus the in-tile part from its Sc2 rows and
            // its dO tile (still in its block: the next commit there is after this
            // tile's third barrier)
            if constexpr (SCN)
                if (jr + 1 < j1) {
                    const T *gtn = (const T *)(smem + ((jr + 1) & 1) * Ly::TB + Ly::oGt);
                    const T *gnn = (const T *)(smem + ((jr + 1) & 1) * Ly::TB + Ly::oG);
#pragma unroll
                    for (int k = 0; k < NQD; ++k)
                        if (w + k * NW_ < 8)
                            dv_finish<T, AL>((w + k * NW_) >> 1, (w + k * NW_) & 1, dvacc[k], gnn, gtn, sSc2, dvp,
                                             a.sg.t, t0 + TT, a.T, vpart);
                }
        }
        __syncthreads();
        if constexpr (P2) {
            // tile j - 1's Q and K rows, then the loads of tile j - 2's; the
            // dV tiles of tile j + 1 (its dO rows stay until this tile's last
            // phase)
            commit_qk((jr + 1) & 1);
            issue_qk((int64_t)max(jr - 2, j0) * TT);
            if (jr + 1 < j1) {
                const T *gtn = (const T *)(smem + ((jr + 1) & 1) * Ly::TB + Ly::oGt);
                const T *gnn = (const T *)(smem + ((jr + 1) & 1) * Ly::TB + Ly::oG);
#pragma unroll
                for (int k = 0; k < NQD; ++k)
                    if (w + k * NW_ < 8)
                        dv_finish<T, AL>((w + k * NW_) >> 1, (w + k * NW_) & 1, dvacc[k], gnn, gtn, sSc2, dvp, a.sg.t,
                                         t0 + TT, a.T, vpart);
            }
        }
        if constexpr (SCN)
            if (jr + 1 < j1) dx_store<T, NW_, XC, AL, XF>(sDproj, sPlT, dkp, a.sg.t, t0 + TT, a.T, xpart, xc0);
        if constexpr (MT2)  // X and Y are read after the next barrier
            for (int q = w; q < 3; q += NW_) m_tile_xy<T, NL>(q, sV, sG, sX, sY);
        f32x4 PKraw[2], PKr[2];  // fp32 P_K (kept for the softmax backward), operand-rounded P_K
        probs_st<KB, AL, PR>(sSpK, sSmK, sg, a.S, jr + 1 < ntiles ? TT : lastv, PKraw);
        PKr[0] = PKraw[0];
        PKr[1] = PKraw[1];
        float kwt[2] = {1.f, 1.f};  // non-causal key weights: P_K' = w_t P_K
        if constexpr (!CAUSAL) {
            if (kwp)
                for (int nt = 0; nt < 2; ++nt) {
                    kwt[nt] = sTok[16 * nt + i];
                    for (int e = 0; e < 4; ++e) PKr[nt][e] *= kwt[nt];
                }
        }
        const Frag<T> Pf = store_ts_operand<T, SP>(sPts, sw, PKr, cst);
        f32x4 dPK[2];
        if constexpr (CAUSAL) {
            f32x4 Wi[2];  // W / (A + eps), the factor of dA
            f32x4 dA[2];
            Frag<T> Wf, Pl, Wl;  // Pl, Wl: the lo parts of P_K (HL) and W (HL, WM)
            if constexpr (HL) {
                f32x4 R[2];
                lo_rem(PKr, R);
                Pl = token_operand<T>(R, cst, po);
            }
            // W's operand, and with HL its lo part
            auto w_operands = [&](const f32x4 (&W)[2]) {
                Wf = store_ts_operand<T, SP>(sWts, sw, W, cst);
                if constexpr (HL || WM) {
                    f32x4 R[2];
                    lo_rem(W, R);
                    Wl = token_operand<T>(R, cst, po);
                }
            };
            if constexpr (GN) {
                f32x4 PQ[2], W[2];
                probs_st<KB, AL, PR>(sSpQ, sSmQ, sg, a.S, jr + 1 < ntiles ? TT : lastv, PQ);
                for (int nt = 0; nt < 2; ++nt) {
                    const float rd = sTok[16 * nt + i], gd = sTok[TT + 16 * nt + i];
                    for (int e = 0; e < 4; ++e) {
                        W[nt][e] = PQ[nt][e] * rd;
                        dA[nt][e] = gd * PQ[nt][e];
                    }
                }
                w_operands(W);
            } else {
                f32x4 PQ[2], Acum[2], W[2], tot, dB[4];
                probs_st<KB, AL, PR>(sSpQ, sSmQ, sg, a.S, jr + 1 < ntiles ? TT : lastv, PQ);
                // forward state at the tile start: end state minus this tile's sums
                if constexpr (BM) {
                    tot = zero4();
                    mma(tot, Pf, cst.ones());
                    if constexpr (HL) mma(tot, Pl, cst.ones());
                    const Frag<T> Pn = neg_frag(Pf);
                    for (int md = 0; md < 4; ++md) {
                        const Frag<T> vo = col_operand<T, NL>(sV, sVt, md);
                        mma(Bm[md], vo, Pn);
                        if constexpr (HL) mma(Bm[md], vo, neg_frag(Pl));
                    }
                    for (int e = 0; e < 4; ++e) Ae[e] -= (double)tot[e];
                } else {
                    if constexpr (is_bf16<T>())
                        tile_sums_bf<NL, HL>(Pf, Pl, cst, sV, sVt, tot, dB);
                    else
                        tile_sums<T>(Pf, cst, sVt, tot, dB);
                    for (int e = 0; e < 4; ++e) {
                        Ae[e] -= (double)tot[e];
                        for (int md = 0; md < 4; ++md) Be[md][e] -= (double)dB[md][e];
                    }
                }
                for (int nt = 0; nt < 2; ++nt) {
                    Acum[nt] = zero4();
                    mma(Acum[nt], Pf, cst.tri_op(nt));
                    if constexpr (HL) mma(Acum[nt], Pl, cst.tri_op(nt));
                }
                float ae[4];
                for (int e = 0; e < 4; ++e) ae[e] = (float)Ae[e] + a.eps;
                for (int nt = 0; nt < 2; ++nt)
                    for (int e = 0; e < 4; ++e) {
                        const float inv = rcp(ae[e] + Acum[nt][e]);
                        W[nt][e] = PQ[nt][e] * inv;
                        Wi[nt][e] = W[nt][e] * inv;
                    }
                w_operands(W);
            }
            store_ut<T, SP>(sUT, sw, Ut, cst, po);
            __syncthreads();  // all waves' P_K, W, U rows in LDS
            // two token blocks: the next tile's rows go to the other block now
            // (its last readers finished before this tile's first barrier);
            // P2: its V and dO rows (the dV tiles of tile j + 1 read them
            // before this barrier), then the loads of tile j - 2's
            if constexpr (P2) {
                commit_vg((jr + 1) & 1);
                issue_vg((int64_t)max(jr - 2, j0) * TT);
            } else if constexpr (NB == 2) {
                commit((int)((jr + 1) & 1));
            }
            // ---- dA = -W G/(A+eps), G[s][t] = sum_d B_start[s][d] g[t][d] + sum_{tau<=t} P_K[tau][s] M[tau][t]
            if constexpr (!GN) {
                Frag<T> Bf[2];
                for (int kk = 0; kk < 2; ++kk) {
                    if constexpr (BM) {
                        Bf[kk] = frag_acc<T>(Bm[2 * kk], Bm[2 * kk + 1]);
                    } else {
                        f32x4 b0, b1;
                        for (int e = 0; e < 4; ++e) {
                            b0[e] = narrow(Be[2 * kk][e]);
                            b1[e] = narrow(Be[2 * kk + 1][e]);
                        }
                        Bf[kk] = frag_acc<T>(b0, b1);
                    }
                }
                for (int nt = 0; nt < 2; ++nt) {
                    f32x4 G = zero4();
                    mma(G, Bf[0], NL::frag_pi(sG, 16 * nt + i, 0));
                    mma(G, Bf[1], NL::frag_pi(sG, 16 * nt + i, 1));
                    const Frag<T> xo = ld_frag_pi(sX + (16 * nt + i) * LDT);
                    mma(G, Pf, xo);
                    if constexpr (HL) mma(G, Pl, xo);
                    for (int e = 0; e < 4; ++e) dA[nt][e] = -Wi[nt][e] * G[e];
                }
            }
            // ---- dP_K[tau][s] = alpha(tau) + sum_d U[s][d] v_tau[d] + sum_{t >= tau} W[t][s] M[tau][t]
            {
                f32x4 alpha[2], tdA;  // alpha(tau): the suffix from this tile on
                suffix_totals(dA, al, alpha, tdA);
                const UOps<T, HL> uo(Ut);
                for (int nt = 0; nt < 2; ++nt) {
                    dPK[nt] = alpha[nt];
                    uo.template apply<NL>(dPK[nt], sV, nt);
                    const Frag<T> yo = ld_frag_pi(sY + (16 * nt + i) * LDT);
                    mma(dPK[nt], Wf, yo);
                    if constexpr (HL || WM) mma(dPK[nt], Wl, yo);
                }
                for (int e = 0; e < 4; ++e) al[e] += tdA[e];
            }
            // ---- U^T[d][s] += sum_t g[t][d] W[t][s]  (the dV tiles read the LDS copy of U)
            for (int md = 0; md < 4; ++md) {
                const Frag<T> go = col_operand<T, NL>(sG, sGt, md);
                mma(Ut[md], go, Wf);
                if constexpr (HL) mma(Ut[md], go, Wl);
            }
            if constexpr (SCN) {
                // the tile's three Sc2 blocks, once each, for its dV tiles in
                // the next iteration
                for (int r = w; r < 3; r += NW_) sc2_tile<T, SP>(r, sWts, sPts, sSc2);
                // and the carried part of its dV tiles (U and P_K rows of this tile)
#pragma unroll
                for (int k = 0; k < NQD; ++k)
                    if (w + k * NW_ < 8) dvacc[k] = dv_part<T, SP>((w + k * NW_) >> 1, (w + k * NW_) & 1, sUT, sPts);
            } else {
                for (int q = w; q < 8; q += NW_)
                    dv_tile<T, SP, CAUSAL, AL>(q >> 1, q & 1, sUT, sPts, sWts, sG, sGt, dvp, a.sg.t, t0, a.T, vpart);
            }
        } else {
            __syncthreads();  // all waves' P_K rows in LDS
            if constexpr (NB == 2) commit((int)((jr + 1) & 1));
            // non-causal: dV^T = U^T P_K^T; dP_K = alpha + v . U (totals)
            for (int q = w; q < 8; q += NW_)
                dv_tile<T, SP, CAUSAL, AL>(q >> 1, q & 1, sUT, sPts, nullptr, nullptr, nullptr, dvp, a.sg.t, t0, a.T, vpart);
            const UOps<T, HL> uo(Ut);
            for (int nt = 0; nt < 2; ++nt) {
                f32x4 c = zero4();
                uo.template apply<NL>(c, sV, nt);
                for (int e = 0; e < 4; ++e) dPK[nt][e] = (c[e] + al[e]) * kwt[nt];  // through the key weight
            }
        }
        {
            if constexpr (KB <= 4) {
                tsum += softhash_bwd<KB, T, PR>(PKraw, dPK, sSpK, sSmK, sThK, sg, a.L, a.inv_temp, sDproj, ho);
            } else {
                softhash_share<KB, T>(PKraw, dPK, wh, sShare);
                __syncthreads();
                tsum += softhash_combine<KB, T, SP, NTH, PR>(sShare, sSpK, sSmK, sThK, z, a.L, a.inv_temp, sDproj);
            }
        }
        // P2: tile j - 1's projections (its Q and K rows arrived in the second
        // phase), for the next iteration
        if constexpr (P2) project2((jr + 1) & 1, (jr + 1) & 1);
        // one token block: the next tile's rows go to it after the tile's
        // last barrier.  The tile's dK is stored in the next iteration (or
        // after the loop).
        if constexpr (NB == 1) {
            __syncthreads();
            commit(0);
        }
    }
    if (j0 < j1) {
        if constexpr (NB == 2) __syncthreads();  // every wave's dproj (and Sc2) rows of the last tile
        dx_store<T, NW_, XC, AL, XF>(sDproj, sPlT, dkp, a.sg.t, (int64_t)j0 * TT, a.T, xpart, xc0);
        if constexpr (SCN) {
            const T *gtn = (const T *)(smem + (j0 & 1) * Ly::TB + Ly::oGt);
            const T *gnn = (const T *)(smem + (j0 & 1) * Ly::TB + Ly::oG);
#pragma unroll
            for (int k = 0; k < NQD; ++k)
                if (w + k * NW_ < 8)
                    dv_finish<T, AL>((w + k * NW_) >> 1, (w + k * NW_) & 1, dvacc[k], gnn, gtn, sSc2, dvp, a.sg.t, (int64_t)j0 * TT, a.T,
                                 vpart);
        }
    }
    const double ts = block_sum_f64<NTH>((double)tsum, sRed);
    if (threadIdx.x == 0) a.tpart[((int64_t)(a.M * a.B * a.H + n) * a.nseg + seg) * a.nslice + z] = ts;
}

// =====================================================================
// Bucket probabilities as an output (for hybrid consumers): P[n][t][s],
// s = l*2^K + r, fp32, from one input x (q's pointer and strides); and the
// backward dP -> dx (dq's pointer and strides; sliced instantiations write
// fp32 partials) with the temperature-gradient partials.
// =====================================================================
// One layout for both directions, except the end-of-kernel block sum's
// scratch [64 * NW_]: the backward reuses its sigmoid rows for it (the last
// tile reads them before its last barrier), which brings it to 4 workgroups
// per CU (backward 1.52 -> 1.38 ms at C4's shape, K=4); the forward, which has
// no block sum, keeps a region of that size, since smaller forward layouts (4
// or 6 workgroups per CU) measured 2.5% slower.
template <typename T, int SP, bool BWD> struct ProbsL {
    static constexpr int NW_ = SP / WB;
    static constexpr int LDN = NatL<T, true>::LD, LDC = ld_of<float>(NCOL), LDDP = sw_ld<T, NCOL>();
    static constexpr size_t oX = 0;
    static constexpr size_t oPl = align16(oX + sizeof(T) * TT * LDN);
    static constexpr size_t oPlLo = align16(oPl + sizeof(T) * NCOL * LDN);
    static constexpr size_t oPlT = align16(oPlLo + sizeof(T) * NCOL * LDN);
    static constexpr size_t oDproj = align16(oPlT + sizeof(T) * D * LDDP);
    static constexpr size_t oSig = align16(oDproj + sizeof(T) * TT * LDDP);  // sp, sm, th
    static_assert(64 * NW_ <= 3 * TT * LDC, "block-sum scratch inside the sigmoid rows");
    static constexpr size_t oRed = BWD ? oSig : align16(oSig + sizeof(float) * 3 * TT * LDC);
    static constexpr size_t oHash = align16(oSig + sizeof(float) * 3 * TT * LDC + (BWD ? 0 : sizeof(float) * 64 * NW_));
    static constexpr size_t oShare = align16(oHash + HashOps<T, 4>::bytes);
    template <int KB> static constexpr size_t bytes() {
        return align16(oShare + (KB > 4 ? WideHash<T, KB>::bytes(NW_) : 0));
    }
};

// the lane's 4 buckets (s0 .. s0+3) of token row p (S fp32 per row)
__device__ __forceinline__ void store_row4(float *row, int s0, int S, const f32x4 &v) {
    if ((S & 3) == 0) {
        if (s0 < S) *reinterpret_cast<f32x4 *>(row + s0) = v;
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (s0 + e < S) row[s0 + e] = v[e];
    }
}
__device__ __forceinline__ f32x4 load_row4(const float *row, int s0, int S) {
    f32x4 v = zero4();
    if ((S & 3) == 0) {
        if (s0 < S) v = *reinterpret_cast<const f32x4 *>(row + s0);
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (s0 + e < S) v[e] = row[s0 + e];
    }
    return v;
}

template <typename T, int SP, int KB, bool BWD>
__global__ __launch_bounds__(threads_of(SP)) void k_probs(Args a) {
    if (a.inv_temp_ptr) a.inv_temp = *a.inv_temp_ptr;  // uniform scalar load
    using Ly = ProbsL<T, SP, BWD>;
    using NL = NatL<T, true>;
    constexpr int NW_ = Ly::NW_, NTH = 64 * NW_, LDC = Ly::LDC, LDDP = Ly::LDDP;
    __shared__ __align__(16) unsigned char smem[Ly::template bytes<KB>()];
    T *sX = (T *)(smem + Ly::oX), *sPl = (T *)(smem + Ly::oPl), *sPlLo = (T *)(smem + Ly::oPlLo);
    T *sPlT = (T *)(smem + Ly::oPlT), *sDproj = (T *)(smem + Ly::oDproj);
    float *sSp = (float *)(smem + Ly::oSig), *sSm = sSp + TT * LDC, *sTh = sSp + 2 * TT * LDC;
    float *sRed = (float *)(smem + Ly::oRed), *sShare = (float *)(smem + Ly::oShare);
    const WgPos wp = wg_pos(a.nseg, a.M * a.B * a.H, a.nslice, sliced<T, KB>());
    if (!wp.live) return;
    const int w = wave_id(), g = lg(), i = li(), sw = WB * w, z = wp.z,
              sg = z * SP + sw;
    const PlaneBlocks pbk(z, SP, KB, a.L, !sliced<T, KB>());  // projection columns of this slice
    const int n = wp.n, seg = wp.seg;
    const int m = n / (a.B * a.H);
    const int ntiles = (int)((a.T + TT - 1) / TT);  // the host bounds T by 2^35
    const int lastv = (int)(a.T - (int64_t)(ntiles - 1) * TT);  // rows of the last tile
    const int j0 = seg * a.tps, j1 = min(ntiles, j0 + a.tps);
    const T *xp = (const T *)a.q + stream_off(a.sq, n, a.B, a.H);
    T *dxp = BWD ? (T *)a.dq + stream_off(a.sg, n, a.B, a.H) : nullptr;
    constexpr int XC = xcols_of(SP, KB);
    constexpr bool XF = xpart_f32(is_bf16<T>(), SP, KB);
    void *xpart = BWD && sliced<T, KB>() ? xpart_at<T, SP, KB>(a.dqpart, z, n, a) : nullptr;
    const int xc0 = ((z * SP) >> KB) * KB;  // first projection column of the slice's tables

    HashOps<T, KB> ho;
    WideHash<T, KB> wh;
    if constexpr (BWD) {
        if constexpr (KB <= 4)
            ho.init((T *)(smem + Ly::oHash), NTH);
        else
            wh.init(sg);
        zero_lds<T>(sDproj, TT * LDDP, NTH);
    }
    load_planes<T, NTH, NL>(a.planes + m * a.planes_m_stride, a.L * a.K, sPl, is_bf16<T>() ? sPlLo : nullptr,
                            BWD ? sPlT : nullptr);
    if constexpr (BWD && KB <= 4) {
        __syncthreads();  // the hash table in LDS; its operand to registers
        ho.cache();
    }
    CarryA<T> tsum = 0;  // this thread's share of sum du * th
    Prefetch<T, NTH> px_;
    if (j0 < j1) px_.issue(xp, a.sq.t, (int64_t)j0 * TT, a.T);
    for (int jt = j0; jt < j1; ++jt) {
        const int64_t t0 = (int64_t)jt * TT;
        __syncthreads();  // the previous tile's readers of sX, sSig, sDproj are done
        px_.template commit<NL>(sX, nullptr);
        if (jt + 1 < j1) px_.issue(xp, a.sq.t, t0 + TT, a.T);  // next tile, in flight during this one
        __syncthreads();
        for (int q = w; q < pbk.tasks(); q += NW_) {
            project_tile<T, NL>(sX, sPl, sPlLo, pbk.mc(q), q & 1, a.inv_temp, sSp, sSm, BWD ? sTh : nullptr);
        }
        __syncthreads();
        f32x4 P[2];
        probs_st<KB>(sSp, sSm, sg, a.S, jt + 1 < ntiles ? TT : lastv, P);
        const int s0 = sg + 4 * g;
        if constexpr (!BWD) {
            for (int nt = 0; nt < 2; ++nt) {
                const int64_t t = t0 + 16 * nt + i;
                if (t < a.T) store_row4(a.probs + ((int64_t)n * a.T + t) * a.S, s0, a.S, P[nt]);
            }
        } else {
            f32x4 dP[2];
            for (int nt = 0; nt < 2; ++nt) {
                const int64_t t = t0 + 16 * nt + i;
                dP[nt] = t < a.T ? load_row4(a.dprobs + ((int64_t)n * a.T + t) * a.S, s0, a.S) : zero4();
            }
            if constexpr (KB <= 4) {
                tsum += softhash_bwd<KB, T>(P, dP, sSp, sSm, sTh, sg, a.L, a.inv_temp, sDproj, ho);
            } else {
                softhash_share<KB, T>(P, dP, wh, sShare);
                __syncthreads();
                tsum += softhash_combine<KB, T, SP, NTH>(sShare, sSp, sSm, sTh, z, a.L, a.inv_temp, sDproj);
            }
            __syncthreads();
            dx_store<T, NW_, XC, false, XF>(sDproj, sPlT, dxp, a.sg.t, t0, a.T, xpart, xc0);
        }
    }
    if constexpr (BWD) {
        const double ts = block_sum_f64<NTH>((double)tsum, sRed);
        if (threadIdx.x == 0) a.tpart[((int64_t)n * a.nseg + seg) * a.nslice + z] = ts;
    }
}

// Partials are read once: nontemporal loads keep them from displacing other
// lines in the caches (measured faster).  4 consecutive elements as fp32.
__device__ __forceinline__ f32x4 part4(const float *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
}
__device__ __forceinline__ f32x4 part4(const bf16 *p) {
    const u32x2 u = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p));
    return f32x4{__uint_as_float(u[0] << 16), __uint_as_float(u[0] & 0xFFFF0000u), __uint_as_float(u[1] << 16),
                 __uint_as_float(u[1] & 0xFFFF0000u)};
}

// The element-wise kernels below run a grid-stride loop over their items:
// their grids are capped at ELEM_BLOCKS workgroups of ELEM_THREADS (one pass
// below N * T of about 2^26 token-heads), so a launch stays far below the
// dispatch packet's 2^32 work-items at any size.
constexpr int ELEM_THREADS = 256;
constexpr int64_t ELEM_BLOCKS = 1 << 20;
__host__ __device__ constexpr unsigned elem_blocks(int64_t items) {
    const int64_t b = (items + ELEM_THREADS - 1) / ELEM_THREADS;
    return (unsigned)(b < ELEM_BLOCKS ? (b > 0 ? b : 1) : ELEM_BLOCKS);
}

// Sum of the per-slice partials [nslice][N][T][D] (element type T) in slice
// order, in fp32, written to the strided output (4 consecutive d per item).
template <typename T>
__global__ __launch_bounds__(ELEM_THREADS) void k_slice_sum(const T *part, int nslice, int64_t N, int64_t Tn, int B,
                                                            int H, Strides so, T *out) {
    const int64_t per = Tn * (D / 4), items = N * per;  // over N * T * D/4
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < items;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t n = idx / per, r = idx % per, t = r / (D / 4);
        const int d0 = 4 * (int)(r % (D / 4));
        const int64_t row = (n * Tn + t) * D + d0, zs = N * Tn * D;
        f32x4 acc = part4(part + row);
        for (int z = 1; z < nslice; ++z) acc += part4(part + z * zs + row);
        store4<T>(out + stream_off(so, (int)n, B, H) + t * so.t + d0, acc);
    }
}

// The same for bf16 partials and a slice count NS known at compile time (8:
// the 8-bit slices of 4 tables): 8 consecutive d per item, 16-byte loads of
// every slice issued together, one 16-byte store.
__device__ __forceinline__ void part8(const bf16 *p, f32x4 &lo, f32x4 &hi) {
    const u32x4 u = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    lo = f32x4{__uint_as_float(u[0] << 16), __uint_as_float(u[0] & 0xFFFF0000u), __uint_as_float(u[1] << 16),
               __uint_as_float(u[1] & 0xFFFF0000u)};
    hi = f32x4{__uint_as_float(u[2] << 16), __uint_as_float(u[2] & 0xFFFF0000u), __uint_as_float(u[3] << 16),
               __uint_as_float(u[3] & 0xFFFF0000u)};
}
template <int NS>
__global__ __launch_bounds__(ELEM_THREADS) void k_slice_sum8(const bf16 *part, int64_t N, int64_t Tn, int B, int H,
                                                             Strides so, bf16 *out) {
    const int64_t per = Tn * (D / 8), items = N * per;  // over N * T * D/8
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < items;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t n = idx / per, r = idx % per, t = r / (D / 8);
        const int d0 = 8 * (int)(r % (D / 8));
        const int64_t row = (n * Tn + t) * D + d0, zs = N * Tn * D;
        f32x4 lo[NS], hi[NS];
#pragma unroll
        for (int z = 0; z < NS; ++z) part8(part + z * zs + row, lo[z], hi[z]);
        f32x4 a = lo[0], b = hi[0];
#pragma unroll
        for (int z = 1; z < NS; ++z) {
            a += lo[z];
            b += hi[z];
        }
        bf16 *o = out + stream_off(so, (int)n, B, H) + t * so.t + d0;
        store4<bf16>(o, a);
        store4<bf16>(o + 4, b);
    }
}

// dX of sliced instantiations: out[n][t][:] = sum over slices z (in order)
// of part[z][n][t][:] . planes[m][c0(z) ..][:] -- per slice one product of
// its dproj columns with planes^T on the matrix cores, the same operands
// (bf16 for bf16 inputs) and fp32 accumulation as dx_store's unsliced path.
// part rows hold XC columns; slice z's columns start at c0(z) = l0(z) K,
// l0(z) = (z SP) >> K, and end at its last table's (at most L K).  One wave
// per DXF_BLK 16-token blocks of a stream (the planes^T operand is loaded
// once per wave): lane (g, i) holds token i, columns 8g .. 8g+7.
constexpr int DXF_BLK = 4;
template <typename T>
__global__ __launch_bounds__(256) void k_dx_finish(const T *part, int nslice, int XC, int SP, int KB, int L,
                                                   const float *planes, int64_t planes_m_stride, int B, int H,
                                                   int64_t N, int64_t Tn, Strides so, T *out) {
    const int64_t wv = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;  // over N * ceil(T / 64)
    const int64_t nblk = (Tn + 16 * DXF_BLK - 1) / (16 * DXF_BLK);
    if (wv >= N * nblk) return;  // whole waves
    const int64_t n = wv / nblk, tw = (wv % nblk) * 16 * DXF_BLK;
    const int g = lg(), i = li();
    const float *pl = planes + (n / (B * H)) * planes_m_stride;
    const int LK = L * KB;
    // planes^T operand of each 16-wide d block: column c = 8g + j, d = 16md + i
    Frag<T> pt[4];
#pragma unroll
    for (int md = 0; md < 4; ++md) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = 8 * g + j < LK ? pl[(int64_t)(8 * g + j) * D + 16 * md + i] : 0.f;
        pt[md] = frag_seq<T>(v);
    }
    for (int tb = 0; tb < DXF_BLK; ++tb) {
    const int64_t t0 = tw + 16 * tb;
    if (t0 >= Tn) break;
    f32x4 acc[4] = {zero4(), zero4(), zero4(), zero4()};
    const int64_t t = t0 + i;
    for (int z = 0; z < nslice; ++z) {
        const int c0 = ((z * SP) >> KB) * KB;
        const int c1 = min(LK, ((((z + 1) * SP - 1) >> KB) + 1) * KB);
        const T *row = part + ((int64_t)z * N * Tn + n * Tn + t) * XC;
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int c = 8 * g + j;
            v[j] = (t < Tn && c >= c0 && c < c1) ? to_f32(row[c - c0]) : 0.f;
        }
        const Frag<T> a = frag_seq<T>(v);
#pragma unroll
        for (int md = 0; md < 4; ++md) mma(acc[md], a, pt[md]);
    }
    // lane (g, i) holds dX[t0 + 4g + e][16md + i]
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int64_t tt = t0 + 4 * g + e;
        if (tt < Tn)
#pragma unroll
            for (int md = 0; md < 4; ++md)
                out[stream_off(so, (int)n, B, H) + tt * so.t + 16 * md + i] = from_f32<T>(acc[md][e]);
    }
    }
}

// dX for bf16 8-bit hashes in slices of 128 buckets: two slices per table
// (slice z holds table z >> 1's 8 columns as fp32 rows, 32 bytes a token), at
// most 4 tables.  Lane (g, i) takes token i and table g's columns: the sum of
// slices 2g and 2g + 1 in fp32 (partials that may cancel, added before any
// rounding), as an fp32-accurate hi + lo bf16 pair (frag_acc_hilo), against
// planes^T rounded to bf16 as in the unsliced kernels.  The product is dX^T,
// with row r of block md holding d = 4r + md: lane (g, i) ends with
// d = 16g .. 16g + 15 of token i (acc[md][e] is d = 16g + 4e + md), stored as
// two 16-byte pieces (fp32 accumulation; the tables' sums meet inside each
// product).
__global__ __launch_bounds__(256) void k_dx_finish8(const float *part, int L, const float *planes,
                                                    int64_t planes_m_stride, int B, int H, int64_t N, int64_t Tn,
                                                    Strides so, bf16 *out) {
    const int64_t wv = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;  // over N * ceil(T / 64)
    const int64_t nblk = (Tn + 16 * DXF_BLK - 1) / (16 * DXF_BLK);
    if (wv >= N * nblk) return;  // whole waves
    const int64_t n = wv / nblk, tw = (wv % nblk) * 16 * DXF_BLK;
    const int g = lg(), i = li();
    const bool live = g < L;  // table g exists
    const float *pl = planes + (n / (B * H)) * planes_m_stride;
    // planes^T operand of block md: column c = 8g + j, row i = d 4i + md
    Frag<bf16> pt[4];
#pragma unroll
    for (int md = 0; md < 4; ++md) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = live ? pl[(int64_t)(8 * g + j) * D + 4 * i + md] : 0.f;
        pt[md] = frag_seq<bf16>(v);
    }
    const int64_t zs = N * Tn * 8;  // elements per slice
    bf16 *op = out + stream_off(so, (int)n, B, H);
    for (int tb = 0; tb < DXF_BLK; ++tb) {
        const int64_t t0 = tw + 16 * tb;
        if (t0 >= Tn) break;
        const int64_t t = t0 + i;
        f32x4 x0 = zero4(), x1 = zero4();
        if (live && t < Tn) {
            const float *row = part + 2 * g * zs + (n * Tn + t) * 8;
            x0 = *reinterpret_cast<const f32x4 *>(row) + *reinterpret_cast<const f32x4 *>(row + zs);
            x1 = *reinterpret_cast<const f32x4 *>(row + 4) + *reinterpret_cast<const f32x4 *>(row + zs + 4);
        }
        Frag<bf16> hi, lo;
        frag_acc_hilo(x0, x1, hi, lo);
        f32x4 acc[4];
#pragma unroll
        for (int md = 0; md < 4; ++md) {
            acc[md] = zero4();
            mma(acc[md], pt[md], hi);
            mma(acc[md], pt[md], lo);
        }
        if (t < Tn) {
            float v[8];
#pragma unroll
            for (int h = 0; h < 2; ++h) {  // d = 16g + 8h .. + 7
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = acc[j & 3][2 * h + (j >> 2)];
                *reinterpret_cast<Frag<bf16> *>(op + t * so.t + 16 * g + 8 * h) = frag_seq<bf16>(v);
            }
        }
    }
}

// den [N][T] = sum of the per-slice partials [nslice][N][T], in slice order.
__global__ __launch_bounds__(ELEM_THREADS) void k_den_sum(const float *denpart, int nslice, int64_t NT, float *den) {
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < NT;
         idx += (int64_t)gridDim.x * blockDim.x) {
        float dn = denpart[idx];
        for (int z = 1; z < nslice; ++z) dn += denpart[z * NT + idx];
        den[idx] = dn;
    }
}

// Global normalisation, sliced instantiations: out = (sum of the slices'
// numerator partials) / max(den, eps), den = sum of the slices' den partials
// [nslice][N][T] (slice order), also written to den [N][T].
template <typename T>
__global__ __launch_bounds__(ELEM_THREADS) void k_slice_sum_gn(const T *part, const float *denpart, int nslice,
                                                               int64_t N, int64_t Tn, int B, int H, Strides so, T *out,
                                                               float *den, float eps) {
    const int64_t per = Tn * (D / 4), items = N * per;  // over N * T * D/4
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < items;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t n = idx / per, r = idx % per, t = r / (D / 4);
        const int d0 = 4 * (int)(r % (D / 4));
        const int64_t row = (n * Tn + t) * D + d0, zs = N * Tn * D, nt = n * Tn + t;
        f32x4 acc = part4(part + row);
        float dn = denpart[nt];
        for (int z = 1; z < nslice; ++z) {
            acc += part4(part + z * zs + row);
            dn += denpart[z * N * Tn + nt];
        }
        const float rc = 1.0f / fmaxf(dn, eps);
        store4<T>(out + stream_off(so, (int)n, B, H) + t * so.t + d0, acc * rc);
        if (d0 == 0) den[nt] = dn;
    }
}

// Bucket-slice GN backward: per token j = n T + t, the slices' shares of
// S = sum_s P_Q G added in slice order, rd = 1 / max(den, eps) and
// gd = dden - [den >= eps] rd^2 S, read by the second k_bwd_reduce pass and
// by k_bwd_out.
__global__ __launch_bounds__(ELEM_THREADS) void k_gn_terms(const float *gsum, int nslice, int64_t NT, const float *den,
                                                           const float *dden, float eps, float *rden, float *gden) {
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < NT; j += (int64_t)gridDim.x * blockDim.x) {
        float sq = gsum[j];
        for (int z = 1; z < nslice; ++z) sq += gsum[z * NT + j];
        const float dn = den[j], rd = 1.0f / fmaxf(dn, eps);
        rden[j] = rd;
        gden[j] = (dden ? dden[j] : 0.f) - (dn >= eps ? rd * rd * sq : 0.f);
    }
}

// grad_inv_temp = sum of all partials, in a fixed order
__global__ void k_temp_sum(const double *tpart, int64_t count, float *out) {
    __shared__ double red[256];
    double acc = 0.0;
    for (int64_t j = threadIdx.x; j < count; j += blockDim.x) acc += tpart[j];
    red[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        double s = 0.0;
        for (int j = 0; j < (int)blockDim.x; ++j) s += red[j];
        *out = (float)s;
    }
}

} // namespace race
