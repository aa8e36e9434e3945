// race_kernels.hip -- gfx950 kernels of the RACE attention operator.
//
// Work decomposition.  A stream n = (m, b, h) is a sequence of T tokens.  It
// is cut into 32-token tiles; consecutive tiles form segments, and one
// 256-thread workgroup walks one (segment, stream) pair.  Per bucket s the
// causal state is the prefix pair (A_s, B_s) = (sum P_K, sum P_K v); inside a
// tile the prefix is rebuilt from the state at the tile start plus a masked
// 32x32 triangle (W = P_Q/(A+eps); O = W B_start + tril(W P_K^T) V).  Across
// tiles the state is carried in MFMA accumulators, across segments by a
// three-phase scan:
//   forward   k_fwd_reduce  per-segment sums of (A,B)        reads K,V
//             k_fwd_scan    exclusive segment prefixes (fp64, kept as state)
//             k_fwd_out     outputs                          reads Q,K,V writes O
//   backward  k_bwd_reduce  forward walk: dQ, per-segment sums of
//                           (alpha, U) = (sum dA, sum W^T g)  reads Q,K,V,dO
//             k_bwd_scan    exclusive segment suffixes
//             k_bwd_out     reverse walk: dK, dV             reads Q,K,V,dO
// The reverse walk of k_bwd_out needs the forward state at every tile start;
// it subtracts each tile's (A,B) sum, recomputed exactly as k_fwd_reduce
// computed it, from the segment's end state in fp64.
// The non-causal operator uses the same kernels with the prefix replaced by
// the full-sequence sums and no triangle terms.
//
// Bucket probabilities are recomputed from Q/K in every kernel (projection on
// MFMA, tanh, then P[t,l,r] = prod_k sigmoid(+-2u_k), which equals the
// reference's softmax over the 2^K corner logits).
#include "race_device.h"

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
    int nseg, tps;   // segments per stream, tiles per segment
    double *fstate;  // [N][nseg+1][SP][D+1] exclusive segment prefixes; [nseg] = totals
    double *fdelta;  // [N][nseg][SP][D+1]
    float *rdelta;   // [N][nseg][SP][D+1]  per-segment (U, alpha) sums
    float *rstate;   // [N][nseg][SP][D+1]  exclusive suffixes (non-causal: totals)
    float *tpart;    // [2][N][nseg] partial sums of dU*th
};

constexpr int SROW = D + 1; // state row: D values of B (or U) then A (or alpha)

__device__ __forceinline__ int64_t stream_off(const Strides &s, int n, int B, int H) {
    const int h = n % H, b = (n / H) % B, m = n / (H * B);
    return (int64_t)m * s.m + (int64_t)b * s.b + (int64_t)h * s.h;
}

__host__ __device__ constexpr size_t align16(size_t x) { return (x + 15) & ~(size_t)15; }
__host__ __device__ constexpr size_t cmax(size_t a, size_t b) { return a > b ? a : b; }

// --------------------------------------------------------------- tile I/O
// Load a [TT][D] token tile (rows t0.. of a stream, row stride st elements);
// rows at or beyond T read as zero.  nat: [TT][ld_of<T>(D)], trn: [D][ld_of<T>(TT)].
template <typename T>
__device__ void load_tile(const T *__restrict__ src, int64_t st, int64_t t0, int64_t Tn, T *nat, T *trn) {
    constexpr int EPC = 16 / sizeof(T);
    constexpr int CPR = D / EPC;
    constexpr int LDN = ld_of<T>(D), LDT = ld_of<T>(TT);
    for (int idx = threadIdx.x; idx < TT * CPR; idx += NT) {
        const int t = idx / CPR, c = idx % CPR;
        uint4 val = make_uint4(0, 0, 0, 0);
        if (t0 + t < Tn) val = *reinterpret_cast<const uint4 *>(src + (t0 + t) * st + c * EPC);
        if (nat) *reinterpret_cast<uint4 *>(nat + t * LDN + c * EPC) = val;
        if (trn) {
            const T *e = reinterpret_cast<const T *>(&val);
#pragma unroll
            for (int j = 0; j < EPC; ++j) trn[(c * EPC + j) * LDT + t] = e[j];
        }
    }
}

// Store a staged [TT][ld_of<T>(D)] tile to rows t0.. (< T) of a stream.
template <typename T>
__device__ void store_tile(T *__restrict__ dst, int64_t st, int64_t t0, int64_t Tn, const T *stage) {
    constexpr int EPC = 16 / sizeof(T);
    constexpr int CPR = D / EPC;
    constexpr int LDN = ld_of<T>(D);
    for (int idx = threadIdx.x; idx < TT * CPR; idx += NT) {
        const int t = idx / CPR, c = idx % CPR;
        if (t0 + t < Tn)
            *reinterpret_cast<uint4 *>(dst + (t0 + t) * st + c * EPC) =
                *reinterpret_cast<const uint4 *>(stage + t * LDN + c * EPC);
    }
}

template <typename T> constexpr bool is_bf16() { return sizeof(T) == 2; }

// Planes [L*K][D] fp32 -> LDS.  pl/pllo: [NCOL][ld_of<T>(D)] (bf16 keeps a
// hi/lo split so the projection is close to fp32), plt: [D][ld_of<T>(NCOL)].
template <typename T>
__device__ void load_planes(const float *__restrict__ planes, int LK, T *pl, T *pllo, T *plt) {
    constexpr int LDN = ld_of<T>(D), LDC = ld_of<T>(NCOL);
    for (int idx = threadIdx.x; idx < NCOL * D; idx += NT) {
        const int c = idx / D, d = idx % D;
        const float w = c < LK ? planes[c * D + d] : 0.f;
        const T hi = from_f32<T>(w);
        if (pl) pl[c * LDN + d] = hi;
        if (pllo) pllo[c * LDN + d] = from_f32<T>(w - to_f32(hi));
        if (plt) plt[d * LDC + c] = hi;
    }
}

// One 16x16 projection tile (rows 16*mt.., columns 16*nc..) of X . planes^T,
// then th = tanh, the sigmoid pair of 2*th*inv_temp into sp/sm [TT][ld_of<float>(NCOL)]
// and (optionally) th into sth.
template <typename T>
__device__ void project_tile(const T *sx, const T *pl, const T *pllo, int mt, int nc, float inv_temp,
                             float *sp, float *sm, float *sth) {
    constexpr int LDN = ld_of<T>(D), LDC = ld_of<float>(NCOL);
    f32x4 acc = zero4();
    tile_mma(acc, sx + 16 * mt * LDN, LDN, pl + 16 * nc * LDN, LDN, D / 32);
    if constexpr (is_bf16<T>()) tile_mma(acc, sx + 16 * mt * LDN, LDN, pllo + 16 * nc * LDN, LDN, D / 32);
    const int i = lane_id() & 15, g = lane_id() >> 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int t = 16 * mt + 4 * g + e, c = 16 * nc + i;
        const float th = tanhf(acc[e]);
        float a, b;
        sigmoid_pair(2.f * th * inv_temp, a, b);
        sp[t * LDC + c] = a;
        sm[t * LDC + c] = b;
        if (sth) sth[t * LDC + c] = th;
    }
}

// Bucket probability P[t, s] from the sigmoid tables; s = l*R + r.
__device__ __forceinline__ float prob_at(const float *sp, const float *sm, int t, int s, int K) {
    constexpr int LDC = ld_of<float>(NCOL);
    const int l = s >> K, r = s & ((1 << K) - 1);
    const float *p = sp + t * LDC + l * K;
    const float *q = sm + t * LDC + l * K;
    float v = 1.f;
    for (int k = 0; k < K; ++k) v *= ((r >> (K - 1 - k)) & 1) ? p[k] : q[k];
    return v;
}

// P_K of a tile into pk [TT][ld_of<T>(SP)] and/or pkt [SP][ld_of<T>(TT)];
// zero for padded buckets (s >= S) and tokens at or beyond T.
template <typename T, int SP>
__device__ void softhash_tile(const float *sp, const float *sm, int K, int S, int64_t t0, int64_t Tn, T *pk,
                              T *pkt) {
    constexpr int LDP = ld_of<T>(SP), LDT = ld_of<T>(TT);
    for (int idx = threadIdx.x; idx < TT * SP; idx += NT) {
        const int s = idx % SP, t = idx / SP;
        float p = 0.f;
        if (s < S && t0 + t < Tn) p = prob_at(sp, sm, t, s, K);
        const T pv = from_f32<T>(p);
        if (pk) pk[t * LDP + s] = pv;
        if (pkt) pkt[s * LDT + t] = pv;
    }
}

// Softmax/corner/tanh backward of one tile: dP [TT][ld_of<float>(SP)] ->
// dproj [TT][ld_of<T>(NCOL)] (columns < L*K); returns this thread's sum of du*th.
template <typename T, int SP>
__device__ float softhash_bwd_tile(const float *sp, const float *sm, const float *sth, const float *dP, int L,
                                   int K, int64_t t0, int64_t Tn, float inv_temp, T *dproj) {
    constexpr int LDC = ld_of<float>(NCOL), LDA = ld_of<float>(SP), LDDP = ld_of<T>(NCOL);
    const int R = 1 << K;
    float tsum = 0.f;
    for (int idx = threadIdx.x; idx < TT * L; idx += NT) {
        const int t = idx / L, l = idx % L;
        float du[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) du[k] = 0.f;
        if (t0 + t < Tn) {
            float dot = 0.f;
            for (int r = 0; r < R; ++r) dot += prob_at(sp, sm, t, l * R + r, K) * dP[t * LDA + l * R + r];
            for (int r = 0; r < R; ++r) {
                const float w = prob_at(sp, sm, t, l * R + r, K) * (dP[t * LDA + l * R + r] - dot);
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    if (k < K) du[k] += ((r >> (K - 1 - k)) & 1) ? w : -w;
            }
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if (k < K) {
                const float th = sth[t * LDC + l * K + k];
                tsum += du[k] * th;
                dproj[t * LDDP + l * K + k] = from_f32<T>(du[k] * inv_temp * (1.f - th * th));
            }
        }
    }
    return tsum;
}

// dX tile = dproj . planes  (rows 16*mt, cols 16*nd), into a staging tile.
template <typename T>
__device__ void dx_tile(const T *dproj, const T *plt, int mt, int nd, T *stage) {
    constexpr int LDDP = ld_of<T>(NCOL), LDN = ld_of<T>(D);
    f32x4 acc = zero4();
    tile_mma(acc, dproj + 16 * mt * LDDP, LDDP, plt + 16 * nd * LDDP, LDDP, NCOL / 32);
    st_tile(stage + 16 * mt * LDN + 16 * nd, LDN, acc);
}

// Sum of a wave-ordered per-thread value over the workgroup (fixed order).
__device__ float block_sum(float v, float *scratch) {
    scratch[threadIdx.x] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        float s = 0.f;
        for (int j = 0; j < NT; ++j) s += scratch[j];
        scratch[0] = s;
    }
    __syncthreads();
    const float r = scratch[0];
    __syncthreads();
    return r;
}

// The carry tiles of a wave: q = wave + NW*j, (ms, nd) = (q / 4, q % 4) over
// the [SP][D] state.  Lane holds state[16ms + 4g + e][16nd + i].
template <int SP> struct Carry {
    static constexpr int NTL = SP / 16 * 4 / NW;
    __device__ static int ms(int j) { return (wave_id() + NW * j) >> 2; }
    __device__ static int nd(int j) { return (wave_id() + NW * j) & 3; }
};

// One tile's (A,B) sums: dB = P_K^T V for this wave's carry tiles (fp32 MFMA
// from zero) -- shared by k_fwd_reduce and k_bwd_out so that both get
// bit-identical values.
template <typename T, int SP>
__device__ __forceinline__ f32x4 tile_dB(const T *pkt, const T *vt, int j) {
    constexpr int LDT = ld_of<T>(TT);
    f32x4 c = zero4();
    tile_mma(c, pkt + 16 * Carry<SP>::ms(j) * LDT, LDT, vt + 16 * Carry<SP>::nd(j) * LDT, LDT, 1);
    return c;
}
// ... and the per-bucket A sum, summed in token order by thread s.
template <typename T>
__device__ __forceinline__ float tile_dA(const T *pkt, int s) {
    constexpr int LDT = ld_of<T>(TT);
    float run = 0.f;
    for (int t = 0; t < TT; ++t) run += to_f32(pkt[s * LDT + t]);
    return run;
}

// =====================================================================
// k_fwd_reduce: per-segment (A, B) sums (fp64 over fp32 tile sums).
// =====================================================================
template <typename T, int SP> struct FwdReduceL {
    static constexpr int LDN = ld_of<T>(D), LDT = ld_of<T>(TT), LDC = ld_of<float>(NCOL);
    static constexpr size_t oK = 0;
    static constexpr size_t oVt = align16(oK + sizeof(T) * TT * LDN);
    static constexpr size_t oPkt = align16(oVt + sizeof(T) * D * LDT);
    static constexpr size_t oPl = align16(oPkt + sizeof(T) * SP * LDT);
    static constexpr size_t oPlLo = align16(oPl + sizeof(T) * NCOL * LDN);
    static constexpr size_t oSp = align16(oPlLo + sizeof(T) * NCOL * LDN);
    static constexpr size_t oSm = align16(oSp + sizeof(float) * TT * LDC);
    static constexpr size_t bytes = align16(oSm + sizeof(float) * TT * LDC);
};

template <typename T, int SP>
__global__ __launch_bounds__(NT) void k_fwd_reduce(Args a) {
    using Ly = FwdReduceL<T, SP>;
    __shared__ __align__(16) unsigned char smem[Ly::bytes];
    T *sK = (T *)(smem + Ly::oK), *sVt = (T *)(smem + Ly::oVt), *sPkt = (T *)(smem + Ly::oPkt);
    T *sPl = (T *)(smem + Ly::oPl), *sPlLo = (T *)(smem + Ly::oPlLo);
    float *sSp = (float *)(smem + Ly::oSp), *sSm = (float *)(smem + Ly::oSm);
    constexpr int NTL = Carry<SP>::NTL;

    const int n = blockIdx.y, seg = blockIdx.x;
    const int m = n / (a.B * a.H);
    const int64_t ntiles = (a.T + TT - 1) / TT;
    const int64_t j0 = (int64_t)seg * a.tps, j1 = min(ntiles, j0 + a.tps);
    const T *kp = (const T *)a.k + stream_off(a.sk, n, a.B, a.H);
    const T *vp = (const T *)a.v + stream_off(a.sv, n, a.B, a.H);

    load_planes<T>(a.planes + m * a.planes_m_stride, a.L * a.K, sPl, is_bf16<T>() ? sPlLo : nullptr, nullptr);
    double accB[NTL][4];
    for (int j = 0; j < NTL; ++j)
        for (int e = 0; e < 4; ++e) accB[j][e] = 0.0;
    double accA = 0.0;

    for (int64_t jt = j0; jt < j1; ++jt) {
        const int64_t t0 = jt * TT;
        __syncthreads();
        load_tile<T>(kp, a.sk.t, t0, a.T, sK, nullptr);
        load_tile<T>(vp, a.sv.t, t0, a.T, nullptr, sVt);
        __syncthreads();
        project_tile<T>(sK, sPl, sPlLo, wave_id() >> 1, wave_id() & 1, a.inv_temp, sSp, sSm, nullptr);
        __syncthreads();
        softhash_tile<T, SP>(sSp, sSm, a.K, a.S, t0, a.T, nullptr, sPkt);
        __syncthreads();
        if (threadIdx.x < SP) accA += (double)tile_dA<T>(sPkt, threadIdx.x);
        for (int j = 0; j < NTL; ++j) {
            const f32x4 c = tile_dB<T, SP>(sPkt, sVt, j);
            for (int e = 0; e < 4; ++e) accB[j][e] += (double)c[e];
        }
    }
    double *out = a.fdelta + ((int64_t)n * a.nseg + seg) * SP * SROW;
    const int i = lane_id() & 15, g = lane_id() >> 4;
    for (int j = 0; j < NTL; ++j)
        for (int e = 0; e < 4; ++e)
            out[(16 * Carry<SP>::ms(j) + 4 * g + e) * SROW + 16 * Carry<SP>::nd(j) + i] = accB[j][e];
    if (threadIdx.x < SP) out[threadIdx.x * SROW + D] = accA;
}

// exclusive prefix over segments; [nseg] receives the total
__global__ void k_fwd_scan(double *fstate, const double *fdelta, int nseg, int elems) {
    const int n = blockIdx.y, e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= elems) return;
    double acc = 0.0;
    for (int s = 0; s < nseg; ++s) {
        fstate[((int64_t)n * (nseg + 1) + s) * elems + e] = acc;
        acc += fdelta[((int64_t)n * nseg + s) * elems + e];
    }
    fstate[((int64_t)n * (nseg + 1) + nseg) * elems + e] = acc;
}

// =====================================================================
// k_fwd_out: outputs.
// =====================================================================
template <typename T, int SP, bool CAUSAL> struct FwdOutL {
    static constexpr int LDN = ld_of<T>(D), LDT = ld_of<T>(TT), LDP = ld_of<T>(SP), LDC = ld_of<float>(NCOL);
    static constexpr size_t oQ = 0;  // Q tile, then output staging
    static constexpr size_t oK = align16(oQ + sizeof(T) * TT * LDN);
    static constexpr size_t oVt = align16(oK + (CAUSAL ? sizeof(T) * TT * LDN : 0));
    static constexpr size_t oPk = align16(oVt + (CAUSAL ? sizeof(T) * D * LDT : 0));
    static constexpr size_t oPkt = align16(oPk + (CAUSAL ? sizeof(T) * TT * LDP : 0));
    static constexpr size_t oW = align16(oPkt + (CAUSAL ? sizeof(T) * SP * LDT : 0));
    static constexpr size_t oBct = align16(oW + sizeof(T) * TT * LDP);
    static constexpr size_t oSc = align16(oBct + sizeof(T) * D * LDP);
    static constexpr size_t oPl = align16(oSc + (CAUSAL ? sizeof(T) * TT * LDT : 0));
    static constexpr size_t oPlLo = align16(oPl + sizeof(T) * NCOL * LDN);
    static constexpr size_t oSig = align16(oPlLo + sizeof(T) * NCOL * LDN);  // [2 tensors][2][TT][LDC]
    static constexpr size_t oAc = align16(oSig + sizeof(float) * 4 * TT * LDC);
    static constexpr size_t bytes = align16(oAc + sizeof(double) * SP);
};

template <typename T, int SP, bool CAUSAL>
__global__ __launch_bounds__(NT) void k_fwd_out(Args a) {
    using Ly = FwdOutL<T, SP, CAUSAL>;
    constexpr int LDN = Ly::LDN, LDT = Ly::LDT, LDP = Ly::LDP, LDC = Ly::LDC;
    __shared__ __align__(16) unsigned char smem[Ly::bytes];
    T *sQ = (T *)(smem + Ly::oQ), *sK = (T *)(smem + Ly::oK), *sVt = (T *)(smem + Ly::oVt);
    T *sPk = (T *)(smem + Ly::oPk), *sPkt = (T *)(smem + Ly::oPkt), *sW = (T *)(smem + Ly::oW);
    T *sBct = (T *)(smem + Ly::oBct), *sSc = (T *)(smem + Ly::oSc);
    T *sPl = (T *)(smem + Ly::oPl), *sPlLo = (T *)(smem + Ly::oPlLo);
    float *sSig = (float *)(smem + Ly::oSig);
    float *sSpQ = sSig, *sSmQ = sSig + TT * LDC, *sSpK = sSig + 2 * TT * LDC, *sSmK = sSig + 3 * TT * LDC;
    double *sAc = (double *)(smem + Ly::oAc);
    T *sO = sQ;
    constexpr int NTL = Carry<SP>::NTL;

    const int n = blockIdx.y, seg = blockIdx.x;
    const int m = n / (a.B * a.H);
    const int64_t ntiles = (a.T + TT - 1) / TT;
    const int64_t j0 = (int64_t)seg * a.tps, j1 = min(ntiles, j0 + a.tps);
    const T *qp = (const T *)a.q + stream_off(a.sq, n, a.B, a.H);
    const T *kp = (const T *)a.k + stream_off(a.sk, n, a.B, a.H);
    const T *vp = (const T *)a.v + stream_off(a.sv, n, a.B, a.H);
    T *op = (T *)a.out + stream_off(a.so, n, a.B, a.H);
    const int i = lane_id() & 15, g = lane_id() >> 4, w = wave_id();

    load_planes<T>(a.planes + m * a.planes_m_stride, a.L * a.K, sPl, is_bf16<T>() ? sPlLo : nullptr, nullptr);
    // carried state: causal = prefix at the segment start, non-causal = totals
    const double *st = a.fstate + ((int64_t)n * (a.nseg + 1) + (CAUSAL ? seg : a.nseg)) * SP * SROW;
    f32x4 accB[NTL];
    for (int j = 0; j < NTL; ++j) {
        for (int e = 0; e < 4; ++e)
            accB[j][e] = (float)st[(16 * Carry<SP>::ms(j) + 4 * g + e) * SROW + 16 * Carry<SP>::nd(j) + i];
        st_tile_T(sBct + 16 * Carry<SP>::nd(j) * LDP + 16 * Carry<SP>::ms(j), LDP, accB[j]);
    }
    if (threadIdx.x < SP) sAc[threadIdx.x] = st[threadIdx.x * SROW + D];

    for (int64_t jt = j0; jt < j1; ++jt) {
        const int64_t t0 = jt * TT;
        __syncthreads();
        load_tile<T>(qp, a.sq.t, t0, a.T, sQ, nullptr);
        if constexpr (CAUSAL) {
            load_tile<T>(kp, a.sk.t, t0, a.T, sK, nullptr);
            load_tile<T>(vp, a.sv.t, t0, a.T, nullptr, sVt);
        }
        __syncthreads();
        project_tile<T>(sQ, sPl, sPlLo, w >> 1, w & 1, a.inv_temp, sSpQ, sSmQ, nullptr);
        if constexpr (CAUSAL) project_tile<T>(sK, sPl, sPlLo, w >> 1, w & 1, a.inv_temp, sSpK, sSmK, nullptr);
        __syncthreads();
        if constexpr (CAUSAL) {
            softhash_tile<T, SP>(sSpK, sSmK, a.K, a.S, t0, a.T, sPk, sPkt);
            __syncthreads();
        }
        if (threadIdx.x < SP) {  // W = P_Q / (A(t) + eps)
            const int s = threadIdx.x;
            const float a0 = (float)sAc[s];
            float run = 0.f;
            for (int t = 0; t < TT; ++t) {
                if constexpr (CAUSAL) run += to_f32(sPkt[s * LDT + t]);
                const float pq = (s < a.S && t0 + t < a.T) ? prob_at(sSpQ, sSmQ, t, s, a.K) : 0.f;
                sW[t * LDP + s] = from_f32<T>(pq / (a0 + run + a.eps));
            }
            if constexpr (CAUSAL) sAc[s] += (double)run;
        }
        __syncthreads();
        if constexpr (CAUSAL) {  // Sc = tril(W P_K^T): waves 0-2 the lower tiles, wave 3 zeroes tile (0,1)
            const int mt = w == 0 ? 0 : 1, nt = w == 2 ? 1 : 0;
            if (w < 3) {
                f32x4 c = zero4();
                tile_mma(c, sW + 16 * mt * LDP, LDP, sPk + 16 * nt * LDP, LDP, SP / 32);
                for (int e = 0; e < 4; ++e)
                    if (16 * nt + i > 16 * mt + 4 * g + e) c[e] = 0.f;
                st_tile(sSc + 16 * mt * LDT + 16 * nt, LDT, c);
            } else {
                st_tile(sSc + 16, LDT, zero4());
            }
            __syncthreads();
        }
        f32x4 oacc[2];
        for (int j = 0; j < 2; ++j) {
            const int q = w + NW * j, mt = q >> 2, nd = q & 3;
            oacc[j] = zero4();
            tile_mma(oacc[j], sW + 16 * mt * LDP, LDP, sBct + 16 * nd * LDP, LDP, SP / 32);
            if constexpr (CAUSAL) tile_mma(oacc[j], sSc + 16 * mt * LDT, LDT, sVt + 16 * nd * LDT, LDT, 1);
        }
        if constexpr (CAUSAL)
            for (int j = 0; j < NTL; ++j)
                tile_mma(accB[j], sPkt + 16 * Carry<SP>::ms(j) * LDT, LDT, sVt + 16 * Carry<SP>::nd(j) * LDT, LDT, 1);
        __syncthreads();
        for (int j = 0; j < 2; ++j) {
            const int q = w + NW * j, mt = q >> 2, nd = q & 3;
            st_tile(sO + 16 * mt * LDN + 16 * nd, LDN, oacc[j]);
        }
        if constexpr (CAUSAL)
            for (int j = 0; j < NTL; ++j)
                st_tile_T(sBct + 16 * Carry<SP>::nd(j) * LDP + 16 * Carry<SP>::ms(j), LDP, accB[j]);
        __syncthreads();
        store_tile<T>(op, a.so.t, t0, a.T, sO);
    }
}

// =====================================================================
// k_bwd_reduce: forward walk.  dQ, and per-segment sums of
// alpha = sum_t dA and U = sum_t W^T g.
// =====================================================================
template <typename T, int SP, bool CAUSAL> struct BwdReduceL {
    static constexpr int LDN = ld_of<T>(D), LDT = ld_of<T>(TT), LDC = ld_of<float>(NCOL), LDA = ld_of<float>(SP),
                         LDDP = ld_of<T>(NCOL);
    static constexpr size_t oQ = 0;  // Q tile, then dQ staging
    static constexpr size_t oK = align16(oQ + sizeof(T) * TT * LDN);
    static constexpr size_t oV = align16(oK + (CAUSAL ? sizeof(T) * TT * LDN : 0));
    static constexpr size_t oG = align16(oV + (CAUSAL ? sizeof(T) * TT * LDN : 0));
    static constexpr size_t oVt = align16(oG + sizeof(T) * TT * LDN);
    static constexpr size_t oGt = align16(oVt + (CAUSAL ? sizeof(T) * D * LDT : 0));
    static constexpr size_t oPkt = align16(oGt + sizeof(T) * D * LDT);
    static constexpr size_t oWt = align16(oPkt + (CAUSAL ? sizeof(T) * SP * LDT : 0));
    static constexpr size_t oBc = align16(oWt + sizeof(T) * SP * LDT);
    static constexpr size_t oHm = align16(oBc + sizeof(T) * SP * LDN);
    static constexpr size_t oDA = align16(oHm + (CAUSAL ? sizeof(T) * TT * LDT : 0));
    static constexpr size_t oDproj = align16(oDA + sizeof(float) * TT * LDA);
    static constexpr size_t oPl = align16(oDproj + sizeof(T) * TT * LDDP);
    static constexpr size_t oPlLo = align16(oPl + sizeof(T) * NCOL * LDN);
    static constexpr size_t oPlT = align16(oPlLo + sizeof(T) * NCOL * LDN);
    static constexpr size_t oSig = align16(oPlT + sizeof(T) * D * LDDP);  // [Q sp, Q sm, Q th, K sp, K sm]
    static constexpr size_t oAc = align16(oSig + sizeof(float) * 5 * TT * LDC);
    static constexpr size_t oAl = align16(oAc + sizeof(double) * SP);
    static constexpr size_t oRed = align16(oAl + sizeof(double) * SP);
    static constexpr size_t bytes = align16(oRed + sizeof(float) * NT);
};

template <typename T, int SP, bool CAUSAL>
__global__ __launch_bounds__(NT) void k_bwd_reduce(Args a) {
    using Ly = BwdReduceL<T, SP, CAUSAL>;
    constexpr int LDN = Ly::LDN, LDT = Ly::LDT, LDC = Ly::LDC, LDA = Ly::LDA, LDDP = Ly::LDDP;
    __shared__ __align__(16) unsigned char smem[Ly::bytes];
    T *sQ = (T *)(smem + Ly::oQ), *sK = (T *)(smem + Ly::oK), *sV = (T *)(smem + Ly::oV);
    T *sG = (T *)(smem + Ly::oG), *sVt = (T *)(smem + Ly::oVt), *sGt = (T *)(smem + Ly::oGt);
    T *sPkt = (T *)(smem + Ly::oPkt), *sWt = (T *)(smem + Ly::oWt), *sBc = (T *)(smem + Ly::oBc);
    T *sHm = (T *)(smem + Ly::oHm), *sDproj = (T *)(smem + Ly::oDproj);
    T *sPl = (T *)(smem + Ly::oPl), *sPlLo = (T *)(smem + Ly::oPlLo), *sPlT = (T *)(smem + Ly::oPlT);
    float *sDA = (float *)(smem + Ly::oDA), *sSig = (float *)(smem + Ly::oSig);
    float *sSpQ = sSig, *sSmQ = sSig + TT * LDC, *sThQ = sSig + 2 * TT * LDC;
    float *sSpK = sSig + 3 * TT * LDC, *sSmK = sSig + 4 * TT * LDC;
    double *sAc = (double *)(smem + Ly::oAc), *sAl = (double *)(smem + Ly::oAl);
    float *sRed = (float *)(smem + Ly::oRed);
    T *sStage = sQ;
    constexpr int NTL = Carry<SP>::NTL;

    const int n = blockIdx.y, seg = blockIdx.x;
    const int m = n / (a.B * a.H);
    const int64_t ntiles = (a.T + TT - 1) / TT;
    const int64_t j0 = (int64_t)seg * a.tps, j1 = min(ntiles, j0 + a.tps);
    const T *qp = (const T *)a.q + stream_off(a.sq, n, a.B, a.H);
    const T *kp = (const T *)a.k + stream_off(a.sk, n, a.B, a.H);
    const T *vp = (const T *)a.v + stream_off(a.sv, n, a.B, a.H);
    const T *gp = (const T *)a.dout + stream_off(a.sdo, n, a.B, a.H);
    T *dqp = (T *)a.dq + stream_off(a.sg, n, a.B, a.H);
    const int i = lane_id() & 15, g = lane_id() >> 4, w = wave_id();

    load_planes<T>(a.planes + m * a.planes_m_stride, a.L * a.K, sPl, is_bf16<T>() ? sPlLo : nullptr, sPlT);
    for (int idx = threadIdx.x; idx < TT * LDDP; idx += NT) sDproj[idx] = from_f32<T>(0.f);
    const double *st = a.fstate + ((int64_t)n * (a.nseg + 1) + (CAUSAL ? seg : a.nseg)) * SP * SROW;
    f32x4 accB[NTL], accU[NTL];
    for (int j = 0; j < NTL; ++j) {
        accU[j] = zero4();
        for (int e = 0; e < 4; ++e)
            accB[j][e] = (float)st[(16 * Carry<SP>::ms(j) + 4 * g + e) * SROW + 16 * Carry<SP>::nd(j) + i];
        st_tile(sBc + 16 * Carry<SP>::ms(j) * LDN + 16 * Carry<SP>::nd(j), LDN, accB[j]);
    }
    if (threadIdx.x < SP) {
        sAc[threadIdx.x] = st[threadIdx.x * SROW + D];
        sAl[threadIdx.x] = 0.0;
    }
    float tsum = 0.f;

    for (int64_t jt = j0; jt < j1; ++jt) {
        const int64_t t0 = jt * TT;
        __syncthreads();
        load_tile<T>(qp, a.sq.t, t0, a.T, sQ, nullptr);
        load_tile<T>(gp, a.sdo.t, t0, a.T, sG, sGt);
        if constexpr (CAUSAL) {
            load_tile<T>(kp, a.sk.t, t0, a.T, sK, nullptr);
            load_tile<T>(vp, a.sv.t, t0, a.T, sV, sVt);
        }
        __syncthreads();
        project_tile<T>(sQ, sPl, sPlLo, w >> 1, w & 1, a.inv_temp, sSpQ, sSmQ, sThQ);
        if constexpr (CAUSAL) project_tile<T>(sK, sPl, sPlLo, w >> 1, w & 1, a.inv_temp, sSpK, sSmK, nullptr);
        __syncthreads();
        if constexpr (CAUSAL) {
            softhash_tile<T, SP>(sSpK, sSmK, a.K, a.S, t0, a.T, nullptr, sPkt);
            __syncthreads();
        }
        if (threadIdx.x < SP) {  // W^T into sWt
            const int s = threadIdx.x;
            const float a0 = (float)sAc[s];
            float run = 0.f;
            for (int t = 0; t < TT; ++t) {
                if constexpr (CAUSAL) run += to_f32(sPkt[s * LDT + t]);
                const float pq = (s < a.S && t0 + t < a.T) ? prob_at(sSpQ, sSmQ, t, s, a.K) : 0.f;
                sWt[s * LDT + t] = from_f32<T>(pq / (a0 + run + a.eps));
            }
        }
        if constexpr (CAUSAL) {  // Hm = tril(g V^T) (tau <= t)
            const int mt = w == 0 ? 0 : 1, nt = w == 2 ? 1 : 0;
            if (w < 3) {
                f32x4 c = zero4();
                tile_mma(c, sG + 16 * mt * LDN, LDN, sV + 16 * nt * LDN, LDN, D / 32);
                for (int e = 0; e < 4; ++e)
                    if (16 * nt + i > 16 * mt + 4 * g + e) c[e] = 0.f;
                st_tile(sHm + 16 * mt * LDT + 16 * nt, LDT, c);
            } else {
                st_tile(sHm + 16, LDT, zero4());
            }
        }
        __syncthreads();
        // G[t,s] = g_t . B_s(t) = g B_start^T + tril(g V^T) P_K
        for (int q = w; q < 2 * SP / 16; q += NW) {
            const int mt = q & 1, ns = q >> 1;
            f32x4 c = zero4();
            tile_mma(c, sG + 16 * mt * LDN, LDN, sBc + 16 * ns * LDN, LDN, D / 32);
            if constexpr (CAUSAL) tile_mma(c, sHm + 16 * mt * LDT, LDT, sPkt + 16 * ns * LDT, LDT, 1);
            st_tile(sDA + 16 * mt * LDA + 16 * ns, LDA, c);
        }
        for (int j = 0; j < NTL; ++j) {
            tile_mma(accU[j], sWt + 16 * Carry<SP>::ms(j) * LDT, LDT, sGt + 16 * Carry<SP>::nd(j) * LDT, LDT, 1);
            if constexpr (CAUSAL)
                tile_mma(accB[j], sPkt + 16 * Carry<SP>::ms(j) * LDT, LDT, sVt + 16 * Carry<SP>::nd(j) * LDT, LDT,
                         1);
        }
        __syncthreads();
        if (threadIdx.x < SP) {  // dP_Q = G/(A+eps) in place; alpha += sum_t -W G/(A+eps)
            const int s = threadIdx.x;
            const float a0 = (float)sAc[s];
            float run = 0.f, sda = 0.f;
            for (int t = 0; t < TT; ++t) {
                if constexpr (CAUSAL) run += to_f32(sPkt[s * LDT + t]);
                const float inv = 1.f / (a0 + run + a.eps);
                const float pq = (s < a.S && t0 + t < a.T) ? prob_at(sSpQ, sSmQ, t, s, a.K) : 0.f;
                const float G = sDA[t * LDA + s];
                sDA[t * LDA + s] = G * inv;
                sda -= pq * inv * G * inv;
            }
            sAl[s] += (double)sda;
            if constexpr (CAUSAL) sAc[s] += (double)run;
        }
        if constexpr (CAUSAL)
            for (int j = 0; j < NTL; ++j)
                st_tile(sBc + 16 * Carry<SP>::ms(j) * LDN + 16 * Carry<SP>::nd(j), LDN, accB[j]);
        __syncthreads();
        tsum += softhash_bwd_tile<T, SP>(sSpQ, sSmQ, sThQ, sDA, a.L, a.K, t0, a.T, a.inv_temp, sDproj);
        __syncthreads();
        for (int j = 0; j < 2; ++j) {
            const int q = w + NW * j;
            dx_tile<T>(sDproj, sPlT, q >> 2, q & 3, sStage);
        }
        __syncthreads();
        store_tile<T>(dqp, a.sg.t, t0, a.T, sStage);
    }
    float *out = a.rdelta + ((int64_t)n * a.nseg + seg) * SP * SROW;
    for (int j = 0; j < NTL; ++j)
        for (int e = 0; e < 4; ++e)
            out[(16 * Carry<SP>::ms(j) + 4 * g + e) * SROW + 16 * Carry<SP>::nd(j) + i] = accU[j][e];
    __syncthreads();
    if (threadIdx.x < SP) out[threadIdx.x * SROW + D] = (float)sAl[threadIdx.x];
    const float ts = block_sum(tsum, sRed);
    if (threadIdx.x == 0) a.tpart[(int64_t)n * a.nseg + seg] = ts;
}

// exclusive suffix over segments (causal) or totals (non-causal)
__global__ void k_bwd_scan(float *rstate, const float *rdelta, int nseg, int elems, int causal) {
    const int n = blockIdx.y, e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= elems) return;
    double acc = 0.0;
    if (causal) {
        for (int s = nseg - 1; s >= 0; --s) {
            rstate[((int64_t)n * nseg + s) * elems + e] = (float)acc;
            acc += rdelta[((int64_t)n * nseg + s) * elems + e];
        }
    } else {
        for (int s = 0; s < nseg; ++s) acc += rdelta[((int64_t)n * nseg + s) * elems + e];
        for (int s = 0; s < nseg; ++s) rstate[((int64_t)n * nseg + s) * elems + e] = (float)acc;
    }
}

// =====================================================================
// k_bwd_out: reverse walk.  dK, dV.
// =====================================================================
template <typename T, int SP, bool CAUSAL> struct BwdOutL {
    static constexpr int LDN = ld_of<T>(D), LDT = ld_of<T>(TT), LDP = ld_of<T>(SP), LDC = ld_of<float>(NCOL),
                         LDA = ld_of<float>(SP), LDDP = ld_of<T>(NCOL);
    // region X: {Q, K} during projection; {Hm, HmT, Sc2} in the middle; {stage, dproj} at the end
    static constexpr size_t xsz = cmax(cmax(sizeof(T) * 2 * TT * LDN, sizeof(T) * 3 * TT * LDT),
                                       align16(sizeof(T) * TT * LDN) + sizeof(T) * TT * LDDP);
    static constexpr size_t oX = 0;
    static constexpr size_t oV = align16(oX + xsz);
    static constexpr size_t oG = align16(oV + sizeof(T) * TT * LDN);
    static constexpr size_t oVt = align16(oG + (CAUSAL ? sizeof(T) * TT * LDN : 0));
    static constexpr size_t oGt = align16(oVt + (CAUSAL ? sizeof(T) * D * LDT : 0));
    static constexpr size_t oPk = align16(oGt + (CAUSAL ? sizeof(T) * D * LDT : 0));
    static constexpr size_t oPkt = align16(oPk + sizeof(T) * TT * LDP);
    static constexpr size_t oW = align16(oPkt + (CAUSAL ? sizeof(T) * SP * LDT : 0));
    static constexpr size_t oWt = align16(oW + (CAUSAL ? sizeof(T) * TT * LDP : 0));
    static constexpr size_t oBs = align16(oWt + (CAUSAL ? sizeof(T) * SP * LDT : 0));
    static constexpr size_t oUt = align16(oBs + (CAUSAL ? sizeof(T) * SP * LDN : 0));
    static constexpr size_t oDA = align16(oUt + sizeof(T) * D * LDP);
    static constexpr size_t oPl = align16(oDA + sizeof(float) * TT * LDA);
    static constexpr size_t oPlLo = align16(oPl + sizeof(T) * NCOL * LDN);
    static constexpr size_t oPlT = align16(oPlLo + (is_bf16<T>() ? sizeof(T) * NCOL * LDN : 0));
    static constexpr size_t oSig = align16(oPlT + sizeof(T) * D * LDDP);  // [K sp, K sm, K th, Q sp, Q sm]
    static constexpr size_t oAe = align16(oSig + sizeof(float) * (CAUSAL ? 5 : 3) * TT * LDC);
    static constexpr size_t oAl = align16(oAe + sizeof(double) * SP);
    static constexpr size_t oRed = align16(oAl + sizeof(float) * SP);
    static constexpr size_t bytes = align16(oRed + sizeof(float) * NT);
};

template <typename T, int SP, bool CAUSAL>
__global__ __launch_bounds__(NT) void k_bwd_out(Args a) {
    using Ly = BwdOutL<T, SP, CAUSAL>;
    constexpr int LDN = Ly::LDN, LDT = Ly::LDT, LDP = Ly::LDP, LDC = Ly::LDC, LDA = Ly::LDA, LDDP = Ly::LDDP;
    __shared__ __align__(16) unsigned char smem[Ly::bytes];
    T *sQ = (T *)(smem + Ly::oX), *sK = sQ + TT * LDN;
    T *sHm = (T *)(smem + Ly::oX), *sHmT = sHm + TT * LDT, *sSc2 = sHm + 2 * TT * LDT;
    T *sStage = (T *)(smem + Ly::oX), *sDproj = (T *)(smem + Ly::oX + align16(sizeof(T) * TT * LDN));
    T *sV = (T *)(smem + Ly::oV), *sG = (T *)(smem + Ly::oG), *sVt = (T *)(smem + Ly::oVt);
    T *sGt = (T *)(smem + Ly::oGt), *sPk = (T *)(smem + Ly::oPk), *sPkt = (T *)(smem + Ly::oPkt);
    T *sW = (T *)(smem + Ly::oW), *sWt = (T *)(smem + Ly::oWt), *sBs = (T *)(smem + Ly::oBs);
    T *sUt = (T *)(smem + Ly::oUt);
    T *sPl = (T *)(smem + Ly::oPl), *sPlLo = (T *)(smem + Ly::oPlLo), *sPlT = (T *)(smem + Ly::oPlT);
    float *sDA = (float *)(smem + Ly::oDA), *sSig = (float *)(smem + Ly::oSig);
    float *sSpK = sSig, *sSmK = sSig + TT * LDC, *sThK = sSig + 2 * TT * LDC;
    float *sSpQ = sSig + 3 * TT * LDC, *sSmQ = sSig + 4 * TT * LDC;
    double *sAe = (double *)(smem + Ly::oAe);
    float *sAl = (float *)(smem + Ly::oAl), *sRed = (float *)(smem + Ly::oRed);
    constexpr int NTL = Carry<SP>::NTL;

    const int n = blockIdx.y, seg = blockIdx.x;
    const int m = n / (a.B * a.H);
    const int64_t ntiles = (a.T + TT - 1) / TT;
    const int64_t j0 = (int64_t)seg * a.tps, j1 = min(ntiles, j0 + a.tps);
    const T *qp = (const T *)a.q + stream_off(a.sq, n, a.B, a.H);
    const T *kp = (const T *)a.k + stream_off(a.sk, n, a.B, a.H);
    const T *vp = (const T *)a.v + stream_off(a.sv, n, a.B, a.H);
    const T *gp = (const T *)a.dout + stream_off(a.sdo, n, a.B, a.H);
    T *dkp = (T *)a.dk + stream_off(a.sg, n, a.B, a.H);
    T *dvp = (T *)a.dv + stream_off(a.sg, n, a.B, a.H);
    const int i = lane_id() & 15, g = lane_id() >> 4, w = wave_id();

    load_planes<T>(a.planes + m * a.planes_m_stride, a.L * a.K, sPl, is_bf16<T>() ? sPlLo : nullptr, sPlT);
    // reverse carries (U, alpha) at the segment end; forward state at the segment end
    const float *rs = a.rstate + ((int64_t)n * a.nseg + seg) * SP * SROW;
    const double *fs = a.fstate + ((int64_t)n * (a.nseg + 1) + seg + 1) * SP * SROW;
    f32x4 accU[NTL];
    double accB[NTL][4];
    for (int j = 0; j < NTL; ++j) {
        for (int e = 0; e < 4; ++e) {
            const int r = (16 * Carry<SP>::ms(j) + 4 * g + e) * SROW + 16 * Carry<SP>::nd(j) + i;
            accU[j][e] = rs[r];
            accB[j][e] = CAUSAL ? fs[r] : 0.0;
        }
        st_tile_T(sUt + 16 * Carry<SP>::nd(j) * LDP + 16 * Carry<SP>::ms(j), LDP, accU[j]);
    }
    if (threadIdx.x < SP) {
        sAl[threadIdx.x] = rs[threadIdx.x * SROW + D];
        if (CAUSAL) sAe[threadIdx.x] = fs[threadIdx.x * SROW + D];
    }
    float tsum = 0.f;

    for (int64_t jr = j1 - 1; jr >= j0; --jr) {
        const int64_t t0 = jr * TT;
        __syncthreads();
        load_tile<T>(kp, a.sk.t, t0, a.T, sK, nullptr);
        load_tile<T>(vp, a.sv.t, t0, a.T, sV, CAUSAL ? sVt : nullptr);
        if constexpr (CAUSAL) {
            load_tile<T>(qp, a.sq.t, t0, a.T, sQ, nullptr);
            load_tile<T>(gp, a.sdo.t, t0, a.T, sG, sGt);
        }
        __syncthreads();
        project_tile<T>(sK, sPl, sPlLo, w >> 1, w & 1, a.inv_temp, sSpK, sSmK, sThK);
        if constexpr (CAUSAL) project_tile<T>(sQ, sPl, sPlLo, w >> 1, w & 1, a.inv_temp, sSpQ, sSmQ, nullptr);
        __syncthreads();
        softhash_tile<T, SP>(sSpK, sSmK, a.K, a.S, t0, a.T, sPk, CAUSAL ? sPkt : nullptr);
        __syncthreads();
        if constexpr (CAUSAL) {
            // forward state at the tile start: end state minus this tile's sums (fp64)
            for (int j = 0; j < NTL; ++j) {
                const f32x4 c = tile_dB<T, SP>(sPkt, sVt, j);
                for (int e = 0; e < 4; ++e) accB[j][e] -= (double)c[e];
                f32x4 b;
                for (int e = 0; e < 4; ++e) b[e] = (float)accB[j][e];
                st_tile(sBs + 16 * Carry<SP>::ms(j) * LDN + 16 * Carry<SP>::nd(j), LDN, b);
            }
            if (threadIdx.x < SP) {
                const int s = threadIdx.x;
                const double as = sAe[s] - (double)tile_dA<T>(sPkt, s);
                sAe[s] = as;
                const float a0 = (float)as;
                float run = 0.f;
                for (int t = 0; t < TT; ++t) {
                    run += to_f32(sPkt[s * LDT + t]);
                    const float pq = (s < a.S && t0 + t < a.T) ? prob_at(sSpQ, sSmQ, t, s, a.K) : 0.f;
                    const T wv = from_f32<T>(pq / (a0 + run + a.eps));
                    sW[t * LDP + s] = wv;
                    sWt[s * LDT + t] = wv;
                }
            }
            __syncthreads();
            // region X now holds Hm [t][tau] (tau <= t), HmT [tau][t], Sc2 [tau][t] (t >= tau)
            for (int q = w; q < 8; q += NW) {
                const int kind = q >> 2, sub = q & 3;  // sub: 0 (0,0), 1 (1,0), 2 (1,1), 3 zero tile
                const int mt = sub == 0 ? 0 : 1, nt = sub == 2 ? 1 : 0;
                if (kind == 0) {
                    if (sub < 3) {
                        f32x4 c = zero4();
                        tile_mma(c, sG + 16 * mt * LDN, LDN, sV + 16 * nt * LDN, LDN, D / 32);
                        for (int e = 0; e < 4; ++e)
                            if (16 * nt + i > 16 * mt + 4 * g + e) c[e] = 0.f;
                        st_tile(sHm + 16 * mt * LDT + 16 * nt, LDT, c);
                        st_tile_T(sHmT + 16 * nt * LDT + 16 * mt, LDT, c);
                    } else {
                        st_tile(sHm + 16, LDT, zero4());
                        st_tile(sHmT + 16 * LDT, LDT, zero4());
                    }
                } else {
                    // Sc2[tau][t] = sum_s P_K[tau,s] W[t,s] for t >= tau: tiles (tau-tile, t-tile)
                    const int mtau = sub == 2 ? 1 : 0, ntt = sub == 0 ? 0 : 1;
                    if (sub < 3) {
                        f32x4 c = zero4();
                        tile_mma(c, sPk + 16 * mtau * LDP, LDP, sW + 16 * ntt * LDP, LDP, SP / 32);
                        for (int e = 0; e < 4; ++e)
                            if (16 * ntt + i < 16 * mtau + 4 * g + e) c[e] = 0.f;
                        st_tile(sSc2 + 16 * mtau * LDT + 16 * ntt, LDT, c);
                    } else {
                        st_tile(sSc2 + 16 * LDT, LDT, zero4());
                    }
                }
            }
            __syncthreads();
            // G = g B_start^T + tril(g V^T) P_K
            for (int q = w; q < 2 * SP / 16; q += NW) {
                const int mt = q & 1, ns = q >> 1;
                f32x4 c = zero4();
                tile_mma(c, sG + 16 * mt * LDN, LDN, sBs + 16 * ns * LDN, LDN, D / 32);
                tile_mma(c, sHm + 16 * mt * LDT, LDT, sPkt + 16 * ns * LDT, LDT, 1);
                st_tile(sDA + 16 * mt * LDA + 16 * ns, LDA, c);
            }
            __syncthreads();
            if (threadIdx.x < SP) {  // dA = -W G/(A+eps), then alpha(tau) = alpha_end + suffix sum
                const int s = threadIdx.x;
                const float a0 = (float)sAe[s];
                float run = 0.f;
                for (int t = 0; t < TT; ++t) {
                    run += to_f32(sPkt[s * LDT + t]);
                    const float inv = 1.f / (a0 + run + a.eps);
                    const float pq = (s < a.S && t0 + t < a.T) ? prob_at(sSpQ, sSmQ, t, s, a.K) : 0.f;
                    sDA[t * LDA + s] = -pq * inv * sDA[t * LDA + s] * inv;
                }
                float al = sAl[s];
                for (int t = TT - 1; t >= 0; --t) {
                    al += sDA[t * LDA + s];
                    sDA[t * LDA + s] = al;
                }
                sAl[s] = al;
            }
            __syncthreads();
        }
        // dP_K[tau,s] = alpha(tau) + v_tau . U_s(tau)
        for (int q = w; q < 2 * SP / 16; q += NW) {
            const int mt = q & 1, ns = q >> 1;
            f32x4 c = zero4();
            tile_mma_bT(c, sV + 16 * mt * LDN, LDN, sUt + 16 * ns, LDP, D / 32);
            if constexpr (CAUSAL) tile_mma(c, sHmT + 16 * mt * LDT, LDT, sWt + 16 * ns * LDT, LDT, 1);
            for (int e = 0; e < 4; ++e) {
                const int t = 16 * mt + 4 * g + e, s = 16 * ns + i;
                const float al = CAUSAL ? sDA[t * LDA + s] : sAl[s];
                sDA[t * LDA + s] = c[e] + al;
            }
        }
        // dV[tau] = sum_s P_K[tau,s] U_s(tau)
        f32x4 vacc[2];
        for (int j = 0; j < 2; ++j) {
            const int q = w + NW * j, mt = q >> 2, nd = q & 3;
            vacc[j] = zero4();
            tile_mma(vacc[j], sPk + 16 * mt * LDP, LDP, sUt + 16 * nd * LDP, LDP, SP / 32);
            if constexpr (CAUSAL) tile_mma(vacc[j], sSc2 + 16 * mt * LDT, LDT, sGt + 16 * nd * LDT, LDT, 1);
        }
        if constexpr (CAUSAL)
            for (int j = 0; j < NTL; ++j)
                tile_mma(accU[j], sWt + 16 * Carry<SP>::ms(j) * LDT, LDT, sGt + 16 * Carry<SP>::nd(j) * LDT, LDT, 1);
        __syncthreads();
        for (int j = 0; j < 2; ++j) {
            const int q = w + NW * j;
            st_tile(sStage + 16 * (q >> 2) * LDN + 16 * (q & 3), LDN, vacc[j]);
        }
        if constexpr (CAUSAL)
            for (int j = 0; j < NTL; ++j)
                st_tile_T(sUt + 16 * Carry<SP>::nd(j) * LDP + 16 * Carry<SP>::ms(j), LDP, accU[j]);
        for (int idx = threadIdx.x; idx < TT * LDDP; idx += NT) sDproj[idx] = from_f32<T>(0.f);
        __syncthreads();
        store_tile<T>(dvp, a.sg.t, t0, a.T, sStage);
        tsum += softhash_bwd_tile<T, SP>(sSpK, sSmK, sThK, sDA, a.L, a.K, t0, a.T, a.inv_temp, sDproj);
        __syncthreads();
        for (int j = 0; j < 2; ++j) {
            const int q = w + NW * j;
            dx_tile<T>(sDproj, sPlT, q >> 2, q & 3, sStage);
        }
        __syncthreads();
        store_tile<T>(dkp, a.sg.t, t0, a.T, sStage);
    }
    const float ts = block_sum(tsum, sRed);
    if (threadIdx.x == 0) a.tpart[(int64_t)(a.M * a.B * a.H + n) * a.nseg + seg] = ts;
}

// grad_inv_temp = sum of all partials, in a fixed order
__global__ void k_temp_sum(const float *tpart, int64_t count, float *out) {
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
