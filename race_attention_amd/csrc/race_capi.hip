// race_capi.hip -- the extern "C" boundary declared in include/race_attention.h.
//
// Validates descriptors and pointers on the host (shape, alignment and stride
// checks happen before any launch, so a kernel never sees a shape it does not
// assume), plans the segment decomposition, carves the caller's workspace and
// enqueues the kernels on the caller's stream.  No allocation, no
// synchronisation, no global mutable state besides the thread-local error.
#include <stdarg.h>
#include <stdio.h>

#include <cmath>
#include <mutex>
#include <string>
#include <type_traits>

#include "../../include/race_attention.h"
#include "prefix_mean.hip"
#include "race_kernels.hip"

namespace race {
namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int ok() {
    g_err.clear();
    return RACE_OK;
}

constexpr int64_t kTargetBlocks = 2048;  // workgroups per forward phase (256 CUs x 8)
// The backward's tile kernels hold one workgroup per CU (LDS): fewer, longer
// segments there amortise each workgroup's set-up (state rows, planes,
// constant tables, the first tile's load) over more tiles.  A backward
// segment is fmul forward segments, so its boundaries are forward ones.
constexpr int64_t kTargetBlocksBwd = 512;
// Longest segment, forward or backward, in 32-token tiles (8192 tokens).
// The bf16 kernels carry B in fp32 MFMA accumulators through a segment:
// k_fwd_reduce and k_bwd_reduce add tile sums from the segment's start,
// and k_bwd_out re-derives B(t) by subtracting them from the fp64 state at
// the segment's end.  Those roundings are relative to the state the walk
// starts from, while B(t) early in a sequence can be far below it (V with a
// non-zero mean makes |B| grow linearly in t), so the walk length must not
// grow with T: long sequences add segments instead.  At 256 tiles the
// walks' error stays below the bf16 operand rounding of B (measured: dK of
// the first tokens equals that of one-tile walks; it grows from 512 tiles).
constexpr int64_t kMaxSegTiles = 256;

struct Plan {
    int SP = 0, S = 0, R = 0, nslice = 1, Spad = 0;
    bool parts = false;  // partial outputs + slice sum (sliced<T, KB>() instantiations)
    int64_t N = 0, ntiles = 0;
    int nseg = 0, tps = 0;
    int fnseg = 0, fmul = 1;  // forward segments; forward segments per segment of this plan
    size_t esize = 0;
    size_t state_bytes = 0, fws = 0, bws = 0;
    size_t fws_core = 0, bws_core = 0, part_bytes = 0;  // partial-output buffers follow the core
    size_t xpart_bytes = 0;  // sliced dX partials (dproj columns), one buffer each for dQ and dK
    // global normalisation: den partials after the forward workspace; rden
    // and gden [N][T] after the backward workspace, then (sliced) the slices'
    // shares of sum_s P_Q dO.B_s [nslice][N][T]
    size_t gfws = 0, gbws = 0, tok_bytes = 0;
};

// Bucket slices: a workgroup handles SP buckets (bf16: 32, 64 or 128; fp32:
// 32, the LDS capacity of the backward tile kernels).  bf16 with K <= 4 and
// L*2^K <= 128 runs one slice of the padded bucket count; everything else
// runs ceil(S / SP) slices whose partial outputs are summed.
void slice_plan(int dtype, int K, int S, int &SP, int &nslice) {
    if (dtype == RACE_DTYPE_BF16 && K <= 4 && S <= 128) {
        SP = (S + 31) / 32 * 32;
        if (SP == 96) SP = 128;
        nslice = 1;
        return;
    }
    SP = dtype == RACE_DTYPE_BF16 ? 128 : 32;
    nslice = (S + SP - 1) / SP;
}

// Work-items of a 1-D launch: the dispatch packet counts them in 32 bits.
constexpr int64_t kMaxWorkItems = 0xFFFFFFFFll;

// bwd: the backward's plan (longer segments of whole forward ones, at most
// kMaxSegTiles); it rejects an explicit seg_tiles above kMaxSegTiles.
// walks: the automatic plan of a call whose state a backward may walk (every
// call but the no-allocation forward and the probability outputs) caps its
// segments at kMaxSegTiles.
int make_plan(const race_desc *d, Plan &p, bool bwd = false, bool walks = true) {
    if (!d) return fail(RACE_E_INVALID, "descriptor is NULL");
    if (d->dtype != RACE_DTYPE_F32 && d->dtype != RACE_DTYPE_BF16)
        return fail(RACE_E_INVALID, "dtype %d is not RACE_DTYPE_F32 or RACE_DTYPE_BF16", d->dtype);
    if (d->M < 1 || d->B < 1 || d->T < 1 || d->H < 1)
        return fail(RACE_E_INVALID, "M, B, T, H must be >= 1 (got %lld, %lld, %lld, %lld)", (long long)d->M,
                    (long long)d->B, (long long)d->T, (long long)d->H);
    if (d->D != D) return fail(RACE_E_UNSUPPORTED, "head dim D=%lld unsupported (this build: D=64)", (long long)d->D);
    // the kernels count tiles of 32 tokens in 32-bit integers
    if (d->T > (1ll << 35))
        return fail(RACE_E_UNSUPPORTED, "T=%lld tokens per sequence unsupported (T <= 2^35)", (long long)d->T);
    if (d->L < 1 || d->K < 1) return fail(RACE_E_INVALID, "L and K must be >= 1 (got L=%d K=%d)", d->L, d->K);
    if (d->K > 8) return fail(RACE_E_UNSUPPORTED, "K=%d hash bits unsupported (K <= 8)", d->K);
    if (d->L * d->K > NCOL)
        return fail(RACE_E_UNSUPPORTED, "L*K=%d projection columns unsupported (L*K <= %d)", d->L * d->K, NCOL);
    if (!(d->eps >= 0.f) || d->eps > 1e30f) return fail(RACE_E_INVALID, "eps must be finite and >= 0");
    if (!d->inv_temp_ptr && (!(d->inv_temp == d->inv_temp) || d->inv_temp > 1e30f || d->inv_temp < -1e30f))
        return fail(RACE_E_INVALID, "inv_temp must be finite");
    if (d->inv_temp_ptr && (uintptr_t)d->inv_temp_ptr % 4)
        return fail(RACE_E_INVALID, "inv_temp_ptr is not 4-byte aligned");
    if (d->planes_m_stride < 0) return fail(RACE_E_INVALID, "planes_m_stride must be >= 0");
    if (d->phases < 0 || d->phases > 7) return fail(RACE_E_INVALID, "phases must be a RACE_PHASE_* bitmask");
    p.R = 1 << d->K;
    p.S = d->L * p.R;
    slice_plan(d->dtype, d->K, p.S, p.SP, p.nslice);
    p.Spad = p.nslice * p.SP;
    p.parts = d->dtype != RACE_DTYPE_BF16 || d->K > 4;
    p.N = d->M * d->B * d->H;
    if (p.N > 65535) return fail(RACE_E_UNSUPPORTED, "M*B*H=%lld streams exceed 65535", (long long)p.N);
    p.ntiles = (d->T + TT - 1) / TT;
    int64_t tps;
    if (d->seg_tiles > 0) {
        if (bwd && d->seg_tiles > kMaxSegTiles)
            return fail(RACE_E_UNSUPPORTED,
                        "seg_tiles=%d exceeds %lld tiles: the backward's fp32 walks of the forward state are "
                        "bounded by the segment length", d->seg_tiles, (long long)kMaxSegTiles);
        tps = d->seg_tiles;
    } else {
        const int64_t per = p.N * p.nslice;  // workgroups per segment index
        int64_t nseg = (kTargetBlocks + per - 1) / per;
        if (nseg > p.ntiles) nseg = p.ntiles;
        tps = (p.ntiles + nseg - 1) / nseg;
        if (walks && tps > kMaxSegTiles) tps = kMaxSegTiles;
    }
    p.tps = (int)(tps < p.ntiles ? tps : p.ntiles);
    const int64_t nseg = (p.ntiles + p.tps - 1) / p.tps;
    if (nseg > (1 << 30)) return fail(RACE_E_UNSUPPORTED, "too many segments");
    // the tile kernels' grids: (nseg, N) of threads_of(SP)-thread workgroups,
    // or (sliced) 1-D over whole blocks of 8 (segment, stream) groups x slices
    const int64_t wgs = p.parts ? (nseg * p.N + 7) / 8 * 8 * p.nslice : nseg;
    if (wgs * threads_of(p.SP) > kMaxWorkItems)
        return fail(RACE_E_UNSUPPORTED, "%lld segments x %lld streams x %d bucket slices exceed one launch's 2^32 "
                    "work-items", (long long)nseg, (long long)p.N, p.nslice);
    p.nseg = (int)nseg;
    p.fnseg = p.nseg;
    p.esize = d->dtype == RACE_DTYPE_BF16 ? 2 : 4;
    const size_t blk = (size_t)p.Spad * SROW;
    p.state_bytes = (size_t)p.N * (p.fnseg + 1) * blk * sizeof(double);
    p.fws_core = align16((size_t)p.N * p.fnseg * blk * sizeof(double));
    if (bwd && d->seg_tiles <= 0) {
        // backward segments of fmul forward ones (one segment when that
        // covers the sequence); explicit seg_tiles keeps the forward's
        // (a segment is at most kMaxSegTiles long: m * tps tiles, or the whole
        // sequence when that is shorter)
        int64_t m = (int64_t)p.fnseg * p.N * p.nslice / kTargetBlocksBwd;
        if (walks && p.ntiles > kMaxSegTiles && m > kMaxSegTiles / p.tps) m = kMaxSegTiles / p.tps;
        if (m > 1) {
            const int64_t tb = (int64_t)p.tps * m;
            p.fmul = m < p.fnseg ? (int)m : p.fnseg;
            p.tps = (int)(tb < p.ntiles ? tb : p.ntiles);
            p.nseg = (int)((p.ntiles + p.tps - 1) / p.tps);
        }
    }
    p.bws_core = 2 * (size_t)p.N * p.nseg * blk * sizeof(float) +
                 align16(2 * (size_t)p.N * p.nseg * p.nslice * sizeof(double));
    // k_dx_finish runs one 64-lane wave per 64 tokens of a stream
    if (p.parts && (p.N * ((d->T + 16 * DXF_BLK - 1) / (16 * DXF_BLK)) + 3) / 4 * 256 > kMaxWorkItems)
        return fail(RACE_E_UNSUPPORTED, "M*B*H*T=%lld token-heads exceed one dX launch's 2^32 work-items",
                    (long long)(p.N * d->T));
    p.part_bytes = p.parts ? align16((size_t)p.nslice * p.N * d->T * D * p.esize) : 0;
    const size_t xesize = xpart_f32(d->dtype == RACE_DTYPE_BF16, p.SP, d->K) ? sizeof(float) : p.esize;
    p.xpart_bytes = p.parts ? align16((size_t)p.nslice * p.N * d->T * xcols_of(p.SP, d->K) * xesize) : 0;
    p.fws = p.fws_core + p.part_bytes;                         // partial O
    p.bws = p.bws_core + 2 * p.xpart_bytes + p.part_bytes;     // dproj columns for dQ, dK; partial dV
    p.tok_bytes = align16((size_t)p.N * d->T * sizeof(float));
    p.gfws = p.fws + (p.parts ? p.nslice * p.tok_bytes : 0);
    p.gbws = p.bws + 2 * p.tok_bytes + (p.parts ? p.nslice * p.tok_bytes : 0);  // + the slices' gsum
    return RACE_OK;
}

// Largest token stride (elements) whose lane byte offsets inside a 32-token
// tile, ((TT - 1) * stride + D) * esize, fit the kernels' 32-bit offsets and
// the 2^31 - 1 byte record size of k_fwd_out's buffer stores.  It also keeps a
// tile's byte stride TT * stride * esize below 2^32, which the kernels' tile
// base addresses (tile index times that stride, a 32 x 32-bit product) need.
int64_t max_token_stride(size_t esize) { return (0x7FFFFFFFll / (int64_t)esize - D) / (TT - 1); }

int check_tensor(const char *name, const void *ptr, const int64_t *st, size_t esize, int64_t T) {
    if (!ptr) return fail(RACE_E_INVALID, "%s is NULL", name);
    if ((uintptr_t)ptr % 16) return fail(RACE_E_INVALID, "%s is not 16-byte aligned", name);
    for (int j = 0; j < 4; ++j) {
        if (st[j] < 0) return fail(RACE_E_INVALID, "%s stride %d is negative", name, j);
        if ((st[j] * (int64_t)esize) % 16)
            return fail(RACE_E_INVALID, "%s stride %d (%lld elements) is not a multiple of 16 bytes", name, j,
                        (long long)st[j]);
    }
    if (T > 1 && st[2] < D)
        return fail(RACE_E_INVALID, "%s token stride %lld overlaps rows", name, (long long)st[2]);
    if (st[2] > max_token_stride(esize))  // lane byte offsets within a 32-token tile are 32-bit
        return fail(RACE_E_UNSUPPORTED, "%s token stride %lld exceeds %lld elements (32-bit tile offsets)", name,
                    (long long)st[2], (long long)max_token_stride(esize));
    return RACE_OK;
}

// A tensor the call writes: as check_tensor, and no two (m, b, t, h) rows
// may share memory through a zero stride or heads closer than D elements
// (workgroups of different streams would race on the same rows).
int check_out(const char *name, const void *ptr, const int64_t *st, size_t esize, const race_desc *d) {
    int rc = check_tensor(name, ptr, st, esize, d->T);
    if (rc) return rc;
    const int64_t sz[4] = {d->M, d->B, d->T, d->H};
    static const char *dim[4] = {"M", "B", "T", "H"};
    for (int j = 0; j < 4; ++j)
        if (sz[j] > 1 && st[j] == 0)
            return fail(RACE_E_INVALID, "%s is written but has stride 0 over %s (size %lld)", name, dim[j],
                        (long long)sz[j]);
    if (d->H > 1 && st[3] < D)
        return fail(RACE_E_INVALID, "%s head stride %lld overlaps rows (< D)", name, (long long)st[3]);
    return RACE_OK;
}

Strides strides_of(const int64_t *s) { return Strides{s[0], s[1], s[2], s[3]}; }

Args base_args(const race_desc *d, const Plan &p, const float *planes) {
    Args a{};
    a.sq = strides_of(d->q_stride);
    a.sk = strides_of(d->k_stride);
    a.sv = strides_of(d->v_stride);
    a.so = strides_of(d->o_stride);
    a.sdo = strides_of(d->do_stride);
    a.sg = strides_of(d->g_stride);
    a.planes = planes;
    a.planes_m_stride = d->planes_m_stride;
    a.M = (int)d->M;
    a.B = (int)d->B;
    a.H = (int)d->H;
    a.L = d->L;
    a.K = d->K;
    a.R = p.R;
    a.S = p.S;
    a.T = d->T;
    a.eps = d->eps;
    a.inv_temp = d->inv_temp;
    a.inv_temp_ptr = d->inv_temp_ptr;
    a.nseg = p.nseg;
    a.tps = p.tps;
    a.fnseg = p.fnseg;
    a.fmul = p.fmul;
    a.nslice = p.nslice;
    a.Spad = p.Spad;
    return a;
}

int launched(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(RACE_E_LAUNCH, "%s: %s", what, hipGetErrorString(e));
    return ok();
}

bool run_phase(const race_desc *d, int ph) { return d->phases == 0 || (d->phases & ph); }

// Launch grid of the tile kernels (their wg_pos): (nseg, N) unsliced; sliced,
// 1-D over blocks of 8 (segment, stream) groups times the slices.
dim3 tile_grid(const Plan &p) {
    if (!p.parts) return dim3((unsigned)p.nseg, (unsigned)p.N, 1);
    return dim3((unsigned)(((int64_t)p.nseg * p.N + 7) / 8 * 8 * p.nslice), 1, 1);
}

template <typename T>
void slice_sum(const Plan &p, const race_desc *d, const void *part, const int64_t *st, void *out, hipStream_t s) {
    if constexpr (std::is_same<T, bf16>::value) {
        if (p.nslice == 8) {  // the 8-bit slices of 4 tables
            const int64_t n8 = p.N * d->T * (D / 8);
            k_slice_sum8<8><<<elem_blocks(n8), ELEM_THREADS, 0, s>>>((const bf16 *)part, p.N, d->T, (int)d->B,
                                                                     (int)d->H, Strides{st[0], st[1], st[2], st[3]},
                                                                     (bf16 *)out);
            return;
        }
    }
    const int64_t n4 = p.N * d->T * (D / 4);
    k_slice_sum<T><<<elem_blocks(n4), ELEM_THREADS, 0, s>>>((const T *)part, p.nslice, p.N, d->T, (int)d->B, (int)d->H,
                                                                Strides{st[0], st[1], st[2], st[3]}, (T *)out);
}

// dX (dQ, dK, the probability backward's dx) of sliced instantiations from
// the slices' dproj columns
template <typename T>
void dx_finish(const Plan &p, const race_desc *d, const void *part, const Args &a, const int64_t *st, void *out,
               hipStream_t s) {
    const int64_t waves = p.N * ((d->T + 16 * DXF_BLK - 1) / (16 * DXF_BLK));  // one wave per 64 tokens
    if constexpr (std::is_same<T, bf16>::value) {
        // 8-bit hashes, slices of 128 buckets: two slices per table, 8 fp32
        // columns each (the plan gives L <= 4 and 2L slices whenever this holds)
        if (xpart_f32(true, p.SP, d->K)) {
            k_dx_finish8<<<(unsigned)((waves + 3) / 4), 256, 0, s>>>(
                (const float *)part, d->L, a.planes, a.planes_m_stride, (int)d->B, (int)d->H, p.N, d->T,
                Strides{st[0], st[1], st[2], st[3]}, (bf16 *)out);
            return;
        }
    }
    k_dx_finish<T><<<(unsigned)((waves + 3) / 4), 256, 0, s>>>(
        (const T *)part, p.nslice, xcols_of(p.SP, d->K), p.SP, d->K, d->L, a.planes, a.planes_m_stride, (int)d->B,
        (int)d->H, p.N, d->T, Strides{st[0], st[1], st[2], st[3]}, (T *)out);
}

// Whole-tile instantiations (template flag AL of the tile kernels): compiled
// for the causal bf16 slices of 128 buckets at 4 and 8 hash bits, and used
// when every tile holds TT tokens (T % TT == 0) and every bucket of every
// slice is one of the S buckets, so no load, store or probability needs a
// row or bucket guard.  Elsewhere the template argument is false and both
// branches below launch the same kernel.
template <typename T, int SP, int KB> constexpr bool al_compiled() {
    return std::is_same<T, bf16>::value && SP == 128 && (KB == 4 || KB == 8);
}
bool whole_tiles(const race_desc *d, const Plan &p) { return d->T % TT == 0 && p.S == p.Spad; }

// The causal F1 operator walks the forward state B back through each backward
// segment (k_bwd_out); its whole-tile bf16 instantiations do it in fp32, the
// others in fp64 (race_kernels.hip walk_f64).  A table's logits differ by at
// most 2 K |inv_temp| (|tanh| <= 1 per bit), so at most e^(2 K |inv_temp|)
// separates its largest and smallest probability: above K |inv_temp| = 2
// (e^4), or with a temperature on the device, whole tiles take the segment
// sums from the generic k_fwd_reduce (fp64) and walk B in fp64 in the
// whole-tile k_bwd_out.  The forward and the backward of one descriptor choose
// alike.
bool exact_walk(const race_desc *d) {
    return d->causal && (d->inv_temp_ptr != nullptr || (double)d->K * std::fabs((double)d->inv_temp) > 2.0);
}

template <typename T, int SP, int KB> int fwd_impl(const race_desc *d, const Plan &p, Args a, hipStream_t s) {
    const dim3 grid = tile_grid(p);
    constexpr bool ALC = al_compiled<T, SP, KB>();
    const bool al = ALC && whole_tiles(d, p);
    if (run_phase(d, RACE_PHASE_REDUCE)) {
        if (al && !exact_walk(d))
            k_fwd_reduce<T, SP, KB, ALC><<<grid, threads_of(SP), 0, s>>>(a);
        else
            k_fwd_reduce<T, SP, KB><<<grid, threads_of(SP), 0, s>>>(a);
    }
    const int elems = p.Spad * SROW;
    if (run_phase(d, RACE_PHASE_SCAN))
        k_fwd_scan<<<dim3((elems + SCAN_THREADS - 1) / SCAN_THREADS, (unsigned)p.N), SCAN_THREADS, 0, s>>>(a.fstate, a.fdelta, p.nseg, elems);
    if (run_phase(d, RACE_PHASE_OUT)) {
        if (d->causal && al)
            k_fwd_out<T, SP, true, KB, false, ALC><<<grid, threads_of(SP), 0, s>>>(a);
        else if (d->causal)
            k_fwd_out<T, SP, true, KB, false><<<grid, threads_of(SP), 0, s>>>(a);
        else
            k_fwd_out<T, SP, false, KB, false><<<grid, threads_of(SP), 0, s>>>(a);
        if (sliced<T, KB>()) {
            slice_sum<T>(p, d, a.opart, d->o_stride, a.out, s);
            if (a.den) {
                const int64_t nt = p.N * d->T;
                k_den_sum<<<elem_blocks(nt), ELEM_THREADS, 0, s>>>(a.denpart, p.nslice, nt, a.den);
            }
        }
    }
    return launched("race_fwd");
}

template <typename T, int SP, int KB>
int bwd_impl(const race_desc *d, const Plan &p, Args a, float *grad_inv_temp, hipStream_t s) {
    const dim3 grid = tile_grid(p);
    constexpr bool ALC = al_compiled<T, SP, KB>();
    const bool al = ALC && whole_tiles(d, p);
    if (run_phase(d, RACE_PHASE_REDUCE)) {
        if (d->causal && al)
            k_bwd_reduce<T, SP, true, KB, false, ALC><<<grid, threads_of(SP), 0, s>>>(a);
        else if (d->causal)
            k_bwd_reduce<T, SP, true, KB, false><<<grid, threads_of(SP), 0, s>>>(a);
        else
            k_bwd_reduce<T, SP, false, KB, false><<<grid, threads_of(SP), 0, s>>>(a);
        if (sliced<T, KB>()) dx_finish<T>(p, d, a.dqpart, a, d->g_stride, a.dq, s);
    }
    const int elems = p.Spad * SROW;
    if (run_phase(d, RACE_PHASE_SCAN))
        k_bwd_scan<<<dim3((elems + SCAN_THREADS - 1) / SCAN_THREADS, (unsigned)p.N), SCAN_THREADS, 0, s>>>(a.rstate, a.rdelta, p.nseg, elems,
                                                                            d->causal);
    if (run_phase(d, RACE_PHASE_OUT)) {
        if (d->causal && al && exact_walk(d))
            k_bwd_out<T, SP, true, KB, false, ALC, true><<<grid, threads_of(SP), 0, s>>>(a);
        else if (d->causal && al)
            k_bwd_out<T, SP, true, KB, false, ALC><<<grid, threads_of(SP), 0, s>>>(a);
        else if (d->causal)
            k_bwd_out<T, SP, true, KB, false><<<grid, threads_of(SP), 0, s>>>(a);
        else
            k_bwd_out<T, SP, false, KB, false><<<grid, threads_of(SP), 0, s>>>(a);
        if (sliced<T, KB>()) {
            dx_finish<T>(p, d, a.dkpart, a, d->g_stride, a.dk, s);
            slice_sum<T>(p, d, a.dvpart, d->g_stride, a.dv, s);
        }
        if (grad_inv_temp) k_temp_sum<<<1, 256, 0, s>>>(a.tpart, 2 * p.N * p.nseg * p.nslice, grad_inv_temp);
    }
    return launched("race_bwd");
}

// Global normalisation (causal): the F1 reduce and scan kernels, then the GN
// readout; its den partials (sliced) are summed with the numerators.  Whole
// tiles run the whole-tile instantiations, as F1 does.
template <typename T, int SP, int KB> int gn_fwd_impl(const race_desc *d, const Plan &p, Args a, hipStream_t s) {
    const dim3 grid = tile_grid(p);
    constexpr bool ALC = al_compiled<T, SP, KB>();
    // the segment sums are F1's (the same kernel): its whole-tile instantiation where it applies
    if (run_phase(d, RACE_PHASE_REDUCE)) {
        if (ALC && whole_tiles(d, p))
            k_fwd_reduce<T, SP, KB, ALC><<<grid, threads_of(SP), 0, s>>>(a);
        else
            k_fwd_reduce<T, SP, KB><<<grid, threads_of(SP), 0, s>>>(a);
    }
    const int elems = p.Spad * SROW;
    if (run_phase(d, RACE_PHASE_SCAN))
        k_fwd_scan<<<dim3((elems + SCAN_THREADS - 1) / SCAN_THREADS, (unsigned)p.N), SCAN_THREADS, 0, s>>>(a.fstate, a.fdelta, p.nseg, elems);
    if (run_phase(d, RACE_PHASE_OUT)) {
        if (ALC && whole_tiles(d, p))
            k_fwd_out<T, SP, true, KB, true, ALC><<<grid, threads_of(SP), 0, s>>>(a);
        else
            k_fwd_out<T, SP, true, KB, true><<<grid, threads_of(SP), 0, s>>>(a);
        if (sliced<T, KB>()) {
            const int64_t n4 = p.N * d->T * (D / 4);
            k_slice_sum_gn<T><<<elem_blocks(n4), ELEM_THREADS, 0, s>>>(
                (const T *)a.opart, a.denpart, p.nslice, p.N, d->T, (int)d->B, (int)d->H, strides_of(d->o_stride), (T *)a.out,
                a.den, d->eps);
        }
    }
    return launched("race_fwd_global");
}

// The GN backward: k_bwd_reduce also forms the per-token terms
// (1/max(den, eps) and dL/d den, from out, dout, den, dden) that k_bwd_out reads.
template <typename T, int SP, int KB>
int gn_bwd_impl(const race_desc *d, const Plan &p, Args a, float *grad_beta, hipStream_t s) {
    const dim3 grid = tile_grid(p);
    constexpr bool ALC = al_compiled<T, SP, KB>();
    const bool al = ALC && whole_tiles(d, p);
    if (run_phase(d, RACE_PHASE_REDUCE)) {
        if constexpr (sliced<T, KB>()) {
            // each slice's share of sum_s P_Q G per token, then rd and gd
            if (al)
                k_bwd_reduce<T, SP, true, KB, true, ALC, true><<<grid, threads_of(SP), 0, s>>>(a);
            else
                k_bwd_reduce<T, SP, true, KB, true, false, true><<<grid, threads_of(SP), 0, s>>>(a);
            const int64_t nt = p.N * d->T;
            k_gn_terms<<<elem_blocks(nt), ELEM_THREADS, 0, s>>>(a.gsum, p.nslice, nt, a.den, a.dden, d->eps, a.rden,
                                                                a.gden);
        }
        if (al)
            k_bwd_reduce<T, SP, true, KB, true, ALC><<<grid, threads_of(SP), 0, s>>>(a);
        else
            k_bwd_reduce<T, SP, true, KB, true><<<grid, threads_of(SP), 0, s>>>(a);
        if (sliced<T, KB>()) dx_finish<T>(p, d, a.dqpart, a, d->g_stride, a.dq, s);
    }
    const int elems = p.Spad * SROW;
    if (run_phase(d, RACE_PHASE_SCAN))
        k_bwd_scan<<<dim3((elems + SCAN_THREADS - 1) / SCAN_THREADS, (unsigned)p.N), SCAN_THREADS, 0, s>>>(a.rstate, a.rdelta, p.nseg, elems, 1);
    if (run_phase(d, RACE_PHASE_OUT)) {
        if (al)
            k_bwd_out<T, SP, true, KB, true, ALC><<<grid, threads_of(SP), 0, s>>>(a);
        else
            k_bwd_out<T, SP, true, KB, true><<<grid, threads_of(SP), 0, s>>>(a);
        if (sliced<T, KB>()) {
            dx_finish<T>(p, d, a.dkpart, a, d->g_stride, a.dk, s);
            slice_sum<T>(p, d, a.dvpart, d->g_stride, a.dv, s);
        }
        if (grad_beta) k_temp_sum<<<1, 256, 0, s>>>(a.tpart, 2 * p.N * p.nseg * p.nslice, grad_beta);
    }
    return launched("race_bwd_global");
}

// Compiled (dtype, slice buckets, hash bits) combinations: every K in 1..8
// with the slice sizes slice_plan() picks (L*K <= 32).
#define RACE_FOR_COMBOS(X)                                                                                          \
    X(bf16, 32, 1) X(bf16, 64, 1) X(bf16, 32, 2) X(bf16, 64, 2) X(bf16, 32, 3) X(bf16, 64, 3) X(bf16, 128, 3)       \
    X(bf16, 32, 4) X(bf16, 64, 4) X(bf16, 128, 4) X(bf16, 128, 5) X(bf16, 128, 6) X(bf16, 128, 7) X(bf16, 128, 8)   \
    X(float, 32, 1) X(float, 32, 2) X(float, 32, 3) X(float, 32, 4) X(float, 32, 5) X(float, 32, 6) X(float, 32, 7)  \
    X(float, 32, 8)

template <typename T> int fwd_dispatch(const race_desc *d, const Plan &p, const Args &a, hipStream_t s) {
#define X(TT_, SP_, KB_)                                                                                             \
    if (std::is_same<T, TT_>::value && p.SP == SP_ && d->K == KB_) return fwd_impl<TT_, SP_, KB_>(d, p, a, s);
    RACE_FOR_COMBOS(X)
#undef X
    return fail(RACE_E_UNSUPPORTED, "bucket count / hash bits combination not compiled");
}

template <typename T>
int bwd_dispatch(const race_desc *d, const Plan &p, const Args &a, float *git, hipStream_t s) {
#define X(TT_, SP_, KB_)                                                                                             \
    if (std::is_same<T, TT_>::value && p.SP == SP_ && d->K == KB_) return bwd_impl<TT_, SP_, KB_>(d, p, a, git, s);
    RACE_FOR_COMBOS(X)
#undef X
    return fail(RACE_E_UNSUPPORTED, "bucket count / hash bits combination not compiled");
}

template <typename T> int gn_fwd_dispatch(const race_desc *d, const Plan &p, const Args &a, hipStream_t s) {
#define X(TT_, SP_, KB_)                                                                                             \
    if (std::is_same<T, TT_>::value && p.SP == SP_ && d->K == KB_) return gn_fwd_impl<TT_, SP_, KB_>(d, p, a, s);
    RACE_FOR_COMBOS(X)
#undef X
    return fail(RACE_E_UNSUPPORTED, "bucket count / hash bits combination not compiled");
}

template <typename T> int gn_bwd_dispatch(const race_desc *d, const Plan &p, const Args &a, float *gb, hipStream_t s) {
#define X(TT_, SP_, KB_)                                                                                             \
    if (std::is_same<T, TT_>::value && p.SP == SP_ && d->K == KB_) return gn_bwd_impl<TT_, SP_, KB_>(d, p, a, gb, s);
    RACE_FOR_COMBOS(X)
#undef X
    return fail(RACE_E_UNSUPPORTED, "bucket count / hash bits combination not compiled");
}

// Bucket probabilities (forward) and dP -> dx (backward)
template <typename T, int SP, int KB> int probs_impl(const race_desc *d, const Plan &p, Args a, bool bwd,
                                                     float *grad_inv_temp, hipStream_t s) {
    const dim3 grid = tile_grid(p);
    if (!bwd) {
        k_probs<T, SP, KB, false><<<grid, threads_of(SP), 0, s>>>(a);
        return launched("race_probs");
    }
    k_probs<T, SP, KB, true><<<grid, threads_of(SP), 0, s>>>(a);
    if (sliced<T, KB>()) dx_finish<T>(p, d, a.dqpart, a, d->g_stride, a.dq, s);
    if (grad_inv_temp) k_temp_sum<<<1, 256, 0, s>>>(a.tpart, p.N * p.nseg * p.nslice, grad_inv_temp);
    return launched("race_probs_bwd");
}

template <typename T>
int probs_dispatch(const race_desc *d, const Plan &p, const Args &a, bool bwd, float *git, hipStream_t s) {
#define X(TT_, SP_, KB_)                                                                                             \
    if (std::is_same<T, TT_>::value && p.SP == SP_ && d->K == KB_) return probs_impl<TT_, SP_, KB_>(d, p, a, bwd, git, s);
    RACE_FOR_COMBOS(X)
#undef X
    return fail(RACE_E_UNSUPPORTED, "bucket count / hash bits combination not compiled");
}

// workspace of race_probs_bwd: temperature partials, then fp32 dx partials (sliced)
size_t probs_ws_core(const Plan &p) { return align16((size_t)p.N * p.nseg * p.nslice * sizeof(double)); }

int check_gn(const race_desc *d) {
    if (d->causal != 1)
        return fail(RACE_E_UNSUPPORTED, "global normalisation is implemented for the causal operator only");
    if (!(d->eps > 0.f)) return fail(RACE_E_INVALID, "eps (the floor of den) must be > 0 for global normalisation");
    return RACE_OK;
}

int check_den(const char *name, const float *p) {
    if (!p) return fail(RACE_E_INVALID, "%s is NULL", name);
    if ((uintptr_t)p % 4) return fail(RACE_E_INVALID, "%s is not 4-byte aligned", name);
    return RACE_OK;
}

// Checks and Args of a backward call (race_bwd, race_bwd_ex)
int bwd_args(const race_desc *d, const Plan &p, const void *q, const void *k, const void *v, const float *planes,
             const void *dout, const void *state, void *dq, void *dk, void *dv, void *ws, size_t ws_bytes, Args &a) {
    int rc;
    if ((rc = check_tensor("q", q, d->q_stride, p.esize, d->T)) || (rc = check_tensor("k", k, d->k_stride, p.esize, d->T)) ||
        (rc = check_tensor("v", v, d->v_stride, p.esize, d->T)) ||
        (rc = check_tensor("dout", dout, d->do_stride, p.esize, d->T)) ||
        (rc = check_out("dq", dq, d->g_stride, p.esize, d)) || (rc = check_out("dk", dk, d->g_stride, p.esize, d)) ||
        (rc = check_out("dv", dv, d->g_stride, p.esize, d)))
        return rc;
    if (!planes) return fail(RACE_E_INVALID, "planes is NULL");
    if (!state) return fail(RACE_E_INVALID, "state is NULL");
    if (!ws || ws_bytes < p.bws)
        return fail(RACE_E_WORKSPACE, "workspace %zu bytes < required %zu", ws_bytes, p.bws);
    a = base_args(d, p, planes);
    a.q = q;
    a.k = k;
    a.v = v;
    a.dout = dout;
    a.dq = dq;
    a.dk = dk;
    a.dv = dv;
    a.fstate = (double *)state;
    const size_t blk = (size_t)p.N * p.nseg * p.Spad * SROW;
    a.rdelta = (float *)ws;
    a.rstate = a.rdelta + blk;
    a.tpart = (double *)(a.rstate + blk);  // blk is even: 8-byte aligned
    if (p.parts) {
        float *part = (float *)((char *)ws + p.bws_core);
        a.dqpart = part;
        a.dkpart = (char *)part + p.xpart_bytes;
        a.dvpart = (char *)part + 2 * p.xpart_bytes;
    }
    return RACE_OK;
}

// prefix mean: segment length so that NS * nseg ~ 4096 waves
int64_t pm_tseg(int64_t NS, int64_t T) {
    int64_t nseg = (4096 + NS - 1) / NS;
    if (nseg > T) nseg = T;
    if (nseg < 1) nseg = 1;
    return (T + nseg - 1) / nseg;
}

int pm_check(const void *a, const char *na, int64_t NS, int64_t T, int64_t D) {
    if (!a) return fail(RACE_E_INVALID, "%s is NULL", na);
    if (NS < 1 || T < 1 || D < 1) return fail(RACE_E_INVALID, "NS, T, D must be >= 1");
    if (D > 64 * PM_MAXC) return fail(RACE_E_UNSUPPORTED, "D=%lld unsupported (D <= %d)", (long long)D, 64 * PM_MAXC);
    if (NS > 65535) return fail(RACE_E_UNSUPPORTED, "NS=%lld exceeds 65535", (long long)NS);
    return RACE_OK;
}

// ---------------------------------------------------------------- no-allocation forward
// race_fwd_noalloc keeps the forward's segment sums and segment state in one
// file-scope device array instead of caller buffers.  In host code `scratch`
// names a host-side stand-in: kernels get the device address that
// hipGetSymbolAddress returns for the current device (each GPU holds its own
// copy of the array), looked up once per device and cached.
static __device__ __align__(256) unsigned char scratch[RACE_NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mu;
constexpr int kMaxDevices = 64;
void *g_scratch_ptr[kMaxDevices];

int scratch_address(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(RACE_E_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(RACE_E_UNSUPPORTED, "device ordinal %d >= %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(RACE_E_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return RACE_OK;
}

constexpr size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
size_t noalloc_need(const Plan &p) { return align256(p.state_bytes) + p.fws; }

// Plan of the no-allocation forward: the descriptor's seg_tiles if set, else
// the default segmentation, coarsened (longer segments) until the state and
// the segment sums fit the scratch array.  Returns RACE_E_UNSUPPORTED with the
// bytes needed when even one segment per stream does not fit.
int noalloc_plan(const race_desc *d, race_desc &dd, Plan &p) {
    if (!d) return fail(RACE_E_INVALID, "descriptor is NULL");
    dd = *d;
    int rc = make_plan(&dd, p, false, false);
    if (rc) return rc;
    if (d->seg_tiles <= 0 && noalloc_need(p) > RACE_NOALLOC_SCRATCH_BYTES) {
        // state (nseg + 1 rows) and sums (nseg rows) of N * Spad * (D+1) fp64 each
        const size_t row = (size_t)p.N * p.Spad * SROW * sizeof(double);
        const size_t fixed = p.part_bytes + row + 512;
        const int64_t nseg = fixed < RACE_NOALLOC_SCRATCH_BYTES
                                 ? (int64_t)((RACE_NOALLOC_SCRATCH_BYTES - fixed) / (2 * row)) : 0;
        if (nseg >= 1) {
            dd.seg_tiles = (int32_t)((p.ntiles + nseg - 1) / nseg);
            if ((rc = make_plan(&dd, p, false, false))) return rc;
        }
    }
    if (noalloc_need(p) > RACE_NOALLOC_SCRATCH_BYTES)
        return fail(RACE_E_UNSUPPORTED,
                    "race_fwd_noalloc: this call needs %zu bytes of scratch (state %zu, segment sums and partial "
                    "outputs %zu); the no-allocation forward holds %zu -- use race_fwd with caller buffers",
                    noalloc_need(p), p.state_bytes, p.fws, (size_t)RACE_NOALLOC_SCRATCH_BYTES);
    return RACE_OK;
}

} // namespace
} // namespace race

using namespace race;

extern "C" {

size_t race_state_bytes(const race_desc *d) {
    Plan p;
    if (make_plan(d, p) != RACE_OK) return 0;
    ok();
    return p.state_bytes;
}

size_t race_fwd_workspace_bytes(const race_desc *d) {
    Plan p;
    if (make_plan(d, p) != RACE_OK) return 0;
    ok();
    return p.fws;
}

size_t race_bwd_workspace_bytes(const race_desc *d) {
    Plan p;
    if (make_plan(d, p, true) != RACE_OK) return 0;
    ok();
    return p.bws;
}

int race_fwd(const race_desc *d, const void *q, const void *k, const void *v, const float *planes, void *out,
             void *state, void *ws, size_t ws_bytes, void *stream) {
    Plan p;
    int rc = make_plan(d, p);
    if (rc) return rc;
    if ((rc = check_tensor("q", q, d->q_stride, p.esize, d->T)) || (rc = check_tensor("k", k, d->k_stride, p.esize, d->T)) ||
        (rc = check_tensor("v", v, d->v_stride, p.esize, d->T)) || (rc = check_out("out", out, d->o_stride, p.esize, d)))
        return rc;
    if (!planes) return fail(RACE_E_INVALID, "planes is NULL");
    if (!state) return fail(RACE_E_INVALID, "state is NULL");
    if (!ws || ws_bytes < p.fws)
        return fail(RACE_E_WORKSPACE, "workspace %zu bytes < required %zu", ws_bytes, p.fws);
    Args a = base_args(d, p, planes);
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.fstate = (double *)state;
    a.fdelta = (double *)ws;
    a.opart = p.parts ? (void *)((char *)ws + p.fws_core) : nullptr;
    hipStream_t s = (hipStream_t)stream;
    if (d->dtype == RACE_DTYPE_BF16) return fwd_dispatch<bf16>(d, p, a, s);
    return fwd_dispatch<float>(d, p, a, s);
}

int race_bwd(const race_desc *d, const void *q, const void *k, const void *v, const float *planes,
             const void *dout, const void *state, void *dq, void *dk, void *dv, float *grad_inv_temp, void *ws,
             size_t ws_bytes, void *stream) {
    Plan p;
    int rc = make_plan(d, p, true);
    if (rc) return rc;
    Args a;
    if ((rc = bwd_args(d, p, q, k, v, planes, dout, state, dq, dk, dv, ws, ws_bytes, a))) return rc;
    hipStream_t s = (hipStream_t)stream;
    if (d->dtype == RACE_DTYPE_BF16) return bwd_dispatch<bf16>(d, p, a, grad_inv_temp, s);
    return bwd_dispatch<float>(d, p, a, grad_inv_temp, s);
}

size_t race_probs_bwd_workspace_bytes(const race_desc *d) {
    Plan p;
    if (make_plan(d, p, false, false) != RACE_OK) return 0;
    ok();
    return probs_ws_core(p) + p.xpart_bytes;
}

int race_probs(const race_desc *d, const void *x, const float *planes, float *P, void *stream) {
    Plan p;
    int rc = make_plan(d, p, false, false);
    if (rc || (rc = check_tensor("x", x, d->q_stride, p.esize, d->T)) || (rc = check_den("P", P))) return rc;
    if (!planes) return fail(RACE_E_INVALID, "planes is NULL");
    Args a = base_args(d, p, planes);
    a.q = x;
    a.probs = P;
    hipStream_t s = (hipStream_t)stream;
    if (d->dtype == RACE_DTYPE_BF16) return probs_dispatch<bf16>(d, p, a, false, nullptr, s);
    return probs_dispatch<float>(d, p, a, false, nullptr, s);
}

int race_probs_bwd(const race_desc *d, const void *x, const float *planes, const float *dP, void *dx,
                   float *grad_inv_temp, void *ws, size_t ws_bytes, void *stream) {
    Plan p;
    int rc = make_plan(d, p, false, false);
    if (rc || (rc = check_tensor("x", x, d->q_stride, p.esize, d->T)) || (rc = check_den("dP", dP)) ||
        (rc = check_out("dx", dx, d->g_stride, p.esize, d)))
        return rc;
    if (!planes) return fail(RACE_E_INVALID, "planes is NULL");
    const size_t need = probs_ws_core(p) + p.xpart_bytes;
    if (!ws || ws_bytes < need) return fail(RACE_E_WORKSPACE, "workspace %zu bytes < required %zu", ws_bytes, need);
    Args a = base_args(d, p, planes);
    a.q = x;
    a.dq = dx;
    a.dprobs = dP;
    a.tpart = (double *)ws;
    a.dqpart = p.parts ? (char *)ws + probs_ws_core(p) : nullptr;
    hipStream_t s = (hipStream_t)stream;
    if (d->dtype == RACE_DTYPE_BF16) return probs_dispatch<bf16>(d, p, a, true, grad_inv_temp, s);
    return probs_dispatch<float>(d, p, a, true, grad_inv_temp, s);
}

size_t race_fwd_ex_workspace_bytes(const race_desc *d) {
    Plan p;
    if (make_plan(d, p) != RACE_OK) return 0;
    ok();
    return p.gfws;  // den partials per slice, like the global mode
}

int race_fwd_ex(const race_desc *d, const void *q, const void *k, const void *v, const float *planes,
                const float *kmask, void *out, float *den, void *state, void *ws, size_t ws_bytes, void *stream) {
    Plan p;
    int rc = make_plan(d, p);
    if (rc) return rc;
    if (d->causal && (kmask || den))
        return fail(RACE_E_UNSUPPORTED, "key weights and den are implemented for the non-causal operator");
    if ((rc = check_tensor("q", q, d->q_stride, p.esize, d->T)) || (rc = check_tensor("k", k, d->k_stride, p.esize, d->T)) ||
        (rc = check_tensor("v", v, d->v_stride, p.esize, d->T)) || (rc = check_out("out", out, d->o_stride, p.esize, d)) ||
        (kmask && (rc = check_den("kmask", kmask))) || (den && (rc = check_den("den", den))))
        return rc;
    if (!planes) return fail(RACE_E_INVALID, "planes is NULL");
    if (!state) return fail(RACE_E_INVALID, "state is NULL");
    const size_t need = den ? p.gfws : p.fws;
    if (!ws || ws_bytes < need) return fail(RACE_E_WORKSPACE, "workspace %zu bytes < required %zu", ws_bytes, need);
    Args a = base_args(d, p, planes);
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.kw = kmask;
    a.den = den;
    a.fstate = (double *)state;
    a.fdelta = (double *)ws;
    a.opart = p.parts ? (void *)((char *)ws + p.fws_core) : nullptr;
    a.denpart = p.parts && den ? (float *)((char *)ws + p.fws) : nullptr;
    hipStream_t s = (hipStream_t)stream;
    if (d->dtype == RACE_DTYPE_BF16) return fwd_dispatch<bf16>(d, p, a, s);
    return fwd_dispatch<float>(d, p, a, s);
}

int race_bwd_ex(const race_desc *d, const void *q, const void *k, const void *v, const float *planes,
                const float *kmask, const void *dout, const float *dden, const void *state, void *dq, void *dk,
                void *dv, float *grad_inv_temp, void *ws, size_t ws_bytes, void *stream) {
    Plan p;
    int rc = make_plan(d, p, true);
    if (rc) return rc;
    if (d->causal && (kmask || dden))
        return fail(RACE_E_UNSUPPORTED, "key weights and den are implemented for the non-causal operator");
    if ((kmask && (rc = check_den("kmask", kmask))) || (dden && (rc = check_den("dden", dden)))) return rc;
    Args a;
    if ((rc = bwd_args(d, p, q, k, v, planes, dout, state, dq, dk, dv, ws, ws_bytes, a))) return rc;
    a.kw = kmask;
    a.dden = dden;
    hipStream_t s = (hipStream_t)stream;
    if (d->dtype == RACE_DTYPE_BF16) return bwd_dispatch<bf16>(d, p, a, grad_inv_temp, s);
    return bwd_dispatch<float>(d, p, a, grad_inv_temp, s);
}

size_t race_fwd_global_workspace_bytes(const race_desc *d) {
    Plan p;
    if (make_plan(d, p) != RACE_OK) return 0;
    ok();
    return p.gfws;
}

size_t race_bwd_global_workspace_bytes(const race_desc *d) {
    Plan p;
    if (make_plan(d, p, true) != RACE_OK) return 0;
    ok();
    return p.gbws;
}

int race_fwd_global(const race_desc *d, const void *q, const void *k, const void *v, const float *planes, void *out,
                    float *den, void *state, void *ws, size_t ws_bytes, void *stream) {
    Plan p;
    int rc = make_plan(d, p);
    if (rc || (rc = check_gn(d))) return rc;
    if ((rc = check_tensor("q", q, d->q_stride, p.esize, d->T)) || (rc = check_tensor("k", k, d->k_stride, p.esize, d->T)) ||
        (rc = check_tensor("v", v, d->v_stride, p.esize, d->T)) || (rc = check_out("out", out, d->o_stride, p.esize, d)) ||
        (rc = check_den("den", den)))
        return rc;
    if (!planes) return fail(RACE_E_INVALID, "planes is NULL");
    if (!state) return fail(RACE_E_INVALID, "state is NULL");
    if (!ws || ws_bytes < p.gfws)
        return fail(RACE_E_WORKSPACE, "workspace %zu bytes < required %zu", ws_bytes, p.gfws);
    Args a = base_args(d, p, planes);
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.den = den;
    a.fstate = (double *)state;
    a.fdelta = (double *)ws;
    a.opart = p.parts ? (void *)((char *)ws + p.fws_core) : nullptr;
    a.denpart = p.parts ? (float *)((char *)ws + p.fws) : nullptr;
    hipStream_t s = (hipStream_t)stream;
    if (d->dtype == RACE_DTYPE_BF16) return gn_fwd_dispatch<bf16>(d, p, a, s);
    return gn_fwd_dispatch<float>(d, p, a, s);
}

int race_bwd_global(const race_desc *d, const void *q, const void *k, const void *v, const float *planes,
                    const void *out, const float *den, const void *dout, const float *dden, const void *state,
                    void *dq, void *dk, void *dv, float *grad_beta, void *ws, size_t ws_bytes, void *stream) {
    Plan p;
    int rc = make_plan(d, p, true);
    if (rc || (rc = check_gn(d))) return rc;
    if ((rc = check_tensor("q", q, d->q_stride, p.esize, d->T)) || (rc = check_tensor("k", k, d->k_stride, p.esize, d->T)) ||
        (rc = check_tensor("v", v, d->v_stride, p.esize, d->T)) ||
        (rc = check_tensor("out", out, d->o_stride, p.esize, d->T)) ||
        (rc = check_tensor("dout", dout, d->do_stride, p.esize, d->T)) ||
        (rc = check_out("dq", dq, d->g_stride, p.esize, d)) || (rc = check_out("dk", dk, d->g_stride, p.esize, d)) ||
        (rc = check_out("dv", dv, d->g_stride, p.esize, d)) || (rc = check_den("den", den)) ||
        (dden && (rc = check_den("dden", dden))))
        return rc;
    if (!planes) return fail(RACE_E_INVALID, "planes is NULL");
    if (!state) return fail(RACE_E_INVALID, "state is NULL");
    if (!ws || ws_bytes < p.gbws)
        return fail(RACE_E_WORKSPACE, "workspace %zu bytes < required %zu", ws_bytes, p.gbws);
    Args a = base_args(d, p, planes);
    a.q = q;
    a.k = k;
    a.v = v;
    a.dout = dout;
    a.dq = dq;
    a.dk = dk;
    a.dv = dv;
    a.fstate = (double *)state;
    const size_t blk = (size_t)p.N * p.nseg * p.Spad * SROW;
    a.rdelta = (float *)ws;
    a.rstate = a.rdelta + blk;
    a.tpart = (double *)(a.rstate + blk);  // blk is even: 8-byte aligned
    if (p.parts) {
        float *part = (float *)((char *)ws + p.bws_core);
        a.dqpart = part;
        a.dkpart = (char *)part + p.xpart_bytes;
        a.dvpart = (char *)part + 2 * p.xpart_bytes;
    }
    a.out = const_cast<void *>(out);  // read only (the GN per-token terms)
    a.den = const_cast<float *>(den);
    a.dden = dden;
    a.rden = (float *)((char *)ws + p.bws);
    a.gden = (float *)((char *)ws + p.bws + p.tok_bytes);
    a.gsum = p.parts ? (float *)((char *)ws + p.bws + 2 * p.tok_bytes) : nullptr;
    hipStream_t s = (hipStream_t)stream;
    if (d->dtype == RACE_DTYPE_BF16) return gn_bwd_dispatch<bf16>(d, p, a, grad_beta, s);
    return gn_bwd_dispatch<float>(d, p, a, grad_beta, s);
}

size_t race_prefix_mean_workspace_bytes(int64_t NS, int64_t T, int64_t D) {
    if (NS < 1 || T < 1 || D < 1) return 0;
    const int64_t tseg = pm_tseg(NS, T), nseg = (T + tseg - 1) / tseg;
    const size_t row = (size_t)(D + 1) * sizeof(double);
    // forward: delta + state; backward adds invA, alpha, rdelta, rstate
    return (size_t)NS * nseg * row + (size_t)NS * (nseg + 1) * row + 2 * (size_t)NS * T * sizeof(double) +
           2 * (size_t)NS * nseg * row;
}

int race_prefix_mean_fwd(const float *w, const float *v, float *E, int64_t NS, int64_t T, int64_t D, double eps,
                         void *ws, size_t ws_bytes, void *stream) {
    int rc;
    if ((rc = pm_check(w, "w", NS, T, D)) || (rc = pm_check(v, "v", NS, T, D)) || (rc = pm_check(E, "E", NS, T, D)))
        return rc;
    const size_t need = race_prefix_mean_workspace_bytes(NS, T, D);
    if (!ws || ws_bytes < need) return fail(RACE_E_WORKSPACE, "workspace %zu bytes < required %zu", ws_bytes, need);
    const int64_t tseg = pm_tseg(NS, T);
    const int nseg = (int)((T + tseg - 1) / tseg);
    double *delta = (double *)ws;
    double *state = delta + NS * nseg * (D + 1);
    hipStream_t s = (hipStream_t)stream;
    const int elems = (int)(D + 1);
    k_pm_reduce<<<dim3(nseg, (unsigned)NS), 64, 0, s>>>(w, v, delta, T, (int)D, tseg, nseg);
    k_pm_scan<<<dim3((elems + 255) / 256, (unsigned)NS), 256, 0, s>>>(state, delta, nseg, elems);
    k_pm_out<<<dim3(nseg, (unsigned)NS), 64, 0, s>>>(w, v, E, state, T, (int)D, tseg, nseg, eps);
    return launched("race_prefix_mean_fwd");
}

int race_prefix_mean_bwd(const float *w, const float *v, const float *gE, float *gW, float *gV, int64_t NS,
                         int64_t T, int64_t D, double eps, void *ws, size_t ws_bytes, void *stream) {
    int rc;
    if ((rc = pm_check(w, "w", NS, T, D)) || (rc = pm_check(v, "v", NS, T, D)) ||
        (rc = pm_check(gE, "gE", NS, T, D)) || (rc = pm_check(gW, "gW", NS, T, D)) ||
        (rc = pm_check(gV, "gV", NS, T, D)))
        return rc;
    const size_t need = race_prefix_mean_workspace_bytes(NS, T, D);
    if (!ws || ws_bytes < need) return fail(RACE_E_WORKSPACE, "workspace %zu bytes < required %zu", ws_bytes, need);
    const int64_t tseg = pm_tseg(NS, T);
    const int nseg = (int)((T + tseg - 1) / tseg);
    double *delta = (double *)ws;
    double *state = delta + NS * nseg * (D + 1);
    double *invA = state + NS * (nseg + 1) * (D + 1);
    double *alpha = invA + NS * T;
    double *rdelta = alpha + NS * T;
    double *rstate = rdelta + NS * nseg * (D + 1);
    hipStream_t s = (hipStream_t)stream;
    const int elems = (int)(D + 1);
    const dim3 grid(nseg, (unsigned)NS);
    k_pm_reduce<<<grid, 64, 0, s>>>(w, v, delta, T, (int)D, tseg, nseg);
    k_pm_scan<<<dim3((elems + 255) / 256, (unsigned)NS), 256, 0, s>>>(state, delta, nseg, elems);
    k_pm_bw_fwd<<<grid, 64, 0, s>>>(w, v, gE, state, invA, alpha, rdelta, T, (int)D, tseg, nseg, eps);
    k_pm_rscan<<<dim3((elems + 255) / 256, (unsigned)NS), 256, 0, s>>>(rstate, rdelta, nseg, elems);
    k_pm_bw_rev<<<grid, 64, 0, s>>>(w, v, gE, invA, alpha, rstate, gW, gV, T, (int)D, tseg, nseg);
    return launched("race_prefix_mean_bwd");
}

int race_fwd_noalloc(const race_desc *d, const void *q, const void *k, const void *v, const float *planes,
                     void *out, void *stream) {
    race_desc dd;
    Plan p;
    int rc = noalloc_plan(d, dd, p);
    if (rc) return rc;
    if ((rc = check_tensor("q", q, d->q_stride, p.esize, d->T)) || (rc = check_tensor("k", k, d->k_stride, p.esize, d->T)) ||
        (rc = check_tensor("v", v, d->v_stride, p.esize, d->T)) || (rc = check_out("out", out, d->o_stride, p.esize, d)))
        return rc;
    if (!planes) return fail(RACE_E_INVALID, "planes is NULL");
    void *base = nullptr;
    if ((rc = scratch_address(&base))) return rc;
    Args a = base_args(&dd, p, planes);
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.fstate = (double *)base;
    a.fdelta = (double *)((char *)base + align256(p.state_bytes));
    a.opart = p.parts ? (void *)((char *)a.fdelta + p.fws_core) : nullptr;
    hipStream_t s = (hipStream_t)stream;
    if (d->dtype == RACE_DTYPE_BF16) return fwd_dispatch<bf16>(&dd, p, a, s);
    return fwd_dispatch<float>(&dd, p, a, s);
}

const char *race_last_error(void) { return g_err.c_str(); }

int race_abi_version(void) { return 3; }

} // extern "C"
