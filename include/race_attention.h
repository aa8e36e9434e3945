/*
 * race_attention.h -- C ABI of the MI355X (gfx950) RACE attention operator.
 *
 * Plain C: pointers, sizes, int status codes, no C++ or torch types.  Every
 * entry point returns RACE_OK (0) or a negative RACE_E_* code and leaves a
 * thread-local message readable through race_last_error().  Calls are
 * enqueued on the given HIP stream (a hipStream_t passed as void*; NULL is the
 * default stream); they allocate nothing -- the caller passes the state and
 * workspace buffers sized by the *_bytes queries.  Results are deterministic
 * (no floating-point atomics).
 *
 * Semantics ("F1", per-bucket normalised RACE; misc/race.py:63-142 causal,
 * misc/vit.py:918-978 non-causal, in the reference repository):
 *   streams n = (m*B + b)*H + h over q/k/v [M,B,T,H,D];
 *   th = tanh(<x, plane_{l,k}>), u = th * inv_temp,
 *   P[t,l,r] = softmax_r(sum_k c[r,k] u_k) with c[r,k] = +1 iff bit (K-1-k) of r;
 *   causal: A_s(t) = sum_{tau<=t} P_K, B_s(t) = sum_{tau<=t} P_K v;
 *   non-causal: the same sums over all tau;
 *   out_t = sum_{s < L*2^K} P_Q[t,s] B_s(t) / (A_s(t) + eps).
 */
#ifndef RACE_ATTENTION_H
#define RACE_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RACE_OK 0
#define RACE_E_INVALID (-1)     /* bad descriptor, shape, stride or pointer */
#define RACE_E_UNSUPPORTED (-2) /* valid request outside what this build implements */
#define RACE_E_WORKSPACE (-3)   /* workspace smaller than the *_bytes query */
#define RACE_E_LAUNCH (-4)      /* HIP error when enqueuing a kernel */

#define RACE_PHASE_REDUCE 1 /* k_fwd_reduce / k_bwd_reduce: per-segment sums */
#define RACE_PHASE_SCAN 2   /* segment prefix (forward) / suffix (backward) scan */
#define RACE_PHASE_OUT 4    /* k_fwd_out / k_bwd_out (+ temperature-gradient sum) */

#define RACE_DTYPE_F32 0
#define RACE_DTYPE_BF16 1

/* Operator descriptor.  Strides are in elements, over the (M, B, T, H)
 * dimensions of a [M,B,T,H,D] tensor whose D dimension is contiguous; a zero
 * M stride expresses the reference's M-fold expand (misc/race.py:167-168). */
typedef struct race_desc {
    int64_t M, B, T, H, D;    /* estimators, batch, tokens (T <= 2^35), heads, head dim (D = 64) */
    int32_t L, K;             /* hash tables, hash bits per table (R = 2^K buckets) */
    int32_t causal;           /* 1: prefix (causal) aggregation, 0: full sequence */
    int32_t dtype;            /* RACE_DTYPE_F32 or RACE_DTYPE_BF16 for q/k/v/out/grads */
    float eps;                /* added to every bucket denominator (1e-6 in the reference) */
    float inv_temp;           /* 1/tau: causal reference 1/sqrt(D), non-causal 1/exp(logit_temp) */
    int64_t planes_m_stride;  /* fp32 elements between per-estimator [L][K][D] plane blocks; 0 = shared */
    int64_t q_stride[4], k_stride[4], v_stride[4];
    int64_t o_stride[4];      /* forward output */
    int64_t do_stride[4];     /* upstream gradient */
    int64_t g_stride[4];      /* dq, dk, dv */
    int32_t seg_tiles;        /* 32-token tiles per scan segment, forward and backward; 0 = automatic
                                 (the backward then joins whole forward segments into fewer ones).
                                 Automatic segments are at most 256 tiles at any T, and the
                                 backward calls reject an explicit value above 256: the
                                 whole-tile bf16 kernels walk B in fp32 through a segment, so
                                 long sequences add segments instead of lengthening the walks. */
    int32_t phases;           /* 0 = run every kernel of the call; otherwise a bitmask of
                                 RACE_PHASE_* to run a subset (per-kernel timing); subsets of
                                 one call must be enqueued in phase order on one stream */
    const float *inv_temp_ptr; /* nullable: a device fp32 scalar read by the kernels in place of
                                 inv_temp (a learnable temperature, misc/vit.py:923, stays on the
                                 GPU: no host read per call); it must hold a finite value when
                                 the call's kernels run.  NULL: the inv_temp field is used. */
} race_desc;

/* Bytes of the forward->backward state buffer (per-segment prefix carries,
 * fp64).  race_fwd writes it; race_bwd reads it. */
size_t race_state_bytes(const race_desc *d);

/* Scratch bytes needed by race_fwd / race_bwd. */
size_t race_fwd_workspace_bytes(const race_desc *d);
size_t race_bwd_workspace_bytes(const race_desc *d);

/* Forward.  Replaces the body of BatchedACE.forward (misc/race.py:63-142;
 * misc/vit.py:918-978) and the unbound fused CUDA forward
 * race_fused_fwd (kernels/gpu/forward_kernel.cu:64-96), computing the
 * projection and soft hash in-kernel instead of taking probabilities.
 * planes: fp32 [L][K][D] (or [M][L][K][D] with planes_m_stride = L*K*D). */
int race_fwd(const race_desc *d, const void *q, const void *k, const void *v,
             const float *planes, void *out, void *state, void *ws,
             size_t ws_bytes, void *stream);

/* Backward.  Replaces the autograd backward of BatchedACE.forward and the CUDA
 * backward pair race_bwd_kq_noscan / race_bwd_v_noscan
 * (kernels/gpu/backward_kernels.cu:145-176, :232-256) and the CPU kernel's
 * race_prefix_mean_flat_bw (kernels/cpu/race_pref.cpp:104-220), recomputing
 * the bucket probabilities from q/k.  grad_inv_temp (nullable, device fp32
 * scalar) receives dL/d(inv_temp). */
int race_bwd(const race_desc *d, const void *q, const void *k, const void *v,
             const float *planes, const void *dout, const void *state,
             void *dq, void *dk, void *dv, float *grad_inv_temp, void *ws,
             size_t ws_bytes, void *stream);

/* ---------------------------------------------------------------------
 * Padded batches and the den output (non-causal F1): the forms of
 * BatchedACE.forward(..., mask) (misc/classification.py:576-592) and of
 * _ace_with_denom (misc/classification.py:641-659, misc/vit.py:1452-1510).
 *   kmask: fp32 [B][T] per-token key weights, shared by heads and
 *          estimators (nullable = 1): P_K'[t,s] = kmask[b][t] * P_K[t,s]
 *          feeds A and B.  The reference's mask also multiplies V, P_Q and
 *          the output; those are elementwise on the inputs and outputs and
 *          stay with the caller.
 *   den:   fp32 [M*B*H][T] (nullable), den_t = sum_s P_Q[t,s] A_s,
 *          unclamped (the reference clamps it at eps).
 *   dden:  its upstream gradient (nullable = 0).
 * Non-causal only (d->causal = 1 with kmask, den or dden returns
 * RACE_E_UNSUPPORTED); state and backward workspace as race_fwd/race_bwd.
 * --------------------------------------------------------------------- */
size_t race_fwd_ex_workspace_bytes(const race_desc *d);
int race_fwd_ex(const race_desc *d, const void *q, const void *k, const void *v,
                const float *planes, const float *kmask, void *out, float *den,
                void *state, void *ws, size_t ws_bytes, void *stream);
int race_bwd_ex(const race_desc *d, const void *q, const void *k, const void *v,
                const float *planes, const float *kmask, const void *dout,
                const float *dden, const void *state, void *dq, void *dk,
                void *dv, float *grad_inv_temp, void *ws, size_t ws_bytes,
                void *stream);

/* ---------------------------------------------------------------------
 * Bucket probabilities as an output, for the hybrid consumers that read
 * them (race_bucket_probs_from_qk, misc/arxiv_64K.py:1580-1644;
 * race_avg_bucket_probs_from_x, misc/vit.py:3193-3262):
 *   P[n][t][l*2^K + r] = softmax_r(sum_k c[r,k] tanh(<x_t, plane_{l,k}>) inv_temp),
 * fp32 [M*B*H][T][L*2^K] contiguous (stream-major), from one input x read
 * with d->q_stride (d->causal is not used).  race_probs_bwd turns dP into dx
 * (d->g_stride) and grad_inv_temp (nullable, device fp32 scalar).
 * --------------------------------------------------------------------- */
size_t race_probs_bwd_workspace_bytes(const race_desc *d);
int race_probs(const race_desc *d, const void *x, const float *planes, float *P,
               void *stream);
int race_probs_bwd(const race_desc *d, const void *x, const float *planes,
                   const float *dP, void *dx, float *grad_inv_temp, void *ws,
                   size_t ws_bytes, void *stream);

/* ---------------------------------------------------------------------
 * Global normalisation ("F2", causal only): one normaliser per token
 * instead of one per bucket, the readout of CausalRACEAttention
 * (misc/elsaa_causal_complete.py:438-586) and of its Triton kernel
 * (misc/race_kernel.py:8-124):
 *   P as above with inv_temp = beta (logits = beta * sum_k c[r,k] th_k,
 *   misc/elsaa_causal_complete.py:483-490);
 *   num_t = sum_s P_Q[t,s] B_s(t),  den_t = sum_s P_Q[t,s] A_s(t)
 *           (sums over all L tables and 2^K corners);
 *   out_t = num_t / max(den_t, eps)   (eps = the floor, 1e-6 in the reference).
 * den is fp32 [M*B*H][T], stream-major (stream n = (m*B + b)*H + h),
 * contiguous.  The state buffer is race_state_bytes() as for race_fwd.
 * --------------------------------------------------------------------- */
size_t race_fwd_global_workspace_bytes(const race_desc *d);
size_t race_bwd_global_workspace_bytes(const race_desc *d);

/* Forward.  Replaces race_chunkwise_triton_forward (misc/race_kernel.py:126-163)
 * together with the phi / chunk-state / division steps of
 * CausalRACEAttention.forward (misc/elsaa_causal_complete.py:492-544):
 * writes out and den (unclamped; the module's d_token is den's mean over
 * heads divided by L, clamped at 1e-6). */
int race_fwd_global(const race_desc *d, const void *q, const void *k,
                    const void *v, const float *planes, void *out, float *den,
                    void *state, void *ws, size_t ws_bytes, void *stream);

/* Backward.  Replaces _RaceChunkwiseTritonFn.backward
 * (misc/elsaa_causal_complete.py:392-436) and the autograd of the module's
 * phi and division: out and den are the forward's outputs, dout the
 * gradient of out, dden (nullable = zero) the gradient of den, fp32 like den.
 * grad_beta (nullable, device fp32 scalar) receives dL/d(beta).  dL/d den
 * is formed from the kernels' bucket sums (sum_s P_Q dout.B_s; bucket slices:
 * summed over the slices by a pre-pass), so out is validated but not read. */
int race_bwd_global(const race_desc *d, const void *q, const void *k,
                    const void *v, const float *planes, const void *out,
                    const float *den, const void *dout, const float *dden,
                    const void *state, void *dq, void *dk, void *dv,
                    float *grad_beta, void *ws, size_t ws_bytes, void *stream);

/* Causal prefix mean over flat streams, the reference CPU kernel's operator
 * (race_prefix_mean_flat, kernels/cpu/race_pref.cpp:36-101):
 * w [NS][T], v [NS][T][D], E [NS][T][D], all fp32 contiguous;
 * E[n,t,:] = (sum_{tau<=t} w v) / (sum_{tau<=t} w + eps). */
size_t race_prefix_mean_workspace_bytes(int64_t NS, int64_t T, int64_t D);
int race_prefix_mean_fwd(const float *w, const float *v, float *E, int64_t NS,
                         int64_t T, int64_t D, double eps, void *ws,
                         size_t ws_bytes, void *stream);

/* Its backward (race_prefix_mean_flat_bw, kernels/cpu/race_pref.cpp:104-220):
 * gW [NS][T], gV [NS][T][D] from gE [NS][T][D]. */
int race_prefix_mean_bwd(const float *w, const float *v, const float *gE,
                         float *gW, float *gV, int64_t NS, int64_t T,
                         int64_t D, double eps, void *ws, size_t ws_bytes,
                         void *stream);

/* ---------------------------------------------------------------------
 * No-allocation forward.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory or pass workspaces (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same semantics and kernels as race_fwd, but the forward's segment state and
 * segment sums live in a file-scope device array of the library of
 * RACE_NOALLOC_SCRATCH_BYTES bytes per GPU (held until the process ends), so
 * the caller passes only inputs and outputs; there is no state for a later
 * race_bwd (forward only, e.g. inference).
 *   - seg_tiles = 0 picks the default segmentation, coarsened until it fits
 *     the array; an explicit seg_tiles is used as given (results are then
 *     bit-identical to race_fwd with the same descriptor).
 *   - A call whose scratch would exceed the array (fp32 or K > 4 inputs write
 *     per-slice partial outputs of nslice * M*B*H * T * D * element-size bytes)
 *     returns RACE_E_UNSUPPORTED and names the bytes it needs.
 *   - Every call on one GPU shares that GPU's array: calls that overlap on
 *     one GPU (concurrent streams or threads) race and must be serialised by
 *     the caller.  Nothing in the array needs clearing between calls.
 * --------------------------------------------------------------------- */
#define RACE_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int race_fwd_noalloc(const race_desc *d, const void *q, const void *k, const void *v,
                     const float *planes, void *out, void *stream);

/* Message for the last failing call on this thread ("" if none). */
const char *race_last_error(void);

/* ABI version (increments on incompatible changes; 3 added inv_temp_ptr). */
int race_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* RACE_ATTENTION_H */
