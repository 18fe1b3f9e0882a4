/*
 * mpattn.h -- C ABI of the MI355X (gfx950) multi-pathway attention library
 * (libmpattn.so).
 *
 * The op: for batch b, head h, query i and key j
 *
 *   s_ij = scale * <R_i q_self_i, R_j k_self_j>   if chain[b,i] == chain[b,j]
 *        = scale * <q_multi_i, k_multi_j>         otherwise
 *   s_ij = -inf                                   if key j is padded
 *   P_i  = softmax_j(s_i)          (one softmax over both pathways)
 *   O_i  = sum_j P_ij * (v_self_j if same chain else v_multi_j)
 *
 * R_p is the rotary embedding at global position p (half-split layout,
 * inv_freq = 10000^(-2i/D)); it is applied only when rope == MPATTN_ROPE_FUSED.
 * A query row whose keys are all padded produces O_i = 0.
 *
 * Reference interfaces (molecular-william/mint_plus, which binds no FFI; these
 * entry points replace the Python/Triton functions named on each one):
 *   mpattn_fwd  -> mint_plus/models/kernels/multi_pathway_attention.py:184
 *                  (fused_multi_pathway_attention), its fp16 twin
 *                  multi_pathway_attention_fp16.py:148, and the eager combine
 *                  mint_plus/models/modules_plus.py:155-201
 *   mpattn_bwd  -> mint_plus/models/kernels/multi_pathway_attention_bwd.py:15
 *                  (fused_multi_pathway_attention_bwd)
 *   mpattn_combine_fwd / mpattn_combine_bwd
 *               -> mint_plus/models/kernels/__init__.py:179 and :247
 *                  (fused_multimer_combine / fused_multimer_combine_bwd)
 *
 * Conventions
 *   - The caller owns and allocates every device buffer (outputs and the
 *     workspaces). The library never allocates, never synchronises, and
 *     keeps no mutable global state (apart from mpattn_fwd_noalloc's static
 *     scratch and its per-device address): calls on different streams are
 *     independent.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = default stream).
 *   - All tensors are 4-D (B, H, L, D) views given by a base pointer and
 *     element strides for b, h and t; the head-dim stride must be 1.
 *     This admits the (L, B, 3E) projection output without a copy. Rows
 *     start 16-byte aligned, and the kernels address rows with 32-bit byte
 *     offsets from each (b, h) base: L * stride_t * element size must stay
 *     below 2^31 (likewise L * mask_stride_q for a dense chain mask in the
 *     backward). Larger requests return MPATTN_ERR_UNSUPPORTED.
 *   - Return 0 on success, a negative MPATTN_ERR_* code on error. Arguments
 *     are validated before anything is enqueued.
 */
#ifndef MPATTN_H
#define MPATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MPATTN_VERSION 6

enum {
    MPATTN_OK = 0,
    MPATTN_ERR_INVALID = -1,      /* bad pointer, shape, stride or enum   */
    MPATTN_ERR_UNSUPPORTED = -2,  /* valid request this build cannot do   */
    MPATTN_ERR_LAUNCH = -3,       /* the HIP runtime rejected the launch  */
};

enum { MPATTN_BF16 = 0, MPATTN_FP16 = 1, MPATTN_FP32 = 2 };

enum {
    MPATTN_ROPE_NONE = 0,   /* q/k used as given (caller rotated/scaled)   */
    MPATTN_ROPE_FUSED = 1,  /* rotate q_self/k_self by global position     */
};

/* 4-D (B, H, L, D) view; strides in elements, head-dim stride is 1. */
typedef struct mpattn_tensor {
    const void *ptr;
    int64_t stride_b, stride_h, stride_t;
} mpattn_tensor;

typedef struct mpattn_fwd_params {
    mpattn_tensor q_self, k_self, v_self;   /* self pathway                 */
    mpattn_tensor q_multi, k_multi, v_multi;/* multimer (cross) pathway     */
    mpattn_tensor out;                      /* written; same dtype          */
    float *lse;              /* optional (B,H,L) fp32 log-sum-exp, or NULL  */
    /* Pathway selection: exactly one of chain_id / chain_mask is non-NULL.
     * chain_id  : (B, L) int32, contiguous.
     * chain_mask: (B, L, L) uint8/bool, element strides below; nonzero means
     *             "different chains" (the reference's self_attn_mask).     */
    const int32_t *chain_id;
    const uint8_t *chain_mask;
    int64_t mask_stride_b, mask_stride_q, mask_stride_k;
    const uint8_t *key_pad;  /* optional (B, L) contiguous, nonzero = pad   */
    /* RoPE tables (L, D/2) fp32 contiguous: cos/sin of p * inv_freq[i].
     * Required when rope == MPATTN_ROPE_FUSED, ignored otherwise.          */
    const float *rope_cos, *rope_sin;
    int32_t B, H, L, D;
    int32_t dtype;           /* MPATTN_BF16 / MPATTN_FP16 / MPATTN_FP32      */
    int32_t rope;            /* MPATTN_ROPE_NONE / MPATTN_ROPE_FUSED         */
    float scale;             /* logit scale (> 0), e.g. D^-1/2               */
    int32_t sqrt_softmax;    /* 1: O = sum sqrt(P) V (muS variant)           */
    float dropout_p;         /* attention dropout in [0, 1) (with sqrt_softmax
                                it drops the sqrt(P) weights)              */
    void *workspace;         /* >= mpattn_fwd_workspace_size() bytes, 256-byte
                                aligned; contents need no initialisation   */
    int64_t workspace_bytes;
    uint64_t dropout_seed;   /* seed of the dropout mask (see below)         */
} mpattn_fwd_params;

typedef struct mpattn_bwd_params {
    mpattn_tensor q_self, k_self, v_self, q_multi, k_multi, v_multi;
    mpattn_tensor out;        /* forward output O                           */
    mpattn_tensor grad_out;   /* dO                                         */
    const float *lse;         /* (B,H,L) fp32 from mpattn_fwd               */
    mpattn_tensor dq_self, dk_self, dv_self, dq_multi, dk_multi, dv_multi;
    const int32_t *chain_id;
    const uint8_t *chain_mask;
    int64_t mask_stride_b, mask_stride_q, mask_stride_k;
    const uint8_t *key_pad;
    const float *rope_cos, *rope_sin;
    void *workspace;          /* >= mpattn_bwd_workspace_size() bytes, 16-byte
                                 aligned; contents need no initialisation  */
    int64_t workspace_bytes;  /* size of the buffer at workspace            */
    int32_t B, H, L, D;
    int32_t dtype, rope;
    float scale;
    int32_t sqrt_softmax;
    float dropout_p;          /* the forward's dropout_p and dropout_seed    */
    uint64_t dropout_seed;
} mpattn_bwd_params;

/* Attention dropout. Element (b, h, i, j) of the weights that multiply V
 * (P, or sqrt(P) with sqrt_softmax) is kept, and scaled by 1 / (1 - dropout_p),
 * when
 *   r = fmix32(fmix32(lo ^ (b*H + h) * 0xC2B2AE3D ^ i * 0x9E3779B1)
 *              ^ (j * 0x85EBCA77 + hi))
 * has (r >> 8) >= round(dropout_p * 2^24), with lo / hi the low / high 32 bits
 * of dropout_seed and fmix32 the MurmurHash3 32-bit finaliser (x ^= x >> 16;
 * x *= 0x85EBCA6B; x ^= x >> 13; x *= 0xC2B2AE35; x ^= x >> 16), all in
 * unsigned 32-bit arithmetic. The row sums of the softmax use P before
 * dropout. The backward with the same seed regenerates the mask. */

/* Workspace bytes mpattn_fwd needs (chain-id staging; RoPE-rotated K_self
 * when rope == MPATTN_ROPE_FUSED; per-32x32-block codes of a dense chain
 * mask, B * (L/32 rounded up to even)^2 bytes, reserved in every case). */
int64_t mpattn_fwd_workspace_size(int32_t B, int32_t H, int32_t L, int32_t D, int32_t dtype,
                                  int32_t rope);

/* Forward. Replaces fused_multi_pathway_attention
 * (mint_plus/models/kernels/multi_pathway_attention.py:184-279) and
 * fused_multi_pathway_attention_fp16 (multi_pathway_attention_fp16.py:148). */
int mpattn_fwd(const mpattn_fwd_params *p, void *stream);

/* No-allocation forward. No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same arguments and result
 * as mpattn_fwd, except that workspace / workspace_bytes are ignored: the
 * workspace is a static device array of MPATTN_NOALLOC_SCRATCH_BYTES bytes
 * that the library holds on every GPU it runs on until the process ends.
 * It calls no allocating routine. Shapes whose workspace
 * (mpattn_fwd_workspace_size) exceeds the array return
 * MPATTN_ERR_UNSUPPORTED. All calls on one GPU share the array: calls that
 * overlap in time on one GPU (different streams or threads) race. */
#define MPATTN_NOALLOC_SCRATCH_BYTES (48ll << 20)
int mpattn_fwd_noalloc(const mpattn_fwd_params *p, void *stream);

/* Workspace bytes mpattn_bwd needs for (B, H, L). */
int64_t mpattn_bwd_workspace_size(int32_t B, int32_t H, int32_t L, int32_t D);

/* Backward: all six gradients, deterministic (no atomics). Replaces
 * fused_multi_pathway_attention_bwd
 * (mint_plus/models/kernels/multi_pathway_attention_bwd.py:15-59). */
int mpattn_bwd(const mpattn_bwd_params *p, void *stream);

/* Materialised-logit combine. Logit tensors are (B, H, L, L) views given as
 * mpattn_tensor with stride_t = query-row stride and unit key stride; they
 * share the values' dtype. chain_mask (B, L, L) is required (nonzero =
 * different chains). Any L >= 1; head dim D a multiple of 8, at most 64. */
typedef struct mpattn_combine_fwd_params {
    mpattn_tensor intra_logits, inter_logits;  /* pre-softmax, padded = -inf */
    mpattn_tensor intra_values, inter_values;  /* (B, H, L, D)               */
    mpattn_tensor out;                         /* (B, H, L, D), written      */
    float *lse;              /* optional (B,H,L) fp32 log-sum-exp, or NULL  */
    const uint8_t *chain_mask;
    int64_t mask_stride_b, mask_stride_q, mask_stride_k;
    int32_t B, H, L, D;
    int32_t dtype;
    float dropout_p;         /* attention dropout in [0, 1)                  */
    uint64_t dropout_seed;   /* the mask of mpattn_fwd's dropout definition */
} mpattn_combine_fwd_params;

typedef struct mpattn_combine_bwd_params {
    mpattn_tensor intra_logits, inter_logits, intra_values, inter_values;
    mpattn_tensor grad_out;                    /* dO (B, H, L, D)            */
    mpattn_tensor d_intra_logits, d_inter_logits;  /* (B, H, L, L), written  */
    mpattn_tensor d_intra_values, d_inter_values;  /* (B, H, L, D), written  */
    const uint8_t *chain_mask;
    int64_t mask_stride_b, mask_stride_q, mask_stride_k;
    void *workspace;         /* >= mpattn_combine_bwd_workspace_size() bytes,
                                256-byte aligned                            */
    int64_t workspace_bytes; /* size of the buffer at workspace             */
    int32_t B, H, L, D;
    int32_t dtype;
    float dropout_p;         /* the forward's dropout_p and dropout_seed    */
    uint64_t dropout_seed;
    /* Optional (no counterpart in the reference, whose backward recomputes
     * the row statistics): the forward's (B,H,L) fp32 log-sum-exp (from
     * mpattn_combine_fwd's lse) and its output O. With lse non-NULL the
     * backward takes LSE from it and Delta = dO . O from out, instead of a
     * statistics pass over both logit tensors; NULL: that pass runs. */
    const float *lse;
    mpattn_tensor out;       /* (B, H, L, D), read when lse is non-NULL     */
} mpattn_combine_bwd_params;

/* Forward of the combine: O = softmax(where(mask, inter, intra)) split by
 * pathway times (Vs, Vm). Replaces fused_multimer_combine
 * (mint_plus/models/kernels/__init__.py:179-242); no power-of-2 limit on L. */
int mpattn_combine_fwd(const mpattn_combine_fwd_params *p, void *stream);

/* Workspace bytes mpattn_combine_bwd needs (row statistics). */
int64_t mpattn_combine_bwd_workspace_size(int32_t B, int32_t H, int32_t L, int32_t D);

/* Backward of the combine: gradients of both logit tensors and both value
 * tensors, deterministic. Replaces fused_multimer_combine_bwd
 * (mint_plus/models/kernels/__init__.py:247-286). */
int mpattn_combine_bwd(const mpattn_combine_bwd_params *p, void *stream);

/* Human-readable message for an MPATTN_ERR_* code, and the detail of the
 * most recent validation failure on the calling thread. */
const char *mpattn_strerror(int code);
const char *mpattn_last_error(void);
int mpattn_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MPATTN_H */
