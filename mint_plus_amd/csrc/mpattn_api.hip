// C-ABI entry points of libmpattn.so: argument validation and dispatch.
//
// Validation mirrors the reference wrappers' asserts
// (mint_plus/models/kernels/multi_pathway_attention.py:224-227,
// mint_plus/models/kernels/__init__.py:203) and adds the layout rules the
// vectorised kernels rely on (16-byte aligned rows).
#include <stdarg.h>
#include <stdio.h>
#include <math.h>

#include "mpattn_common.h"

namespace mpattn {
hipError_t launch_fwd16(const mpattn_fwd_params& p, hipStream_t stream);
int64_t fwd_workspace_bytes(int B, int H, int L, int D, int dtype, int rope);
hipError_t launch_fwd32(const mpattn_fwd_params& p, hipStream_t stream);
hipError_t launch_bwd(const mpattn_bwd_params& p, hipStream_t stream);
int64_t bwd_workspace_bytes(int B, int H, int L, int D);
hipError_t launch_combine_fwd(const mpattn_combine_fwd_params& p, float* lse, hipStream_t stream);
hipError_t launch_combine_bwd(const mpattn_combine_bwd_params& p, hipStream_t stream);
int64_t combine_bwd_workspace_bytes(int B, int H, int L);
}  // namespace mpattn

namespace {

thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int elt_size(int dtype) { return dtype == MPATTN_FP32 ? 4 : 2; }

// Every row start must be 16-byte aligned: base pointer aligned and all
// strides multiples of 16 bytes.
int check_tensor(const mpattn_tensor& t, const char* name, int esize, bool out) {
    if (!t.ptr) return fail(MPATTN_ERR_INVALID, "%s: null pointer", name);
    if ((uintptr_t)t.ptr % 16) return fail(MPATTN_ERR_UNSUPPORTED, "%s: base not 16-byte aligned", name);
    const int64_t q = 16 / esize;
    if (t.stride_b % q || t.stride_h % q || t.stride_t % q)
        return fail(MPATTN_ERR_UNSUPPORTED, "%s: strides must be multiples of %lld elements", name,
                    (long long)q);
    if (t.stride_b < 0 || t.stride_h < 0 || t.stride_t < 0)
        return fail(MPATTN_ERR_UNSUPPORTED, "%s: negative stride", name);
    (void)out;
    return MPATTN_OK;
}

// The kernels address rows with 32-bit byte offsets from each (b, h) base
// (the DMA copies take a 32-bit per-lane offset); the last row's end must fit.
int check_row_offsets(const mpattn_tensor* const* ts, const char* const* names, int n, int L, int esize) {
    for (int i = 0; i < n; ++i)
        if ((int64_t)L * ts[i]->stride_t * esize + 64 * esize > 0x7fffffffLL)
            return fail(MPATTN_ERR_UNSUPPORTED, "%s: L * stride_t too large for 32-bit row offsets", names[i]);
    return MPATTN_OK;
}

int check_common(int B, int H, int L, int D, int dtype, int rope, float scale,
                 const int32_t* chain_id, const uint8_t* chain_mask, int64_t msb, int64_t msq,
                 int64_t msk, const float* rc, const float* rs, int sqrt_softmax) {
    if (B < 1 || H < 1 || L < 1) return fail(MPATTN_ERR_INVALID, "B, H, L must be >= 1 (got %d, %d, %d)", B, H, L);
    if (dtype != MPATTN_BF16 && dtype != MPATTN_FP16 && dtype != MPATTN_FP32)
        return fail(MPATTN_ERR_INVALID, "unknown dtype %d", dtype);
    if (D != 16 && D != 24 && D != 32 && D != 64)
        return fail(MPATTN_ERR_UNSUPPORTED, "head dim %d not supported (16, 24, 32, 64)", D);
    if (rope != MPATTN_ROPE_NONE && rope != MPATTN_ROPE_FUSED)
        return fail(MPATTN_ERR_INVALID, "unknown rope mode %d", rope);
    if (!(scale > 0.f) || !isfinite(scale)) return fail(MPATTN_ERR_INVALID, "scale must be finite and > 0");
    if ((chain_id == nullptr) == (chain_mask == nullptr))
        return fail(MPATTN_ERR_INVALID, "exactly one of chain_id / chain_mask must be given");
    if (chain_id && (uintptr_t)chain_id % 4) return fail(MPATTN_ERR_INVALID, "chain_id misaligned");
    if (chain_mask && (msb < 0 || msq < 0 || msk < 0))
        return fail(MPATTN_ERR_UNSUPPORTED, "chain_mask: negative stride");
    if (rope == MPATTN_ROPE_FUSED) {
        if (!rc || !rs) return fail(MPATTN_ERR_INVALID, "rope tables required for fused RoPE");
        if ((uintptr_t)rc % 16 || (uintptr_t)rs % 16)
            return fail(MPATTN_ERR_UNSUPPORTED, "rope tables not 16-byte aligned");
    }
    if (sqrt_softmax != 0 && sqrt_softmax != 1) return fail(MPATTN_ERR_INVALID, "sqrt_softmax must be 0/1");
    // Every launch stays below 2^32 work-items (HIP's limit per grid): at
    // most 24 per padded row (the backward's prep: up to 8 for Delta and 12
    // for the RoPE rotations), and with a dense mask 1/16 per mask element
    // plus 64 per batch row and query (its label and block checks).
    // (in double: the products of extreme arguments overflow int64)
    const double lim = 4294967295.0, Lp = (double)(((int64_t)L + 127) / 128 * 128);
    const double rows = (double)B * H * Lp;
    const bool mask_big = chain_mask && (double)B * Lp * (Lp / 16) + (double)B * Lp * 64 > lim;
    if (rows * 24 > lim || mask_big || (int64_t)L * 4 > 0x7fffffffLL)
        return fail(MPATTN_ERR_UNSUPPORTED, "problem too large for one launch");
    return MPATTN_OK;
}

// Attention dropout: p in [0, 1) (every element type, with or without
// sqrt-softmax).
int check_dropout(float p, int dtype, int sqrt_softmax) {
    (void)dtype;
    (void)sqrt_softmax;
    if (!(p >= 0.f && p < 1.f)) return fail(MPATTN_ERR_INVALID, "dropout_p must be in [0, 1) (got %g)", (double)p);
    return MPATTN_OK;
}

// Shape, dtype and mask checks shared by the combine entry points.
int check_combine(int B, int H, int L, int D, int dtype, const uint8_t* mask, int64_t msb,
                  int64_t msq, int64_t msk, float dropout_p) {
    if (B < 1 || H < 1 || L < 1) return fail(MPATTN_ERR_INVALID, "B, H, L must be >= 1 (got %d, %d, %d)", B, H, L);
    if (dtype != MPATTN_BF16 && dtype != MPATTN_FP16 && dtype != MPATTN_FP32)
        return fail(MPATTN_ERR_INVALID, "unknown dtype %d", dtype);
    if (D < 8 || D > 64 || D % 8)
        return fail(MPATTN_ERR_UNSUPPORTED, "combine: head dim %d not supported (multiple of 8, <= 64)", D);
    if (!mask) return fail(MPATTN_ERR_INVALID, "chain_mask required");
    if (msb < 0 || msq < 0 || msk < 0) return fail(MPATTN_ERR_UNSUPPORTED, "chain_mask: negative stride");
    if (!(dropout_p >= 0.f && dropout_p < 1.f))
        return fail(MPATTN_ERR_INVALID, "dropout_p must be in [0, 1) (got %g)", (double)dropout_p);
    // every launch below 2^32 work-items: at most 8 per row (the backward's
    // Delta from the forward's output; the others take 2 to 4)
    if ((double)B * H * (((int64_t)L + 127) / 128 * 128) * 8 > 4294967295.0)
        return fail(MPATTN_ERR_UNSUPPORTED, "problem too large for one launch");
    return MPATTN_OK;
}

// Argument checks of mpattn_fwd / mpattn_fwd_noalloc (everything but the
// workspace).
int validate_fwd(const mpattn_fwd_params* p) {
    if (!p) return fail(MPATTN_ERR_INVALID, "null params");
    int rc = check_common(p->B, p->H, p->L, p->D, p->dtype, p->rope, p->scale, p->chain_id,
                          p->chain_mask, p->mask_stride_b, p->mask_stride_q, p->mask_stride_k,
                          p->rope_cos, p->rope_sin, p->sqrt_softmax);
    if (rc) return rc;
    if ((rc = check_dropout(p->dropout_p, p->dtype, p->sqrt_softmax))) return rc;
    const int es = elt_size(p->dtype);
    const mpattn_tensor* ts[7] = {&p->q_self, &p->k_self, &p->v_self, &p->q_multi,
                                  &p->k_multi, &p->v_multi, &p->out};
    const char* names[7] = {"q_self", "k_self", "v_self", "q_multi", "k_multi", "v_multi", "out"};
    for (int i = 0; i < 7; ++i)
        if ((rc = check_tensor(*ts[i], names[i], es, i == 6))) return rc;
    if (p->lse && (uintptr_t)p->lse % 4) return fail(MPATTN_ERR_INVALID, "lse misaligned");
    // Rows are addressed with 32-bit byte offsets from each (b, h) base.
    if ((rc = check_row_offsets(ts, names, 6, p->L, es))) return rc;
    return MPATTN_OK;
}

int launch_fwd_any(const mpattn_fwd_params& p, void* stream) {
    hipError_t e;
    if (p.dtype == MPATTN_FP32) {
        e = mpattn::launch_fwd32(p, (hipStream_t)stream);
    } else {
        e = mpattn::launch_fwd16(p, (hipStream_t)stream);
    }
    if (e != hipSuccess) return fail(MPATTN_ERR_LAUNCH, "fwd launch: %s", hipGetErrorString(e));
    return MPATTN_OK;
}

}  // namespace

namespace mpattn {
// Shared with the no-allocation entry point (mpattn_noalloc.hip).
int api_validate_fwd(const mpattn_fwd_params* p) { return validate_fwd(p); }
int api_launch_fwd(const mpattn_fwd_params& p, void* stream) { return launch_fwd_any(p, stream); }
void api_clear_error() { g_last_error[0] = 0; }
int api_fail(int code, const char* msg) { return fail(code, "%s", msg); }
}  // namespace mpattn

extern "C" {

int mpattn_version(void) { return MPATTN_VERSION; }

const char* mpattn_last_error(void) { return g_last_error; }

const char* mpattn_strerror(int code) {
    switch (code) {
        case MPATTN_OK: return "success";
        case MPATTN_ERR_INVALID: return "invalid argument";
        case MPATTN_ERR_UNSUPPORTED: return "unsupported configuration";
        case MPATTN_ERR_LAUNCH: return "kernel launch failed";
    }
    return "unknown error";
}

int mpattn_fwd(const mpattn_fwd_params* p, void* stream) {
    g_last_error[0] = 0;
    int rc = validate_fwd(p);
    if (rc) return rc;
    {
        const int64_t need = mpattn::fwd_workspace_bytes(p->B, p->H, p->L, p->D, p->dtype, p->rope);
        if (!p->workspace || (uintptr_t)p->workspace % 256 || p->workspace_bytes < need)
            return fail(MPATTN_ERR_INVALID, "workspace: need %lld bytes, 256-byte aligned (got %lld)",
                        (long long)need, (long long)p->workspace_bytes);
    }
    return launch_fwd_any(*p, stream);
}

int64_t mpattn_fwd_workspace_size(int32_t B, int32_t H, int32_t L, int32_t D, int32_t dtype,
                                  int32_t rope) {
    if (B < 1 || H < 1 || L < 1) return -1;
    return mpattn::fwd_workspace_bytes(B, H, L, D, dtype, rope);
}

int64_t mpattn_bwd_workspace_size(int32_t B, int32_t H, int32_t L, int32_t D) {
    if (B < 1 || H < 1 || L < 1) return -1;
    return mpattn::bwd_workspace_bytes(B, H, L, D);
}

int mpattn_bwd(const mpattn_bwd_params* p, void* stream) {
    g_last_error[0] = 0;
    if (!p) return fail(MPATTN_ERR_INVALID, "null params");
    int rc = check_common(p->B, p->H, p->L, p->D, p->dtype, p->rope, p->scale, p->chain_id,
                          p->chain_mask, p->mask_stride_b, p->mask_stride_q, p->mask_stride_k,
                          p->rope_cos, p->rope_sin, p->sqrt_softmax);
    if (rc) return rc;
    if ((rc = check_dropout(p->dropout_p, p->dtype, p->sqrt_softmax))) return rc;
    const int es = elt_size(p->dtype);
    const mpattn_tensor* ts[14] = {&p->q_self,  &p->k_self,   &p->v_self,  &p->q_multi, &p->k_multi,
                                   &p->v_multi, &p->out,      &p->grad_out, &p->dq_self, &p->dk_self,
                                   &p->dv_self, &p->dq_multi, &p->dk_multi, &p->dv_multi};
    const char* names[14] = {"q_self", "k_self", "v_self", "q_multi", "k_multi", "v_multi", "out",
                             "grad_out", "dq_self", "dk_self", "dv_self", "dq_multi", "dk_multi",
                             "dv_multi"};
    for (int i = 0; i < 14; ++i)
        if ((rc = check_tensor(*ts[i], names[i], es, i >= 8))) return rc;
    if (!p->lse || (uintptr_t)p->lse % 4) return fail(MPATTN_ERR_INVALID, "lse required (fp32, aligned)");
    if ((rc = check_row_offsets(ts, names, 14, p->L, es))) return rc;
    if (p->chain_mask &&
        (int64_t)p->L * p->mask_stride_q + (int64_t)p->L * p->mask_stride_k + 16 > 0x7fffffffLL)
        return fail(MPATTN_ERR_UNSUPPORTED, "chain_mask: L * mask_stride_q too large for 32-bit row offsets");
    {
        const int64_t need = mpattn::bwd_workspace_bytes(p->B, p->H, p->L, p->D);
        if (!p->workspace || (uintptr_t)p->workspace % 16 || p->workspace_bytes < need)
            return fail(MPATTN_ERR_INVALID, "workspace: need %lld bytes, 16-byte aligned (got %lld)",
                        (long long)need, (long long)p->workspace_bytes);
    }
    hipError_t e = mpattn::launch_bwd(*p, (hipStream_t)stream);
    if (e == hipErrorInvalidValue) return fail(MPATTN_ERR_UNSUPPORTED, "bwd: configuration not built");
    if (e != hipSuccess) return fail(MPATTN_ERR_LAUNCH, "bwd launch: %s", hipGetErrorString(e));
    return MPATTN_OK;
}

int mpattn_combine_fwd(const mpattn_combine_fwd_params* p, void* stream) {
    g_last_error[0] = 0;
    if (!p) return fail(MPATTN_ERR_INVALID, "null params");
    int rc = check_combine(p->B, p->H, p->L, p->D, p->dtype, p->chain_mask, p->mask_stride_b,
                           p->mask_stride_q, p->mask_stride_k, p->dropout_p);
    if (rc) return rc;
    const int es = elt_size(p->dtype);
    const mpattn_tensor* ts[5] = {&p->intra_logits, &p->inter_logits, &p->intra_values,
                                  &p->inter_values, &p->out};
    const char* names[5] = {"intra_logits", "inter_logits", "intra_values", "inter_values", "out"};
    for (int i = 2; i < 5; ++i)
        if ((rc = check_tensor(*ts[i], names[i], es, i == 4))) return rc;
    for (int i = 0; i < 2; ++i)
        if (!ts[i]->ptr || ts[i]->stride_b < 0 || ts[i]->stride_h < 0 || ts[i]->stride_t < 0)
            return fail(MPATTN_ERR_INVALID, "%s: null pointer or negative stride", names[i]);
    if (p->lse && (uintptr_t)p->lse % 4) return fail(MPATTN_ERR_INVALID, "lse misaligned");
    hipError_t e = mpattn::launch_combine_fwd(*p, p->lse, (hipStream_t)stream);
    if (e != hipSuccess) return fail(MPATTN_ERR_LAUNCH, "combine fwd launch: %s", hipGetErrorString(e));
    return MPATTN_OK;
}

int64_t mpattn_combine_bwd_workspace_size(int32_t B, int32_t H, int32_t L, int32_t D) {
    (void)D;
    if (B < 1 || H < 1 || L < 1) return -1;
    return mpattn::combine_bwd_workspace_bytes(B, H, L);
}

int mpattn_combine_bwd(const mpattn_combine_bwd_params* p, void* stream) {
    g_last_error[0] = 0;
    if (!p) return fail(MPATTN_ERR_INVALID, "null params");
    int rc = check_combine(p->B, p->H, p->L, p->D, p->dtype, p->chain_mask, p->mask_stride_b,
                           p->mask_stride_q, p->mask_stride_k, p->dropout_p);
    if (rc) return rc;
    const int es = elt_size(p->dtype);
    const mpattn_tensor* vt[5] = {&p->intra_values, &p->inter_values, &p->grad_out,
                                  &p->d_intra_values, &p->d_inter_values};
    const char* vn[5] = {"intra_values", "inter_values", "grad_out", "d_intra_values",
                         "d_inter_values"};
    for (int i = 0; i < 5; ++i)
        if ((rc = check_tensor(*vt[i], vn[i], es, i >= 3))) return rc;
    const mpattn_tensor* lt[4] = {&p->intra_logits, &p->inter_logits, &p->d_intra_logits,
                                  &p->d_inter_logits};
    const char* ln[4] = {"intra_logits", "inter_logits", "d_intra_logits", "d_inter_logits"};
    for (int i = 0; i < 4; ++i)
        if (!lt[i]->ptr || lt[i]->stride_b < 0 || lt[i]->stride_h < 0 || lt[i]->stride_t < 0)
            return fail(MPATTN_ERR_INVALID, "%s: null pointer or negative stride", ln[i]);
    if (p->lse) {  // the forward's statistics: LSE and its output O
        if ((uintptr_t)p->lse % 4) return fail(MPATTN_ERR_INVALID, "lse misaligned");
        if ((rc = check_tensor(p->out, "out", es, false))) return rc;
    }
    {
        const int64_t need = mpattn::combine_bwd_workspace_bytes(p->B, p->H, p->L);
        if (!p->workspace || (uintptr_t)p->workspace % 256 || p->workspace_bytes < need)
            return fail(MPATTN_ERR_INVALID, "workspace: need %lld bytes, 256-byte aligned (got %lld)",
                        (long long)need, (long long)p->workspace_bytes);
    }
    hipError_t e = mpattn::launch_combine_bwd(*p, (hipStream_t)stream);
    if (e != hipSuccess) return fail(MPATTN_ERR_LAUNCH, "combine bwd launch: %s", hipGetErrorString(e));
    return MPATTN_OK;
}

}  // extern "C"
