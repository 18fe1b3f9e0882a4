// fp32 backward of the multi-pathway attention for gfx950 (the ESM-2 8M model
// trains in fp32; the tolerance is 1e-4 max-abs, so every product and sum
// stays in fp32 on v_mfma_f32_32x32x2f32 and nothing is rounded to 16 bits).
//
// Same gradients as the 16-bit backward (mpattn_bwd.hip, which also runs the
// prep kernel for this path: Delta = dO . O, LSE * log2(e), chain summaries
// and, with fused RoPE, the forward's fp32 operands R(q_self) * f, R(k_self),
// q_multi * f):
//
//   P_ij = exp2(c s_ij - LSE2_i)      s_ij = Q_sel,i . K_sel,j
//   softmax:       dV_j += P_ij dO_i,  dS_ij = P_ij (dP_ij - Delta_i)
//   sqrt-softmax:  w_ij = sqrt(P_ij) (the fp32 forward's weight),
//                  dV_j += w_ij dO_i,  dS_ij = w_ij (dP_ij - w_ij Delta_i) / 2
//   dP_ij = dO_i . V_sel,j;  dQ_i = scale sum_j dS_ij K_sel,j;
//   dK_j = kmul sum_i dS_ij Q_sel,i;  R^T applied to dQ_self and dK_self.
//   With dropout (keep mask Z, r = 1 / (1 - p)): dV takes r Z w and dP_ij
//   becomes r Z_ij dO_i . V_sel,j (the forward's definition in mpattn.h).
//
// One launch, bwd32_kernel, runs dK/dV workgroups and then dQ workgroups.
// Both split the work by pathway: a workgroup computes the gradients
// of one pathway only, so it needs one pathway's operands and accumulators
// (half the registers; a (query, key) pair contributes to exactly one
// pathway). Workgroups of the two pathways of one row block are adjacent in
// dispatch order, so they share their XCD's L2.
//
//  * dK/dV (key-stationary): 4 wavefronts x 32 keys. K and V of
//    the wave's keys sit in registers as MFMA B operands (lane l: dims
//    2*kk + l/32 of key l%32). 32-query subtiles of Q, dO, LSE2, Delta and
//    chain ids stream through LDS, double-buffered. S = Q K^T and dP = dO V^T
//    read query rows in the order pi(r) = 2*(4*(r/8) + r%4) + (r/4)%2, so
//    slot i of lane half hh holds query 2*i + hh: the B operand of step i of
//    dV^T += dO^T P and dK^T += Q^T dS.
//  * dQ (query-stationary): the fp32 forward's structure
//    (S^T = K Q^T with Q in registers), plus dP^T = V dO^T and
//    dQ^T += K^T dS^T.
// Subtiles are classified from the prep kernel's chain summaries: all pairs on
// the other pathway (skipped), all on this one (no per-pair selection), or
// mixed. No atomics: results are bitwise reproducible.
#include "mpattn_bwd.h"

namespace mpattn {
namespace {

constexpr int kTB = 32;  // rows per staged subtile

__device__ __forceinline__ f32x16 mma32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

struct RowSrc {
    const float* base;  // row 0 of this (b, h)
    int64_t st;         // row stride (floats)
};

__device__ __forceinline__ RowSrc tensor_rows(const mpattn_tensor& t, int b, int h) {
    return {(const float*)t.ptr + b * t.stride_b + h * t.stride_h, t.stride_t};
}

// Rotated / folded operands in the workspace: [B][H][Lp][D], rows past L zero.
__device__ __forceinline__ RowSrc ws_rows(const void* ws, int b, int h, int H, int Lp, int D) {
    return {(const float*)ws + ((int64_t)b * H + h) * Lp * D, D};
}

// Slot order of the row-major operand reads (see the header).
__device__ __forceinline__ int slot_perm(int r) { return 2 * (4 * (r / 8) + r % 4) + ((r / 4) & 1); }

// Mode of a (query block, key block) pair for pathway PW from the chain
// summaries {min chain, max chain, count}: 0 skip, 1 every pair on PW,
// 2 mixed (per-pair selection). `kclean`: the key block has no padded keys.
template <int PW, bool DENSE>
__device__ __forceinline__ int pair_mode(int qmin, int qmax, int kmin, int kmax, bool kclean) {
    if (DENSE || !kclean) return 2;
    const bool same = kmin == kmax && qmin == qmax && kmin == qmin;
    const bool cross = kmax < qmin || kmin > qmax;
    if (same) return PW == 0 ? 1 : 0;
    if (cross) return PW == 1 ? 1 : 0;
    return 2;
}

// Store 32 rows r0.. of a transposed accumulator (rows = head dims, columns =
// the wave's 32 rows of dst) times `mul`; rows >= L are skipped, rows with a
// clear bit in `live` are written as zeros; `rope` applies R_r^T.
template <int D>
__device__ void store_rows32(const f32x16* acc, float* scratch, const mpattn_tensor& dst, int b, int h,
                             int r0, int L, float mul, bool rope, const float* cos_tab,
                             const float* sin_tab, uint32_t live) {
    constexpr int NDB = (D + 31) / 32;
    constexpr int LD = NDB * 32 + 1;
    constexpr int H2 = D / 2;
    const int lane = threadIdx.x & 63, hh = lane >> 5, ql = lane & 31;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) scratch[ql * LD + db * 32 + 8 * (i / 4) + 4 * hh + (i % 4)] = acc[db][i] * mul;
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    constexpr int NC = D / 4;
    for (int it = lane; it < kTB * NC; it += 64) {
        const int row = it / NC, d0 = (it % NC) * 4;
        const int r = r0 + row;
        if (r >= L) continue;
        const bool lv = (live >> row) & 1u;
        float x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int d = d0 + u;
            x[u] = lv ? scratch[row * LD + d] : 0.f;
            if (rope && lv) {
                const bool lo = d < H2;
                const int dp = lo ? d + H2 : d - H2;
                const int fi = lo ? d : dp;
                // transpose of x*cos + rotate_half(x)*sin
                x[u] = rope_rot(x[u], scratch[row * LD + dp], cos_tab[(int64_t)r * H2 + fi],
                                sin_tab[(int64_t)r * H2 + fi], !lo);
            }
        }
        float* out = (float*)dst.ptr + b * dst.stride_b + h * dst.stride_h + (int64_t)r * dst.stride_t;
        *reinterpret_cast<f32x4*>(out + d0) = f32x4{x[0], x[1], x[2], x[3]};
    }
    __builtin_amdgcn_wave_barrier();
}

// Stage rows r0..r0+31 of two row sources into LDS tiles (row stride RS);
// rows past `nrows` are clamped (their weights are zero).
template <int D, int RS>
__device__ __forceinline__ void stage_two(float* st, RowSrc s0, RowSrc s1, int r0, int nrows, int tid) {
    constexpr int C4 = D / 4;
    for (int it = tid; it < 2 * kTB * C4; it += 256) {
        const int ten = it / (kTB * C4);
        const int rem = it % (kTB * C4);
        const int r = rem / C4, d0 = (rem % C4) * 4;
        const int row = min(r0 + r, nrows - 1);
        const RowSrc s = ten ? s1 : s0;
        const f32x4 x = *reinterpret_cast<const f32x4*>(s.base + row * s.st + d0);
        float* dst = st + ten * kTB * RS + r * RS + d0;
        dst[0] = x[0];
        dst[1] = x[1];
        dst[2] = x[2];
        dst[3] = x[3];
    }
}

template <int D>
struct Shape32 {
    static constexpr int NK = D / 2;           // MFMA steps over head dims
    static constexpr int NDB = (D + 31) / 32;  // 32-dim blocks of the transposed accumulators
    static constexpr int RS = D + 1;           // LDS row stride (floats), odd: no bank conflicts
    static constexpr int TILE = kTB * RS;
    static constexpr int STAGE = 2 * TILE;     // two row tiles per buffer
    static constexpr int SCR = 4 * kTB * (NDB * 32 + 1);  // epilogue scratch, 4 waves
    static constexpr int SMEM = 2 * STAGE > SCR ? 2 * STAGE : SCR;
};

// ---------------------------------------------------------------------------
// dK / dV of pathway PW for 128 keys.
// ---------------------------------------------------------------------------
template <int D, bool ROPE, bool DENSE, bool SQRT, bool DROP, int PW>
__device__ void dkdv32_body(const BwdArgs& a, float* smem, int* sint, int kb, int b, int h) {
    using S = Shape32<D>;
    constexpr int NK = S::NK, NDB = S::NDB, RS = S::RS, TILE = S::TILE;
    const mpattn_bwd_params& p = a.p;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kl = lane & 31, hh = lane >> 5;
    const int L = p.L, H = p.H, Lp = a.Lp;
    const int kw0 = kb * 128 + wave * 32;
    const int key = kw0 + kl;
    const bool kvalid = key < L;

    // This wave's keys: operands, chain, padding.
    const RowSrc ksrc = PW == 0 ? (ROPE ? ws_rows(a.krot, b, h, H, Lp, D) : tensor_rows(p.k_self, b, h))
                                : tensor_rows(p.k_multi, b, h);
    const RowSrc vsrc = tensor_rows(PW == 0 ? p.v_self : p.v_multi, b, h);
    float kf[NK], vf[NK];
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
        kf[kk] = kvalid ? ksrc.base[key * ksrc.st + 2 * kk + hh] : 0.f;
        vf[kk] = kvalid ? vsrc.base[key * vsrc.st + 2 * kk + hh] : 0.f;
    }
    const int ke = kvalid ? a.keff[(int64_t)b * Lp + key] : kPadChain;
    const bool kpad = ke == kPadChain;
    const uint32_t key_live = (uint32_t)(__ballot(!kpad) & 0xffffffffull);
    // Wave-uniform chain range of the live keys (a wave past L has none).
    // Padded keys need no per-pair test here: their lanes get P = 0.
    int kmin = 0, kmax = -1;
    if (kw0 < L) {
        const int4 ks = reinterpret_cast<const int4*>(a.ksum)[(int64_t)b * (Lp / 32) + kw0 / 32];
        kmin = __builtin_amdgcn_readfirstlane(ks.x);
        kmax = __builtin_amdgcn_readfirstlane(ks.y);
    }
    const bool wave_live = key_live != 0;

    const RowSrc qsrc = PW == 0 ? (ROPE ? ws_rows(a.qrot, b, h, H, Lp, D) : tensor_rows(p.q_self, b, h))
                                : (ROPE ? ws_rows(a.qmf, b, h, H, Lp, D) : tensor_rows(p.q_multi, b, h));
    const RowSrc gsrc = tensor_rows(p.grad_out, b, h);
    const float* lse2 = a.lse2 + ((int64_t)b * H + h) * Lp;
    const float* delta = a.delta + ((int64_t)b * H + h) * Lp;
    const int* qcid = a.qcid + (int64_t)b * Lp;
    const uint8_t* mcol = nullptr;  // dense mask column of this lane's key
    if constexpr (DENSE) mcol = p.chain_mask + (int64_t)b * p.mask_stride_b + (int64_t)(kvalid ? key : 0) * p.mask_stride_k;

    // sint: per buffer lse2[32], delta (as bits)[32], qcid[32]
    auto stage_in = [&](int t, int bf) {
        const int q0 = t * kTB;
        stage_two<D, RS>(smem + bf * S::STAGE, qsrc, gsrc, q0, L, tid);
        if (tid < kTB) {
            int* si = sint + bf * 3 * kTB;
            si[tid] = __float_as_int(lse2[q0 + tid]);  // q0 + tid < Lp
            si[kTB + tid] = __float_as_int(delta[q0 + tid]);
            si[2 * kTB + tid] = qcid[q0 + tid];
        }
    };

    f32x16 dv[NDB], dk[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) dv[db][i] = dk[db][i] = 0.f;

    const int perm = slot_perm(kl);
    const float c = a.c;
    const int4* qsum = reinterpret_cast<const int4*>(a.qsum) + (int64_t)b * (Lp / 32);
    const int nsub = (L + kTB - 1) / kTB;
    stage_in(0, 0);
    __syncthreads();
    for (int t = 0; t < nsub; ++t) {
        const int bf = t & 1;
        if (t + 1 < nsub) stage_in(t + 1, bf ^ 1);
        const float* qt = smem + bf * S::STAGE;  // Q_pw rows
        const float* gt = qt + TILE;             // dO rows
        const int* si = sint + bf * 3 * kTB;
        const int4 qs = qsum[t];
        const int mode = wave_live ? pair_mode<PW, DENSE>(__builtin_amdgcn_readfirstlane(qs.x),
                                                          __builtin_amdgcn_readfirstlane(qs.y), kmin, kmax,
                                                          true)
                                   : 0;
        if (mode != 0) {
            f32x16 s, dp;
#pragma unroll
            for (int i = 0; i < 16; ++i) s[i] = dp[i] = 0.f;
#pragma unroll
            for (int kk = 0; kk < NK; ++kk) {
                s = mma32(qt[perm * RS + 2 * kk + hh], kf[kk], s);
                dp = mma32(gt[perm * RS + 2 * kk + hh], vf[kk], dp);
            }
            f32x16 wv, ds;  // weight of dO in dV; dS
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int ql = 2 * i + hh;
                bool on = !kpad;
                if (mode == 2) {
                    bool same;
                    if constexpr (DENSE) {
                        const int q = t * kTB + ql;
                        same = !(q < L && kvalid && mcol[(int64_t)q * p.mask_stride_q] != 0);
                    } else {
                        same = si[2 * kTB + ql] == ke;
                    }
                    on = on && (same == (PW == 0));
                }
                const float l2 = __int_as_float(si[ql]);
                const float dl = __int_as_float(si[kTB + ql]);
                const float pr = on ? fast_exp2(s[i] * c + l2) : 0.f;  // (l2, dl: -LSE2, -Delta)
                const float w = SQRT ? sqrtf(pr) : pr;
                float dpi = dp[i];
                bool keep = true;
                if constexpr (DROP) {
                    keep = drop_keep(drop_row(a.drop.lo, (uint32_t)(b * p.H + h), (uint32_t)(t * kTB + ql)),
                                     a.drop.hi, (uint32_t)key, a.drop.thr);
                    dpi = keep ? dpi * a.drop.rkeep : 0.f;
                }
                wv[i] = keep ? w : 0.f;  // (1 / (1 - p) applied when dV is stored)
                ds[i] = SQRT ? 0.5f * w * (dpi + w * dl) : w * (dpi + dl);
            }
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                const int d = db * 32 + kl;
#pragma unroll
                for (int kk = 0; kk < 16; ++kk) {
                    const float go = d < D ? gt[(2 * kk + hh) * RS + d] : 0.f;
                    const float qv = d < D ? qt[(2 * kk + hh) * RS + d] : 0.f;
                    dv[db] = mma32(go, wv[kk], dv[db]);
                    dk[db] = mma32(qv, ds[kk], dk[db]);
                }
            }
        }
        __syncthreads();
    }

    float* scratch = smem + wave * kTB * (NDB * 32 + 1);
    const mpattn_tensor& dvt = PW == 0 ? p.dv_self : p.dv_multi;
    const mpattn_tensor& dkt = PW == 0 ? p.dk_self : p.dk_multi;
    if (kw0 < L) {
        store_rows32<D>(dv, scratch, dvt, b, h, kw0, L, DROP ? a.drop.rkeep : 1.0f, false, nullptr, nullptr,
                        key_live);
        store_rows32<D>(dk, scratch, dkt, b, h, kw0, L, a.kmul, ROPE && PW == 0, p.rope_cos, p.rope_sin,
                        key_live);
    }
}

// ---------------------------------------------------------------------------
// dQ of pathway PW for 128 queries.
// ---------------------------------------------------------------------------
template <int D, bool ROPE, bool DENSE, bool SQRT, bool DROP, int PW>
__device__ void dq32_body(const BwdArgs& a, float* smem, int* sint, int qb, int b, int h) {
    using S = Shape32<D>;
    constexpr int NK = S::NK, NDB = S::NDB, RS = S::RS, TILE = S::TILE;
    const mpattn_bwd_params& p = a.p;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ql = lane & 31, hh = lane >> 5;
    const int L = p.L, H = p.H, Lp = a.Lp;
    const int qw0 = qb * 128 + wave * 32;
    const int q = qw0 + ql;
    const bool qvalid = q < L;

    const RowSrc qsrc = PW == 0 ? (ROPE ? ws_rows(a.qrot, b, h, H, Lp, D) : tensor_rows(p.q_self, b, h))
                                : (ROPE ? ws_rows(a.qmf, b, h, H, Lp, D) : tensor_rows(p.q_multi, b, h));
    const RowSrc gsrc = tensor_rows(p.grad_out, b, h);
    float qf[NK], gf[NK];
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
        qf[kk] = qvalid ? qsrc.base[q * qsrc.st + 2 * kk + hh] : 0.f;
        gf[kk] = qvalid ? gsrc.base[q * gsrc.st + 2 * kk + hh] : 0.f;
    }
    const int64_t rowi = ((int64_t)b * H + h) * Lp + (qvalid ? q : 0);
    const float l2 = qvalid ? a.lse2[rowi] : -INFINITY;  // -LSE2
    const float dl = qvalid ? a.delta[rowi] : 0.f;
    const uint32_t drow = DROP ? drop_row(a.drop.lo, (uint32_t)(b * H + h), (uint32_t)q) : 0u;
    const int cq = qvalid ? a.qcid[(int64_t)b * Lp + q] : 0;
    int qmin = 0, qmax = -1;
    if (qw0 < L) {
        const int4 qs = reinterpret_cast<const int4*>(a.qsum)[(int64_t)b * (Lp / 32) + qw0 / 32];
        qmin = __builtin_amdgcn_readfirstlane(qs.x);
        qmax = __builtin_amdgcn_readfirstlane(qs.y);
    }
    const bool wave_live = qw0 < L;
    const uint8_t* mrow = nullptr;
    if constexpr (DENSE) mrow = p.chain_mask + (int64_t)b * p.mask_stride_b + (int64_t)(qvalid ? q : 0) * p.mask_stride_q;

    const RowSrc ksrc = PW == 0 ? (ROPE ? ws_rows(a.krot, b, h, H, Lp, D) : tensor_rows(p.k_self, b, h))
                                : tensor_rows(p.k_multi, b, h);
    const RowSrc vsrc = tensor_rows(PW == 0 ? p.v_self : p.v_multi, b, h);
    const int* keff = a.keff + (int64_t)b * Lp;
    auto stage_in = [&](int t, int bf) {
        const int k0 = t * kTB;
        stage_two<D, RS>(smem + bf * S::STAGE, ksrc, vsrc, k0, L, tid);
        if (tid < kTB) sint[bf * kTB + tid] = keff[k0 + tid];  // k0 + tid < Lp
    };

    f32x16 dq[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) dq[db][i] = 0.f;

    const int perm = slot_perm(ql);
    const float c = a.c;
    const int4* ksum = reinterpret_cast<const int4*>(a.ksum) + (int64_t)b * (Lp / 32);
    const int nsub = (L + kTB - 1) / kTB;
    stage_in(0, 0);
    __syncthreads();
    for (int t = 0; t < nsub; ++t) {
        const int bf = t & 1;
        if (t + 1 < nsub) stage_in(t + 1, bf ^ 1);
        const float* kt = smem + bf * S::STAGE;  // K_pw rows
        const float* vt = kt + TILE;             // V_pw rows
        const int* kc = sint + bf * kTB;
        const int4 ks = ksum[t];
        const int npad = __builtin_amdgcn_readfirstlane(ks.z);
        const int mode = wave_live && npad < kTB
                             ? pair_mode<PW, DENSE>(qmin, qmax, __builtin_amdgcn_readfirstlane(ks.x),
                                                    __builtin_amdgcn_readfirstlane(ks.y), npad == 0)
                             : 0;
        if (mode != 0) {
            f32x16 s, dp;
#pragma unroll
            for (int i = 0; i < 16; ++i) s[i] = dp[i] = 0.f;
#pragma unroll
            for (int kk = 0; kk < NK; ++kk) {
                s = mma32(kt[perm * RS + 2 * kk + hh], qf[kk], s);
                dp = mma32(vt[perm * RS + 2 * kk + hh], gf[kk], dp);
            }
            f32x16 ds;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int kl = 2 * i + hh;
                bool on = true;
                if (mode == 2) {
                    const int ck = kc[kl];
                    bool same;
                    if constexpr (DENSE) {
                        const int kg = t * kTB + kl;
                        same = !(kg < L && qvalid && mrow[(int64_t)kg * p.mask_stride_k] != 0);
                    } else {
                        same = ck == cq;
                    }
                    on = ck != kPadChain && (same == (PW == 0));
                }
                const float pr = on ? fast_exp2(s[i] * c + l2) : 0.f;  // (l2, dl: -LSE2, -Delta)
                const float w = SQRT ? sqrtf(pr) : pr;
                float dpi = dp[i];
                if constexpr (DROP)
                    dpi = drop_keep(drow, a.drop.hi, (uint32_t)(t * kTB + kl), a.drop.thr) ? dpi * a.drop.rkeep : 0.f;
                ds[i] = SQRT ? 0.5f * w * (dpi + w * dl) : w * (dpi + dl);
            }
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                const int d = db * 32 + ql;
#pragma unroll
                for (int kk = 0; kk < 16; ++kk) {
                    const float kv = d < D ? kt[(2 * kk + hh) * RS + d] : 0.f;
                    dq[db] = mma32(kv, ds[kk], dq[db]);
                }
            }
        }
        __syncthreads();
    }

    float* scratch = smem + wave * kTB * (NDB * 32 + 1);
    if (qw0 < L)
        store_rows32<D>(dq, scratch, PW == 0 ? p.dq_self : p.dq_multi, b, h, qw0, L, p.scale,
                        ROPE && PW == 0, p.rope_cos, p.rope_sin, 0xffffffffu);
}

// dK/dV and dQ in one grid (same inputs, disjoint outputs): workgroups
// [0, nkv) compute dK/dV, one per (key block, pathway, b*H + h), the rest
// dQ, one per (query block, pathway, b*H + h). At the 8M shape each half
// has fewer workgroups than the GPU has CUs, so the two run side by side.
template <int D, bool ROPE, bool DENSE, bool SQRT, bool DROP>
__global__ __launch_bounds__(256) void bwd32_kernel(const BwdArgs a, int nkv) {
    __shared__ float smem[Shape32<D>::SMEM];
    __shared__ int sint[2 * 3 * kTB];
    const int nb = (a.p.L + 127) / 128;
    const int bid = blockIdx.x;
    const bool kv = bid < nkv;
    const int g = kv ? xcd_remap(bid, nkv) : xcd_remap(bid - nkv, (int)gridDim.x - nkv);
    const int pw = g & 1, rest = g >> 1;
    const int rb = rest % nb, bh = rest / nb;
    const int b = bh / a.p.H, h = bh % a.p.H;
    if (kv) {
        if (pw == 0) dkdv32_body<D, ROPE, DENSE, SQRT, DROP, 0>(a, smem, sint, rb, b, h);
        else dkdv32_body<D, ROPE, DENSE, SQRT, DROP, 1>(a, smem, sint, rb, b, h);
    } else {
        if (pw == 0) dq32_body<D, ROPE, DENSE, SQRT, DROP, 0>(a, smem, sint, rb, b, h);
        else dq32_body<D, ROPE, DENSE, SQRT, DROP, 1>(a, smem, sint, rb, b, h);
    }
}

template <int D, bool ROPE, bool DENSE, bool SQRT, bool DROP>
hipError_t launch32(const BwdArgs& a, hipStream_t stream) {
    const int nb = (a.p.L + 127) / 128;
    const unsigned grid = (unsigned)(2 * (int64_t)a.p.B * a.p.H * nb);
    hipLaunchKernelGGL((bwd32_kernel<D, ROPE, DENSE, SQRT, DROP>), dim3(2 * grid), dim3(256), 0, stream, a,
                       (int)grid);
    return hipGetLastError();
}

template <int D, bool DROP>
hipError_t dispatch32_d(const BwdArgs& a, hipStream_t s) {
    const bool rope = a.p.rope == MPATTN_ROPE_FUSED, dense = a.p.chain_mask != nullptr;
    const bool sq = a.p.sqrt_softmax != 0;
#define MPATTN_B32(R, DN, SQ) return launch32<D, R, DN, SQ, DROP>(a, s)
    if (rope) {
        if (dense) { if (sq) MPATTN_B32(true, true, true); MPATTN_B32(true, true, false); }
        if (sq) MPATTN_B32(true, false, true);
        MPATTN_B32(true, false, false);
    }
    if (dense) { if (sq) MPATTN_B32(false, true, true); MPATTN_B32(false, true, false); }
    if (sq) MPATTN_B32(false, false, true);
    MPATTN_B32(false, false, false);
#undef MPATTN_B32
}

template <int D>
hipError_t dispatch32(const BwdArgs& a, hipStream_t s) {
    if (a.p.dropout_p > 0.f) return dispatch32_d<D, true>(a, s);
    return dispatch32_d<D, false>(a, s);
}

}  // namespace

hipError_t launch_bwd32(const BwdArgs& a, hipStream_t stream) {
    switch (a.p.D) {
        case 16: return dispatch32<16>(a, stream);
        case 24: return dispatch32<24>(a, stream);
        case 32: return dispatch32<32>(a, stream);
        case 64: return dispatch32<64>(a, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace mpattn
