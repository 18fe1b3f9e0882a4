// Backward multi-pathway attention for gfx950 (16-bit inputs, fp32 accumulate).
//
// Gradients of the op defined in include/mpattn.h, following the softmax
// backward of the reference eager path (autograd through
// mint_plus/models/modules_plus.py:178-194 and attention.py:186-236):
//
//   P_ij  = exp(s_ij - LSE_i)                 (LSE saved by the forward)
//   dV_j  = sum_i P_ij dO_i                  (into V_self or V_multi by pathway)
//   dP_ij = dO_i . V_sel(ij),j
//   dS_ij = P_ij (dP_ij - Delta_i),           Delta_i = dO_i . O_i
//   with dropout (keep mask Z, r = 1/(1-p), regenerated from the seed):
//   dV_j = r sum_i Z_ij P_ij dO_i,  dP_ij = r Z_ij dO_i . V_sel(ij),j
//   dQ_i  = scale sum_j dS_ij K_sel,j ;  dK_j = scale sum_i dS_ij Q_sel,i
//   and R_p^T applied to dQ_self / dK_self with fused RoPE.
//
// This is the exact gradient; the reference's Triton backward
// (mint_plus/models/kernels/multi_pathway_attention_bwd.py:123-271) takes the
// softmax row sum per key tile and applies the scale twice, and is not
// followed. No atomics: dK/dV and dQ come from separate workgroups, so
// results are bitwise reproducible.
//
// Launches:
//  1. bwd_prep_kernel: chain staging for keys (as the forward) and queries,
//     Delta and LSE*log2(e) per query, RoPE-rotated Q_self/K_self.
//  2. bwd_kernel: dK/dV workgroups, then dQ workgroups, in one grid.
//     dK/dV (key-stationary, one pathway per workgroup: a pair
//     contributes to one pathway only, so a workgroup holds that pathway's
//     operands and accumulators): each wavefront keeps K and V of 32 keys in
//     registers (MFMA B operands) and streams 64-query stages of Q (of the
//     pathway) and dO through LDS. S and dP come out with lane = key and
//     slot = query (query rows read bit-2/3-swapped), which is directly the A
//     operand of dV += P^T dO and dK += dS^T Q; dO^T and Q^T are transpose
//     reads of the row-major tiles.
//     dQ (query-stationary): the forward's structure plus dP^T = V dO^T
//     and dQ^T += K^T dS^T.
#include <type_traits>

#include "mpattn_bwd.h"

namespace mpattn {

template <int N> using IC = std::integral_constant<int, N>;

int64_t bwd_workspace_bytes(int B, int H, int L, int D) {
    // Sized for the largest element type and fused RoPE: callers allocate
    // once regardless of the mode.
    return bwd_ws_layout(B, H, L, D, 4, true).total;
}

// ---------------------------------------------------------------------------
// Prep: chain staging, Delta / LSE2 rows, RoPE of Q_self and K_self.
// ---------------------------------------------------------------------------
// Prep work split: lanes per row for Delta (8 dims each, a power of two) and
// threads per row for the RoPE rotation.
template <int D> constexpr int kPrepLanes = D <= 16 ? 2 : (D <= 32 ? 4 : 8);
template <int D> constexpr int kRotItems = (D / 2) % 8 == 0 ? D / 16 : 1;

template <typename T, int D, bool ROPE, bool DENSE>
__global__ __launch_bounds__(256) void bwd_prep_kernel(const BwdArgs a, float* lse2, float* delta,
                                                       int* keff, int* ksum, int* qcid, int* qsum,
                                                       T* qrot, T* krot, T* qmf, int nchain, int nrow) {
    typedef typename Elt<T>::v8 v8;
    const mpattn_bwd_params& p = a.p;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int L = p.L, Lp = a.Lp;
    const int bid = blockIdx.x;
    if (bid < nchain) {
        const int ngrp = Lp / 64;
        const int gid = bid * 4 + wave;
        if (gid >= p.B * ngrp) return;
        const int b = gid / ngrp, k0 = (gid % ngrp) * 64;
        const int kg = k0 + lane;
        // (dense masks: the row labels for batch rows whose mask is a chain
        // partition, which run the chain-id kernels; 0 for the others)
        const int cid = kg >= L ? 0
                        : !DENSE ? p.chain_id[(int64_t)b * L + kg]
                        : (a.gate && a.gate[b]) ? a.label[(int64_t)b * L + kg] : 0;
        const bool pad = kg >= L || (p.key_pad && p.key_pad[(int64_t)b * L + kg]);
        const int ke = pad ? kPadChain : cid;
        keff[(int64_t)b * Lp + kg] = ke;
        qcid[(int64_t)b * Lp + kg] = cid;
        const int hh = lane >> 5;
        {
            const int mn = half_min_i(pad ? INT32_MAX : cid);
            const int mx = half_max_i(pad ? INT32_MIN : cid);
            const uint64_t padm = __ballot(pad);
            if ((lane & 31) == 0) {
                int* o = ksum + ((int64_t)b * (Lp / 32) + (k0 >> 5) + hh) * 4;
                o[0] = mn;
                o[1] = mx;
                o[2] = __popcll(hh ? (padm >> 32) : (padm & 0xffffffffull));
                o[3] = 0;
            }
        }
        {
            const bool qv = kg < L;
            const int mn = half_min_i(qv ? cid : INT32_MAX);
            const int mx = half_max_i(qv ? cid : INT32_MIN);
            const uint64_t inval = __ballot(!qv);
            if ((lane & 31) == 0) {
                int* o = qsum + ((int64_t)b * (Lp / 32) + (k0 >> 5) + hh) * 4;
                o[0] = mn;
                o[1] = mx;
                o[2] = __popcll(hh ? (inval >> 32) : (inval & 0xffffffffull));
                o[3] = 0;
            }
        }
        return;
    }
    if (bid < nchain + nrow) {
        // Delta and LSE2 per (b, h, row < Lp): kPrepLanes<D> lanes per row,
        // each with 8 dims, so a wave's loads cover whole rows.
        constexpr int NPL = kPrepLanes<D>;
        const int64_t item = (int64_t)(bid - nchain) * 256 + tid;
        const int64_t row = item / NPL;
        const int c = (int)(item % NPL);
        if (row >= (int64_t)p.B * p.H * Lp) return;  // (whole row groups)
        const int t = (int)(row % Lp);
        const int bh = (int)(row / Lp);
        const int b = bh / p.H, h = bh % p.H;
        float dl = 0.f;
        if (t < L && c * 8 < D) {
            const T* orow = (const T*)p.out.ptr + b * p.out.stride_b + h * p.out.stride_h +
                            (int64_t)t * p.out.stride_t;
            const T* grow = (const T*)p.grad_out.ptr + b * p.grad_out.stride_b +
                            h * p.grad_out.stride_h + (int64_t)t * p.grad_out.stride_t;
            float x[8], y[8];
            load8f<T>(orow, c * 8, x);
            load8f<T>(grow, c * 8, y);
#pragma unroll
            for (int u = 0; u < 8; ++u) dl += x[u] * y[u];
        }
#pragma unroll
        for (int o = NPL / 2; o >= 1; o >>= 1) dl += __shfl_xor(dl, o);
        if (c == 0) {
            float l2 = INFINITY;
            if (t < L) {
                const float lse = p.lse[((int64_t)b * p.H + h) * L + t];
                // A row whose keys are all padded has LSE = -inf and no probabilities.
                l2 = lse == -INFINITY ? INFINITY : lse * a.lmul;
            }
            // stored negated: the key-stationary kernel starts its S and dP
            // accumulators from them (P = exp2(S' ), dS = P dP')
            lse2[row] = -l2;
            delta[row] = -dl;
        }
        return;
    }
    if constexpr (ROPE) {
        // The forward's MFMA operands (mpattn_fwd.hip, fused RoPE): Q_self
        // rotated and times the logit factor, K_self rotated, Q_multi times
        // the logit factor, each rounded once from the same fp32 values
        // (rope_rot). Items: Q_self, K_self, Q_multi in thirds;
        // kRotItems<D> threads per row, each with an 8-dim chunk and its
        // RoPE partner chunk (D = 24: one thread per row).
        constexpr int H2 = D / 2, NPC = kRotItems<D>;
        const int64_t rows = (int64_t)p.B * p.H * Lp;
        int64_t item = (int64_t)(bid - nchain - nrow) * 256 + tid;
        if (item >= 3 * rows * NPC) return;
        const int which = (int)(item / (rows * NPC));  // 0 Q_self, 1 K_self, 2 Q_multi
        item -= (int64_t)which * rows * NPC;
        const int64_t row = item / NPC;
        const int pc = (int)(item % NPC);
        const int t = (int)(row % Lp);
        const int bh = (int)(row / Lp);
        const int b = bh / p.H, h = bh % p.H;
        const mpattn_tensor& src_t = which == 0 ? p.q_self : which == 1 ? p.k_self : p.q_multi;
        const T* src = (const T*)src_t.ptr + b * src_t.stride_b + h * src_t.stride_h + (int64_t)t * src_t.stride_t;
        T* dst = (which == 0 ? qrot : which == 1 ? krot : qmf) + row * D;
        const float mul = which == 1 ? 1.0f : a.qmul;
        if constexpr (H2 % 8 == 0) {
            const int d0 = pc * 8;
            float lo[8], hi[8];
            if (t < L) {
                float x[8], y[8];
                load8f<T>(src, d0, x);
                load8f<T>(src, d0 + H2, y);
                if (which == 2) {
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        lo[u] = x[u] * mul;
                        hi[u] = y[u] * mul;
                    }
                } else {
                    const float* cr = p.rope_cos + (int64_t)t * H2 + d0;
                    const float* sr = p.rope_sin + (int64_t)t * H2 + d0;
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        lo[u] = rope_rot(x[u], y[u], cr[u], sr[u], true) * mul;
                        hi[u] = rope_rot(y[u], x[u], cr[u], sr[u], false) * mul;
                    }
                }
            } else {
#pragma unroll
                for (int u = 0; u < 8; ++u) lo[u] = hi[u] = 0.f;
            }
            *reinterpret_cast<v8*>(dst + d0) = pack8<T>(lo);
            *reinterpret_cast<v8*>(dst + d0 + H2) = pack8<T>(hi);
        } else {
#pragma unroll
            for (int d0 = 0; d0 < D; d0 += 8) {
                float x[8];
                if (t < L) load8_rot<T, D>(src, p.rope_cos, p.rope_sin, t, d0, mul, which != 2, x);
                else
                    for (int u = 0; u < 8; ++u) x[u] = 0.f;
                *reinterpret_cast<v8*>(dst + d0) = pack8<T>(x);
            }
        }
    }
}

// Logit gradient from the recomputed weight w (P, or sqrt(P) for
// sqrt-softmax), dw = dO . V_sel and delta = dO . O:
//   softmax:       dS = P (dP - delta)
//   sqrt-softmax:  dS = W dW / 2 - P delta / 2 = W (dW - W delta) / 2
template <bool SQRT>
__device__ __forceinline__ float dscore_t(float w, float dw, float ndelta) {
    if constexpr (SQRT) return 0.5f * w * fmaf(w, ndelta, dw);
    return w * (dw + ndelta);
}

// Shapes shared by the two gradient kernels.
template <int D> struct BwdShape {
    static constexpr int DP = D <= 16 ? 16 : (D <= 32 ? 32 : 64);  // MFMA K over head dims
    static constexpr int NKK = DP / 16;
    static constexpr int NDB = DP <= 32 ? 1 : 2;  // 32-column blocks of head dims
};

// Stage the wave's 32 x D fp32 result tile `acc` (layout: lane l holds column
// db*32 + l%32 of rows 8*(i/4) + 4*hh + i%4, or the transposed layout when
// TRANS) through LDS scratch and write rows r0 .. r0+31 of `dst` (rows >= L
// skipped), optionally rotated back by RoPE (R_p^T, p = row index) and scaled.
template <typename T, int D, bool TRANS>
__device__ void store_rows(const f32x16* acc, float* scratch, const mpattn_tensor& dst, int b, int h,
                           int r0, int L, float mul, bool rope, const float* cos_tab,
                           const float* sin_tab, uint32_t rowmask = 0xffffffffu) {
    using BS = BwdShape<D>;
    typedef typename Elt<T>::v8 v8;
    const int lane = threadIdx.x & 63, hh = lane >> 5, ql = lane & 31;
    constexpr int LD = BS::NDB * 32 + 1;  // padded row stride (floats)
#pragma unroll
    for (int db = 0; db < BS::NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = 8 * (i / 4) + 4 * hh + (i % 4);
            // TRANS: accumulator rows are head dims, columns rows of dst.
            const int row = TRANS ? ql : m;
            const int col = TRANS ? db * 32 + m : db * 32 + ql;
            scratch[row * LD + col] = acc[db][i] * mul;
        }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    // lane -> (row, 8-wide chunk) items
    constexpr int NCHK = D / 8;
    for (int it = lane; it < 32 * NCHK; it += 64) {
        const int row = it / NCHK, d0 = (it % NCHK) * 8;
        const int r = r0 + row;
        if (r >= L) continue;
        float x[8];
        const bool live = (rowmask >> row) & 1u;
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = live ? scratch[row * LD + d0 + u] : 0.f;
        if (rope && live) {
            constexpr int H2 = D / 2;
            const float* cr = cos_tab + (int64_t)r * H2;
            const float* sr = sin_tab + (int64_t)r * H2;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int d = d0 + u;
                const bool lo = d < H2;
                const int dp = lo ? d + H2 : d - H2;
                const int fi = lo ? d : dp;
                const float y = scratch[row * LD + dp];
                // transpose of x*cos + rotate_half(x)*sin
                x[u] = x[u] * cr[fi] + (lo ? y : -y) * sr[fi];
            }
        }
        T* out = (T*)dst.ptr + b * dst.stride_b + h * dst.stride_h + (int64_t)r * dst.stride_t;
        *reinterpret_cast<v8*>(out + d0) = pack8<T>(x);
    }
    __builtin_amdgcn_wave_barrier();
}

// ---------------------------------------------------------------------------
// dK / dV: key-stationary.
// ---------------------------------------------------------------------------
// Stage layout of the dK/dV kernel (one pathway per workgroup): Q of the
// pathway and dO tiles, the aux rows, and (dense mask) the mask tile.
template <int D, int W, bool DENSE> struct DkdvStage {
    using TS = TileShape<D>;
    static constexpr int NTEN = 2;  // Q of the workgroup's pathway, dO
    static constexpr int AUX = 4 * kBS * 4;  // lse2, delta, qcid (+ spare) floats/ints
    // Dense mask: the stage's tile of mask bytes, kBS query rows x the
    // workgroup's 32 W keys, copied with the stage (when a.mdma).
    static constexpr int MROW = 32 * W;
    static constexpr int MSK = DENSE ? kBS * MROW : 0;
    static constexpr int STAGE = NTEN * TS::TILE + AUX + MSK;
    // Copies run NBUF-1 stages ahead (three buffers where they fit in 64 KB).
    static constexpr int NBUF = 3 * STAGE <= 65536 ? 3 : 2;
    static constexpr int SMEM = NBUF * STAGE > W * 32 * 65 * 4 ? NBUF * STAGE : W * 32 * 65 * 4;
};

// The gradients of pathway PW for the 32 W keys of key block kblk of (b, h):
// a (query, key) pair contributes to exactly one pathway, so the workgroup
// needs that pathway's K / V operands and accumulators only, and its stage
// tiles hold Q of that pathway and dO.
template <typename T, int D, int W, bool ROPE, bool DENSE, bool SQRT, bool DROP, int PW>
__device__ __forceinline__ void dkdv_body(const BwdArgs& a, char* smem, uint64_t* wmask, int kblk, int bh) {
    using TS = TileShape<D>;
    using BS = BwdShape<D>;
    using E = Elt<T>;
    using SL = DkdvStage<D, W, DENSE>;
    typedef typename E::v8 v8;
    typedef short s4 __attribute__((ext_vector_type(4)));
    constexpr int NTEN = SL::NTEN;
    constexpr int TOT = NTEN * TS::NI;
    constexpr int NJ = (TOT + W - 1) / W;  // copies per wave (the last may be idle)
    constexpr int AUX = SL::AUX;
    constexpr int MROW = SL::MROW;
    constexpr int MSK = SL::MSK;
    constexpr int STAGE = SL::STAGE;
    constexpr int NBUF = SL::NBUF;
    static_assert(!DENSE || (kBS * MROW) % (1024 * W) == 0, "mask tile copies split evenly over the waves");
    const mpattn_bwd_params& p = a.p;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ql = lane & 31, hh = lane >> 5;
    const int L = p.L, H = p.H, Lp = a.Lp;
    const int b = bh / H, h = bh % H;
    const int kw0 = kblk * 32 * W + wave * 32;  // first key of this wave
    const int key = kw0 + ql;                   // this lane's key (B operand column)

    auto base = [&](const mpattn_tensor& t) { return (const T*)t.ptr + b * t.stride_b + h * t.stride_h; };
    // Q and K of the pathway (with fused RoPE: the prep kernel's folded,
    // rotated operands), V of the pathway, dO
    const T* const q_p = PW == 0 ? (ROPE ? (const T*)a.qrot + (int64_t)bh * Lp * D : base(p.q_self))
                                 : (ROPE ? (const T*)a.qmf + (int64_t)bh * Lp * D : base(p.q_multi));
    const int64_t q_t = ROPE ? D : (PW == 0 ? p.q_self.stride_t : p.q_multi.stride_t);
    const T* const do_p = base(p.grad_out);
    const T* const k_p = PW == 0 ? (ROPE ? (const T*)a.krot + (int64_t)bh * Lp * D : base(p.k_self))
                                 : base(p.k_multi);
    const int64_t k_t = PW == 0 ? (ROPE ? D : p.k_self.stride_t) : p.k_multi.stride_t;
    const T* const v_p = base(PW == 0 ? p.v_self : p.v_multi);
    const int64_t v_t = PW == 0 ? p.v_self.stride_t : p.v_multi.stride_t;
    const float* const lse2_bh = a.lse2 + (int64_t)bh * Lp;
    const float* const delta_bh = a.delta + (int64_t)bh * Lp;
    const int* const qcid_b = a.qcid + (int64_t)b * Lp;
    const int4* const qsum_b = reinterpret_cast<const int4*>(a.qsum) + (int64_t)b * (Lp / 32);

    // ---- key-side registers: B operands K[key][dims kk*16 + 8*hh + (0..7)] ----
    v8 kf[BS::NKK], vf[BS::NKK];
    const bool kin = key < L;
    // Dense mask tile: the workgroup's first key, and this lane's byte
    // offset in a tile row. The last 16-key chunk that holds keys < L is
    // copied from L - 16 (never past a row), so its bytes sit shifted.
    const int mkb0 = kblk * MROW;
    int mkoff = key - mkb0;
    {
        const int rem = L - mkb0;
        if (rem < MROW && rem % 16 != 0 && mkoff / 16 == rem / 16) mkoff += 16 - rem % 16;
        if (!kin) mkoff = 0;
    }
    const uint8_t* const mask_b = DENSE ? p.chain_mask + (int64_t)b * p.mask_stride_b : nullptr;
#pragma unroll
    for (int kk = 0; kk < BS::NKK; ++kk) {
        const int d0 = kk * 16 + hh * 8;
        float x[8];
        if (kin && d0 < D) load8f<T>(k_p + (int64_t)key * k_t, d0, x);
        else for (int u = 0; u < 8; ++u) x[u] = 0.f;
        kf[kk] = pack8<T>(x);
        if (kin && d0 < D) load8f<T>(v_p + (int64_t)key * v_t, d0, x);
        else for (int u = 0; u < 8; ++u) x[u] = 0.f;
        vf[kk] = pack8<T>(x);
    }
    const int ckey = kin ? a.keff[(int64_t)b * Lp + key] : kPadChain;  // kPadChain if padded
    const bool kvalid = ckey != kPadChain;
    const int kc_min = __builtin_amdgcn_readfirstlane(wave_min_i(kvalid ? ckey : INT32_MAX));
    const int kc_max = __builtin_amdgcn_readfirstlane(wave_max_i(kvalid ? ckey : INT32_MIN));
    // Keys on several chains: no query stage is skipped and every pass is
    // masked, and the workgroup's stage barriers wait for this wavefront,
    // so it issues ahead of the wavefronts it shares a SIMD with.
    if (kc_min < kc_max) __builtin_amdgcn_s_setprio(3);
    // Padded keys are not masked in the loop: a lane's probabilities enter only
    // its own key's rows of dV and dK, which the epilogue writes as zeros.
    const uint32_t key_live = (uint32_t)__builtin_amdgcn_ballot_w64(kvalid);
    const bool any_live = key_live != 0;

    // ---- accumulators of the workgroup's pathway ----
    f32x16 dv[BS::NDB], dk[BS::NDB];
#pragma unroll
    for (int db = 0; db < BS::NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) dv[db][i] = dk[db][i] = 0.f;
    // ---- DMA plan (as the forward) ----
    const char* dsb[NJ];
    unsigned dstr[NJ], dlds[NJ], dloff[NJ];
    auto dma_slot = [&](int j, int& r, int& cb) {
        const int slot = ((wave + j * W) % TS::NI) * 64 + lane;
        r = slot / TS::NCH;
        cb = TS::swz(r, slot % TS::NCH) * 16;
    };
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int ins = min(wave + j * W, TOT - 1);
        const int ten = ins / TS::NI, part = ins % TS::NI;
        int r, cb;
        dma_slot(j, r, cb);
        const T* tb = ten == 0 ? q_p : do_p;
        const int64_t ts = ten == 0 ? q_t : p.grad_out.stride_t;
        dsb[j] = (const char*)tb;
        dstr[j] = (unsigned)(ts * (int64_t)sizeof(T));
        dlds[j] = ten * TS::TILE + part * 1024;
        dloff[j] = r * dstr[j] + cb;
    }
    const unsigned smem_base = lds_addr(smem);
    // aux copy of this wave: 0 lse2, 1 delta, 2 qcid, 3 (spare: qcid again)
    const int aux = wave & 3;
    const char* aux_src = aux == 0 ? (const char*)lse2_bh : aux == 1 ? (const char*)delta_bh : (const char*)qcid_b;
    auto issue = [&](int s, int bf) {
        const int q0 = s * kBS;
        const unsigned lb = smem_base + bf * STAGE;
        unsigned voff[NJ];
        if (q0 + kBS <= L) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) voff[j] = (unsigned)q0 * dstr[j] + dloff[j];
        } else {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                int r, cb;
                dma_slot(j, r, cb);
                voff[j] = (unsigned)min(q0 + r, L - 1) * dstr[j] + cb;
            }
        }
        const int m0v = m0_save();
#pragma unroll
        for (int j = 0; j < NJ; ++j)
            if (TOT % W == 0 || wave + j * W < TOT) dma16(dsb[j], voff[j], lb + dlds[j]);
        dma4(aux_src, (unsigned)(q0 + lane) * 4u, lb + NTEN * TS::TILE + aux * kBS * 4);
        if constexpr (DENSE) {
            if (a.mdma) {
                // Copy m: tile rows 8m .. 8m+7, 16-byte chunk lane % 8 of each
                // (rows past L read row L-1; chunks past L read from L - 16).
#pragma unroll
                for (int m = wave; m < MSK / 1024; m += W) {
                    const int row = min(q0 + m * 8 + (lane >> 3), L - 1);
                    const int cst = min(mkb0 + (lane & 7) * 16, L - 16);
                    dma16(mask_b, (unsigned)((int64_t)row * p.mask_stride_q + cst),
                          lb + NTEN * TS::TILE + AUX + m * 1024);
                }
            }
        }
        m0_restore(m0v);
    };

    // ---- operand readers ----
    const int qrow = swapped_row(ql);
    int roff[BS::NKK];
#pragma unroll
    for (int kk = 0; kk < BS::NKK; ++kk) {
        const int cch = 2 * kk + hh;
        roff[kk] = cch < TS::NCH ? qrow * TS::RB + TS::swz(qrow, cch) * 16 : 0;
    }
    const int tg = lane >> 4, ti = lane & 15;
    int toff[BS::NDB][2];
#pragma unroll
    for (int db = 0; db < BS::NDB; ++db) {
        int e = 8 * db + 4 * (tg & 1) + (ti & 3);
        if (8 * e >= TS::RB) e = ti & 3;
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
            const int row = 8 * (tg >> 1) + 4 * rr + (ti >> 2);
            toff[db][rr] = row * TS::RB + TS::swz(row, e >> 1) * 16 + (e & 1) * 8;
        }
    }
    v8 zero8;
#pragma unroll
    for (int t = 0; t < 8; ++t) zero8[t] = (T)0.f;
    // A operand: rows (queries) of tile `ten`, bit-swapped order.
    auto rop = [&](const char* stage, int ten, int st, int kk) -> v8 {
        if (2 * kk + hh >= TS::NCH) return zero8;
        return *reinterpret_cast<const v8*>(stage + ten * TS::TILE + st * 32 * TS::RB + roff[kk]);
    };
    // B operand: tile^T, lane -> column d = db*32 + l%32, 8 rows 16*cc + 8*hh + j.
    auto top = [&](const char* stage, int ten, int st, int cc, int db) -> v8 {
        s4 half[2];
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
            const char* ptr = stage + ten * TS::TILE + (st * 32 + 16 * cc) * TS::RB + toff[db][rr];
            half[rr] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)(ptr));
        }
        const v8 r8 = __builtin_bit_cast(v8, __builtin_shufflevector(half[0], half[1], 0, 1, 2, 3, 4, 5, 6, 7));
        if constexpr (D % 32 == 0) return r8;
        return db * 32 + (lane & 31) < D ? r8 : zero8;
    };
    // per-slot query data (slot i -> query st*32 + 16*(i/8) + 8*hh + i%8)
    auto aux16 = [&](const char* stage, int which, int st, float* out) {
        const float* base_f = (const float*)(stage + NTEN * TS::TILE + which * kBS * 4);
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const int ql0 = st * 32 + 16 * cc + 8 * hh;
            const f32x4 x0 = *reinterpret_cast<const f32x4*>(base_f + ql0);
            const f32x4 x1 = *reinterpret_cast<const f32x4*>(base_f + ql0 + 4);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                out[8 * cc + t] = x0[t];
                out[8 * cc + 4 + t] = x1[t];
            }
        }
    };

    const float c = a.c;
    auto dscore = [](float w, float dw, float ndelta) { return dscore_t<SQRT>(w, dw, ndelta); };
    auto mma_kloop = [&](const v8* aop, const v8* bop) {
        f32x16 acc;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.f;
#pragma unroll
        for (int kk = 0; kk < BS::NKK; ++kk) acc = E::mma(aop[kk], bop[kk], acc);
        return acc;
    };
    // The same product accumulated onto acc0.
    auto mma_kloop_c = [&](const v8* aop, const v8* bop, f32x16 acc) {
#pragma unroll
        for (int kk = 0; kk < BS::NKK; ++kk) acc = E::mma(aop[kk], bop[kk], acc);
        return acc;
    };
    // With fused RoPE the logit factor is folded into Q (c = 1), so without
    // sqrt-softmax and dropout the accumulators of S and dP start from the
    // slots' -LSE2 and -Delta: P = exp2(S') and dS = P * dP' need no VALU
    // work besides the exp2 and one multiply.
    constexpr bool FOLDC = ROPE && !SQRT && !DROP;

    // One pass over a subtile of 32 queries. masked: only the pairs on PW
    // count (a subtile with queries or keys on several chains); the others
    // get an infinite LSE, so their probabilities are 0.
    auto pass = [&](bool masked, const char* stage, int st, int q0) {
        float l2[16], dl[16];  // -LSE2 and -Delta of the slots' queries
        aux16(stage, 0, st, l2);
        aux16(stage, 1, st, dl);
        if (masked) {
            int qc[16];
            {
                float tmp[16];
                aux16(stage, 2, st, tmp);
#pragma unroll
                for (int i = 0; i < 16; ++i) qc[i] = __builtin_bit_cast(int, tmp[i]);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                bool same;
                if constexpr (DENSE) {
                    const int ql_ = st * 32 + 16 * (i / 8) + 8 * hh + (i % 8);
                    const int qg = q0 + ql_;
                    bool mb;
                    if (a.mdma) {
                        mb = *(reinterpret_cast<const uint8_t*>(stage + NTEN * TS::TILE + AUX) + ql_ * MROW + mkoff) != 0;
                    } else {
                        mb = p.chain_mask[(int64_t)b * p.mask_stride_b + (int64_t)qg * p.mask_stride_q +
                                          (int64_t)key * p.mask_stride_k] != 0;
                    }
                    same = !(qg < L && kin && mb);
                } else {
                    same = qc[i] == ckey;
                }
                if (same != (PW == 0)) l2[i] = -INFINITY;
            }
        }
        v8 qa[BS::NKK], doa[BS::NKK], ka[BS::NKK], va[BS::NKK];
#pragma unroll
        for (int kk = 0; kk < BS::NKK; ++kk) {
            doa[kk] = rop(stage, 1, st, kk);
            qa[kk] = rop(stage, 0, st, kk);
            ka[kk] = kf[kk];
            va[kk] = vf[kk];
        }
        float pv[16], dsv[16];
        if constexpr (FOLDC) {
            f32x16 a0, a1;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                a0[i] = l2[i];
                a1[i] = dl[i];
            }
            const f32x16 sv = mma_kloop_c(qa, ka, a0);   // S - LSE2
            const f32x16 dp = mma_kloop_c(doa, va, a1);  // dP - Delta
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                pv[i] = fast_exp2(sv[i]);
                dsv[i] = pv[i] * dp[i];
            }
        } else {
        const f32x16 sv = mma_kloop(qa, ka);
        const f32x16 dp = mma_kloop(doa, va);
        // Dropout: dP of dropped entries is 0, kept ones scaled by 1/(1-p);
        // the dV operand is Z*P (the 1/(1-p) goes into the dV store).
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float pm = fast_exp2(fmaf(sv[i], c, l2[i]));
            float dpi = dp[i];
            bool keep = true;
            if constexpr (DROP) {
                const int qg = q0 + st * 32 + 16 * (i / 8) + 8 * hh + (i % 8);
                keep = drop_keep(drop_row(a.drop.lo, (uint32_t)bh, (uint32_t)qg), a.drop.hi, (uint32_t)key,
                                 a.drop.thr);
                dpi = keep ? dpi * a.drop.rkeep : 0.f;
            }
            dsv[i] = dscore(pm, dpi, dl[i]);
            pv[i] = keep ? pm : 0.f;
        }
        }
        // dV += P^T dO ; dK += dS^T Q, per 16-query chunk cc
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const v8 p8 = pack8<T>(pv + 8 * cc), ds8 = pack8<T>(dsv + 8 * cc);
#pragma unroll
            for (int db = 0; db < BS::NDB; ++db) {
                dv[db] = E::mma(p8, top(stage, 1, st, cc, db), dv[db]);
                dk[db] = E::mma(ds8, top(stage, 0, st, cc, db), dk[db]);
            }
        }
    };

    // 0 / 1: every pair of the subtile on the self / multimer pathway; 2:
    // both; 3: nothing to do (no valid query or no valid key).
    auto qmode = [&](int qmin, int qmax, int ninval) {
        if (ninval == 32 || !any_live) return 3;
        if (!DENSE) {
            if (qmin == qmax && kc_min == kc_max && qmin == kc_min) return 0;
            if (qmax < kc_min || qmin > kc_max) return 1;
        }
        return 2;
    };

    // Every wave runs every stage, also one whose keys are all padded: the
    // stage copies are split over the waves and the barriers are block-wide.
    const int nst = (L + kBS - 1) / kBS;
    // Query summaries of a window of 64 subtiles (32 stages), one per lane,
    // read with readlane: a summary load inside the stage would wait for
    // the next stage's copies too. The window moves once per 32 stages.
    auto sum_window = [&](int first) {
        int4 v = {0, 0, 32, 0};
        if (first + lane < Lp / 32) v = qsum_b[first + lane];
        return v;
    };
    // vector-memory instructions one issue() puts in flight (uniform)
    int ncp = 1;
#pragma unroll
    for (int j = 0; j < NJ; ++j) ncp += (TOT % W == 0 || wave + j * W < TOT) ? 1 : 0;
    if constexpr (DENSE) {
        if (a.mdma)
            for (int m = wave; m < MSK / 1024; m += W) ++ncp;
    }
    // Stages with work for this workgroup's pathway (some wave has a subtile
    // whose pairs include pathway PW): up to 64 stages (lane = stage), the
    // other stages are neither copied nor waited for. Longer rows run every
    // stage.
    uint64_t smask = ~0ull;
    if (nst <= 64) {
        bool need = false;
        if (lane < nst) {
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const int sb = 2 * lane + st;
                int4 v = {0, 0, 32, 0};
                if (sb < Lp / 32) v = qsum_b[sb];
                const int md = qmode(v.x, v.y, v.z);
                need = need || md == 2 || md == PW;
            }
        }
        wmask[wave] = __builtin_amdgcn_ballot_w64(need);
        __syncthreads();
        smask = 0;
#pragma unroll
        for (int w = 0; w < W; ++w) smask |= wmask[w];
    }
    // first stage with work after stage `after` (nst if none)
    auto next_stage = [&](int after) -> int {
        const int s1 = after + 1;
        if (nst > 64) return s1;
        if (s1 >= nst) return nst;
        const uint64_t m = smask & (~0ull << s1);
        return m ? __builtin_ctzll(m) : nst;
    };
    int sub0 = 0;
    int4 qsw = sum_window(0);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // (compiler-visible) the window has landed
    int up[NBUF];  // the next NBUF stages with work (nst past the last)
    up[0] = next_stage(-1);
#pragma unroll
    for (int t = 1; t < NBUF; ++t) up[t] = up[t - 1] < nst ? next_stage(up[t - 1]) : nst;
#pragma unroll
    for (int t = 0; t < NBUF - 1; ++t)
        if (up[t] < nst) issue(up[t], t);
    int bf = 0;
    while (up[0] < nst) {
        const int s = up[0];
        // stage s's copies have landed (later stages' may stay in flight)
        if (NBUF == 3 && up[1] < nst) wait_vm_var(ncp);
        else wait_vm<0>();
        stage_barrier();
        if (2 * s - sub0 >= 64) {
            sub0 = 2 * s;
            qsw = sum_window(sub0);
            __builtin_amdgcn_s_waitcnt(0x0F70);  // (drains the copies in flight too; rare)
        }
        if (up[NBUF - 1] < nst) issue(up[NBUF - 1], bf == 0 ? NBUF - 1 : bf - 1);
#pragma unroll
        for (int t = 0; t < NBUF - 1; ++t) up[t] = up[t + 1];
        up[NBUF - 1] = up[NBUF - 2] < nst ? next_stage(up[NBUF - 2]) : nst;
        const char* stage = smem + bf * STAGE;
        const int q0 = s * kBS;
        int md2[2];
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const int i = 2 * s + st - sub0;
            md2[st] = qmode(__builtin_amdgcn_readlane(qsw.x, i), __builtin_amdgcn_readlane(qsw.y, i),
                            __builtin_amdgcn_readlane(qsw.z, i));
        }
        // One pass per subtile with pairs on PW (masked when the subtile
        // mixes pathways).
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const int md = st ? md2[1] : md2[0];
            if (md == 2 || md == PW) pass(md == 2, stage, st, q0);
        }
        bf = bf + 1 == NBUF ? 0 : bf + 1;
    }
    wait_vm<0>();
    stage_barrier();  // stage buffers become epilogue scratch

    float* scratch = (float*)(smem + wave * 32 * 65 * 4);
    const float vmul = DROP ? a.drop.rkeep : 1.0f;
    store_rows<T, D, false>(dv, scratch, PW == 0 ? p.dv_self : p.dv_multi, b, h, kw0, L, vmul, false, nullptr,
                            nullptr, key_live);
    store_rows<T, D, false>(dk, scratch, PW == 0 ? p.dk_self : p.dk_multi, b, h, kw0, L, a.kmul, ROPE && PW == 0,
                            p.rope_cos, p.rope_sin, key_live);
}

// ---------------------------------------------------------------------------
// dQ: query-stationary.
// ---------------------------------------------------------------------------
// Stage layout of the dQ kernel (one pathway per workgroup): K and V tiles
// of the pathway.
template <int D, int W> struct DqStage {
    static constexpr int NTEN = 2;  // K, V of the workgroup's pathway
    static constexpr int STAGE = NTEN * TileShape<D>::TILE;
    static constexpr int NBUF = 2;
    static constexpr int SMEM = NBUF * STAGE > W * 32 * 65 * 4 ? NBUF * STAGE : W * 32 * 65 * 4;
};

// dQ of pathway PW for the 32 W queries of query block qblk of (b, h).
template <typename T, int D, int W, bool ROPE, bool DENSE, bool SQRT, bool DROP, int PW>
__device__ __forceinline__ void dq_body(const BwdArgs& a, char* smem, int (*scid)[DqStage<D, W>::NBUF][kBS],
                                        uint64_t* wmask, int qblk, int bh) {
    using TS = TileShape<D>;
    using BS = BwdShape<D>;
    using E = Elt<T>;
    using SL = DqStage<D, W>;
    typedef typename E::v8 v8;
    typedef short s4 __attribute__((ext_vector_type(4)));
    constexpr int NTEN = SL::NTEN;
    constexpr int TOT = NTEN * TS::NI;
    constexpr int NJ = (TOT + W - 1) / W;  // copies per wave (the last may be idle)
    constexpr int STAGE = SL::STAGE;
    const mpattn_bwd_params& p = a.p;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ql = lane & 31, hh = lane >> 5;
    const int L = p.L, H = p.H, Lp = a.Lp;
    const int b = bh / H, h = bh % H;
    const int qw0 = qblk * 32 * W + wave * 32;
    const int q = qw0 + ql;
    const bool qin = q < L;

    auto base = [&](const mpattn_tensor& t) { return (const T*)t.ptr + b * t.stride_b + h * t.stride_h; };
    const T* const q_p = PW == 0 ? (ROPE ? (const T*)a.qrot + (int64_t)bh * Lp * D : base(p.q_self))
                                 : (ROPE ? (const T*)a.qmf + (int64_t)bh * Lp * D : base(p.q_multi));
    const int64_t q_t = ROPE ? D : (PW == 0 ? p.q_self.stride_t : p.q_multi.stride_t);
    const T* const do_p = base(p.grad_out);
    const T* const k_p = PW == 0 ? (ROPE ? (const T*)a.krot + (int64_t)bh * Lp * D : base(p.k_self))
                                 : base(p.k_multi);
    const int64_t k_t = PW == 0 ? (ROPE ? D : p.k_self.stride_t) : p.k_multi.stride_t;
    const T* const v_p = base(PW == 0 ? p.v_self : p.v_multi);
    const int64_t v_t = PW == 0 ? p.v_self.stride_t : p.v_multi.stride_t;
    const int* const keff_b = a.keff + (int64_t)b * Lp;
    const int4* const ksum_b = reinterpret_cast<const int4*>(a.ksum) + (int64_t)b * (Lp / 32);

    // ---- query-side registers (B operands) ----
    v8 qf[BS::NKK], dof[BS::NKK];
#pragma unroll
    for (int kk = 0; kk < BS::NKK; ++kk) {
        const int d0 = kk * 16 + hh * 8;
        float x[8];
        const bool ok = qin && d0 < D;
        if (ok) load8f<T>(q_p + (int64_t)q * q_t, d0, x);
        else for (int u = 0; u < 8; ++u) x[u] = 0.f;
        qf[kk] = pack8<T>(x);
        if (ok) load8f<T>(do_p + (int64_t)q * p.grad_out.stride_t, d0, x);
        else for (int u = 0; u < 8; ++u) x[u] = 0.f;
        dof[kk] = pack8<T>(x);
    }
    const float l2 = qin ? a.lse2[(int64_t)bh * Lp + q] : -INFINITY;  // -LSE2
    const uint32_t drow = DROP ? drop_row(a.drop.lo, (uint32_t)bh, (uint32_t)q) : 0u;
    // dP of dropped entries is 0, kept ones scaled by 1/(1-p); key of slot i
    // of subtile st: k0 + st*32 + 16*(i/8) + 8*hh + i%8.
    auto dpe = [&](float dp, int kg) {
        if constexpr (!DROP) return dp;
        return drop_keep(drow, a.drop.hi, (uint32_t)kg, a.drop.thr) ? dp * a.drop.rkeep : 0.f;
    };
    const float dl = qin ? a.delta[(int64_t)bh * Lp + q] : 0.f;  // -Delta
    int cq = 0, cq_min = 0, cq_max = 0;
    const uint8_t* mrow = nullptr;
    if constexpr (!DENSE) {
        cq = qin ? p.chain_id[(int64_t)b * L + q] : 0;
        cq_min = __builtin_amdgcn_readfirstlane(wave_min_i(qin ? cq : INT32_MAX));
        cq_max = __builtin_amdgcn_readfirstlane(wave_max_i(qin ? cq : INT32_MIN));
        // Queries on several chains: every subtile is masked and the stage
        // barriers wait for this wavefront (as in dK/dV).
        if (cq_min < cq_max) __builtin_amdgcn_s_setprio(3);
    } else {
        mrow = p.chain_mask + (int64_t)b * p.mask_stride_b + (int64_t)(qin ? q : 0) * p.mask_stride_q;
    }

    f32x16 dq[BS::NDB];
#pragma unroll
    for (int db = 0; db < BS::NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) dq[db][i] = 0.f;

    // ---- DMA plan ----
    const char* dsb[NJ];
    unsigned dstr[NJ], dlds[NJ], dloff[NJ];
    auto dma_slot = [&](int j, int& r, int& cb) {
        const int slot = ((wave + j * W) % TS::NI) * 64 + lane;
        r = slot / TS::NCH;
        cb = TS::swz(r, slot % TS::NCH) * 16;
    };
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int ins = min(wave + j * W, TOT - 1);
        const int ten = ins / TS::NI, part = ins % TS::NI;
        int r, cb;
        dma_slot(j, r, cb);
        const T* tb = ten == 0 ? k_p : v_p;
        const int64_t ts = ten == 0 ? k_t : v_t;
        dsb[j] = (const char*)tb;
        dstr[j] = (unsigned)(ts * (int64_t)sizeof(T));
        dlds[j] = ten * TS::TILE + part * 1024;
        dloff[j] = r * dstr[j] + cb;
    }
    const unsigned smem_base = lds_addr(smem);
    const unsigned scid_base = lds_addr(&scid[wave][0][0]);
    auto issue = [&](int s, int bf) {
        const int k0 = s * kBS;
        const unsigned lb = smem_base + bf * STAGE;
        unsigned voff[NJ];
        if (k0 + kBS <= L) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) voff[j] = (unsigned)k0 * dstr[j] + dloff[j];
        } else {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                int r, cb;
                dma_slot(j, r, cb);
                voff[j] = (unsigned)min(k0 + r, L - 1) * dstr[j] + cb;
            }
        }
        const int m0v = m0_save();
#pragma unroll
        for (int j = 0; j < NJ; ++j)
            if (TOT % W == 0 || wave + j * W < TOT) dma16(dsb[j], voff[j], lb + dlds[j]);
        dma4(keff_b, (unsigned)(k0 + lane) * 4u, scid_base + bf * kBS * 4);
        m0_restore(m0v);
    };

    // ---- operand readers ----
    const int krow = swapped_row(ql);
    int roff[BS::NKK];
#pragma unroll
    for (int kk = 0; kk < BS::NKK; ++kk) {
        const int cch = 2 * kk + hh;
        roff[kk] = cch < TS::NCH ? krow * TS::RB + TS::swz(krow, cch) * 16 : 0;
    }
    const int tg = lane >> 4, ti = lane & 15;
    int toff[BS::NDB][2];
#pragma unroll
    for (int db = 0; db < BS::NDB; ++db) {
        int e = 8 * db + 4 * (tg & 1) + (ti & 3);
        if (8 * e >= TS::RB) e = ti & 3;
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
            const int row = 8 * (tg >> 1) + 4 * rr + (ti >> 2);
            toff[db][rr] = row * TS::RB + TS::swz(row, e >> 1) * 16 + (e & 1) * 8;
        }
    }
    v8 zero8;
#pragma unroll
    for (int t = 0; t < 8; ++t) zero8[t] = (T)0.f;
    auto rop = [&](const char* stage, int ten, int st, int kk) -> v8 {
        if (2 * kk + hh >= TS::NCH) return zero8;
        return *reinterpret_cast<const v8*>(stage + ten * TS::TILE + st * 32 * TS::RB + roff[kk]);
    };
    auto top = [&](const char* stage, int ten, int st, int cc, int db) -> v8 {
        s4 half[2];
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
            const char* ptr = stage + ten * TS::TILE + (st * 32 + 16 * cc) * TS::RB + toff[db][rr];
            half[rr] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)(ptr));
        }
        const v8 r8 = __builtin_bit_cast(v8, __builtin_shufflevector(half[0], half[1], 0, 1, 2, 3, 4, 5, 6, 7));
        if constexpr (D % 32 == 0) return r8;
        return db * 32 + (lane & 31) < D ? r8 : zero8;
    };
    const float c = a.c;
    auto dscore = [](float w, float dw, float ndelta) { return dscore_t<SQRT>(w, dw, ndelta); };
    auto mma_kloop = [&](const v8* aop, const v8* bop) {
        f32x16 acc;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.f;
#pragma unroll
        for (int kk = 0; kk < BS::NKK; ++kk) acc = E::mma(aop[kk], bop[kk], acc);
        return acc;
    };
    // With fused RoPE (logit factor folded into Q, c = 1), no sqrt-softmax
    // and no dropout, the S accumulators start from the query's -LSE2
    // (loop-invariant, the lane's query): P = exp2(S').
    constexpr bool FOLDC = ROPE && !SQRT && !DROP;
    f32x16 nl2v;
#pragma unroll
    for (int i = 0; i < 16; ++i) nl2v[i] = l2;
    auto s_of = [&](const v8* aop, const v8* bop) {
        if constexpr (FOLDC) {
            f32x16 acc = nl2v;
#pragma unroll
            for (int kk = 0; kk < BS::NKK; ++kk) acc = E::mma(aop[kk], bop[kk], acc);
            return acc;
        }
        return mma_kloop(aop, bop);
    };
    // probability of slot value x of S (or S' when folded)
    auto prob = [&](float x) { return FOLDC ? fast_exp2(x) : fast_exp2(fmaf(x, c, l2)); };
    f32x16 ndlv;
#pragma unroll
    for (int i = 0; i < 16; ++i) ndlv[i] = dl;
    auto dp_of = [&](const v8* aop, const v8* bop) {
        if constexpr (FOLDC) {
            f32x16 acc = ndlv;
#pragma unroll
            for (int kk = 0; kk < BS::NKK; ++kk) acc = E::mma(aop[kk], bop[kk], acc);
            return acc;
        }
        return mma_kloop(aop, bop);
    };
    const float dlx = FOLDC ? 0.f : dl;  // -Delta left for dscore (0 when folded)

    // One 32-key subtile of pathway PW; masked: the subtile mixes pathways
    // (or holds padded keys), so only its pairs on PW count.
    uint64_t mcur[2][2], mnxt[2][2];  // dense mask words (see mload below)
    auto subtile = [&](const char* stage, const int* cid, int st, bool masked, int k0) {
        v8 ka[BS::NKK], va[BS::NKK];
#pragma unroll
        for (int kk = 0; kk < BS::NKK; ++kk) {
            ka[kk] = rop(stage, 0, st, kk);
            va[kk] = rop(stage, 1, st, kk);
        }
        const f32x16 sv = s_of(ka, qf);
        const f32x16 dp = dp_of(va, dof);
        // dS of every pair, then (masked) the pairs off the pathway set to 0
        // in place: a select, so an overflowed P off the pathway is dropped
        // whole, and both kinds of subtile feed one dQ product (the
        // accumulators keep their registers across the branch).
        float dsv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float pv = prob(sv[i]);
            dsv[i] = FOLDC ? pv * dp[i] : dscore(pv, dpe(dp[i], k0 + st * 32 + 16 * (i / 8) + 8 * hh + (i % 8)), dlx);
        }
        if (masked) {
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const int kl = st * 32 + 16 * cc + 8 * hh;
                const i32x4 c0 = *reinterpret_cast<const i32x4*>(&cid[kl]);
                const i32x4 c1 = *reinterpret_cast<const i32x4*>(&cid[kl + 4]);
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const int ck = t < 4 ? c0[t & 3] : c1[t & 3];
                    const int i = 8 * cc + t;
                    bool sm_;
                    if constexpr (DENSE) {
                        // mask word prefetched one stage ahead (key kl + t)
                        const uint64_t mw = st ? mcur[1][cc] : mcur[0][cc];
                        sm_ = ((mw >> (8 * t)) & 0xffu) == 0;
                    } else {
                        sm_ = ck == cq;
                    }
                    const bool on = ck != kPadChain && sm_ == (PW == 0);
                    dsv[i] = on ? dsv[i] : 0.f;
                }
            }
        }
        // dQ^T += K^T dS^T
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const v8 ds8 = pack8<T>(dsv + 8 * cc);
#pragma unroll
            for (int db = 0; db < BS::NDB; ++db) dq[db] = E::mma(top(stage, 0, st, cc, db), ds8, dq[db]);
        }
    };

    auto kmode = [&](int kmin, int kmax, int npad) {
        if (npad == 32) return 3;
        if (!DENSE && npad == 0) {
            if (kmin == kmax && cq_min == cq_max && kmin == cq_min) return 0;
            if (kmax < cq_min || kmin > cq_max) return 1;
        }
        return 2;
    };

    const int nst = (L + kBS - 1) / kBS;
    // Dense mask: each lane's mask bytes of a stage (8 keys per subtile half,
    // keys past L read as 0) are loaded one stage ahead, before the next copy
    // is issued, and land by the compiler-visible wait at the stage top.
    auto mload = [&](int s, uint64_t (*m)[2]) {
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const int kg = s * kBS + st * 32 + 16 * cc + 8 * hh;
                uint64_t w = 0;
                if (a.mvec && kg + 8 <= L) {
                    w = *reinterpret_cast<const uint64_t*>(mrow + kg);
                } else {
                    for (int t = 0; t < 8; ++t)
                        if (kg + t < L && mrow[(int64_t)(kg + t) * p.mask_stride_k] != 0) w |= 0xffull << (8 * t);
                }
                m[st][cc] = w;
            }
    };
    // Key stages with work for this workgroup's pathway (as in the dK/dV
    // kernel: up to 64 stages, lane = stage; all-padded key stages have none).
    uint64_t smask = ~0ull;
    if (nst <= 64) {
        bool need = false;
        if (lane < nst) {
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const int sb = 2 * lane + st;
                int4 v = {0, 0, 32, 0};
                if (sb < Lp / 32) v = ksum_b[sb];
                const int md = kmode(v.x, v.y, v.z);
                need = need || md == 2 || md == PW;
            }
        }
        wmask[wave] = __builtin_amdgcn_ballot_w64(need);
        __syncthreads();
        smask = 0;
#pragma unroll
        for (int w = 0; w < W; ++w) smask |= wmask[w];
    }
    auto next_stage = [&](int after) -> int {
        const int s1 = after + 1;
        if (nst > 64) return s1;
        if (s1 >= nst) return nst;
        const uint64_t m = smask & (~0ull << s1);
        return m ? __builtin_ctzll(m) : nst;
    };
    // Key summaries of a window of 64 subtiles (32 stages), one per lane,
    // read with readlane (as in the dK/dV kernel).
    auto sum_window = [&](int first) {
        int4 v = {0, 0, 32, 0};
        if (first + lane < Lp / 32) v = ksum_b[first + lane];
        return v;
    };
    int sub0 = 0;
    int4 ksw = sum_window(0);
    int cur = next_stage(-1);
    int nxt = cur < nst ? next_stage(cur) : nst;
    if constexpr (DENSE)
        if (cur < nst) mload(cur, mcur);
    if (cur < nst) issue(cur, 0);
    int bf = 0;
    while (cur < nst) {
        const int s = cur;
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), compiler-visible
        stage_barrier();
        if (2 * s - sub0 >= 64) {
            sub0 = 2 * s;
            ksw = sum_window(sub0);
            __builtin_amdgcn_s_waitcnt(0x0F70);  // before the next copy is issued
        }
        if constexpr (DENSE)
            if (nxt < nst) mload(nxt, mnxt);
        if (nxt < nst) issue(nxt, bf ^ 1);
        const char* stage = smem + bf * STAGE;
        const int* cid = &scid[wave][bf][0];
        const int k0 = s * kBS;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const int i = 2 * s + st - sub0;
            const int md = kmode(__builtin_amdgcn_readlane(ksw.x, i), __builtin_amdgcn_readlane(ksw.y, i),
                                 __builtin_amdgcn_readlane(ksw.z, i));
            if (md == PW || md == 2) subtile(stage, cid, st, md == 2, k0);
        }
        if constexpr (DENSE) {
#pragma unroll
            for (int st = 0; st < 2; ++st)
#pragma unroll
                for (int cc = 0; cc < 2; ++cc) mcur[st][cc] = mnxt[st][cc];
        }
        cur = nxt;
        nxt = cur < nst ? next_stage(cur) : nst;
        bf ^= 1;
    }
    wait_vm<0>();
    stage_barrier();

    float* scratch = (float*)(smem + wave * 32 * 65 * 4);
    store_rows<T, D, true>(dq, scratch, PW == 0 ? p.dq_self : p.dq_multi, b, h, qw0, L, p.scale, ROPE && PW == 0,
                           p.rope_cos, p.rope_sin);
}

// dK/dV and dQ in one grid (they read the same prep outputs and write
// disjoint gradients): workgroups [0, nkv) run dK/dV, one per (key block,
// pathway, b*H + h), the rest dQ, one per (query block, pathway, b*H + h);
// the two pathways of a block are neighbours in dispatch order (their
// tiles share the XCD's L2). dQ workgroups fill the last round of dK/dV's
// instead of waiting for a grid boundary. One LDS allocation serves
// whichever body the workgroup runs.
template <typename T, int D, int W, bool ROPE, bool DENSE, bool SQRT, bool DROP>
__global__ __launch_bounds__(W * 64) void bwd_kernel(const BwdArgs a, int nkv) {
    using SK = DkdvStage<D, W, DENSE>;
    using SQ = DqStage<D, W>;
    constexpr int SMEM = SK::SMEM > SQ::SMEM ? SK::SMEM : SQ::SMEM;
    __shared__ __attribute__((aligned(1024))) char smem[SMEM];
    __shared__ __attribute__((aligned(16))) int scid[W][SQ::NBUF][kBS];
    __shared__ uint64_t wmask[W];
    const int nb = (a.p.L + 32 * W - 1) / (32 * W);
    const int bid = blockIdx.x;
    const bool kv = bid < nkv;
    int blk, bh;
    if (kv)
        dispatch_order_at(bid, nkv, 2 * nb, a.p.H, nullptr, 0, 0, 1, false, (int64_t)3 * a.p.L * D * sizeof(T),
                          2 << 20, blk, bh);
    else
        dispatch_order_at(bid - nkv, (int)gridDim.x - nkv, 2 * nb, a.p.H, nullptr, 0, 0, 1, false,
                          (int64_t)2 * a.p.L * D * sizeof(T), 4 << 20, blk, bh);
    if (a.gate && ((a.gate_want == 0 && a.gate[a.p.B] == 0) ||  // (every row a partition)
                   (a.gate[bh / a.p.H] != 0) != (a.gate_want != 0)))
        return;  // (uniform)
    if (kv) {
        if (blk & 1) dkdv_body<T, D, W, ROPE, DENSE, SQRT, DROP, 1>(a, smem, wmask, blk >> 1, bh);
        else dkdv_body<T, D, W, ROPE, DENSE, SQRT, DROP, 0>(a, smem, wmask, blk >> 1, bh);
    } else {
        if (blk & 1) dq_body<T, D, W, ROPE, DENSE, SQRT, DROP, 1>(a, smem, scid, wmask, blk >> 1, bh);
        else dq_body<T, D, W, ROPE, DENSE, SQRT, DROP, 0>(a, smem, scid, wmask, blk >> 1, bh);
    }
}

// ---------------------------------------------------------------------------
template <typename T, int D, bool ROPE, bool DENSE, bool SQRT, bool DROP>
static hipError_t launch_bwd_t(const mpattn_bwd_params& p, hipStream_t stream) {
    constexpr int W = 4;
    BwdArgs a;
    a.p = p;
    const int Lp = rup(p.L, kBS);
    a.Lp = Lp;
    // With fused RoPE the forward folds the logit factor into Q (both
    // pathways); the backward recomputes the logits from the same folded,
    // rounded operands (prep kernel), so c = 1 and dK = (scale / f) dS^T Qf.
    // The fp32 forward takes sqrt-softmax as the square root of the full
    // softmax (logit factor not halved), and so does the fp32 backward.
    constexpr bool F32 = std::is_same<T, float>::value;
    const float f = p.scale * kLog2e * (SQRT && !F32 ? 0.5f : 1.0f);
    a.c = ROPE ? 1.0f : f;
    a.qmul = f;
    a.kmul = ROPE ? p.scale / f : p.scale;
    a.lmul = kLog2e * (SQRT && !F32 ? 0.5f : 1.0f);
    a.drop = drop_cfg(p.dropout_p, p.dropout_seed);
    a.mvec = p.chain_mask && p.mask_stride_k == 1 && (uintptr_t)p.chain_mask % 8 == 0 && p.mask_stride_b % 8 == 0 &&
             p.mask_stride_q % 8 == 0;
    a.mdma = p.chain_mask && p.mask_stride_k == 1 && (uintptr_t)p.chain_mask % 16 == 0 && p.mask_stride_b % 16 == 0 &&
             p.mask_stride_q % 16 == 0 && p.L >= 16 && (int64_t)p.L * p.mask_stride_q < ((int64_t)1 << 31);
    const BwdWs ws = bwd_ws_layout(p.B, p.H, p.L, D, sizeof(T), ROPE);
    char* w = (char*)p.workspace;
    float* lse2 = (float*)(w + ws.lse2);
    float* delta = (float*)(w + ws.delta);
    int* keff = (int*)(w + ws.keff);
    int* ksum = (int*)(w + ws.ksum);
    int* qcid = (int*)(w + ws.qcid);
    int* qsum = (int*)(w + ws.qsum);
    T* qrot = (T*)(w + ws.qrot);
    T* krot = (T*)(w + ws.krot);
    T* qmf = (T*)(w + ws.qmf);
    a.lse2 = lse2;
    a.delta = delta;
    a.keff = keff;
    a.ksum = ksum;
    a.qcid = qcid;
    a.qsum = qsum;
    a.qrot = qrot;
    a.krot = krot;
    a.qmf = qmf;
    a.label = nullptr;
    a.gate = nullptr;
    a.gate_want = 0;
    hipError_t e;
    if (DENSE && !F32) {
        // Row labels of the mask and the check that it is their "different
        // chain" relation: those batch rows run the chain-id kernels.
        int* label = (int*)(w + ws.label);
        int* valid = (int*)(w + ws.valid);
        if ((e = launch_mask_labels(p.chain_mask, p.mask_stride_b, p.mask_stride_q, p.mask_stride_k, p.B, p.L, label,
                                    valid, a.mvec, true, stream)) != hipSuccess)
            return e;
        a.label = label;
        a.gate = valid;
    }
    const int nchain = (p.B * (Lp / 64) + 3) / 4;
    const int nrow = (int)(((int64_t)p.B * p.H * Lp * kPrepLanes<D> + 255) / 256);
    const int nrot = ROPE ? (int)((3 * (int64_t)p.B * p.H * Lp * kRotItems<D> + 255) / 256) : 0;
    hipLaunchKernelGGL((bwd_prep_kernel<T, D, ROPE, DENSE>), dim3(nchain + nrow + nrot), dim3(256), 0, stream,
                       a, lse2, delta, keff, ksum, qcid, qsum, qrot, krot, qmf, nchain, nrow);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if constexpr (F32) {
        return launch_bwd32(a, stream);
    } else {
    const int nb = (p.L + 32 * W - 1) / (32 * W);
    const unsigned grid = (unsigned)((int64_t)p.B * p.H * nb);
    if (DENSE) {
        BwdArgs ac = a;
        ac.p.chain_id = a.label;
        ac.p.chain_mask = nullptr;
        ac.gate_want = 1;
        hipLaunchKernelGGL((bwd_kernel<T, D, W, ROPE, false, SQRT, DROP>), dim3(4 * grid), dim3(W * 64), 0, stream,
                           ac, (int)(2 * grid));
        if ((e = hipGetLastError()) != hipSuccess) return e;
        a.gate_want = 0;
    }
    hipLaunchKernelGGL((bwd_kernel<T, D, W, ROPE, DENSE, SQRT, DROP>), dim3(4 * grid), dim3(W * 64), 0, stream, a,
                       (int)(2 * grid));
    return hipGetLastError();
    }
}

template <typename T, int D>
static hipError_t dispatch_bwd_d(const mpattn_bwd_params& p, hipStream_t s) {
    const bool rope = p.rope == MPATTN_ROPE_FUSED;
    const bool dense = p.chain_mask != nullptr;
    // fp32: dropout is handled by the fp32 kernels' own dispatch.
    const bool drop = p.dropout_p > 0.f && !std::is_same<T, float>::value;
    if (p.sqrt_softmax) {
        if (drop) {
            if (rope) return dense ? launch_bwd_t<T, D, true, true, true, true>(p, s) : launch_bwd_t<T, D, true, false, true, true>(p, s);
            return dense ? launch_bwd_t<T, D, false, true, true, true>(p, s) : launch_bwd_t<T, D, false, false, true, true>(p, s);
        }
        if (rope) return dense ? launch_bwd_t<T, D, true, true, true, false>(p, s) : launch_bwd_t<T, D, true, false, true, false>(p, s);
        return dense ? launch_bwd_t<T, D, false, true, true, false>(p, s) : launch_bwd_t<T, D, false, false, true, false>(p, s);
    }
    if (drop) {
        if (rope) return dense ? launch_bwd_t<T, D, true, true, false, true>(p, s) : launch_bwd_t<T, D, true, false, false, true>(p, s);
        return dense ? launch_bwd_t<T, D, false, true, false, true>(p, s) : launch_bwd_t<T, D, false, false, false, true>(p, s);
    }
    if (rope) return dense ? launch_bwd_t<T, D, true, true, false, false>(p, s) : launch_bwd_t<T, D, true, false, false, false>(p, s);
    return dense ? launch_bwd_t<T, D, false, true, false, false>(p, s) : launch_bwd_t<T, D, false, false, false, false>(p, s);
}

template <typename T>
static hipError_t dispatch_bwd_t(const mpattn_bwd_params& p, hipStream_t s) {
    switch (p.D) {
        case 16: return dispatch_bwd_d<T, 16>(p, s);
        case 24: return dispatch_bwd_d<T, 24>(p, s);
        case 32: return dispatch_bwd_d<T, 32>(p, s);
        case 64: return dispatch_bwd_d<T, 64>(p, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_bwd(const mpattn_bwd_params& p, hipStream_t stream) {
    if (p.dtype == MPATTN_FP32) return dispatch_bwd_t<float>(p, stream);
    if (p.dtype == MPATTN_BF16) return dispatch_bwd_t<bf16_t>(p, stream);
    return dispatch_bwd_t<fp16_t>(p, stream);
}


}  // namespace mpattn
