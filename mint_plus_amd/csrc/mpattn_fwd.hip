// Forward multi-pathway attention for gfx950 (16-bit inputs, fp32 accumulate).
//
// Follows the math of the reference eager combine
// (mint_plus/models/modules_plus.py:155-201 with the fp32 softmax of
// mint_plus/models/mu_scaling/layer.py:159) and the flash-style contract of
// mint_plus/models/kernels/multi_pathway_attention.py:32-181, re-designed for
// CDNA4. Two launches:
//
// 1. fwd_prep_kernel (memory-bound, small): effective chain id per key (the
//    chain id, or kPadChain for padded keys and keys past L), a per-32-key
//    summary (min/max chain id over valid keys, number of padded keys) and,
//    with fused RoPE, K_self rotated once into the workspace.
//
// 2. fwd_kernel:
//  * A workgroup of W wavefronts (8 for D <= 32) owns 32*W consecutive queries
//    of one (b, h); each wavefront owns 32 of them. Q is loaded once, RoPE and
//    the logit scale applied in fp32.
//  * Keys stream through a ring of NBUF LDS stages of 64 keys. A stage has
//    room for K_self, K_multi, V_self, V_multi tiles, copied by
//    global_load_lds (16 bytes per lane, straight into LDS); only the tiles of
//    the pathways some wavefront of the workgroup needs are copied. Copies run
//    NBUF-1 stages ahead; one barrier per stage. Rows are stored densely with
//    their 16-byte chunks XOR-swizzled by row to spread LDS banks.
//  * Per 32-key subtile a wavefront computes S^T = K Q^T with
//    v_mfma_f32_32x32x16 (rows = keys, columns = queries): lane l holds 16
//    logits of query l%32, so the softmax statistics are in-lane. K rows are
//    read with bits 2 and 3 of the row index swapped, which makes accumulator
//    slot i of lane half hh the key 16*(i/8) + 8*hh + i%8: the probabilities
//    are then already the B operand of O^T += V^T P^T. The V^T operand comes
//    from the row-major V tile via ds_read_b64_tr_b16.
//  * Subtiles are classified from per-32-key and per-32-query chain summaries:
//    pure self / pure multimer (one pathway), straddle (keys on one chain,
//    queries on several: pathway chosen per lane), general (mixed or padded
//    keys: both logits, selected per element), skip (all keys padded). Stages
//    whose two subtiles share one pure pathway take the fast path.
//  * Softmax in base 2 without a running max: p = exp2(s2) relative to a
//    reference m_ref = 0. A stage whose row sum leaves (0, 2^64] takes a rare
//    fix-up path that recomputes it against the stage's max and moves m_ref
//    (the wavefront then subtracts m_ref with one FMA per logit).
//  * Row sums come from v_dot2_f32_bf16 on the rounded probabilities (the
//    values the PV MFMA consumes).
#include <type_traits>

#include "mpattn_common.h"

namespace mpattn {

constexpr int kBN = 64;  // keys per LDS stage

inline int round_up(int x, int m) { return (x + m - 1) / m * m; }

// Workspace layout (offsets 256-byte aligned):
//   keff int32 [B][Lp]          effective chain id per key
//   ksum int32 [B][Lp/32][4]    keys: min chain, max chain (valid keys), #padded, 0
//   qsum int32 [B][Lp/32][4]    queries: min chain, max chain (queries < L), 0, 0
//   krot T     [B][H][Lp][D]    RoPE-rotated K_self (fused RoPE only)
struct FwdWs {
    int64_t keff, ksum, qsum, krot, total;
};

inline FwdWs fwd_ws_layout(int B, int H, int L, int D, int esize, bool rope) {
    const int64_t Lp = round_up(L, kBN);
    auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
    FwdWs w;
    w.keff = 0;
    w.ksum = al(w.keff + (int64_t)B * Lp * 4);
    w.qsum = al(w.ksum + (int64_t)B * (Lp / 32) * 16);
    w.krot = al(w.qsum + (int64_t)B * (Lp / 32) * 16);
    w.total = al(w.krot + (rope ? (int64_t)B * H * Lp * D * esize : 0));
    return w;
}

int64_t fwd_workspace_bytes(int B, int H, int L, int D, int dtype, int rope) {
    const int es = dtype == MPATTN_FP32 ? 4 : 2;
    return fwd_ws_layout(B, H, L, D, es, rope == MPATTN_ROPE_FUSED).total;
}

struct FwdArgs {
    mpattn_fwd_params p;
    const int* keff;
    const int* ksum;
    const int* qsum;
    const void* krot;
    int Lp;
    float qmul;    // factor applied to q while loading (scale*log2e when fused, else 1)
    float c;       // base-2 factor applied to raw logits (1 when fused)
};

// ---------------------------------------------------------------------------
// Prep: chain staging (blocks [0, nchain)) and K_self rotation (the rest).
// ---------------------------------------------------------------------------
template <typename T, int D, bool ROPE, bool DENSE>
__global__ __launch_bounds__(256) void fwd_prep_kernel(const mpattn_fwd_params p, int* keff,
                                                       int* ksum, int* qsum, T* krot, int Lp, int nchain) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int L = p.L;
    if ((int)blockIdx.x < nchain) {
        const int ngrp = Lp / 64;
        const int gid = blockIdx.x * 4 + wave;
        if (gid >= p.B * ngrp) return;
        const int b = gid / ngrp, k0 = (gid % ngrp) * 64;
        const int kg = k0 + lane;
        const int chain = kg < L && !DENSE ? p.chain_id[(int64_t)b * L + kg] : 0;
        int cid = kPadChain;
        if (kg < L && !(p.key_pad && p.key_pad[(int64_t)b * L + kg])) cid = chain;
        keff[(int64_t)b * Lp + kg] = cid;
        const bool valid = cid != kPadChain;
        const int mn = half_min_i(valid ? cid : INT32_MAX);
        const int mx = half_max_i(valid ? cid : INT32_MIN);
        const uint64_t padm = __ballot(!valid);
        const int qmn = half_min_i(kg < L ? chain : INT32_MAX);
        const int qmx = half_max_i(kg < L ? chain : INT32_MIN);
        if ((lane & 31) == 0) {
            const int hh = lane >> 5;
            const int64_t blk = (int64_t)b * (Lp / 32) + (k0 >> 5) + hh;
            int* o = ksum + blk * 4;
            o[0] = mn;
            o[1] = mx;
            o[2] = __popcll(hh ? (padm >> 32) : (padm & 0xffffffffull));
            o[3] = 0;
            int* oq = qsum + blk * 4;
            oq[0] = qmn;
            oq[1] = qmx;
            oq[2] = 0;
            oq[3] = 0;
        }
        return;
    }
    if constexpr (ROPE) {
        typedef typename Elt<T>::v8 v8;
        constexpr int H2 = D / 2;
        constexpr int NPC = (H2 % 8 == 0) ? H2 / 8 : 1;  // work items per row
        const int64_t item = (int64_t)(blockIdx.x - nchain) * 256 + tid;
        const int64_t rows = (int64_t)p.B * p.H * Lp;
        if (item >= rows * NPC) return;
        const int64_t row = item / NPC;
        const int pc = (int)(item % NPC);
        const int t = (int)(row % Lp);
        const int bh = (int)(row / Lp);
        const int b = bh / p.H, h = bh % p.H;
        T* dst = krot + row * D;
        const T* src = (const T*)p.k_self.ptr + b * p.k_self.stride_b + h * p.k_self.stride_h +
                       (int64_t)t * p.k_self.stride_t;
        if constexpr (H2 % 8 == 0) {
            const int d0 = pc * 8;
            float lo[8], hi[8];
            if (t < L) {
                float x[8], y[8];
                load8f<T>(src, d0, x);
                load8f<T>(src, d0 + H2, y);
                const float* cr = p.rope_cos + (int64_t)t * H2 + d0;
                const float* sr = p.rope_sin + (int64_t)t * H2 + d0;
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    lo[u] = x[u] * cr[u] - y[u] * sr[u];
                    hi[u] = y[u] * cr[u] + x[u] * sr[u];
                }
            } else {
#pragma unroll
                for (int u = 0; u < 8; ++u) lo[u] = hi[u] = 0.f;
            }
            *reinterpret_cast<v8*>(dst + d0) = pack8<T>(lo);
            *reinterpret_cast<v8*>(dst + d0 + H2) = pack8<T>(hi);
        } else {
            // D = 24: one thread per row.
#pragma unroll
            for (int d0 = 0; d0 < D; d0 += 8) {
                float x[8];
                if (t < L) load8_rot<T, D>(src, p.rope_cos, p.rope_sin, t, d0, 1.0f, true, x);
                else
                    for (int u = 0; u < 8; ++u) x[u] = 0.f;
                *reinterpret_cast<v8*>(dst + d0) = pack8<T>(x);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Main kernel.
// ---------------------------------------------------------------------------
template <int D> struct FwdShape : TileShape<D> {
    static constexpr int DP = D <= 16 ? 16 : (D <= 32 ? 32 : 64);  // MFMA K for QK^T
    static constexpr int NKK = DP / 16;                              // QK MFMAs / subtile
    static constexpr int NDB = DP <= 32 ? 1 : 2;                     // 32-row blocks of O^T
    static constexpr int STAGE = 4 * TileShape<D>::TILE;             // K_s, K_m, V_s, V_m
    static constexpr int W = D == 64 ? 4 : 8;                        // wavefronts per workgroup
};

#ifndef MPATTN_FWD_WAVES
#define MPATTN_FWD_WAVES 4  // register budget: wavefronts per SIMD
#endif
#ifndef MPATTN_FWD_NBUF
#define MPATTN_FWD_NBUF 2  // LDS stages in the copy ring (copies run NBUF-1 stages ahead)
#endif
#ifndef MPATTN_FWD_SPLIT
// Key halves per 32-query block (D <= 32). 2 fills the machine in whole rounds
// at the 150M shape but doubles the per-task prologue and the L2->LDS copies;
// measured on MI355X it is slower (145 us vs 121 us), so the default is 1.
#define MPATTN_FWD_SPLIT 1
#endif

// Row sums above this bound (or not finite) send a stage through the fix-up
// path, which moves the row's reference max. 2^64 keeps every partial sum and
// accumulator far from fp32 overflow.
constexpr float kSumHi = 18446744073709551616.0f;

// SPLIT = 2: two wavefronts per 32-query block, each over half of the keys,
// merged through LDS at the end; each half streams its keys through its own
// LDS ring (both halves share the per-stage barrier).
// SQRT: sqrt-softmax, O = sum_j sqrt(P_ij) V_j. The kernel then works with
// e = exp2(s2 / 2) (the 1/2 is folded into the logit factor), accumulates
// sum e V and sum e^2, and divides by sqrt(sum e^2) at the end.
template <typename T, int D, int W, int SPLIT, int NBUF, bool ROPE, bool DENSE, bool SQRT>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(MPATTN_FWD_WAVES)))
void fwd_kernel(const FwdArgs args) {
    using S = FwdShape<D>;
    using E = Elt<T>;
    typedef typename E::v8 v8;
    typedef typename E::v2 v2;
    typedef short s4 __attribute__((ext_vector_type(4)));
    static_assert(NBUF >= 2 && NBUF <= 4, "LDS stages in flight");
    static_assert(SPLIT == 1 || SPLIT == 2, "key split");
    constexpr int WQ = W / SPLIT;               // 32-query blocks per workgroup
    constexpr int TOT = 4 * S::NI;              // DMA wave-instructions per full stage
    constexpr int NJ = (TOT + WQ - 1) / WQ;     // per wavefront (the last may be idle)
    // With fused RoPE the logit factor scale*log2(e) is folded into Q.
    constexpr bool FOLDED = ROPE;
    const mpattn_fwd_params& p = args.p;

    __shared__ __attribute__((aligned(1024))) char smem[SPLIT * NBUF * S::STAGE];
    __shared__ __attribute__((aligned(16))) int scid[W][NBUF][kBN];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ql = lane & 31, hh = lane >> 5;
    const int L = p.L, H = p.H, Lp = args.Lp;
    const int half = SPLIT == 1 ? 0 : wave / WQ;  // key half of this wavefront
    const int qw = wave - half * WQ;              // its query block in the workgroup
    const int nqb = (L + 32 * WQ - 1) / (32 * WQ);
    const int g = xcd_remap(blockIdx.x, gridDim.x);
    const int qb = g % nqb, bh = g / nqb;
    const int b = bh / H, h = bh % H;
    const int qw0 = qb * 32 * WQ;  // first query of the workgroup
    const int q = qw0 + qw * 32 + ql;
    const bool qvalid = q < L;

    auto base = [&](const mpattn_tensor& t) {
        return (const T*)t.ptr + b * t.stride_b + h * t.stride_h;
    };
    const T* const qs_p = base(p.q_self);
    const T* const qm_p = base(p.q_multi);
    const T* const km_p = base(p.k_multi);
    const T* const vs_p = base(p.v_self);
    const T* const vm_p = base(p.v_multi);
    const T* const ks_p = ROPE ? (const T*)args.krot + (int64_t)bh * Lp * D : base(p.k_self);
    const int64_t ks_t = ROPE ? D : p.k_self.stride_t;
    const int64_t km_t = p.k_multi.stride_t, vs_t = p.v_self.stride_t, vm_t = p.v_multi.stride_t;
    const int* const keff_b = args.keff + (int64_t)b * Lp;
    const int4* const ksum_b = reinterpret_cast<const int4*>(args.ksum) + (int64_t)b * (Lp / 32);

    // ---- DMA plan: copy j of this wavefront covers 16-byte slots
    // [64*part, 64*part + 64) of tile `ten` (0 K_self, 1 K_multi, 2 V_self,
    // 3 V_multi); lane -> (row r, logical chunk c), physical slot swizzled.
    const char* dsb[NJ];  // (b, h) base of the source tensor (uniform)
    unsigned dstr[NJ];    // row stride in bytes (uniform)
    unsigned dlds[NJ];    // LDS offset inside a stage (uniform)
    unsigned dloff[NJ];   // per-lane byte offset of (r, c) relative to row 0
    int drow[NJ], dcol[NJ];
    int dten[NJ];         // tile index, 4 for an idle copy (uniform)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int ins0 = qw + j * WQ;
        const int ins = ins0 < TOT ? ins0 : TOT - 1;
        const int ten = ins / S::NI, part = ins % S::NI;
        const int slot = part * 64 + lane;
        const int r = slot / S::NCH, pc = slot % S::NCH;
        const int cb = S::swz(r, pc) * 16;  // swz is an involution on the chunk index
        const T* tb = ten == 0 ? ks_p : ten == 1 ? km_p : ten == 2 ? vs_p : vm_p;
        const int64_t ts = ten == 0 ? ks_t : ten == 1 ? km_t : ten == 2 ? vs_t : vm_t;
        dsb[j] = (const char*)tb;
        dstr[j] = (unsigned)(ts * (int64_t)sizeof(T));
        dlds[j] = ten * S::TILE + part * 1024;
        drow[j] = r;
        dcol[j] = cb;
        dloff[j] = r * dstr[j] + cb;
        dten[j] = ins0 < TOT ? ten : 4;
    }
    const unsigned smem_base = lds_addr(smem) + half * NBUF * S::STAGE;  // this half's ring
    const unsigned scid_base = lds_addr(&scid[wave][0][0]);

    // ---- copy stage s into buffer bf: only the pathways the workgroup needs ----
    // Returns the number of vector-memory instructions issued (uniform).
    auto issue = [&](int s, int bf, int tiles) -> int {
        const int k0 = s * kBN;
        const unsigned lb = smem_base + bf * S::STAGE;
        unsigned voff[NJ];
        if (k0 + kBN <= L) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) voff[j] = (unsigned)k0 * dstr[j] + dloff[j];
        } else {  // last stage: clamp rows past L to L-1 (their keys are masked)
#pragma unroll
            for (int j = 0; j < NJ; ++j) voff[j] = (unsigned)min(k0 + drow[j], L - 1) * dstr[j] + dcol[j];
        }
        const int m0v = m0_save();
        int n = 1;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
            if ((tiles >> dten[j]) & 1) {
                dma16(dsb[j], voff[j], lb + dlds[j]);
                ++n;
            }
        dma4(keff_b, (unsigned)(k0 + lane) * 4u, scid_base + bf * kBN * 4);
        m0_restore(m0v);
        return n;
    };

    // ---- Q fragments (B operand of S^T = K Q^T): dims kk*16 + 8*hh + [0,8) ----
    v8 qf[2][S::NKK];
#pragma unroll
    for (int pw = 0; pw < 2; ++pw) {
#pragma unroll
        for (int kk = 0; kk < S::NKK; ++kk) {
            float x[8];
            if (qvalid) {
                const T* row = pw == 0 ? qs_p + (int64_t)q * p.q_self.stride_t
                                       : qm_p + (int64_t)q * p.q_multi.stride_t;
                load8_rot<T, D>(row, p.rope_cos, p.rope_sin, q, kk * 16 + hh * 8, args.qmul,
                                ROPE && pw == 0, x);
            } else {
#pragma unroll
                for (int t = 0; t < 8; ++t) x[t] = 0.f;
            }
            qf[pw][kk] = pack8<T>(x);
        }
    }
    // Query chain ranges of this wavefront and of the whole workgroup.
    // (from the per-32-query summaries of the prep kernel: uniform loads)
    int cq = 0, cq_min = 0, cq_max = 0, wq_min = INT32_MAX, wq_max = INT32_MIN;
    if constexpr (!DENSE) {
        cq = qvalid ? p.chain_id[(int64_t)b * L + q] : 0;
        const int4* qsum_b = reinterpret_cast<const int4*>(args.qsum) + (int64_t)b * (Lp / 32) + qw0 / 32;
#pragma unroll
        for (int w = 0; w < WQ; ++w) {
            const int4 qs = qsum_b[w < Lp / 32 - qw0 / 32 ? w : 0];
            if (qw0 + 32 * w < L) {
                wq_min = min(wq_min, qs.x);
                wq_max = max(wq_max, qs.y);
            }
            if (w == qw) {
                cq_min = qs.x;
                cq_max = qs.y;
            }
        }
        wq_min = __builtin_amdgcn_readfirstlane(wq_min);
        wq_max = __builtin_amdgcn_readfirstlane(wq_max);
        cq_min = __builtin_amdgcn_readfirstlane(cq_min);
        cq_max = __builtin_amdgcn_readfirstlane(cq_max);
    }
    const uint8_t* mrow = nullptr;
    if constexpr (DENSE) {
        mrow = p.chain_mask + (int64_t)b * p.mask_stride_b + (int64_t)(qvalid ? q : 0) * p.mask_stride_q;
    }

    // ---- softmax state ----
    // Probabilities are exp2(s2 - m_ref) with s2 = c * s the base-2 logit.
    // m_ref starts at 0 and stays there unless a stage's row sum leaves
    // (0, 2^64]: then the fix-up path sets it from that stage's max and the
    // wavefront switches to the shifted form (one FMA per logit).
    const float c = args.c;  // 1 when FOLDED
    float m_ref = 0.f;
    bool shifted = false;    // wavefront-uniform: some m_ref != 0
    float l_run = 0.f;
    f32x16 o[S::NDB];
#pragma unroll
    for (int db = 0; db < S::NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] = 0.f;

    const int krow = swapped_row(ql);
    v8 zero8;
#pragma unroll
    for (int t = 0; t < 8; ++t) zero8[t] = (T)0.f;

    // Per-lane LDS byte offsets of the MFMA operands inside a tile (the chunk
    // swizzle repeats every 16 rows, so other subtiles only add a constant).
    int koff[S::NKK];
#pragma unroll
    for (int kk = 0; kk < S::NKK; ++kk) {
        const int cch = 2 * kk + hh;
        koff[kk] = cch < S::NCH ? krow * S::RB + S::swz(krow, cch) * 16 : 0;
    }
    // V^T operand via ds_read_b64_tr_b16: lane (group tg, index ti) addresses
    // row 8*(tg>>1) + 4*rr + ti/4 and the 8-byte chunk 8*db + 4*(tg&1) + ti%4
    // (clamped into the row for D < 32; those lanes' values are unused).
    const int tg = lane >> 4, ti = lane & 15;
    int voffv[S::NDB][2];
#pragma unroll
    for (int db = 0; db < S::NDB; ++db) {
        int e = 8 * db + 4 * (tg & 1) + (ti & 3);
        if (8 * e >= S::RB) e = ti & 3;
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
            const int row = 8 * (tg >> 1) + 4 * rr + (ti >> 2);
            voffv[db][rr] = row * S::RB + S::swz(row, e >> 1) * 16 + (e & 1) * 8;
        }
    }

    // Base-2 probability of raw logit x.
    auto prob = [&](float x, bool sh) -> float {
        if (sh) return fast_exp2(fmaf(x, c, -m_ref));
        return fast_exp2(FOLDED ? x : x * c);
    };
    // Probabilities of NS subtiles (slot 8*cc + t -> pb[st][cc][t]) and their
    // row sum over this lane's keys.
    auto probs = [&](auto ns_c, const f32x16* sv, v8 (*pb)[2], bool sh) -> float {
        constexpr int NS = decltype(ns_c)::value;
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        // Pairs are rounded once (v_cvt_pk) and feed both the PV operand and
        // the row sum; two sum chains halve the dependency depth.
        float ls0 = 0.f, ls1 = 0.f;
#pragma unroll
        for (int st = 0; st < NS; ++st)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                v2 pr[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const f32x2 f = {prob(sv[st][8 * cc + 2 * u], sh), prob(sv[st][8 * cc + 2 * u + 1], sh)};
                    pr[u] = __builtin_convertvector(f, v2);
                }
                pb[st][cc] = __builtin_shufflevector(__builtin_shufflevector(pr[0], pr[1], 0, 1, 2, 3),
                                                     __builtin_shufflevector(pr[2], pr[3], 0, 1, 2, 3), 0, 1, 2,
                                                     3, 4, 5, 6, 7);
                if constexpr (SQRT) {
                    ls0 = E::sq2(pr[0], ls0);
                    ls1 = E::sq2(pr[1], ls1);
                    ls0 = E::sq2(pr[2], ls0);
                    ls1 = E::sq2(pr[3], ls1);
                } else {
                    ls0 = E::sum2(pr[0], ls0);
                    ls1 = E::sum2(pr[1], ls1);
                    ls0 = E::sum2(pr[2], ls0);
                    ls1 = E::sum2(pr[3], ls1);
                }
            }
        return ls0 + ls1;
    };
    // Rare path: a lane's stage sum overflowed, or its row has accumulated
    // nothing yet. The stage's logits are recomputed from LDS (`logits`
    // fills sv) and its probabilities redone relative to a reference max
    // taken from them (raised only, once something has been accumulated).
    auto fixup = [&](auto ns_c, auto logits, v8 (*pb)[2]) -> float {
        constexpr int NS = decltype(ns_c)::value;
        f32x16 sv[NS];
        logits(sv);
        float mx = -INFINITY;
#pragma unroll
        for (int st = 0; st < NS; ++st)
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sv[st][i]);
        const float mq = fmaxf(mx, __shfl_xor(mx, 32));  // query max of the stage, raw units
        const float lq = l_run + __shfl_xor(l_run, 32);
        const float ms = mq * c;
        float m_new;
        if (lq > 0.f) m_new = fmaxf(m_ref, ms);
        else m_new = ms > -INFINITY ? ms : m_ref;
        const float alpha = lq > 0.f ? fast_exp2(m_ref - m_new) : 1.0f;
        l_run *= SQRT ? alpha * alpha : alpha;
#pragma unroll
        for (int db = 0; db < S::NDB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
        m_ref = m_new;
        shifted = __builtin_amdgcn_ballot_w64(m_ref != 0.f) != 0;
        return probs(ns_c, sv, pb, true);
    };
    // Stage check: true if any lane needs the fix-up.
    auto needs_fix = [&](float ls) {
        const bool bad = !(ls <= kSumHi) || (l_run + ls == 0.f);
        return __builtin_amdgcn_ballot_w64(bad) != 0;
    };

    // Operand readers with the tile base given.
    auto kop_t = [&](const char* tile, int st, int kk) -> v8 {
        if (2 * kk + hh >= S::NCH) return zero8;  // D = 24: dims [24, 32)
        return *reinterpret_cast<const v8*>(tile + st * 32 * S::RB + koff[kk]);
    };
    auto vop_t = [&](const char* tile, int st, int cc, int db) -> v8 {
        s4 half[2];
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
            const char* ptr = tile + (st * 32 + 16 * cc) * S::RB + voffv[db][rr];
            half[rr] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)(ptr));
        }
        // Whole-vector bitcast: element-wise i16 -> bf16 inserts are mis-lowered.
        return __builtin_bit_cast(v8, __builtin_shufflevector(half[0], half[1], 0, 1, 2, 3, 4, 5, 6, 7));
    };
    // S^T of one subtile from K operands ka and Q operands qa.
    auto qkq = [&](const v8* ka, const v8* qa) -> f32x16 {
        f32x16 sv;
#pragma unroll
        for (int i = 0; i < 16; ++i) sv[i] = 0.f;
#pragma unroll
        for (int kk = 0; kk < S::NKK; ++kk) sv = E::mma(ka[kk], qa[kk], sv);
        return sv;
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;

    // Q operand of the fast path's pathway (changes rarely: at chain edges).
    int cur_pw = 0;
    v8 qcur[S::NKK];
#pragma unroll
    for (int kk = 0; kk < S::NKK; ++kk) qcur[kk] = qf[0][kk];

    // Fast path: both subtiles of the stage on pathway pw, unshifted softmax.
    // Returns false (nothing accumulated) if the stage needs the fix-up.
    auto fast_stage = [&](const char* stage, int pw) -> bool {
        const char* kt = stage + pw * S::TILE;
        const char* vt = stage + (2 + pw) * S::TILE;
        // All LDS operands are read up front: the V reads overlap the softmax.
        v8 ka[2][S::NKK], va[2][2][S::NDB];
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
            for (int kk = 0; kk < S::NKK; ++kk) ka[st][kk] = kop_t(kt, st, kk);
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                for (int db = 0; db < S::NDB; ++db) va[st][cc][db] = vop_t(vt, st, cc, db);
        // keep every LDS read of the stage ahead of the softmax
        __builtin_amdgcn_sched_barrier(0);
        v8 pb[2][2];
        float ls;
        {
            f32x16 sv[2];
#pragma unroll
            for (int st = 0; st < 2; ++st) sv[st] = qkq(ka[st], qcur);
            ls = probs(I2{}, sv, pb, false);
        }
        if (needs_fix(ls)) return false;
        l_run += ls;
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                for (int db = 0; db < S::NDB; ++db) o[db] = E::mma(va[st][cc][db], pb[st][cc], o[db]);
        return true;
    };

    // Both pathways on one subtile, selected per element; handles padded keys.
    auto general = [&](const char* stage, const int* cid, int st, int k0) {
        bool same[16];
        // Selected raw logits (-inf for padded keys) into sv[0]; keys of
        // slot i: st*32 + 16*(i/8) + 8*hh + i%8.
        auto logits = [&](f32x16* sv) {
            v8 ks[S::NKK], km[S::NKK];
#pragma unroll
            for (int kk = 0; kk < S::NKK; ++kk) {
                ks[kk] = kop_t(stage, st, kk);
                km[kk] = kop_t(stage + S::TILE, st, kk);
            }
            const f32x16 ss = qkq(ks, qf[0]), sm = qkq(km, qf[1]);
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const int kl = st * 32 + 16 * cc + 8 * hh;
                const i32x4 c0 = *reinterpret_cast<const i32x4*>(&cid[kl]);
                const i32x4 c1 = *reinterpret_cast<const i32x4*>(&cid[kl + 4]);
                uint32_t mbits = 0;
                if constexpr (DENSE) {
                    const int kg = k0 + kl;
                    for (int t = 0; t < 8; ++t)
                        if (kg + t < L)
                            mbits |= (uint32_t)(mrow[(int64_t)(kg + t) * p.mask_stride_k] != 0) << t;
                }
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const int ck = t < 4 ? c0[t & 3] : c1[t & 3];
                    const int i = 8 * cc + t;
                    const bool sm_ = DENSE ? !((mbits >> t) & 1u) : (ck == cq);
                    same[i] = sm_;
                    const float v = sm_ ? ss[i] : sm[i];
                    sv[0][i] = ck == kPadChain ? -INFINITY : v;
                }
            }
        };
        v8 pb[1][2];
        float ls;
        {
            f32x16 sv[1];
            logits(sv);
            ls = shifted ? probs(I1{}, sv, pb, true) : probs(I1{}, sv, pb, false);
        }
        if (needs_fix(ls)) ls = fixup(I1{}, logits, pb);
        l_run += ls;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            v8 ps, pm;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int i = 8 * cc + t;
                ps[t] = same[i] ? pb[0][cc][t] : (T)0.f;
                pm[t] = same[i] ? (T)0.f : pb[0][cc][t];
            }
#pragma unroll
            for (int db = 0; db < S::NDB; ++db) {
                o[db] = E::mma(vop_t(stage + 2 * S::TILE, st, cc, db), ps, o[db]);
                o[db] = E::mma(vop_t(stage + 3 * S::TILE, st, cc, db), pm, o[db]);
            }
        }
    };

    // One subtile on the slow path. code: 0 pure self, 1 pure multimer,
    // 2 straddle (keys on one chain, queries on several: pathway per lane),
    // 3 general, 4 skip.
    auto slow_subtile = [&](const char* stage, const int* cid, int st, int code, int k0) {
        if (code >= 4) return;
        if (code == 3) {
            general(stage, cid, st, k0);
            return;
        }
        v8 pb[1][2];
        float ls;
        if (code <= 1) {
            const int pw = code;
            const char* kt = stage + pw * S::TILE;
            v8 qa[S::NKK];
#pragma unroll
            for (int kk = 0; kk < S::NKK; ++kk) qa[kk] = pw ? qf[1][kk] : qf[0][kk];
            auto logits = [&](f32x16* sv) {
                v8 kr[S::NKK];
#pragma unroll
                for (int kk = 0; kk < S::NKK; ++kk) kr[kk] = kop_t(kt, st, kk);
                sv[0] = qkq(kr, qa);
            };
            {
                f32x16 sv[1];
                logits(sv);
                ls = shifted ? probs(I1{}, sv, pb, true) : probs(I1{}, sv, pb, false);
            }
            if (needs_fix(ls)) ls = fixup(I1{}, logits, pb);
            l_run += ls;
            const char* vt = stage + (2 + pw) * S::TILE;
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                for (int db = 0; db < S::NDB; ++db) o[db] = E::mma(vop_t(vt, st, cc, db), pb[0][cc], o[db]);
            return;
        }
        // straddle: lane is on the self pathway iff its chain is the keys' chain
        const bool self_lane = cq == cid[st * 32];
        auto logits = [&](f32x16* sv) {
            v8 ks[S::NKK], km[S::NKK];
#pragma unroll
            for (int kk = 0; kk < S::NKK; ++kk) {
                ks[kk] = kop_t(stage, st, kk);
                km[kk] = kop_t(stage + S::TILE, st, kk);
            }
            const f32x16 ss = qkq(ks, qf[0]), sm = qkq(km, qf[1]);
#pragma unroll
            for (int i = 0; i < 16; ++i) sv[0][i] = self_lane ? ss[i] : sm[i];
        };
        {
            f32x16 sv[1];
            logits(sv);
            ls = shifted ? probs(I1{}, sv, pb, true) : probs(I1{}, sv, pb, false);
        }
        if (needs_fix(ls)) ls = fixup(I1{}, logits, pb);
        l_run += ls;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const v8 ps = self_lane ? pb[0][cc] : zero8;
            const v8 pm = self_lane ? zero8 : pb[0][cc];
#pragma unroll
            for (int db = 0; db < S::NDB; ++db) {
                o[db] = E::mma(vop_t(stage + 2 * S::TILE, st, cc, db), ps, o[db]);
                o[db] = E::mma(vop_t(stage + 3 * S::TILE, st, cc, db), pm, o[db]);
            }
        }
    };

    auto subtile_mode = [&](int kmin, int kmax, int npad) -> int {
        if (npad == 32) return 4;
        if (DENSE) return 3;
        if (npad == 0) {
            if (kmax < cq_min || kmin > cq_max) return 1;
            if (kmin == kmax) return cq_min == cq_max ? 0 : 2;
        }
        return 3;
    };

    // Subtile codes of this wavefront for the 64 subtiles from kb0, as three
    // bit masks (mb0..mb2 = code bits), and which pathways the workgroup
    // needs there (nS / nM) so stages copy only those tiles. Each reload is a
    // vector load whose wait also drains the copies in flight: windows move
    // once per 32 stages.
    uint64_t mb0 = 0, mb1 = 0, mb2 = 0, nS = 0, nM = 0;
    auto load_codes = [&](int kb0) {
        const int kb = kb0 + lane;
        int code = 4;
        if (kb < Lp / 32) {
            const int4 sm = ksum_b[kb];
            code = subtile_mode(sm.x, sm.y, sm.z);
        }
        mb0 = __builtin_amdgcn_ballot_w64(code & 1);
        mb1 = __builtin_amdgcn_ballot_w64((code >> 1) & 1);
        mb2 = __builtin_amdgcn_ballot_w64((code >> 2) & 1);
    };
    auto load_needs = [&](int kb0) {
        const int kb = kb0 + lane;
        bool ns = false, nm = false;
        if (kb < Lp / 32) {
            const int4 sm = ksum_b[kb];
            if (sm.z < 32) {
                if (DENSE || sm.z > 0) {
                    ns = nm = true;
                } else {
                    ns = !(sm.y < wq_min || sm.x > wq_max);
                    nm = !(sm.x == sm.y && wq_min == wq_max && sm.x == wq_min);
                }
            }
        }
        nS = __builtin_amdgcn_ballot_w64(ns);
        nM = __builtin_amdgcn_ballot_w64(nm);
    };
    auto code_at = [&](int sub) -> int {
        return (int)((mb0 >> sub) & 1) | (int)(((mb1 >> sub) & 1) << 1) | (int)(((mb2 >> sub) & 1) << 2);
    };

    // ---- main loop over stages ----
    // This wavefront's keys: stages [s_lo, s_lo + s_cnt); both halves run
    // nloop iterations so the barriers pair up.
    const int nst_all = (L + kBN - 1) / kBN;
    const int n0 = SPLIT == 1 ? nst_all : (nst_all + 1) / 2;
    const int s_lo = half ? n0 : 0;
    const int s_cnt = half ? nst_all - n0 : n0;
    const int nloop = n0;
    int kbp = 2 * s_lo, kbi = 2 * s_lo;  // first subtile of the code / need windows
    load_codes(kbp);                     // before any copy is in flight
    load_needs(kbi);
    // Every prologue load (Q, chain ids, summaries) has landed before the first
    // copy is issued. The compiler sees this wait (the copies are inline asm it
    // cannot see), so it adds no vmcnt(0) at later uses, which would also
    // drain the copies in flight.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    // Tiles stage t copies (bit i = tile i): K_self and V_self (bits 0, 2)
    // if any of its subtiles needs the self pathway, K_multi and V_multi
    // (1, 3) for the multimer pathway.
    auto tiles_for = [&](int t) -> int {
        if (2 * t + 1 - kbi >= 64) {
            kbi = 2 * t;
            load_needs(kbi);
        }
        const int nx = 2 * t - kbi;
        const int m = (((nS >> nx) & 3) != 0 ? 5 : 0) | (((nM >> nx) & 3) != 0 ? 10 : 0);
        return __builtin_amdgcn_readfirstlane(m);
    };
    // pend[k]: vector-memory instructions of local stage s + k still in flight.
    int pend[NBUF];
#pragma unroll
    for (int t = 0; t < NBUF; ++t) pend[t] = 0;
#pragma unroll
    for (int t = 0; t < NBUF - 1; ++t)
        if (t < s_cnt) pend[t] = issue(s_lo + t, t, tiles_for(s_lo + t));
    int bf = 0;
    char* const ring = smem + half * NBUF * S::STAGE;
    for (int s = 0; s < nloop; ++s) {
        int allow = 0;  // copies of later stages that may stay in flight
#pragma unroll
        for (int k = 1; k < NBUF - 1; ++k) allow += pend[k];
        wait_vm_var(allow);
        stage_barrier();
#pragma unroll
        for (int k = 0; k < NBUF - 1; ++k) pend[k] = pend[k + 1];
        pend[NBUF - 1] = 0;
        if (s >= s_cnt) continue;  // the shorter half: barrier only
        const int gs = s_lo + s;   // global stage index
        if (2 * gs + 1 - kbp >= 64) {
            kbp = 2 * gs;
            load_codes(kbp);
        }
        const int sub = 2 * gs - kbp;
        const int c0 = code_at(sub), c1 = code_at(sub + 1);
        if (s + NBUF - 1 < s_cnt) {
            const int bn = bf + NBUF - 1 >= NBUF ? bf - 1 : bf + NBUF - 1;
            pend[NBUF - 2] = issue(gs + NBUF - 1, bn, tiles_for(gs + NBUF - 1));
        }

        const char* stage = ring + bf * S::STAGE;
        bool done = false;
        if (c0 == c1 && c0 <= 1 && !shifted) {
            if (c0 != cur_pw) {  // rare: kept a branch (not selects on every stage)
                asm volatile("" ::: "memory");
                cur_pw = c0;
#pragma unroll
                for (int kk = 0; kk < S::NKK; ++kk) qcur[kk] = c0 ? qf[1][kk] : qf[0][kk];
            }
            done = fast_stage(stage, c0);
        }
        if (!done) {
            const int* cid = &scid[wave][bf][0];
            const int k0 = gs * kBN;
#pragma unroll 1
            for (int st = 0; st < 2; ++st) slow_subtile(stage, cid, st, st ? c1 : c0, k0);
        }
        bf = bf + 1 == NBUF ? 0 : bf + 1;
    }

    // ---- merge the two key halves (SPLIT = 2) ----
    if constexpr (SPLIT == 2) {
        // The rings are free once every wavefront passed its last stage.
        stage_barrier();
        constexpr int NV = 16 * S::NDB + 2;  // o, l_run, m_ref per lane
        float* xs = reinterpret_cast<float*>(smem) + (size_t)qw * NV * 64;
        if (half) {
#pragma unroll
            for (int db = 0; db < S::NDB; ++db)
#pragma unroll
                for (int i = 0; i < 16; ++i) xs[(16 * db + i) * 64 + lane] = o[db][i];
            xs[(16 * S::NDB) * 64 + lane] = l_run;
            xs[(16 * S::NDB + 1) * 64 + lane] = m_ref;
        }
        stage_barrier();
        if (half) return;
        const float lb = xs[(16 * S::NDB) * 64 + lane];
        const float mb = xs[(16 * S::NDB + 1) * 64 + lane];
        // A half that accumulated nothing for this query (its sums over both
        // lane halves are 0) neither sets nor rescales the merged reference.
        const float laq = l_run + __shfl_xor(l_run, 32);
        const float lbq = lb + __shfl_xor(lb, 32);
        float m = m_ref;
        if (lbq > 0.f) m = laq > 0.f ? fmaxf(m_ref, mb) : mb;
        const float aa = (laq > 0.f && m_ref != m) ? fast_exp2(m_ref - m) : 1.0f;
        const float ab = (lbq > 0.f && mb != m) ? fast_exp2(mb - m) : 1.0f;
#pragma unroll
        for (int db = 0; db < S::NDB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][i] = o[db][i] * aa + xs[(16 * db + i) * 64 + lane] * ab;
        l_run = SQRT ? l_run * aa * aa + lb * ab * ab : l_run * aa + lb * ab;
        m_ref = m;
    }

    // ---- epilogue: normalise, store O and LSE ----
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const float inv = l_tot > 0.f ? (SQRT ? __frsqrt_rn(l_tot) : 1.0f / l_tot) : 0.f;
    if (qvalid) {
        T* orow = (T*)p.out.ptr + b * p.out.stride_b + h * p.out.stride_h + (int64_t)q * p.out.stride_t;
#pragma unroll
        for (int db = 0; db < S::NDB; ++db)
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const int d = db * 32 + 8 * a + 4 * hh;
                if (d < D) {
                    typename E::v4 v;
#pragma unroll
                    for (int j = 0; j < 4; ++j) v[j] = (T)(o[db][4 * a + j] * inv);
                    *reinterpret_cast<typename E::v4*>(orow + d) = v;
                }
            }
        if (p.lse && hh == 0) {
            p.lse[((int64_t)b * H + h) * L + q] =
                l_tot > 0.f ? ((SQRT ? 2.0f * m_ref : m_ref) + __log2f(l_tot)) * kLn2 : -INFINITY;
        }
    }
}

template <typename T, int D, bool ROPE, bool DENSE, bool SQRT>
static hipError_t launch_fwd(FwdArgs& a, hipStream_t stream) {
    constexpr int W = FwdShape<D>::W;
    // Optional key split for D <= 32 (see MPATTN_FWD_SPLIT). Two LDS stages per
    // ring keep two workgroups per CU with the split (D = 64 tiles are twice as
    // large: two stages, no split).
    constexpr int SPLIT = D == 64 ? 1 : MPATTN_FWD_SPLIT;
    constexpr int NBUF = (D == 64 || SPLIT == 2) ? 2 : MPATTN_FWD_NBUF;
    const mpattn_fwd_params& p = a.p;
    const int Lp = round_up(p.L, kBN);
    a.Lp = Lp;
    const FwdWs ws = fwd_ws_layout(p.B, p.H, p.L, D, sizeof(T), ROPE);
    char* wsb = (char*)p.workspace;
    int* keff = (int*)(wsb + ws.keff);
    int* ksum = (int*)(wsb + ws.ksum);
    int* qsum = (int*)(wsb + ws.qsum);
    T* krot = (T*)(wsb + ws.krot);
    a.keff = keff;
    a.ksum = ksum;
    a.qsum = qsum;
    a.krot = krot;
    const int nchain = (p.B * (Lp / 64) + 3) / 4;
    constexpr int NPC = ((D / 2) % 8 == 0) ? D / 16 : 1;
    const int64_t nrot = ROPE ? ((int64_t)p.B * p.H * Lp * NPC + 255) / 256 : 0;
    hipLaunchKernelGGL((fwd_prep_kernel<T, D, ROPE, DENSE>), dim3((unsigned)(nchain + nrot)), dim3(256), 0,
                       stream, p, keff, ksum, qsum, krot, Lp, nchain);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    constexpr int WQ = W / SPLIT;
    const int nqb = (p.L + 32 * WQ - 1) / (32 * WQ);
    const int64_t grid = (int64_t)p.B * p.H * nqb;
    hipLaunchKernelGGL((fwd_kernel<T, D, W, SPLIT, NBUF, ROPE, DENSE, SQRT>), dim3((unsigned)grid),
                       dim3(W * 64), 0, stream, a);
    return hipGetLastError();
}

// Chain staging for the fp32 kernel (mpattn_fp32.hip): the prep kernel's
// chain blocks only (the fp32 kernel rotates K_self while staging it).
void fwd_ws_offsets(int B, int H, int L, int D, int esize, bool rope, int64_t* keff, int64_t* ksum,
                    int64_t* qsum) {
    const FwdWs w = fwd_ws_layout(B, H, L, D, esize, rope);
    *keff = w.keff;
    *ksum = w.ksum;
    *qsum = w.qsum;
}

hipError_t launch_fwd_prep_f32(const mpattn_fwd_params& p, int* keff, int* ksum, int* qsum, int Lp,
                               hipStream_t stream) {
    const int nchain = (p.B * (Lp / 64) + 3) / 4;
    if (p.chain_mask)
        hipLaunchKernelGGL((fwd_prep_kernel<float, 16, false, true>), dim3((unsigned)nchain), dim3(256), 0,
                           stream, p, keff, ksum, qsum, (float*)nullptr, Lp, nchain);
    else
        hipLaunchKernelGGL((fwd_prep_kernel<float, 16, false, false>), dim3((unsigned)nchain), dim3(256), 0,
                           stream, p, keff, ksum, qsum, (float*)nullptr, Lp, nchain);
    return hipGetLastError();
}

template <typename T, int D>
static hipError_t dispatch_fwd_d(FwdArgs& a, hipStream_t s) {
    const bool rope = a.p.rope == MPATTN_ROPE_FUSED;
    const bool dense = a.p.chain_mask != nullptr;
    if (a.p.sqrt_softmax) {
        if (rope) return dense ? launch_fwd<T, D, true, true, true>(a, s) : launch_fwd<T, D, true, false, true>(a, s);
        return dense ? launch_fwd<T, D, false, true, true>(a, s) : launch_fwd<T, D, false, false, true>(a, s);
    }
    if (rope) return dense ? launch_fwd<T, D, true, true, false>(a, s) : launch_fwd<T, D, true, false, false>(a, s);
    return dense ? launch_fwd<T, D, false, true, false>(a, s) : launch_fwd<T, D, false, false, false>(a, s);
}

template <typename T>
static hipError_t dispatch_fwd_t(FwdArgs& a, hipStream_t s) {
    switch (a.p.D) {
        case 16: return dispatch_fwd_d<T, 16>(a, s);
        case 24: return dispatch_fwd_d<T, 24>(a, s);
        case 32: return dispatch_fwd_d<T, 32>(a, s);
        case 64: return dispatch_fwd_d<T, 64>(a, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_fwd16(const mpattn_fwd_params& p, hipStream_t stream) {
    FwdArgs a;
    a.p = p;
    // Fused RoPE folds scale * log2(e) into Q; caller-rotated q keeps its
    // exact values and the factor is applied per logit.
    // Sqrt-softmax works with exp2 of half the base-2 logit.
    const bool fused = p.rope == MPATTN_ROPE_FUSED;
    const float f = p.scale * kLog2e * (p.sqrt_softmax ? 0.5f : 1.0f);
    a.qmul = fused ? f : 1.0f;
    a.c = fused ? 1.0f : f;
    if (p.dtype == MPATTN_BF16) return dispatch_fwd_t<bf16_t>(a, stream);
    return dispatch_fwd_t<fp16_t>(a, stream);
}

}  // namespace mpattn
