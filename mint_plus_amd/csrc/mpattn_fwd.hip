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
//  * A workgroup of W wavefronts owns 32*W consecutive queries of one (b, h);
//    each wavefront owns 32 of them. Q is loaded once, RoPE and the logit
//    scale applied in fp32.
//  * Keys stream through a ring of NBUF LDS stages of 64 keys. Each stage holds
//    K_self, K_multi, V_self, V_multi tiles copied by global_load_lds (16 bytes
//    per lane, straight into LDS, no register round trip), issued NBUF-1
//    stages ahead of use, one barrier per stage. Rows are stored densely with
//    their 16-byte chunks XOR-swizzled by row to spread LDS banks.
//  * Per 32-key subtile a wavefront computes S^T = K Q^T with
//    v_mfma_f32_32x32x16 (rows = keys, columns = queries): lane l holds 16
//    logits of query l%32, so the softmax row statistics are in-lane. K rows
//    are read with bits 2 and 3 of the row index swapped, which makes
//    accumulator slot i of lane half hh the key 16*(i/8) + 8*hh + i%8: the
//    probabilities are then already the B operand of O^T += V^T P^T. The V^T
//    operand comes from the row-major V tile via ds_read_b64_tr_b16.
//  * Stages are classified from the per-32-key chain summaries and the
//    wavefront's query chain range: pure same-chain stages run only the self
//    pathway, pure cross-chain stages only the multimer pathway (one softmax
//    update over 64 keys); mixed or padded subtiles compute both logits and
//    select per element.
//  * Online softmax in base 2 with a lazily updated reference max: nothing is
//    rescaled unless a row max grows by more than 2^8, and only then do the
//    two lane halves of a query exchange their maxima.
//  * Row sums come from v_dot2_f32_bf16 on the rounded probabilities (the
//    values the PV MFMA consumes). For D < 32 the unused rows of the V^T
//    operand are ones, so the MFMA produces the sum.
#include <type_traits>

#include "mpattn_common.h"

namespace mpattn {

constexpr int kBN = 64;  // keys per LDS stage

inline int round_up(int x, int m) { return (x + m - 1) / m * m; }

// Workspace layout (offsets 256-byte aligned):
//   keff int32 [B][Lp]          effective chain id per key
//   ksum int32 [B][Lp/32][4]    min chain, max chain, #padded, 0
//   krot T     [B][H][Lp][D]    RoPE-rotated K_self (fused RoPE only)
struct FwdWs {
    int64_t keff, ksum, krot, total;
};

inline FwdWs fwd_ws_layout(int B, int H, int L, int D, int esize, bool rope) {
    const int64_t Lp = round_up(L, kBN);
    auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
    FwdWs w;
    w.keff = 0;
    w.ksum = al(w.keff + (int64_t)B * Lp * 4);
    w.krot = al(w.ksum + (int64_t)B * (Lp / 32) * 16);
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
                                                       int* ksum, T* krot, int Lp, int nchain) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int L = p.L;
    if ((int)blockIdx.x < nchain) {
        const int ngrp = Lp / 64;
        const int gid = blockIdx.x * 4 + wave;
        if (gid >= p.B * ngrp) return;
        const int b = gid / ngrp, k0 = (gid % ngrp) * 64;
        const int kg = k0 + lane;
        int cid = kPadChain;
        if (kg < L && !(p.key_pad && p.key_pad[(int64_t)b * L + kg]))
            cid = DENSE ? 0 : p.chain_id[(int64_t)b * L + kg];
        keff[(int64_t)b * Lp + kg] = cid;
        const bool valid = cid != kPadChain;
        const int mn = half_min_i(valid ? cid : INT32_MAX);
        const int mx = half_max_i(valid ? cid : INT32_MIN);
        const uint64_t padm = __ballot(!valid);
        if ((lane & 31) == 0) {
            const int hh = lane >> 5;
            int* o = ksum + ((int64_t)b * (Lp / 32) + (k0 >> 5) + hh) * 4;
            o[0] = mn;
            o[1] = mx;
            o[2] = __popcll(hh ? (padm >> 32) : (padm & 0xffffffffull));
            o[3] = 0;
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
template <int D> struct FwdShape {
    static constexpr int DP = D <= 16 ? 16 : (D <= 32 ? 32 : 64);  // MFMA K for QK^T
    static constexpr int NKK = DP / 16;                              // QK MFMAs / subtile
    static constexpr int NDB = DP <= 32 ? 1 : 2;                     // 32-row blocks of O^T
    static constexpr bool SUM_MFMA = D < 32;                         // ones rows give the sum
    static constexpr int ISUM = 4 * (D / 8);                         // accumulator slot of row D
    static constexpr int RB = D * 2;                                 // LDS row bytes
    static constexpr int NCH = RB / 16;                              // 16-byte chunks per row
    static constexpr int TILE = kBN * RB;                            // bytes per tensor tile
    static constexpr int STAGE = 4 * TILE;
    static constexpr int NI = TILE / 1024;                           // DMA wave-instr per tile
    static constexpr bool POW2 = (NCH & (NCH - 1)) == 0;
    static constexpr int ROWS_PER_256 = 256 / RB;
    // physical 16-byte chunk of logical chunk c in row r
    static __device__ __forceinline__ int swz(int r, int c) {
        if constexpr (POW2) return c ^ ((r / ROWS_PER_256) & (NCH - 1));
        return c;
    }
};

#ifndef MPATTN_FWD_WAVES
#define MPATTN_FWD_WAVES 4  // register budget: wavefronts per SIMD
#endif
#ifndef MPATTN_FWD_NBUF32
#define MPATTN_FWD_NBUF32 2  // LDS stages in flight for D <= 32
#endif

template <typename T, int D, int W, int NBUF, bool ROPE, bool DENSE>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(MPATTN_FWD_WAVES)))
void fwd_kernel(const FwdArgs args) {
    using S = FwdShape<D>;
    using E = Elt<T>;
    typedef typename E::v8 v8;
    typedef typename E::v2 v2;
    typedef short s4 __attribute__((ext_vector_type(4)));
    typedef short s8 __attribute__((ext_vector_type(8)));
    constexpr int TOT = 4 * S::NI;  // DMA instructions per stage
    static_assert(TOT % W == 0, "stage DMA must split evenly over waves");
    constexpr int IPW = TOT / W + 1;  // per wave per stage, incl. the chain ids
    const mpattn_fwd_params& p = args.p;

    __shared__ __attribute__((aligned(1024))) char smem[NBUF * S::STAGE];
    __shared__ __attribute__((aligned(16))) int scid[W][NBUF][kBN];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ql = lane & 31, hh = lane >> 5;
    const int L = p.L, H = p.H, Lp = args.Lp;
    const int nqb = (L + 32 * W - 1) / (32 * W);
    const int g = xcd_remap(blockIdx.x, gridDim.x);
    const int qb = g % nqb, bh = g / nqb;
    const int b = bh / H, h = bh % H;
    const int q = qb * 32 * W + wave * 32 + ql;
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

    // ---- DMA plan: this wave's TOT/W tile copies per stage ----
    // Copy j covers 16-byte slots [64*part, 64*part + 64) of tensor `ten`;
    // lane -> (row r, logical chunk c) with the physical slot swizzled.
    constexpr int NJ = TOT / W;
    const char* dsb[NJ];     // (b, h) base of the source tensor (uniform)
    unsigned dstr[NJ];       // row stride in bytes (uniform)
    unsigned dlds[NJ];       // LDS offset inside a stage (uniform)
    unsigned dloff[NJ];      // per-lane byte offset of (r, c) relative to row 0
    int drow[NJ], dcol[NJ];  // per-lane row and chunk byte offset
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int ins = wave + j * W;
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
    }
    const unsigned smem_base = lds_addr(smem);
    const unsigned scid_base = lds_addr(&scid[wave][0][0]);

    // ---- issue the DMA of stage s into buffer bf ----
    auto issue = [&](int s, int bf) {
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
#pragma unroll
        for (int j = 0; j < NJ; ++j) dma16(dsb[j], voff[j], lb + dlds[j]);
        dma4(keff_b, (unsigned)(k0 + lane) * 4u, scid_base + bf * kBN * 4);
        m0_restore(m0v);
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
    int cq = 0, cq_min = 0, cq_max = 0;
    if constexpr (!DENSE) {
        cq = qvalid ? p.chain_id[(int64_t)b * L + q] : 0;
        cq_min = __builtin_amdgcn_readfirstlane(wave_min_i(qvalid ? cq : INT32_MAX));
        cq_max = __builtin_amdgcn_readfirstlane(wave_max_i(qvalid ? cq : INT32_MIN));
    }
    const uint8_t* mrow = nullptr;
    if constexpr (DENSE) {
        mrow = p.chain_mask + (int64_t)b * p.mask_stride_b + (int64_t)(qvalid ? q : 0) * p.mask_stride_q;
    }

    // ---- online softmax state ----
    // Logits are handled in base-2 units, s2 = c * s. With BIAS (fused RoPE) c
    // is folded into Q in fp32 before its single rounding, and the MFMA itself
    // returns s2 - m_ref through one extra feature (K side 1, Q side -m_ref,
    // m_ref kept bf16-exact): no per-logit FMA. Without BIAS (caller-rotated
    // q/k used as given) s2 - m_ref is one FMA per logit.
    // The bias feature costs one more MFMA on each subtile's dependency chain
    // (QK -> bias -> max -> exp); measured on MI355X at the 150M shape it is
    // slower (182 us vs 153 us) than one FMA per logit, so it stays off.
    constexpr bool BIAS = false;
    const float c = args.c;  // 1 with BIAS
    float m_ref = 0.f;       // reference max (base 2)
    bool started = false;    // wave-uniform: m_ref has been set
    float l_run = 0.f;
    f32x16 o[S::NDB];
#pragma unroll
    for (int db = 0; db < S::NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] = 0.f;

    // K operand row: subtile row ql with bits 2,3 swapped.
    const int krow = (ql & ~12) | ((ql & 4) << 1) | ((ql & 8) >> 1);
    v8 zero8, one8, unit8;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        zero8[t] = (T)0.f;
        one8[t] = (T)1.0f;
        unit8[t] = (T)(t == 0 ? 1.0f : 0.0f);
    }
    // Bias feature: an extra K-chunk (K side: 1 at dim 0 of lane half 0) for
    // D != 24; for D = 24 it is dim 24, inside the zero padding [24, 32).
    const v8 kbias = hh == 0 ? unit8 : zero8;
    v8 qbias = zero8;
    auto set_bias = [&]() {
        const T nb = (T)(-m_ref);
        if constexpr (D == 24) {
            if (hh) {
                qf[0][1][0] = nb;
                qf[1][1][0] = nb;
            }
        } else {
            if (hh == 0) qbias[0] = nb;
        }
    };

    // Per-lane LDS byte offsets of the MFMA operands inside a tile. The chunk
    // swizzle repeats every 16 rows, so moving to another subtile or key chunk
    // only adds a constant.
    // K operand (A of S^T = K Q^T): row krow, dims kk*16 + 8*hh + [0, 8).
    int koff[S::NKK];
#pragma unroll
    for (int kk = 0; kk < S::NKK; ++kk) {
        const int cch = 2 * kk + hh;
        koff[kk] = cch < S::NCH ? krow * S::RB + S::swz(krow, cch) * 16 : 0;
    }
    // V operand (A of O^T += V^T P^T) for d block db via ds_read_b64_tr_b16:
    // lane (group tg, index ti) addresses row 8*(tg>>1) + 4*rr + ti/4 and the
    // 8-byte chunk 8*db + 4*(tg&1) + ti%4 (clamped into the row when D = 24/16;
    // those lanes' results are replaced by the ones rows).
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

    auto kop = [&](const char* stage, int ten, int st, int kk) -> v8 {
        if (2 * kk + hh >= S::NCH) return BIAS ? unit8 : zero8;  // D = 24: dims [24, 32)
        return *reinterpret_cast<const v8*>(stage + ten * S::TILE + st * 32 * S::RB + koff[kk]);
    };
    auto vop = [&](const char* stage, int ten, int st, int cc, int db) -> v8 {
        const int d = db * 32 + (lane & 31);
        s4 half[2];
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
            const char* ptr = stage + ten * S::TILE + (st * 32 + 16 * cc) * S::RB + voffv[db][rr];
            half[rr] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)(ptr));
        }
        // Whole-vector bitcast: element-wise i16 -> bf16 inserts are mis-lowered.
        const v8 r8 = __builtin_bit_cast(v8, __builtin_shufflevector(half[0], half[1], 0, 1, 2, 3, 4, 5, 6, 7));
        if constexpr (D % 32 == 0) return r8;
        return d < D ? r8 : one8;
    };
    // S^T of one subtile for pathway pw from preloaded K operands.
    auto qk = [&](const v8* ka, int pw) -> f32x16 {
        f32x16 sv;
#pragma unroll
        for (int i = 0; i < 16; ++i) sv[i] = 0.f;
#pragma unroll
        for (int kk = 0; kk < S::NKK; ++kk) sv = E::mma(ka[kk], qf[pw][kk], sv);
        if constexpr (BIAS && D != 24) sv = E::mma(kbias, qbias, sv);
        return sv;
    };

    // Reference-max update. `rel` is this lane half's max of s2 - m_ref over
    // the new logits. Rescales (rarely) when a row max exceeds the reference
    // by 2^8; the first stage only sets the reference. Returns true if m_ref
    // moved, with `shift` = new - old (BIAS logits must subtract it).
    auto update = [&](float rel, float& shift) -> bool {
        shift = 0.f;
        const bool need = !started || rel > 8.0f;
        if (__builtin_amdgcn_ballot_w64(need) == 0) return false;
        const float ra = fmaxf(rel, __shfl_xor(rel, 32));
        const bool upd = !started || ra > 8.0f;
        float m_new = upd ? m_ref + ra : m_ref;
        if constexpr (BIAS) m_new = (float)(T)m_new;
        shift = m_new - m_ref;
        const float alpha = started ? fast_exp2(-shift) : 0.f;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < S::NDB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
        m_ref = m_new;
        started = true;
        if constexpr (BIAS) set_bias();
        return true;
    };

    // One pathway over NS consecutive subtiles starting at subtile st0.
    auto pure = [&](auto pw_c, auto ns_c, const char* stage, int st0) {
        constexpr int pw = decltype(pw_c)::value;
        constexpr int NS = decltype(ns_c)::value;
        // All LDS operands of the step are read up front: the V reads then
        // overlap the softmax.
        v8 ka[NS][S::NKK], va[NS][2][S::NDB];
#pragma unroll
        for (int st = 0; st < NS; ++st)
#pragma unroll
            for (int kk = 0; kk < S::NKK; ++kk) ka[st][kk] = kop(stage, pw, st0 + st, kk);
#pragma unroll
        for (int st = 0; st < NS; ++st)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                for (int db = 0; db < S::NDB; ++db) va[st][cc][db] = vop(stage, 2 + pw, st0 + st, cc, db);
        f32x16 sv[NS];
#pragma unroll
        for (int st = 0; st < NS; ++st) sv[st] = qk(ka[st], pw);
        float mx = sv[0][0];
#pragma unroll
        for (int st = 0; st < NS; ++st)
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sv[st][i]);
        float shift;
        const bool moved = update(BIAS ? mx : fmaf(mx, c, -m_ref), shift);
        if constexpr (BIAS) {
            if (moved) {
#pragma unroll
                for (int st = 0; st < NS; ++st)
#pragma unroll
                    for (int i = 0; i < 16; ++i) sv[st][i] -= shift;
            }
        }
        const float mc = m_ref;
#pragma unroll
        for (int st = 0; st < NS; ++st) {
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                float pr[8];
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    pr[t] = fast_exp2(BIAS ? sv[st][8 * cc + t] : fmaf(sv[st][8 * cc + t], c, -mc));
                const v8 pb = pack8<T>(pr);
                if constexpr (!S::SUM_MFMA) {
#pragma unroll
                    for (int t = 0; t < 8; t += 2) l_run = E::sum2(v2{pb[t], pb[t + 1]}, l_run);
                }
#pragma unroll
                for (int db = 0; db < S::NDB; ++db) o[db] = E::mma(va[st][cc][db], pb, o[db]);
            }
        }
    };

    // Both pathways on one subtile, selected per element; handles padded keys.
    auto general = [&](const char* stage, const int* cid, int st, int k0) {
        v8 ks[S::NKK], km[S::NKK];
#pragma unroll
        for (int kk = 0; kk < S::NKK; ++kk) {
            ks[kk] = kop(stage, 0, st, kk);
            km[kk] = kop(stage, 1, st, kk);
        }
        const f32x16 ss = qk(ks, 0), sm = qk(km, 1);
        f32x16 sv;
        bool same[16];
        // keys of slot i: st*32 + 16*(i/8) + 8*hh + i%8
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
                sv[i] = ck == kPadChain ? -INFINITY : v;
            }
        }
        float mx = sv[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) mx = fmaxf(mx, sv[i]);
        float shift;
        const bool moved = update(BIAS ? mx : fmaf(mx, c, -m_ref), shift);
        if constexpr (BIAS) {
            if (moved) {
#pragma unroll
                for (int i = 0; i < 16; ++i) sv[i] -= shift;
            }
        }
        const float mc = m_ref;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            v8 ps, pm;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int i = 8 * cc + t;
                const T pv = (T)fast_exp2(BIAS ? sv[i] : fmaf(sv[i], c, -mc));
                ps[t] = same[i] ? pv : (T)0.f;
                pm[t] = same[i] ? (T)0.f : pv;
            }
            if constexpr (!S::SUM_MFMA) {
#pragma unroll
                for (int t = 0; t < 8; t += 2) {
                    l_run = E::sum2(v2{ps[t], ps[t + 1]}, l_run);
                    l_run = E::sum2(v2{pm[t], pm[t + 1]}, l_run);
                }
            }
#pragma unroll
            for (int db = 0; db < S::NDB; ++db) {
                o[db] = E::mma(vop(stage, 2, st, cc, db), ps, o[db]);
                o[db] = E::mma(vop(stage, 3, st, cc, db), pm, o[db]);
            }
        }
    };

    auto subtile_mode = [&](int kmin, int kmax, int npad) {
        // 0: pure self, 1: pure multimer, 2: general, 3: skip (all padded)
        if (npad == 32) return 3;
        if (!DENSE && npad == 0) {
            if (kmin == kmax && cq_min == cq_max && kmin == cq_min) return 0;
            if (kmax < cq_min || kmin > cq_max) return 1;
        }
        return 2;
    };

    // Pathway codes of 64 consecutive 32-key subtiles starting at kb0, as two
    // bit masks (bit k of mlo / mhi = low / high bit of subtile kb0 + k).
    uint64_t mlo = 0, mhi = 0;
    auto load_modes = [&](int kb0) {
        const int kb = kb0 + lane;
        int code = 3;
        if (kb < Lp / 32) {
            const int4 sm = ksum_b[kb];
            code = subtile_mode(sm.x, sm.y, sm.z);
        }
        mlo = __builtin_amdgcn_ballot_w64(code & 1);
        mhi = __builtin_amdgcn_ballot_w64((code >> 1) & 1);
    };

    // ---- main loop over stages ----
    const int nst = (L + kBN - 1) / kBN;
    load_modes(0);  // before any copy is in flight (its wait drains vmcnt)
#pragma unroll
    for (int t = 0; t < NBUF - 1; ++t)
        if (t < nst) issue(t, t);
    for (int s = 0; s < nst; ++s) {
        const int bf = s % NBUF;
        if constexpr (NBUF == 3) {
            if (s + 1 < nst) wait_vm<IPW>();
            else wait_vm<0>();
        } else {
            wait_vm<0>();
        }
        stage_barrier();
        if (s + NBUF - 1 < nst) issue(s + NBUF - 1, (s + NBUF - 1) % NBUF);

        if (s > 0 && (s & 31) == 0) load_modes(2 * s);
        const int sub = (2 * s) & 63;
        const int m0 = (int)((mlo >> sub) & 1) | (int)(((mhi >> sub) & 1) << 1);
        const int m1 = (int)((mlo >> (sub + 1)) & 1) | (int)(((mhi >> (sub + 1)) & 1) << 1);
        const char* stage = smem + bf * S::STAGE;
        const int* cid = &scid[wave][bf][0];
        const int k0 = s * kBN;
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        if (m0 == 0 && m1 == 0) {
            pure(I0{}, I2{}, stage, 0);
        } else if (m0 == 1 && m1 == 1) {
            pure(I1{}, I2{}, stage, 0);
        } else {
            if (m0 == 0) pure(I0{}, I1{}, stage, 0);
            else if (m0 == 1) pure(I1{}, I1{}, stage, 0);
            else if (m0 == 2) general(stage, cid, 0, k0);
            if (m1 == 0) pure(I0{}, I1{}, stage, 1);
            else if (m1 == 1) pure(I1{}, I1{}, stage, 1);
            else if (m1 == 2) general(stage, cid, 1, k0);
        }
    }

    // ---- epilogue: normalise, store O and LSE ----
    float l_tot;
    if constexpr (S::SUM_MFMA) {
        l_tot = o[0][S::ISUM];
    } else {
        l_tot = l_run + __shfl_xor(l_run, 32);
    }
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
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
                l_tot > 0.f ? (m_ref + __log2f(l_tot)) * kLn2 : -INFINITY;
        }
    }
}

template <typename T, int D, bool ROPE, bool DENSE>
static hipError_t launch_fwd(FwdArgs& a, hipStream_t stream) {
    constexpr int W = 4;
    constexpr int NBUF = D <= 32 ? MPATTN_FWD_NBUF32 : 2;
    const mpattn_fwd_params& p = a.p;
    const int Lp = round_up(p.L, kBN);
    a.Lp = Lp;
    const FwdWs ws = fwd_ws_layout(p.B, p.H, p.L, D, sizeof(T), ROPE);
    char* wsb = (char*)p.workspace;
    int* keff = (int*)(wsb + ws.keff);
    int* ksum = (int*)(wsb + ws.ksum);
    T* krot = (T*)(wsb + ws.krot);
    a.keff = keff;
    a.ksum = ksum;
    a.krot = krot;
    const int nchain = (p.B * (Lp / 64) + 3) / 4;
    constexpr int NPC = ((D / 2) % 8 == 0) ? D / 16 : 1;
    const int64_t nrot = ROPE ? ((int64_t)p.B * p.H * Lp * NPC + 255) / 256 : 0;
    hipLaunchKernelGGL((fwd_prep_kernel<T, D, ROPE, DENSE>), dim3((unsigned)(nchain + nrot)), dim3(256), 0,
                       stream, p, keff, ksum, krot, Lp, nchain);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int nqb = (p.L + 32 * W - 1) / (32 * W);
    const int64_t grid = (int64_t)p.B * p.H * nqb;
    hipLaunchKernelGGL((fwd_kernel<T, D, W, NBUF, ROPE, DENSE>), dim3((unsigned)grid), dim3(W * 64), 0,
                       stream, a);
    return hipGetLastError();
}

template <typename T, int D>
static hipError_t dispatch_fwd_d(FwdArgs& a, hipStream_t s) {
    const bool rope = a.p.rope == MPATTN_ROPE_FUSED;
    const bool dense = a.p.chain_mask != nullptr;
    if (rope) return dense ? launch_fwd<T, D, true, true>(a, s) : launch_fwd<T, D, true, false>(a, s);
    return dense ? launch_fwd<T, D, false, true>(a, s) : launch_fwd<T, D, false, false>(a, s);
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
    const bool fused = p.rope == MPATTN_ROPE_FUSED;
    a.qmul = fused ? p.scale * kLog2e : 1.0f;
    a.c = fused ? 1.0f : p.scale * kLog2e;
    if (p.dtype == MPATTN_BF16) return dispatch_fwd_t<bf16_t>(a, stream);
    return dispatch_fwd_t<fp16_t>(a, stream);
}

}  // namespace mpattn
