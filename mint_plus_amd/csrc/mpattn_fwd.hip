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
//    global_load_lds (16 bytes per lane, straight into LDS); all four are
//    copied (skipping the tiles no wavefront needs saved L2 reads but cost
//    more in branches than it saved). Copies run NBUF-1 stages ahead; one
//    barrier per stage. Rows are stored densely with
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
//    reference m_ref = 0. A stage whose row sum exceeds 2^64 (fp16: 2^15),
//    or leaves the row's running sum at 0 (fp16: at most 2^-6, below which
//    its probabilities are subnormal), takes a rare fix-up path that recomputes
//    it against the stage's max and moves m_ref (the wavefront then
//    subtracts m_ref with one FMA per logit).
//  * Row sums add the fp32 probabilities with VALU adds (v_dot2 would share
//    the matrix-core issue path and serialise with the MFMAs).
#include <type_traits>

#include "mpattn_common.h"

namespace mpattn {

constexpr int kBN = 64;  // keys per LDS stage

inline int round_up(int x, int m) { return (x + m - 1) / m * m; }

// Workspace layout (offsets 256-byte aligned):
//   keff int32 [B][Lp]          effective chain id per key
//   ksum int32 [B][Lp/32][4]    keys: min chain, max chain (valid keys), #padded,
//                               1 if the padded keys are a suffix of the 32
//   qsum int32 [B][Lp/32][4]    queries: min chain, max chain (queries < L), 0, 0
//   krot T     [B][H][Lp][D]    RoPE-rotated K_self (fused RoPE only)
//   mcode u8   [B][Lp/32][Lp/32] dense mask: code of each 32 x 32 block
//   label int32 [B][L]          dense mask: label of each row, the first key
//                               on its chain (min{j : mask[b, i, j] == 0})
//   valid int32 [B + 1]         dense mask: 1 when row b of the mask is the
//                               "different chain" relation of those labels;
//                               valid[B] = 1 when some row is not
struct FwdWs {
    int64_t keff, ksum, qsum, krot, mcode, label, valid, total;
};

inline FwdWs fwd_ws_layout(int B, int H, int L, int D, int esize, bool rope) {
    const int64_t Lp = round_up(L, kBN);
    auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
    FwdWs w;
    w.keff = 0;
    w.ksum = al(w.keff + (int64_t)B * Lp * 4);
    w.qsum = al(w.ksum + (int64_t)B * (Lp / 32) * 16);
    w.krot = al(w.qsum + (int64_t)B * (Lp / 32) * 16);
    w.mcode = al(w.krot + (rope ? (int64_t)B * H * Lp * D * esize : 0));
    w.label = al(w.mcode + (int64_t)B * (Lp / 32) * (Lp / 32));
    w.valid = al(w.label + (int64_t)B * L * 4);
    w.total = al(w.valid + (int64_t)(B + 1) * 4);
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
    DropCfg drop;  // attention dropout (DROP kernels)
    const uint8_t* mcode;  // dense mask block codes (0 all same chain, 1 all different, 2 mixed)
    int mvec;      // dense mask rows readable as aligned 8-byte words
    const int* gate;  // per-batch-row flags (dense masks): run only the rows whose
    int gate_want;    // flag != 0 equals gate_want; null: run every row. With
                      // gate_want == 0, gate[B] != 0 says that some row runs.
};

// ---------------------------------------------------------------------------
// Dense masks: row labels. One wavefront per mask row (b, i < L): the label
// is the first key j with mask[b, i, j] == 0 (the first key on i's chain
// when the mask is a chain partition; L when the row has none). Also sets
// valid[b] = 1, which the check below (or the forward's prep kernel, in the
// same pass as the block codes) clears when a mask entry disagrees.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mask_label_kernel(const uint8_t* mask, int64_t msb, int64_t msq, int64_t msk,
                                                         int B, int L, int* label, int* valid, int vec) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= (int64_t)B * L) return;
    const int b = (int)(row / L), i = (int)(row % L);
    if (i == 0 && lane == 0) {
        valid[b] = 1;
        if (b == 0) valid[B] = 0;
    }
    const uint8_t* r = mask + (int64_t)b * msb + (int64_t)i * msq;
    int lab = L;
    for (int j0 = 0; j0 < L; j0 += 64 * 8) {
        const int j = j0 + lane * 8;
        int first = INT32_MAX;
        if (vec && j + 8 <= L) {
            const uint64_t w = *reinterpret_cast<const uint64_t*>(r + j);
#pragma unroll
            for (int t = 7; t >= 0; --t)
                if (((w >> (8 * t)) & 0xff) == 0) first = j + t;
        } else {
            for (int t = 7; t >= 0; --t)
                if (j + t < L && r[(int64_t)(j + t) * msk] == 0) first = j + t;
        }
        const int m = wave_min_i(first);
        if (m != INT32_MAX) {
            lab = m;
            break;
        }
    }
    if (lane == 0) label[row] = lab;
}

// Check of a dense mask against its row labels: one wavefront per 32 x 32
// block (lane: query row lane/2, 16 keys); valid[b] = 0 when some entry
// with query and key < L differs from (label[q] != label[k]).
__global__ __launch_bounds__(256) void mask_verify_kernel(const uint8_t* mask, int64_t msb, int64_t msq, int64_t msk,
                                                          int B, int L, const int* label, int* valid, int vec) {
    const int lane = threadIdx.x & 63;
    const int nb = (L + 31) / 32;
    const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= (int64_t)B * nb * nb) return;
    const int b = (int)(blk / ((int64_t)nb * nb));
    const int rem = (int)(blk % ((int64_t)nb * nb));
    const int q = (rem / nb) * 32 + (lane >> 1), k0 = (rem % nb) * 32 + (lane & 1) * 16;
    bool bad = false;
    if (q < L) {
        const uint8_t* row = mask + (int64_t)b * msb + (int64_t)q * msq;
        const int* lb = label + (int64_t)b * L;
        const int lq = lb[q];
        if (vec && k0 + 16 <= L) {
            const uint64_t w0 = *reinterpret_cast<const uint64_t*>(row + k0);
            const uint64_t w1 = *reinterpret_cast<const uint64_t*>(row + k0 + 8);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const bool v0 = ((w0 >> (8 * t)) & 0xff) != 0, v1 = ((w1 >> (8 * t)) & 0xff) != 0;
                bad = bad || v0 != (lb[k0 + t] != lq) || v1 != (lb[k0 + 8 + t] != lq);
            }
        } else {
            for (int t = 0; t < 16; ++t)
                if (k0 + t < L) bad = bad || (row[(int64_t)(k0 + t) * msk] != 0) != (lb[k0 + t] != lq);
        }
    }
    if (__builtin_amdgcn_ballot_w64(bad) != 0 && lane == 0) {
        valid[b] = 0;
        valid[B] = 1;
    }
}

hipError_t launch_mask_labels(const uint8_t* mask, int64_t msb, int64_t msq, int64_t msk, int B, int L, int* label,
                              int* valid, int vec, bool verify, hipStream_t stream) {
    hipLaunchKernelGGL(mask_label_kernel, dim3((unsigned)(((int64_t)B * L + 3) / 4)), dim3(256), 0, stream, mask, msb,
                       msq, msk, B, L, label, valid, vec);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !verify) return e;
    const int64_t nb = (L + 31) / 32;
    hipLaunchKernelGGL(mask_verify_kernel, dim3((unsigned)((B * nb * nb + 3) / 4)), dim3(256), 0, stream, mask, msb,
                       msq, msk, B, L, (const int*)label, valid, vec);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Prep: chain staging (blocks [0, nchain)) and K_self rotation (the rest).
// ---------------------------------------------------------------------------
template <typename T, int D, bool ROPE, bool DENSE>
__global__ __launch_bounds__(256) void fwd_prep_kernel(const mpattn_fwd_params p, int* keff,
                                                       int* ksum, int* qsum, T* krot, int Lp, int nchain,
                                                       uint8_t* mcode, int64_t nrot, const int* label,
                                                       int* valid) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int L = p.L;
    if constexpr (DENSE) {
        if ((int64_t)blockIdx.x >= nchain + nrot) {
            // Dense mask: one wave per 32 x 32 block (lane: query row lane/2,
            // 16 keys), code 0 if every entry with query and key < L is 0
            // (same chain), 1 if every one is nonzero, 2 if mixed.
            const int nb = Lp / 32;
            const int64_t blk = ((int64_t)blockIdx.x - nchain - nrot) * 4 + wave;
            if (blk >= (int64_t)p.B * nb * nb) return;
            const int b = (int)(blk / ((int64_t)nb * nb));
            const int rem = (int)(blk % ((int64_t)nb * nb));
            const int q = (rem / nb) * 32 + (lane >> 1), k0 = (rem % nb) * 32 + (lane & 1) * 16;
            // With row labels, each entry is also checked against them:
            // mask != 0 exactly when the labels differ.
            bool any1 = false, any0 = false, bad = false;
            if (q < L) {
                const uint8_t* row = p.chain_mask + (int64_t)b * p.mask_stride_b + (int64_t)q * p.mask_stride_q;
                const bool vec = p.mask_stride_k == 1 && ((uintptr_t)p.chain_mask & 7) == 0 &&
                                 (p.mask_stride_b & 7) == 0 && (p.mask_stride_q & 7) == 0;
                const int* lb = label ? label + (int64_t)b * L : nullptr;
                const int lq = lb ? lb[q] : 0;
                if (vec && k0 + 16 <= L) {
                    const uint64_t w0 = *reinterpret_cast<const uint64_t*>(row + k0);
                    const uint64_t w1 = *reinterpret_cast<const uint64_t*>(row + k0 + 8);
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        const bool v0 = ((w0 >> (8 * t)) & 0xff) != 0, v1 = ((w1 >> (8 * t)) & 0xff) != 0;
                        any1 = any1 || v0 || v1;
                        any0 = any0 || !v0 || !v1;
                        if (lb) bad = bad || v0 != (lb[k0 + t] != lq) || v1 != (lb[k0 + 8 + t] != lq);
                    }
                } else {
                    for (int t = 0; t < 16; ++t)
                        if (k0 + t < L) {
                            const bool v = row[(int64_t)(k0 + t) * p.mask_stride_k] != 0;
                            any1 = any1 || v;
                            any0 = any0 || !v;
                            if (lb) bad = bad || v != (lb[k0 + t] != lq);
                        }
                }
            }
            const bool a1 = __builtin_amdgcn_ballot_w64(any1) != 0, a0 = __builtin_amdgcn_ballot_w64(any0) != 0;
            if (lane == 0) mcode[blk] = a1 ? (a0 ? 2 : 1) : 0;
            if (__builtin_amdgcn_ballot_w64(bad) != 0 && lane == 0) {
                valid[b] = 0;
                valid[p.B] = 1;
            }
            return;
        }
    }
    if ((int)blockIdx.x < nchain) {
        const int ngrp = Lp / 64;
        const int gid = blockIdx.x * 4 + wave;
        if (gid >= p.B * ngrp) return;
        const int b = gid / ngrp, k0 = (gid % ngrp) * 64;
        const int kg = k0 + lane;
        // (dense masks: the row labels stand in for chain ids)
        const int chain = kg >= L ? 0 : !DENSE ? p.chain_id[(int64_t)b * L + kg] : label ? label[(int64_t)b * L + kg] : 0;
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
            const unsigned pm = (unsigned)(hh ? (padm >> 32) : (padm & 0xffffffffull));
            const int np = __popc(pm);
            o[2] = np;
            // 1 when the padded keys are the last np keys of the 32
            o[3] = (np > 0 && np < 32 && pm == (0xffffffffu << (32 - np))) ? 1 : 0;
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
                    lo[u] = rope_rot(x[u], y[u], cr[u], sr[u], true);
                    hi[u] = rope_rot(y[u], x[u], cr[u], sr[u], false);
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
};

#ifndef MPATTN_FWD_QB
// 32-query blocks per wavefront for D <= 32. Two blocks halve the per-stage
// bookkeeping, barriers and LDS operand reads per flop and let the logits of
// one block be computed on the matrix cores while the other block's softmax
// runs on the VALU; the register budget is then 2 wavefronts per SIMD.
#define MPATTN_FWD_QB 1
#endif
#ifndef MPATTN_FWD_NBUF
#define MPATTN_FWD_NBUF 2  // LDS stages in the copy ring (copies run NBUF-1 stages ahead)
#endif

// Launch shape per head dim: W wavefronts per workgroup, QB query blocks per
// wavefront, WPE wavefronts per SIMD (the register budget).
template <int D> struct FwdCfg {
    static constexpr int QB = D == 64 ? 1 : MPATTN_FWD_QB;
    static constexpr int W = QB == 1 ? (D == 64 ? 4 : 8) : 4;
    static constexpr int WPE = QB == 1 ? 4 : 2;
};

// Row sums above this bound (or not finite) send a stage through the fix-up
// path, which moves the row's reference max. 2^64 keeps every partial sum and
// accumulator far from fp32 overflow; for fp16, 2^15 keeps every probability
// (each at most the sum) inside the fp16 range (max 65504) when it is
// rounded for the PV MFMA.
template <typename T> constexpr float sum_hi() {
    return std::is_same<T, fp16_t>::value ? 32768.0f : 18446744073709551616.0f;
}
// fp16 probabilities lose precision below 2^-14 (subnormal) and overflow past
// 65504: a row whose accumulated sum is still at most 2^-6 also takes the
// fix-up, which then lowers the reference toward the row's logits. (bf16
// shares fp32's exponent range: only an empty sum is sent there.)
template <typename T> constexpr float sum_lo() { return std::is_same<T, fp16_t>::value ? 0.015625f : 0.0f; }

template <int N> using IC = std::integral_constant<int, N>;

// Calls f(IC<0>{}), ..., f(IC<N-1>{}): per-block state is indexed by compile-
// time constants only, so it stays in registers.
template <int N, typename F> __device__ __forceinline__ void for_blocks(F&& f) {
    if constexpr (N > 0) {
        for_blocks<N - 1>(f);
        f(IC<N - 1>{});
    }
}

// SQRT: sqrt-softmax, O = sum_j sqrt(P_ij) V_j. The kernel then works with
// e = exp2(s2 / 2) (the 1/2 is folded into the logit factor), accumulates
// sum e V and sum e^2, and divides by sqrt(sum e^2) at the end.
// DROP: attention dropout; the PV operand takes the kept probabilities, the
// row sums all of them, and O is scaled by 1 / (1 - p) at the end.
template <typename T, int D, int W, int QB, int WPE, int NBUF, bool ROPE, bool DENSE, bool SQRT, bool DROP>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(WPE)))
void fwd_kernel(const FwdArgs args) {
    using S = FwdShape<D>;
    using E = Elt<T>;
    typedef typename E::v8 v8;
    typedef typename E::v2 v2;
    typedef short s4 __attribute__((ext_vector_type(4)));
    static_assert(NBUF >= 2 && NBUF <= 4, "LDS stages in flight");
    static_assert(QB == 1 || QB == 2, "query blocks per wavefront");
    constexpr int QW = 32 * QB;              // queries per wavefront
    constexpr int TOT = 4 * S::NI;           // DMA wave-instructions per full stage
    constexpr int NJ = (TOT + W - 1) / W;    // per wavefront (the last may be idle)
    // With fused RoPE the logit factor scale*log2(e) is folded into Q.
    constexpr bool FOLDED = ROPE;
    constexpr float kSumLo = sum_lo<T>();
    constexpr float kSumHi = sum_hi<T>();
    const mpattn_fwd_params& p = args.p;

    __shared__ __attribute__((aligned(1024))) char smem[NBUF * S::STAGE];
    // effective chain ids of each stage's keys (one copy per workgroup, by
    // its last wavefront, which has the fewest tile copies)
    __shared__ __attribute__((aligned(16))) int scid[NBUF][kBN];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ql = lane & 31, hh = lane >> 5;
    const int L = p.L, H = p.H, Lp = args.Lp;
    const int nqb = (L + QW * W - 1) / (QW * W);
    // Gated launch (dense masks): a launch with no batch row to run ends
    // before any other work.
    if (args.gate) {
        if (args.gate_want == 0) {
            if (args.gate[p.B] == 0) return;  // every row is a partition (one scalar load)
        } else {
            bool any = false;
            for (int b0 = 0; b0 < p.B; b0 += 64)
                any = any || __builtin_amdgcn_ballot_w64(b0 + lane < p.B && args.gate[b0 + lane] != 0) != 0;
            if (!any) return;
        }
    }
    // Query blocks whose rows straddle a chain boundary are dispatched first.
    int qb, bh;
    dispatch_order(nqb, H, DENSE ? nullptr : reinterpret_cast<const int4*>(args.qsum), Lp / 32,
                   (L + 31) / 32, QB * W, false, (int64_t)4 * L * D * sizeof(T), 2 << 20, qb, bh);
    const int b = bh / H, h = bh % H;
    if (args.gate && (args.gate[b] != 0) != (args.gate_want != 0)) return;  // (uniform)
    const int qw0 = qb * QW * W;    // first query of the workgroup
    const int qv0 = qw0 + wave * QW;  // first query of this wavefront
    int qrow[QB];
    bool qvalid[QB];
#pragma unroll
    for (int u = 0; u < QB; ++u) {
        qrow[u] = qv0 + 32 * u + ql;
        qvalid[u] = qrow[u] < L;
    }
    uint32_t drow[QB];  // dropout row hashes
#pragma unroll
    for (int u = 0; u < QB; ++u) drow[u] = DROP ? drop_row(args.drop.lo, (uint32_t)bh, (uint32_t)qrow[u]) : 0u;

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
    // When W divides a tile's instruction count, copy j's tile is j*W/NI for
    // every wavefront (a compile-time constant).
    constexpr bool TSTAT = S::NI % W == 0;
    const char* dsb[NJ];  // (b, h) base of the source tensor (uniform)
    unsigned dstr[NJ];    // row stride in bytes (uniform)
    unsigned dlds[NJ];    // LDS offset inside a stage (uniform)
    unsigned dvo[NJ];     // per-lane byte offset of (r, c) from the stage's first row
    int dten[NJ];         // tile index, 4 for an idle copy (uniform)
    // (row, swizzled byte column) of copy j for lane `ln`
    auto dma_rc = [&](int j, int ln, int& r, int& cb) {
        const int ins0 = wave + j * W;
        const int part = (ins0 < TOT ? ins0 : TOT - 1) % S::NI;
        const int slot = part * 64 + ln;
        r = slot / S::NCH;
        cb = S::swz(r, slot % S::NCH) * 16;  // swz is an involution on the chunk index
    };
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int ins0 = wave + j * W;
        const int ins = ins0 < TOT ? ins0 : TOT - 1;
        const int ten = TSTAT ? j * W / S::NI : ins / S::NI;
        const int part = TSTAT ? j * W % S::NI + wave : ins % S::NI;
        int r, cb;
        dma_rc(j, lane, r, cb);
        const T* tb = ten == 0 ? ks_p : ten == 1 ? km_p : ten == 2 ? vs_p : vm_p;
        const int64_t ts = ten == 0 ? ks_t : ten == 1 ? km_t : ten == 2 ? vs_t : vm_t;
        dsb[j] = (const char*)tb;
        dstr[j] = (unsigned)(ts * (int64_t)sizeof(T));
        dlds[j] = ten * S::TILE + part * 1024;
        dvo[j] = r * dstr[j] + cb;
        dten[j] = ins0 < TOT ? ten : 4;
    }
    const char* const keff_c = reinterpret_cast<const char*>(keff_b);
    const unsigned smem_base = lds_addr(smem);
    const unsigned scid_base = lds_addr(&scid[0][0]);
    const bool cidw = wave == W - 1;  // (uniform)

    // ---- copy stage s into buffer bf ----
    // Returns the number of vector-memory instructions issued (uniform).
    // Sources are a uniform 64-bit base (the stage's first row, advanced by
    // scalar adds) plus a per-lane 32-bit offset inside the stage's 64 rows:
    // no per-lane address arithmetic per stage.
    auto issue = [&](int s, int bf) -> int {
        const int k0 = s * kBN;
        const unsigned lb = smem_base + bf * S::STAGE;
        // Each branch issues its own copies (no register merge of the offsets).
        auto copies = [&](const unsigned* vo) {
            const int m0v = m0_save();
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                if (TOT % W == 0 || dten[j] < 4)  // (idle copies of the last round)
                    dma16(dsb[j] + (int64_t)k0 * dstr[j], vo[j], lb + dlds[j]);
            if (cidw) dma4(keff_c + k0 * 4, (unsigned)lane * 4, scid_base + bf * kBN * 4);
            m0_restore(m0v);
        };
        if (k0 + kBN <= L) {
            copies(dvo);
        } else {  // last stage: clamp rows past L to L-1 (their keys are masked)
            unsigned vo[NJ];
            // The lane id comes from an opaque instruction so that (r, cb)
            // are recomputed here instead of occupying registers all loop.
            int ln;
            asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                int r, cb;
                dma_rc(j, ln, r, cb);
                vo[j] = (unsigned)min(r, L - 1 - k0) * dstr[j] + cb;
            }
            copies(vo);
        }
        int n = cidw ? 1 : 0;
#pragma unroll
        for (int j = 0; j < NJ; ++j) n += (TOT % W == 0 || dten[j] < 4) ? 1 : 0;
        return n;
    };

    const int nst = (L + kBN - 1) / kBN;
    int pend[NBUF];
#pragma unroll
    for (int t = 0; t < NBUF; ++t) pend[t] = 0;
    // ---- Q fragments (B operand of S^T = K Q^T): dims kk*16 + 8*hh + [0,8) ----
    // With D/2 a multiple of 8 the raw Q rows (with the RoPE partner chunks
    // and table entries) are loaded first and the stage-0 copy is issued
    // behind them: both are in flight together, and the loads are not queued
    // behind the copy (3-5 % of the call at D = 32 and 64).
    constexpr int H2 = D / 2;
    constexpr bool QEARLY = H2 % 8 == 0;
    v8 qf[QB][2][S::NKK];
    v8 qraw[QB][2][S::NKK], qpar[QB][S::NKK];
    f32x4 qcs[QB][S::NKK][4];
    if constexpr (QEARLY) {
#pragma unroll
        for (int u = 0; u < QB; ++u) {
            const int qr = qvalid[u] ? qrow[u] : 0;
#pragma unroll
            for (int pw = 0; pw < 2; ++pw)
#pragma unroll
                for (int kk = 0; kk < S::NKK; ++kk) {
                    const int d0 = kk * 16 + hh * 8;
                    if (d0 >= D) continue;
                    const T* row = pw == 0 ? qs_p + (int64_t)qr * p.q_self.stride_t
                                           : qm_p + (int64_t)qr * p.q_multi.stride_t;
                    qraw[u][pw][kk] = *reinterpret_cast<const v8*>(row + d0);
                    if (ROPE && pw == 0) {
                        const bool lo = d0 < H2;
                        const int dp = lo ? d0 + H2 : d0 - H2, fi = lo ? d0 : dp;
                        qpar[u][kk] = *reinterpret_cast<const v8*>(row + dp);
                        const float* cr = p.rope_cos + (int64_t)qr * H2 + fi;
                        const float* sr = p.rope_sin + (int64_t)qr * H2 + fi;
                        qcs[u][kk][0] = *reinterpret_cast<const f32x4*>(cr);
                        qcs[u][kk][1] = *reinterpret_cast<const f32x4*>(cr + 4);
                        qcs[u][kk][2] = *reinterpret_cast<const f32x4*>(sr);
                        qcs[u][kk][3] = *reinterpret_cast<const f32x4*>(sr + 4);
                    }
                }
        }
    }
    pend[0] = issue(0, 0);
#pragma unroll
    for (int u = 0; u < QB; ++u)
#pragma unroll
        for (int pw = 0; pw < 2; ++pw)
#pragma unroll
            for (int kk = 0; kk < S::NKK; ++kk) {
                float x[8];
                const int d0 = kk * 16 + hh * 8;
                if (QEARLY) {
                    if (!qvalid[u] || d0 >= D) {
#pragma unroll
                        for (int t = 0; t < 8; ++t) x[t] = 0.f;
                    } else if (ROPE && pw == 0) {
                        const bool lo = d0 < H2;
#pragma unroll
                        for (int t = 0; t < 8; ++t) {
                            const float c = qcs[u][kk][t >> 2][t & 3], sn = qcs[u][kk][2 + (t >> 2)][t & 3];
                            x[t] = rope_rot((float)qraw[u][pw][kk][t], (float)qpar[u][kk][t], c, sn, lo) * args.qmul;
                        }
                    } else {
#pragma unroll
                        for (int t = 0; t < 8; ++t) x[t] = (float)qraw[u][pw][kk][t] * args.qmul;
                    }
                } else if (qvalid[u]) {
                    const T* row = pw == 0 ? qs_p + (int64_t)qrow[u] * p.q_self.stride_t
                                           : qm_p + (int64_t)qrow[u] * p.q_multi.stride_t;
                    load8_rot<T, D>(row, p.rope_cos, p.rope_sin, qrow[u], kk * 16 + hh * 8, args.qmul,
                                    ROPE && pw == 0, x);
                } else {
#pragma unroll
                    for (int t = 0; t < 8; ++t) x[t] = 0.f;
                }
                qf[u][pw][kk] = pack8<T>(x);
            }
    // Query chain range of each block (the prep kernel's per-32-query
    // summaries: uniform loads).
    int cq[QB], cq_min[QB], cq_max[QB];
#pragma unroll
    for (int u = 0; u < QB; ++u) cq[u] = cq_min[u] = cq_max[u] = 0;
    if constexpr (!DENSE) {
#pragma unroll
        for (int u = 0; u < QB; ++u) cq[u] = qvalid[u] ? p.chain_id[(int64_t)b * L + qrow[u]] : 0;
        const int4* qsum_b = reinterpret_cast<const int4*>(args.qsum) + (int64_t)b * (Lp / 32);
#pragma unroll
        for (int u = 0; u < QB; ++u) {
            const int qbk = (qv0 >> 5) + u;  // this block's summary (a block past L reads block 0)
            const int4 qs = qsum_b[qbk < Lp / 32 ? qbk : 0];
            cq_min[u] = qs.x;
            cq_max[u] = qs.y;
        }
#pragma unroll
        for (int u = 0; u < QB; ++u) {
            cq_min[u] = __builtin_amdgcn_readfirstlane(cq_min[u]);
            cq_max[u] = __builtin_amdgcn_readfirstlane(cq_max[u]);
        }
        // A wavefront whose queries span chains runs its subtiles on both
        // pathways, and its workgroup's stage barriers wait for it: it issues
        // ahead of the wavefronts it shares a SIMD with.
        bool qstraddle = false;
#pragma unroll
        for (int u = 0; u < QB; ++u) qstraddle = qstraddle || cq_min[u] != cq_max[u];
        if (qstraddle) __builtin_amdgcn_s_setprio(3);
    }
    const uint8_t* mrow[QB];
#pragma unroll
    for (int u = 0; u < QB; ++u) {
        mrow[u] = nullptr;
        if constexpr (DENSE)
            mrow[u] = p.chain_mask + (int64_t)b * p.mask_stride_b +
                      (int64_t)(qvalid[u] ? qrow[u] : 0) * p.mask_stride_q;
    }
    // Dense mask: each lane's mask bytes of a stage (8 keys per subtile half)
    // are loaded one stage ahead, before the next copy is issued, and land
    // by the compiler-visible wait at the top of the stage that reads them.
    constexpr bool DMP = DENSE && NBUF == 2;
    uint64_t mcur[QB][2][2], mnxt[QB][2][2];
    auto mload = [&](int s, uint64_t (*m)[2][2]) {
#pragma unroll
        for (int u = 0; u < QB; ++u)
#pragma unroll
            for (int st = 0; st < 2; ++st)
#pragma unroll
                for (int cc = 0; cc < 2; ++cc) {
                    const int kg = s * kBN + st * 32 + 16 * cc + 8 * hh;
                    uint64_t w = 0;
                    if (args.mvec && kg + 8 <= L) {
                        w = *reinterpret_cast<const uint64_t*>(mrow[u] + kg);
                    } else {
                        for (int t = 0; t < 8; ++t)
                            if (kg + t < L && mrow[u][(int64_t)(kg + t) * p.mask_stride_k] != 0)
                                w |= 0xffull << (8 * t);
                    }
                    m[u][st][cc] = w;
                }
    };

    // ---- softmax state, per query block ----
    // Probabilities are exp2(s2 - m_ref) with s2 = c * s the base-2 logit.
    // m_ref starts at 0 and stays there unless a stage's row sum leaves
    // (0, 2^64]: then the fix-up path sets it from that stage's max and the
    // block switches to the shifted form (one FMA per logit).
    const float c = args.c;  // 1 when FOLDED
    float m_ref[QB], l_run[QB];
    bool shifted[QB];         // wavefront-uniform: some m_ref != 0
    f32x16 o[QB][S::NDB];
#pragma unroll
    for (int u = 0; u < QB; ++u) {
        m_ref[u] = 0.f;
        l_run[u] = 0.f;
        shifted[u] = false;
#pragma unroll
        for (int db = 0; db < S::NDB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[u][db][i] = 0.f;
    }

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

    // Base-2 probability of raw logit x against reference mr.
    auto prob = [&](float x, bool sh, float mr) -> float {
        if (sh) return fast_exp2(fmaf(x, c, -mr));
        return fast_exp2(FOLDED ? x : x * c);
    };
    // Probabilities of NS subtiles (slot 8*cc + t -> pb[st][cc][t]) and their
    // row sum over this lane's keys.
    // kb: key of slot 0 of the first subtile (slot 8*cc + t of subtile st is
    // key kb + 32*st + 16*cc + t); dr: the block's dropout row hash.
    auto probs = [&](auto ns_c, const f32x16* sv, v8 (*pb)[2], bool sh, float mr, int kb,
                     uint32_t dr) -> float {
        constexpr int NS = decltype(ns_c)::value;
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        // Pairs are rounded once (v_cvt_pk) for the PV operand. The row sum
        // adds the fp32 probabilities with plain VALU adds: v_dot2 on the
        // rounded pairs would issue on the matrix-core path and serialise
        // with the MFMAs of the other wavefronts of the SIMD (measured), where
        // adds run under them. Four sum chains keep the dependency depth low.
        float ls[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < NS; ++st)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                v2 pr[4];
#pragma unroll
                for (int uu = 0; uu < 4; ++uu) {
                    const f32x2 f = {prob(sv[st][8 * cc + 2 * uu], sh, mr),
                                     prob(sv[st][8 * cc + 2 * uu + 1], sh, mr)};
                    pr[uu] = __builtin_convertvector(f, v2);
                    if constexpr (SQRT) {
                        ls[uu] = fmaf(f.x, f.x, ls[uu]);
                        ls[uu] = fmaf(f.y, f.y, ls[uu]);
                    } else {
                        ls[uu] += f.x;
                        ls[uu] += f.y;
                    }
                }
                v2 pv[4];
#pragma unroll
                for (int uu = 0; uu < 4; ++uu) pv[uu] = pr[uu];
                if constexpr (DROP) {
                    const int kj = kb + 32 * st + 16 * cc;
#pragma unroll
                    for (int uu = 0; uu < 4; ++uu) {
                        const bool k0 = drop_keep(dr, args.drop.hi, (uint32_t)(kj + 2 * uu), args.drop.thr);
                        const bool k1 = drop_keep(dr, args.drop.hi, (uint32_t)(kj + 2 * uu + 1), args.drop.thr);
                        const uint32_t m = (k0 ? 0x0000FFFFu : 0u) | (k1 ? 0xFFFF0000u : 0u);
                        pv[uu] = __builtin_bit_cast(v2, __builtin_bit_cast(uint32_t, pr[uu]) & m);
                    }
                }
                pb[st][cc] = __builtin_shufflevector(__builtin_shufflevector(pv[0], pv[1], 0, 1, 2, 3),
                                                     __builtin_shufflevector(pv[2], pv[3], 0, 1, 2, 3), 0, 1, 2,
                                                     3, 4, 5, 6, 7);
            }
        return (ls[0] + ls[1]) + (ls[2] + ls[3]);
    };
    // Rare path: a lane's stage sum overflowed, or its row has accumulated
    // nothing yet. The subtile's logits are recomputed from LDS (`logits`
    // fills sv) and its probabilities redone relative to a reference max
    // taken from them (raised only, once something has been accumulated).
    auto fixup = [&](auto u_c, auto logits, v8 (*pb)[2], int kb) -> float {
        constexpr int u = decltype(u_c)::value;
        f32x16 sv[1];
        logits(sv);
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sv[0][i]);
        const float mq = fmaxf(mx, __shfl_xor(mx, 32));  // query max of the subtile, raw units
        const float lq = l_run[u] + __shfl_xor(l_run[u], 32);
        const float ms = mq * c;
        float m_new;
        if (lq > kSumLo) {
            m_new = fmaxf(m_ref[u], ms);  // raise only
        } else if (lq > 0.f) {
            // Small accumulated sum (fp16): every earlier base-2 logit is at
            // most m_ref + log2(lq) (halved for sqrt-softmax, whose sum holds
            // squares), so lowering the reference to that bound keeps the
            // rescaled sum at most 1.
            m_new = fmaxf(ms, m_ref[u] + (SQRT ? 0.5f : 1.0f) * __log2f(lq));
        } else {
            m_new = ms > -INFINITY ? ms : m_ref[u];
        }
        const float alpha = lq > 0.f ? fast_exp2(m_ref[u] - m_new) : 1.0f;
        l_run[u] *= SQRT ? alpha * alpha : alpha;
#pragma unroll
        for (int db = 0; db < S::NDB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[u][db][i] *= alpha;
        m_ref[u] = m_new;
        shifted[u] = __builtin_amdgcn_ballot_w64(m_new != 0.f) != 0;
        return probs(IC<1>{}, sv, pb, true, m_new, kb, drow[u]);
    };
    // Check: true if any lane of block u needs the fix-up.
    auto needs_fix = [&](float ls, float lr) {
        const bool bad = !(ls <= kSumHi) || (lr + ls <= kSumLo);
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

    // Fast-path row sums on the matrix cores (no dropout, no sqrt-softmax):
    // v_mfma_f32_16x16x32 with the probabilities as the B operand (lane l:
    // column l%16, k-group l/16, i.e. query l%32 and key half l/32 of a
    // 16-key chunk) and a 0/1 selector as A (row m, k-group g: 1 iff m is
    // 0 or 8 for even g, 4 or 12 for odd g). Output row 4*(l/16) of lane l
    // (its accumulator slot 0) is then the chunk's sum for query l%32 over
    // both key halves.
    constexpr bool MSUM = !SQRT && !DROP && !DENSE;
    v8 rsel;
    {
        const int sm = lane & 15, sg = lane >> 4;
        const bool one = (sm & 3) == 0 && ((sm >> 2) & 1) == (sg & 1);
#pragma unroll
        for (int t = 0; t < 8; ++t) rsel[t] = one ? (T)1.0f : (T)0.0f;
    }

    // Q operands of the fast path's pathway (changes rarely: at chain edges).
    int cur_pw = 0;
    v8 qcur[QB][S::NKK];
#pragma unroll
    for (int u = 0; u < QB; ++u)
#pragma unroll
        for (int kk = 0; kk < S::NKK; ++kk) qcur[u][kk] = qf[u][0][kk];

    // Fast path: every block and both subtiles of the stage on pathway pw,
    // unshifted softmax. All blocks' logits are issued first so the matrix
    // cores work on block u+1 while the VALU does block u's softmax. Returns
    // the mask of blocks accumulated; a block that needs the fix-up is left
    // to the slow path.
    // MIXED: the two subtiles are on different pathways (pw0, pw1: a chain
    // edge at key 32 of the stage); the Q operands are then selected per
    // subtile instead of taken from qcur.
    auto fast_stage = [&](auto mixed_c, const char* stage, int pw0, int pw1, int k0) -> int {
        constexpr bool MIXED = decltype(mixed_c)::value;
        const char* const kt[2] = {stage + pw0 * S::TILE, stage + pw1 * S::TILE};
        const char* const vt[2] = {stage + (2 + pw0) * S::TILE, stage + (2 + pw1) * S::TILE};
        // All LDS operands are read up front: the V reads overlap the softmax.
        v8 ka[2][S::NKK], va[2][2][S::NDB];
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
            for (int kk = 0; kk < S::NKK; ++kk) ka[st][kk] = kop_t(kt[st], st, kk);
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                for (int db = 0; db < S::NDB; ++db) va[st][cc][db] = vop_t(vt[st], st, cc, db);
        // keep every LDS read of the stage ahead of the softmax
        __builtin_amdgcn_sched_barrier(0);
        f32x16 sv[QB][2];
#pragma unroll
        for (int u = 0; u < QB; ++u)
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                if constexpr (MIXED) {
                    v8 qa[S::NKK];
#pragma unroll
                    for (int kk = 0; kk < S::NKK; ++kk) qa[kk] = (st ? pw1 : pw0) ? qf[u][1][kk] : qf[u][0][kk];
                    sv[u][st] = qkq(ka[st], qa);
                } else {
                    sv[u][st] = qkq(ka[st], qcur[u]);
                }
            }
        int done = 0;
        for_blocks<QB>([&](auto u_c) {
            constexpr int u = decltype(u_c)::value;
            v8 pb[2][2];
            float ls;
            if constexpr (MSUM) {
                // Row sums of the rounded probabilities on the matrix cores
                // (rsel: selector operand): the full 64-key sum of lane's
                // query, booked half per lane half like the VALU sums.
                probs(IC<2>{}, sv[u], pb, false, 0.f, k0 + 8 * hh, drow[u]);
                f32x4 r = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int st = 0; st < 2; ++st)
#pragma unroll
                    for (int cc = 0; cc < 2; ++cc) r = E::mma16(rsel, pb[st][cc], r);
                ls = 0.5f * r[0];
            } else {
                ls = probs(IC<2>{}, sv[u], pb, false, 0.f, k0 + 8 * hh, drow[u]);
            }
            if (needs_fix(ls, l_run[u])) return;
            l_run[u] += ls;
            done |= 1 << u;
#pragma unroll
            for (int st = 0; st < 2; ++st)
#pragma unroll
                for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                    for (int db = 0; db < S::NDB; ++db) o[u][db] = E::mma(va[st][cc][db], pb[st][cc], o[u][db]);
        });
        return done;
    };

    // Both pathways on one subtile of block u, selected per element; handles
    // padded keys.
    auto general = [&](auto u_c, const char* stage, const int* cid, int st, int k0) {
        constexpr int u = decltype(u_c)::value;
        const int kbs = k0 + 32 * st + 8 * hh;
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
            const f32x16 ss = qkq(ks, qf[u][0]), sm = qkq(km, qf[u][1]);
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const int kl = st * 32 + 16 * cc + 8 * hh;
                const i32x4 c0 = *reinterpret_cast<const i32x4*>(&cid[kl]);
                const i32x4 c1 = *reinterpret_cast<const i32x4*>(&cid[kl + 4]);
                uint32_t mbits = 0;
                if constexpr (DMP) {
                    const uint64_t mw = st ? mcur[u][1][cc] : mcur[u][0][cc];
#pragma unroll
                    for (int t = 0; t < 8; ++t) mbits |= (uint32_t)(((mw >> (8 * t)) & 0xffu) != 0) << t;
                } else if constexpr (DENSE) {
                    const int kg = k0 + kl;
                    for (int t = 0; t < 8; ++t)
                        if (kg + t < L)
                            mbits |= (uint32_t)(mrow[u][(int64_t)(kg + t) * p.mask_stride_k] != 0) << t;
                }
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const int ck = t < 4 ? c0[t & 3] : c1[t & 3];
                    const int i = 8 * cc + t;
                    const bool sm_ = DENSE ? !((mbits >> t) & 1u) : (ck == cq[u]);
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
            ls = shifted[u] ? probs(IC<1>{}, sv, pb, true, m_ref[u], kbs, drow[u])
                            : probs(IC<1>{}, sv, pb, false, 0.f, kbs, drow[u]);
        }
        if (needs_fix(ls, l_run[u])) ls = fixup(u_c, logits, pb, kbs);
        l_run[u] += ls;
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
                o[u][db] = E::mma(vop_t(stage + 2 * S::TILE, st, cc, db), ps, o[u][db]);
                o[u][db] = E::mma(vop_t(stage + 3 * S::TILE, st, cc, db), pm, o[u][db]);
            }
        }
    };

    // One subtile of block u on the slow path. code: 0 pure self, 1 pure
    // multimer, 2 straddle (keys on one chain, queries on several: pathway per
    // lane), 3 general, 4 skip, 5 / 6 pure self / multimer with padded keys.
    auto slow_subtile = [&](auto u_c, const char* stage, const int* cid, int st, int code, int k0) {
        constexpr int u = decltype(u_c)::value;
        const int kbs = k0 + 32 * st + 8 * hh;
        if (code == 4) return;
        if (code == 3) {
            general(u_c, stage, cid, st, k0);
            return;
        }
        v8 pb[1][2];
        float ls;
        if (code <= 1 || code >= 5) {
            const bool masked = code >= 5;
            const int pw = masked ? code - 5 : code;
            const char* kt = stage + pw * S::TILE;
            v8 qa[S::NKK];
#pragma unroll
            for (int kk = 0; kk < S::NKK; ++kk) qa[kk] = pw ? qf[u][1][kk] : qf[u][0][kk];
            auto logits = [&](f32x16* sv) {
                v8 kr[S::NKK];
#pragma unroll
                for (int kk = 0; kk < S::NKK; ++kk) kr[kk] = kop_t(kt, st, kk);
                sv[0] = qkq(kr, qa);
                if (masked) {
#pragma unroll
                    for (int cc = 0; cc < 2; ++cc) {
                        const int kl = st * 32 + 16 * cc + 8 * hh;
                        const i32x4 k0v = *reinterpret_cast<const i32x4*>(&cid[kl]);
                        const i32x4 k1v = *reinterpret_cast<const i32x4*>(&cid[kl + 4]);
#pragma unroll
                        for (int t = 0; t < 8; ++t) {
                            const int ck = t < 4 ? k0v[t & 3] : k1v[t & 3];
                            if (ck == kPadChain) sv[0][8 * cc + t] = -INFINITY;
                        }
                    }
                }
            };
            {
                f32x16 sv[1];
                logits(sv);
                ls = shifted[u] ? probs(IC<1>{}, sv, pb, true, m_ref[u], kbs, drow[u])
                                : probs(IC<1>{}, sv, pb, false, 0.f, kbs, drow[u]);
            }
            if (needs_fix(ls, l_run[u])) ls = fixup(u_c, logits, pb, kbs);
            l_run[u] += ls;
            const char* vt = stage + (2 + pw) * S::TILE;
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                for (int db = 0; db < S::NDB; ++db) o[u][db] = E::mma(vop_t(vt, st, cc, db), pb[0][cc], o[u][db]);
            return;
        }
        // straddle: lane is on the self pathway iff its chain is the keys' chain
        const bool self_lane = cq[u] == cid[st * 32];
        auto logits = [&](f32x16* sv) {
            v8 ks[S::NKK], km[S::NKK];
#pragma unroll
            for (int kk = 0; kk < S::NKK; ++kk) {
                ks[kk] = kop_t(stage, st, kk);
                km[kk] = kop_t(stage + S::TILE, st, kk);
            }
            const f32x16 ss = qkq(ks, qf[u][0]), sm = qkq(km, qf[u][1]);
#pragma unroll
            for (int i = 0; i < 16; ++i) sv[0][i] = self_lane ? ss[i] : sm[i];
        };
        {
            f32x16 sv[1];
            logits(sv);
            ls = shifted[u] ? probs(IC<1>{}, sv, pb, true, m_ref[u], kbs, drow[u])
                            : probs(IC<1>{}, sv, pb, false, 0.f, kbs, drow[u]);
        }
        if (needs_fix(ls, l_run[u])) ls = fixup(u_c, logits, pb, kbs);
        l_run[u] += ls;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const v8 ps = self_lane ? pb[0][cc] : zero8;
            const v8 pm = self_lane ? zero8 : pb[0][cc];
#pragma unroll
            for (int db = 0; db < S::NDB; ++db) {
                o[u][db] = E::mma(vop_t(stage + 2 * S::TILE, st, cc, db), ps, o[u][db]);
                o[u][db] = E::mma(vop_t(stage + 3 * S::TILE, st, cc, db), pm, o[u][db]);
            }
        }
    };

    // Codes 5 / 6: pure self / multimer subtile whose padded keys are a
    // suffix (the padding tail): one pathway with the padded keys masked.
    auto subtile_mode = [&](int kmin, int kmax, int npad, int suffix, int qmin, int qmax) -> int {
        if (npad == 32) return 4;
        if (DENSE) return 3;
        if (npad == 0 || suffix) {
            if (kmax < qmin || kmin > qmax) return npad ? 6 : 1;
            if (kmin == kmax && qmin == qmax) return npad ? 5 : 0;
            if (kmin == kmax && npad == 0) return 2;
        }
        return 3;
    };

    // Subtile codes of each block for the 64 subtiles from kb0, as three bit
    // masks per block (mb0..mb2 = code bits). Each reload is a vector load
    // whose wait also drains the copies in flight: windows move once per 32
    // stages.
    uint64_t mb0[QB], mb1[QB], mb2[QB];
    auto ksum_at = [&](int kb0) -> int4 {
        const int kb = kb0 + lane;
        int4 sm = {0, 0, 32, 0};
        if (kb < Lp / 32) sm = ksum_b[kb];
        return sm;
    };
    // Dense mask: the block code of (this block's 32 queries, subtile kbi)
    // from the prep kernel decides the path like the chain summaries do.
    auto dense_mode = [&](const int4 sm, int mc) -> int {
        if (sm.z == 32) return 4;
        if (mc == 2) return 3;
        if (sm.z == 0) return mc ? 1 : 0;
        if (sm.w) return mc ? 6 : 5;
        return 3;
    };
    auto set_codes = [&](const int4 sm, int kbi) {
#pragma unroll
        for (int u = 0; u < QB; ++u) {
            int code;
            if constexpr (DENSE) {
                const int nb = Lp / 32, qbk = (qv0 >> 5) + u;
                const int mc = kbi < nb ? args.mcode[((int64_t)b * nb + (qbk < nb ? qbk : 0)) * nb + kbi] : 2;
                code = dense_mode(sm, mc);
            } else {
                code = subtile_mode(sm.x, sm.y, sm.z, sm.w, cq_min[u], cq_max[u]);
            }
            mb0[u] = __builtin_amdgcn_ballot_w64(code & 1);
            mb1[u] = __builtin_amdgcn_ballot_w64((code >> 1) & 1);
            mb2[u] = __builtin_amdgcn_ballot_w64((code >> 2) & 1);
        }
    };
    // Control words of a window of 32 stages, one per lane (lane t: stage
    // sw0 + t): the codes of the stage's two subtiles for each query block
    // (3 bits each, block u from bit 6u). Built once per window, read with
    // one readlane per stage. A rebuild's summary load waits for the copies
    // in flight; windows move once per 32 stages.
    int ctrl = 0, sw0 = 0;
    auto build_ctrl = [&](int s0) {
        sw0 = s0;
        const int4 sm = ksum_at(2 * s0);  // lane: subtile 2*s0 + lane
        set_codes(sm, 2 * s0 + lane);
        const int t2 = 2 * (lane & 31);
        int w = 0;
#pragma unroll
        for (int u = 0; u < QB; ++u) {
            const int a = (int)((mb0[u] >> t2) & 1) | (int)(((mb1[u] >> t2) & 1) << 1) |
                          (int)(((mb2[u] >> t2) & 1) << 2);
            const int bb = (int)((mb0[u] >> (t2 + 1)) & 1) | (int)(((mb1[u] >> (t2 + 1)) & 1) << 1) |
                           (int)(((mb2[u] >> (t2 + 1)) & 1) << 2);
            w |= (a | bb << 3) << (6 * u);
        }
        ctrl = w;
    };

    // ---- main loop over stages ----
    if constexpr (DMP) mload(0, mcur);
    build_ctrl(0);
    // Every prologue load (Q, chain ids, summaries) and the stage-0 copy have
    // landed here. The compiler sees this wait (the copies are inline asm it
    // cannot see), so it adds no vmcnt(0) at later uses, which would also
    // drain the copies in flight.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    // Stages after the last one with a valid key (every key padded: a skip
    // for every wavefront, since it depends on the keys only) are not run.
    // The first control window decides; longer sequences run every stage.
    // At least stage 0 runs (its copy is in flight).
    int nrun = nst;
    if (nst <= 32) {
        const uint64_t skip = mb2[0] & ~mb1[0] & ~mb0[0];  // code 4 per subtile (lane)
        const uint64_t live = ~skip & (nst >= 32 ? ~0ull : (1ull << (2 * nst)) - 1);
        nrun = live ? (63 - __builtin_clzll(live)) / 2 + 1 : 1;
    }
    pend[0] = 0;
    // pend[k]: vector-memory instructions of stage s + k still in flight
    // (stage 0 was issued before the prologue and has landed).
#pragma unroll
    for (int t = 1; t < NBUF - 1; ++t)
        if (t < nrun) pend[t] = issue(t, t);
    int bf = 0;
    for (int s = 0; s < nrun; ++s) {
        int allow = 0;  // copies of later stages that may stay in flight
#pragma unroll
        for (int k = 1; k < NBUF - 1; ++k) allow += pend[k];
        if constexpr (DMP) __builtin_amdgcn_s_waitcnt(0x0F70);  // (allow == 0) the mask words too
        else wait_vm_var(allow);
        stage_barrier();
#pragma unroll
        for (int k = 0; k < NBUF - 1; ++k) pend[k] = pend[k + 1];
        pend[NBUF - 1] = 0;
        if (s + NBUF - 1 - sw0 >= 32) build_ctrl(s);
        const int cw = __builtin_amdgcn_readlane(ctrl, s - sw0);
        int c0[QB], c1[QB];
#pragma unroll
        for (int u = 0; u < QB; ++u) {
            c0[u] = (cw >> (6 * u)) & 7;
            c1[u] = (cw >> (6 * u + 3)) & 7;
        }
        if constexpr (DMP)
            if (s + 1 < nrun) mload(s + 1, mnxt);
        if (s + NBUF - 1 < nrun) {
            const int bn = bf + NBUF - 1 >= NBUF ? bf - 1 : bf + NBUF - 1;
            pend[NBUF - 2] = issue(s + NBUF - 1, bn);
        }

        const char* stage = smem + bf * S::STAGE;
        // (dense-mask kernels: both subtiles on one pathway, no mixed stage,
        // which would not fit their register budget)
        bool fast = c0[0] <= 1 && c1[0] <= 1 && (!DENSE || c1[0] == c0[0]);
#pragma unroll
        for (int u = 0; u < QB; ++u) fast = fast && c0[u] == c0[0] && c1[u] == c1[0] && !shifted[u];
        int done = 0;
        if (!DENSE && fast && c0[0] != c1[0]) {
            done = fast_stage(IC<1>{}, stage, c0[0], c1[0], s * kBN);
        } else if (fast) {
            if (c0[0] != cur_pw) {  // rare: kept a branch (not selects on every stage)
                asm volatile("" ::: "memory");
                cur_pw = c0[0];
#pragma unroll
                for (int u = 0; u < QB; ++u)
#pragma unroll
                    for (int kk = 0; kk < S::NKK; ++kk) qcur[u][kk] = cur_pw ? qf[u][1][kk] : qf[u][0][kk];
            }
            done = fast_stage(IC<0>{}, stage, c0[0], c0[0], s * kBN);
        }
        if (done != (1 << QB) - 1) {
            const int* cid = &scid[bf][0];
            const int k0 = s * kBN;
            for_blocks<QB>([&](auto u_c) {
                constexpr int u = decltype(u_c)::value;
                if ((done >> u) & 1) return;
                // Unrolled for chain ids: with an inner loop the accumulators
                // get a second register home and every fast stage pays two
                // copies of them. The dense-mask kernels keep the loop
                // (unrolled, they no longer fit their occupancy).
                if constexpr (DENSE) {
#pragma unroll 1
                    for (int st = 0; st < 2; ++st) slow_subtile(u_c, stage, cid, st, st ? c1[u] : c0[u], k0);
                } else {
#pragma unroll
                    for (int st = 0; st < 2; ++st) slow_subtile(u_c, stage, cid, st, st ? c1[u] : c0[u], k0);
                }
            });
        }
        bf = bf + 1 == NBUF ? 0 : bf + 1;
        if constexpr (DMP) {
#pragma unroll
            for (int u = 0; u < QB; ++u)
#pragma unroll
                for (int st = 0; st < 2; ++st)
#pragma unroll
                    for (int cc = 0; cc < 2; ++cc) mcur[u][st][cc] = mnxt[u][st][cc];
        }
    }

    // ---- epilogue: normalise, store O and LSE ----
#pragma unroll
    for (int u = 0; u < QB; ++u) {
        const float l_tot = l_run[u] + __shfl_xor(l_run[u], 32);
        float inv = l_tot > 0.f ? (SQRT ? __frsqrt_rn(l_tot) : 1.0f / l_tot) : 0.f;
        if constexpr (DROP) inv *= args.drop.rkeep;
        if (qvalid[u]) {
            T* orow = (T*)p.out.ptr + b * p.out.stride_b + h * p.out.stride_h + (int64_t)qrow[u] * p.out.stride_t;
#pragma unroll
            for (int db = 0; db < S::NDB; ++db)
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    const int d = db * 32 + 8 * a + 4 * hh;
                    if (d < D) {
                        typename E::v4 v;
#pragma unroll
                        for (int j = 0; j < 4; ++j) v[j] = (T)(o[u][db][4 * a + j] * inv);
                        *reinterpret_cast<typename E::v4*>(orow + d) = v;
                    }
                }
            if (p.lse && hh == 0) {
                p.lse[((int64_t)b * H + h) * L + qrow[u]] =
                    l_tot > 0.f ? ((SQRT ? 2.0f * m_ref[u] : m_ref[u]) + __log2f(l_tot)) * kLn2 : -INFINITY;
            }
        }
    }
}

template <typename T, int D, bool ROPE, bool DENSE, bool SQRT, bool DROP>
static hipError_t launch_fwd(FwdArgs& a, hipStream_t stream) {
    using C = FwdCfg<D>;
    constexpr int NBUF = D == 64 ? 2 : MPATTN_FWD_NBUF;
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
    uint8_t* mcode = (uint8_t*)(wsb + ws.mcode);
    a.mcode = mcode;
    a.gate = nullptr;
    a.gate_want = 0;
    int* label = DENSE ? (int*)(wsb + ws.label) : nullptr;
    int* valid = DENSE ? (int*)(wsb + ws.valid) : nullptr;
    hipError_t e;
    if (DENSE) {
        // Row labels of the mask, then (prep kernel) the check that the mask
        // is the "different chain" relation of those labels.
        if ((e = launch_mask_labels(p.chain_mask, p.mask_stride_b, p.mask_stride_q, p.mask_stride_k, p.B, p.L, label,
                                    valid, a.mvec, false, stream)) != hipSuccess)
            return e;
    }
    const int64_t nmc = DENSE ? ((int64_t)p.B * (Lp / 32) * (Lp / 32) + 3) / 4 : 0;
    hipLaunchKernelGGL((fwd_prep_kernel<T, D, ROPE, DENSE>), dim3((unsigned)(nchain + nrot + nmc)), dim3(256), 0,
                       stream, p, keff, ksum, qsum, krot, Lp, nchain, mcode, nrot, (const int*)label, valid);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const int nqb = (p.L + 32 * C::QB * C::W - 1) / (32 * C::QB * C::W);
    const int64_t grid = (int64_t)p.B * p.H * nqb;
    if (DENSE) {
        // Batch rows whose mask is a chain partition run the chain-id kernel
        // on the labels (the same pathway for every pair); the others run
        // the dense-mask kernel. Both launches are gated by valid[b].
        FwdArgs ac = a;
        ac.p.chain_id = label;
        ac.p.chain_mask = nullptr;
        ac.gate = valid;
        ac.gate_want = 1;
        hipLaunchKernelGGL((fwd_kernel<T, D, C::W, C::QB, C::WPE, NBUF, ROPE, false, SQRT, DROP>),
                           dim3((unsigned)grid), dim3(C::W * 64), 0, stream, ac);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        a.gate = valid;
        a.gate_want = 0;
    }
    hipLaunchKernelGGL((fwd_kernel<T, D, C::W, C::QB, C::WPE, NBUF, ROPE, DENSE, SQRT, DROP>), dim3((unsigned)grid),
                       dim3(C::W * 64), 0, stream, a);
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
                           stream, p, keff, ksum, qsum, (float*)nullptr, Lp, nchain, (uint8_t*)nullptr, (int64_t)0,
                           (const int*)nullptr, (int*)nullptr);
    else
        hipLaunchKernelGGL((fwd_prep_kernel<float, 16, false, false>), dim3((unsigned)nchain), dim3(256), 0,
                           stream, p, keff, ksum, qsum, (float*)nullptr, Lp, nchain, (uint8_t*)nullptr, (int64_t)0,
                           (const int*)nullptr, (int*)nullptr);
    return hipGetLastError();
}

template <typename T, int D>
static hipError_t dispatch_fwd_d(FwdArgs& a, hipStream_t s) {
    const bool rope = a.p.rope == MPATTN_ROPE_FUSED;
    const bool dense = a.p.chain_mask != nullptr;
    if (a.p.sqrt_softmax) {
        if (a.p.dropout_p > 0.f) {
            if (rope) return dense ? launch_fwd<T, D, true, true, true, true>(a, s) : launch_fwd<T, D, true, false, true, true>(a, s);
            return dense ? launch_fwd<T, D, false, true, true, true>(a, s) : launch_fwd<T, D, false, false, true, true>(a, s);
        }
        if (rope) return dense ? launch_fwd<T, D, true, true, true, false>(a, s) : launch_fwd<T, D, true, false, true, false>(a, s);
        return dense ? launch_fwd<T, D, false, true, true, false>(a, s) : launch_fwd<T, D, false, false, true, false>(a, s);
    }
    if (a.p.dropout_p > 0.f) {
        if (rope) return dense ? launch_fwd<T, D, true, true, false, true>(a, s) : launch_fwd<T, D, true, false, false, true>(a, s);
        return dense ? launch_fwd<T, D, false, true, false, true>(a, s) : launch_fwd<T, D, false, false, false, true>(a, s);
    }
    if (rope) return dense ? launch_fwd<T, D, true, true, false, false>(a, s) : launch_fwd<T, D, true, false, false, false>(a, s);
    return dense ? launch_fwd<T, D, false, true, false, false>(a, s) : launch_fwd<T, D, false, false, false, false>(a, s);
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
    a.drop = drop_cfg(p.dropout_p, p.dropout_seed);
    a.mvec = p.chain_mask && p.mask_stride_k == 1 && (uintptr_t)p.chain_mask % 8 == 0 && p.mask_stride_b % 8 == 0 &&
             p.mask_stride_q % 8 == 0;
    if (p.dtype == MPATTN_BF16) return dispatch_fwd_t<bf16_t>(a, stream);
    return dispatch_fwd_t<fp16_t>(a, stream);
}

}  // namespace mpattn
