// Forward multi-pathway attention for gfx950 (16-bit inputs, fp32 accumulate).
//
// Follows the math of the reference eager combine
// (mint_plus/models/modules_plus.py:155-201 with the fp32 softmax of
// mint_plus/models/mu_scaling/layer.py:159) and the flash-style contract of
// mint_plus/models/kernels/multi_pathway_attention.py:32-181, re-designed for
// CDNA4:
//
// * A workgroup of W wavefronts owns 32*W consecutive queries of one (b, h);
//   each wavefront owns 32 of them.
// * Keys stream through LDS in stages of 64 (two 32-key subtiles). K rows are
//   stored row-major, V is stored transposed (d-major) so that the PV operand
//   is one 16-byte LDS read per lane. RoPE and the logit scale are applied in
//   fp32 while Q is loaded and while K_self is staged.
// * Per 32-key subtile a wavefront computes S^T = K Q^T with
//   v_mfma_f32_32x32x16 (rows = keys, columns = queries). Lane l then holds 16
//   logits of query l%32, so the softmax row max/sum are in-lane reductions
//   plus one exchange with lane l^32. K rows are read in an order that swaps
//   bits 2 and 3 of the row index, which makes accumulator slot i of lane half
//   hh correspond to key 16*(i/8) + 8*hh + i%8: the probabilities are then
//   already laid out as the B operand of O^T += V^T P^T, with no shuffle.
// * Subtiles are classified from the chain-id range of their keys and of the
//   wavefront's queries: pure same-chain subtiles run only the self pathway,
//   pure cross-chain subtiles only the multimer pathway; mixed or padded
//   subtiles compute both logits and select per element.
// * Online softmax in base 2 with a lazily updated reference max: the
//   accumulators are rescaled only when a row max grows by more than 2^8.
// * For D < 32 the unused rows of the V^T operand hold ones, so the MFMA also
//   produces the softmax denominator; otherwise it is summed in fp32.
#include <type_traits>

#include "mpattn_common.h"

namespace mpattn {

constexpr int kBN = 64;  // keys per LDS stage

template <int D> struct FwdShape {
    static constexpr int DP = D <= 16 ? 16 : (D <= 32 ? 32 : 64);  // MFMA K for QK^T
    static constexpr int NKK = DP / 16;                              // QK MFMAs / subtile
    static constexpr int NDB = DP <= 32 ? 1 : 2;                     // 32-row blocks of O^T
    static constexpr int VROWS = NDB * 32;
    static constexpr bool SUM_MFMA = D < 32;                         // ones rows give the sum
    static constexpr int ISUM = 4 * (D / 8);                         // accumulator slot of row D
    static constexpr int KST = DP + 8;                               // LDS row stride, K
    static constexpr int VST = kBN + 8;                              // LDS row stride, V^T
};

struct FwdArgs {
    mpattn_fwd_params p;
    float qmul;   // factor applied to q while loading (scale when fused, else 1)
    float c;      // base-2 factor applied to raw logits
    float lse_mul;// raw logit -> natural-unit logit
};

// Query-side state carried by one wavefront.
template <typename T, int D> struct QFrag {
    typename Elt<T>::v8 f[2][FwdShape<D>::NKK];  // [pathway][k-chunk]
};

template <typename T, int D, int W, bool ROPE, bool DENSE>
__global__ __launch_bounds__(W * 64) void fwd_kernel(const FwdArgs args) {
    using S = FwdShape<D>;
    using E = Elt<T>;
    typedef typename E::v8 v8;
    const mpattn_fwd_params& p = args.p;

    __shared__ __attribute__((aligned(16))) T sK[2][kBN * S::KST];
    __shared__ __attribute__((aligned(16))) T sVt[2][S::VROWS * S::VST];
    __shared__ __attribute__((aligned(16))) int sCid[kBN];
    __shared__ int sSum[2][4];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int ql = lane & 31, hh = lane >> 5;
    const int L = p.L, H = p.H;
    const int nqb = (L + 32 * W - 1) / (32 * W);
    const int g = xcd_remap(blockIdx.x, gridDim.x);
    const int qb = g % nqb, bh = g / nqb;
    const int b = bh / H, h = bh % H;
    const int q = qb * 32 * W + wave * 32 + ql;
    const bool qvalid = q < L;

    // (b, h) base of each operand; pathway 0 = self, 1 = multimer.
    auto base = [&](const mpattn_tensor& t) {
        return (const T*)t.ptr + b * t.stride_b + h * t.stride_h;
    };
    const T* const qs_p = base(p.q_self);
    const T* const qm_p = base(p.q_multi);
    const T* const ks_p = base(p.k_self);
    const T* const km_p = base(p.k_multi);
    const T* const vs_p = base(p.v_self);
    const T* const vm_p = base(p.v_multi);

    // Ones rows of V^T (rows D..VROWS-1) turn the PV MFMA into a row-sum too.
    if constexpr (S::SUM_MFMA) {
        for (int i = tid; i < 2 * (S::VROWS - D) * kBN; i += W * 64) {
            const int pw = i / ((S::VROWS - D) * kBN);
            const int r = i % ((S::VROWS - D) * kBN);
            sVt[pw][(D + r / kBN) * S::VST + r % kBN] = (T)1.0f;
        }
    }

    // ---- Q fragments (B operand of S^T = K Q^T): dims kk*16 + 8*hh + [0,8) ----
    QFrag<T, D> qf;
#pragma unroll
    for (int pw = 0; pw < 2; ++pw) {
#pragma unroll
        for (int kk = 0; kk < S::NKK; ++kk) {
            float x[8];
            if (qvalid) {
                const T* row = pw == 0 ? qs_p + (int64_t)q * p.q_self.stride_t
                                       : qm_p + (int64_t)q * p.q_multi.stride_t;
                load8_rot<T, D>(row, p.rope_cos, p.rope_sin, q,
                                kk * 16 + hh * 8, args.qmul, ROPE && pw == 0, x);
            } else {
#pragma unroll
                for (int t = 0; t < 8; ++t) x[t] = 0.f;
            }
            qf.f[pw][kk] = pack8<T>(x);
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

    const float c = args.c;
    const float th = 8.0f / c;  // rescale threshold in raw logit units (2^8)
    float m_ref = -INFINITY;
    float l_run = 0.f;
    f32x16 o[S::NDB];
#pragma unroll
    for (int db = 0; db < S::NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] = 0.f;

    // Row of the K operand this lane reads: subtile row ql with bits 2,3 swapped.
    const int krow = (ql & ~12) | ((ql & 4) << 1) | ((ql & 8) >> 1);

    for (int k0 = 0; k0 < L; k0 += kBN) {
        __syncthreads();  // previous stage fully consumed
        // ---- stage K (row-major, RoPE on self) ----
        constexpr int KCH = S::DP / 8;  // 8-element chunks per row
        for (int it = tid; it < 2 * kBN * KCH; it += W * 64) {
            const int pw = it / (kBN * KCH);
            const int r = (it / KCH) % kBN;
            const int d0 = (it % KCH) * 8;
            const int kg = k0 + r;
            float x[8];
            if (kg < L) {
                const T* row = pw == 0 ? ks_p + (int64_t)kg * p.k_self.stride_t
                                       : km_p + (int64_t)kg * p.k_multi.stride_t;
                load8_rot<T, D>(row, p.rope_cos, p.rope_sin, kg, d0, 1.0f, ROPE && pw == 0, x);
            } else {
#pragma unroll
                for (int t = 0; t < 8; ++t) x[t] = 0.f;
            }
            *reinterpret_cast<v8*>(&sK[pw][r * S::KST + d0]) = pack8<T>(x);
        }
        // ---- stage V^T (d-major); each item: 2 keys x 8 dims ----
        constexpr int VCH = D / 8;
        for (int it = tid; it < 2 * (kBN / 2) * VCH; it += W * 64) {
            const int pw = it / ((kBN / 2) * VCH);
            const int kp2 = (it / VCH) % (kBN / 2);
            const int d0 = (it % VCH) * 8;
            const int kg = k0 + 2 * kp2;
            const T* vb = pw == 0 ? vs_p : vm_p;
            const int64_t vstr = pw == 0 ? p.v_self.stride_t : p.v_multi.stride_t;
            float x0[8], x1[8];
            if (kg < L) load8f<T>(vb + (int64_t)kg * vstr, d0, x0);
            else for (int t = 0; t < 8; ++t) x0[t] = 0.f;
            if (kg + 1 < L) load8f<T>(vb + (int64_t)(kg + 1) * vstr, d0, x1);
            else for (int t = 0; t < 8; ++t) x1[t] = 0.f;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                typename Elt<T>::v2 pr2;
                pr2[0] = (T)x0[t];
                pr2[1] = (T)x1[t];
                *reinterpret_cast<typename Elt<T>::v2*>(&sVt[pw][(d0 + t) * S::VST + 2 * kp2]) = pr2;
            }
        }
        // ---- chain ids / padding, and per-subtile summary (wave 0) ----
        if (wave == 0) {
            const int kg = k0 + lane;
            int cid = kPadChain;
            if (kg < L && !(p.key_pad && p.key_pad[(int64_t)b * L + kg])) {
                cid = DENSE ? 0 : p.chain_id[(int64_t)b * L + kg];
            }
            sCid[lane] = cid;
            const bool valid = cid != kPadChain;
            const int mn = half_min_i(valid ? cid : INT32_MAX);
            const int mx = half_max_i(valid ? cid : INT32_MIN);
            const uint64_t padm = __ballot(!valid);
            if ((lane & 31) == 0) {
                sSum[hh][0] = mn;
                sSum[hh][1] = mx;
                sSum[hh][2] = __popcll(hh ? (padm >> 32) : (padm & 0xffffffffull));
            }
        }
        __syncthreads();

#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const int kmin = __builtin_amdgcn_readfirstlane(sSum[st][0]);
            const int kmax = __builtin_amdgcn_readfirstlane(sSum[st][1]);
            const int npad = __builtin_amdgcn_readfirstlane(sSum[st][2]);
            if (npad == 32) continue;
            int mode = 2;  // 0: pure self, 1: pure multimer, 2: general
            if (!DENSE && npad == 0) {
                if (kmin == kmax && cq_min == cq_max && kmin == cq_min) mode = 0;
                else if (kmax < cq_min || kmin > cq_max) mode = 1;
            }
            const int kbase = st * 32;
            const int krd = (kbase + krow) * S::KST + hh * 8;  // K operand offset

            // Online softmax (base 2, lazy rescale): updates m_ref / l_run / o
            // for this subtile's logits and returns the unnormalised weights.
            auto softmax_step = [&](const f32x16& sv, float pr[16]) {
                float mx = sv[0];
#pragma unroll
                for (int i = 1; i < 16; ++i) mx = fmaxf(mx, sv[i]);
                mx = fmaxf(mx, __shfl_xor(mx, 32));
                const bool need = mx > m_ref + th;
                if (__any(need)) {
                    const float m_new = need ? mx : m_ref;
                    const float alpha = need ? fast_exp2((m_ref - m_new) * c) : 1.0f;
                    m_ref = m_new;
                    l_run *= alpha;
#pragma unroll
                    for (int db = 0; db < S::NDB; ++db)
#pragma unroll
                        for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
                }
                const float mc = m_ref * c;
#pragma unroll
                for (int i = 0; i < 16; ++i) pr[i] = fast_exp2(fmaf(sv[i], c, -mc));
            };

            // One pathway for the whole subtile.
            auto pure = [&](auto pw_c) {
                constexpr int pw = decltype(pw_c)::value;
                f32x16 sv;
#pragma unroll
                for (int i = 0; i < 16; ++i) sv[i] = 0.f;
#pragma unroll
                for (int kk = 0; kk < S::NKK; ++kk) {
                    const v8 a = *reinterpret_cast<const v8*>(&sK[pw][krd + kk * 16]);
                    sv = E::mma(a, qf.f[pw][kk], sv);
                }
                float pr[16];
                softmax_step(sv, pr);
                v8 pb[2];
#pragma unroll
                for (int cc = 0; cc < 2; ++cc) pb[cc] = pack8<T>(&pr[8 * cc]);
                if constexpr (!S::SUM_MFMA) {
#pragma unroll
                    for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                        for (int t = 0; t < 8; ++t) l_run += (float)pb[cc][t];
                }
#pragma unroll
                for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                    for (int db = 0; db < S::NDB; ++db) {
                        const v8 a = *reinterpret_cast<const v8*>(
                            &sVt[pw][(db * 32 + ql) * S::VST + kbase + 16 * cc + 8 * hh]);
                        o[db] = E::mma(a, pb[cc], o[db]);
                    }
            };

            // Both pathways, selected per element; handles padded keys.
            auto general = [&]() {
                f32x16 ss, sm, sv;
#pragma unroll
                for (int i = 0; i < 16; ++i) { ss[i] = 0.f; sm[i] = 0.f; }
#pragma unroll
                for (int kk = 0; kk < S::NKK; ++kk) {
                    const v8 as = *reinterpret_cast<const v8*>(&sK[0][krd + kk * 16]);
                    const v8 am = *reinterpret_cast<const v8*>(&sK[1][krd + kk * 16]);
                    ss = E::mma(as, qf.f[0][kk], ss);
                    sm = E::mma(am, qf.f[1][kk], sm);
                }
                bool same[16];
                // keys of slot i: kbase + 16*(i/8) + 8*hh + i%8
#pragma unroll
                for (int cc = 0; cc < 2; ++cc) {
                    const int kl = kbase + 16 * cc + 8 * hh;
                    const i32x4 c0 = *reinterpret_cast<const i32x4*>(&sCid[kl]);
                    const i32x4 c1 = *reinterpret_cast<const i32x4*>(&sCid[kl + 4]);
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
                float pr[16];
                softmax_step(sv, pr);
                v8 ps[2], pm[2];
#pragma unroll
                for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        const int i = 8 * cc + t;
                        const T pv = (T)pr[i];
                        if constexpr (!S::SUM_MFMA) l_run += (float)pv;
                        ps[cc][t] = same[i] ? pv : (T)0.f;
                        pm[cc][t] = same[i] ? (T)0.f : pv;
                    }
#pragma unroll
                for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                    for (int db = 0; db < S::NDB; ++db) {
                        const int off = (db * 32 + ql) * S::VST + kbase + 16 * cc + 8 * hh;
                        const v8 a0 = *reinterpret_cast<const v8*>(&sVt[0][off]);
                        const v8 a1 = *reinterpret_cast<const v8*>(&sVt[1][off]);
                        o[db] = E::mma(a0, ps[cc], o[db]);
                        o[db] = E::mma(a1, pm[cc], o[db]);
                    }
            };

            if (mode == 0) pure(std::integral_constant<int, 0>{});
            else if (mode == 1) pure(std::integral_constant<int, 1>{});
            else general();
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
                l_tot > 0.f ? m_ref * args.lse_mul + logf(l_tot) : -INFINITY;
        }
    }
}

template <typename T, int D, bool ROPE, bool DENSE>
static hipError_t launch_fwd(const FwdArgs& a, hipStream_t stream) {
    constexpr int W = 4;
    const int nqb = (a.p.L + 32 * W - 1) / (32 * W);
    const int64_t grid = (int64_t)a.p.B * a.p.H * nqb;
    hipLaunchKernelGGL((fwd_kernel<T, D, W, ROPE, DENSE>), dim3((unsigned)grid), dim3(W * 64), 0,
                       stream, a);
    return hipGetLastError();
}

template <typename T, int D>
static hipError_t dispatch_fwd_d(const FwdArgs& a, hipStream_t s) {
    const bool rope = a.p.rope == MPATTN_ROPE_FUSED;
    const bool dense = a.p.chain_mask != nullptr;
    if (rope) return dense ? launch_fwd<T, D, true, true>(a, s) : launch_fwd<T, D, true, false>(a, s);
    return dense ? launch_fwd<T, D, false, true>(a, s) : launch_fwd<T, D, false, false>(a, s);
}

template <typename T>
static hipError_t dispatch_fwd_t(const FwdArgs& a, hipStream_t s) {
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
    const bool fused = p.rope == MPATTN_ROPE_FUSED;
    a.qmul = fused ? p.scale : 1.0f;
    a.c = fused ? kLog2e : p.scale * kLog2e;
    a.lse_mul = fused ? 1.0f : p.scale;
    if (p.dtype == MPATTN_BF16) return dispatch_fwd_t<bf16_t>(a, stream);
    return dispatch_fwd_t<fp16_t>(a, stream);
}

}  // namespace mpattn
