// fp32 multi-pathway attention forward for gfx950 (the ESM-2 8M model runs
// in fp32). Same op and contract as the 16-bit kernels (include/mpattn.h);
// the tolerance here is 1e-4 max-abs against an fp64 reference, so every
// product and sum stays in fp32 and probabilities are not rounded.
//
// * One workgroup of 4 wavefronts owns 128 queries of one (b, h); each
//   wavefront owns 32. Q (RoPE and the logit factor applied) sits in
//   registers in the MFMA B-operand layout of v_mfma_f32_32x32x2_f32: lane l
//   holds dims 2*kk + l/32 of query l%32 (RoPE pairs dims d and d + D/2,
//   which have the same parity, so each lane rotates its own dims).
// * Keys stream through LDS in subtiles of 32 (K_self rotated while it is
//   staged, K_multi, V_self, V_multi, chain ids), double-buffered.
// * S^T = K Q^T (rows = keys, columns = queries). K rows are read in the
//   order pi(r) = 2*(4*(r/8) + r%4) + (r/4)%2, so accumulator slot i of lane
//   half hh holds key 2*i + hh: exactly the B operand of step i of
//   O^T += V^T P^T.
// * Subtiles are classified from the chain summaries of the prep kernel
//   (pure self / pure multimer / general / all padded), as in the 16-bit
//   forward. Online softmax in base 2 with an exact running max.
#include "mpattn_common.h"

namespace mpattn {

// Shared with the 16-bit forward (mpattn_fwd.hip).
int64_t fwd_workspace_bytes(int B, int H, int L, int D, int dtype, int rope);
hipError_t launch_fwd_prep_f32(const mpattn_fwd_params& p, int* keff, int* ksum, int* qsum, int Lp,
                               hipStream_t stream);
void fwd_ws_offsets(int B, int H, int L, int D, int esize, bool rope, int64_t* keff, int64_t* ksum,
                    int64_t* qsum);

namespace {

constexpr int kKB = 32;  // keys per subtile

__device__ __forceinline__ f32x16 mma32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// DROP: attention dropout (the definition in mpattn.h): the weights that
// multiply V are the kept ones, the row sum takes all of them, and O is
// scaled by 1 / (1 - p).
template <int D, bool ROPE, bool DENSE, bool SQRT, bool DROP>
__global__ __launch_bounds__(256) void fwd32_kernel(const mpattn_fwd_params p, const int* keff,
                                                    const int* ksum, const int* qsum, int Lp,
                                                    float qmul, float c, DropCfg drop) {
    constexpr int W = 4;
    constexpr int H2 = D / 2;
    constexpr int NK = D / 2;             // MFMA steps over head dims
    constexpr int NDB = (D + 31) / 32;    // 32-row blocks of O^T
    constexpr int RS = D + 1;             // LDS row stride (floats), odd: no bank conflicts
    constexpr int TILE = kKB * RS;        // floats per staged tile
    constexpr int STAGE = 4 * TILE;

    __shared__ float smem[2][STAGE];
    __shared__ int scid[2][kKB];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ql = lane & 31, hh = lane >> 5;
    const int L = p.L, H = p.H;
    const int nqb = (L + 32 * W - 1) / (32 * W);
    const int g = xcd_remap(blockIdx.x, gridDim.x);
    const int qb = g % nqb, bh = g / nqb;
    const int b = bh / H, h = bh % H;
    const int qw0 = qb * 32 * W;
    const int q = qw0 + wave * 32 + ql;
    const bool qvalid = q < L;
    const uint32_t drow = DROP ? drop_row(drop.lo, (uint32_t)bh, (uint32_t)q) : 0u;

    auto base = [&](const mpattn_tensor& t) {
        return (const float*)t.ptr + b * t.stride_b + h * t.stride_h;
    };
    const float* ks_p = base(p.k_self);
    const float* km_p = base(p.k_multi);
    const float* vs_p = base(p.v_self);
    const float* vm_p = base(p.v_multi);

    // ---- Q operands: lane holds dims 2*kk + hh ----
    float qf[2][NK];
#pragma unroll
    for (int pw = 0; pw < 2; ++pw) {
        const mpattn_tensor& qt = pw == 0 ? p.q_self : p.q_multi;
        const float* row = base(qt) + (int64_t)(qvalid ? q : 0) * qt.stride_t;
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) {
            const int d = 2 * kk + hh;
            float x = qvalid ? row[d] : 0.f;
            if (ROPE && pw == 0 && qvalid) {
                const bool lo = d < H2;
                const int fi = lo ? d : d - H2;
                const float y = row[lo ? d + H2 : d - H2];
                const float cs = p.rope_cos[(int64_t)q * H2 + fi], sn = p.rope_sin[(int64_t)q * H2 + fi];
                x = rope_rot(x, y, cs, sn, lo);
            }
            qf[pw][kk] = x * qmul;
        }
    }
    int cq = 0, cq_min = 0, cq_max = 0;
    if constexpr (!DENSE) {
        cq = qvalid ? p.chain_id[(int64_t)b * L + q] : 0;
        // this wavefront's 32-query block (clamped: a block past Lp has no queries)
        const int blk = min(qw0 / 32 + wave, Lp / 32 - 1);
        const int4 qs = reinterpret_cast<const int4*>(qsum)[(int64_t)b * (Lp / 32) + blk];
        cq_min = __builtin_amdgcn_readfirstlane(qs.x);
        cq_max = __builtin_amdgcn_readfirstlane(qs.y);
    }
    const uint8_t* mrow = nullptr;
    if constexpr (DENSE)
        mrow = p.chain_mask + (int64_t)b * p.mask_stride_b + (int64_t)(qvalid ? q : 0) * p.mask_stride_q;

    // ---- staging of subtile t into buffer bf (all 256 threads) ----
    auto stage_in = [&](int t, int bf) {
        const int k0 = t * kKB;
        float* st = smem[bf];
        constexpr int C4 = D / 4;  // float4 chunks per row
        for (int it = tid; it < 4 * kKB * C4; it += 256) {
            const int ten = it / (kKB * C4);
            const int rem = it % (kKB * C4);
            const int r = rem / C4, d0 = (rem % C4) * 4;
            const int key = min(k0 + r, L - 1);  // rows past L are masked later
            const float* src = ten == 0 ? ks_p : ten == 1 ? km_p : ten == 2 ? vs_p : vm_p;
            const int64_t stt = ten == 0 ? p.k_self.stride_t : ten == 1 ? p.k_multi.stride_t
                                : ten == 2 ? p.v_self.stride_t : p.v_multi.stride_t;
            const float* rowp = src + (int64_t)key * stt;
            float4 x = *reinterpret_cast<const float4*>(rowp + d0);
            if (ROPE && ten == 0) {
                const bool lo = d0 < H2;
                const int fi = lo ? d0 : d0 - H2;
                const float4 y = *reinterpret_cast<const float4*>(rowp + (lo ? d0 + H2 : d0 - H2));
                const float4 cs = *reinterpret_cast<const float4*>(p.rope_cos + (int64_t)key * H2 + fi);
                const float4 sn = *reinterpret_cast<const float4*>(p.rope_sin + (int64_t)key * H2 + fi);
                x.x = rope_rot(x.x, y.x, cs.x, sn.x, lo);
                x.y = rope_rot(x.y, y.y, cs.y, sn.y, lo);
                x.z = rope_rot(x.z, y.z, cs.z, sn.z, lo);
                x.w = rope_rot(x.w, y.w, cs.w, sn.w, lo);
            }
            float* dst = st + ten * TILE + r * RS + d0;
            dst[0] = x.x;
            dst[1] = x.y;
            dst[2] = x.z;
            dst[3] = x.w;
        }
        if (tid < kKB) scid[bf][tid] = keff[(int64_t)b * Lp + k0 + tid];
    };

    // K row read for accumulator row r (see the header).
    const int perm = 2 * (4 * (ql / 8) + ql % 4) + ((ql / 4) & 1);

    float m_run = -INFINITY;  // running max, base 2
    float l_run = 0.f;
    f32x16 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] = 0.f;

    auto qk = [&](const float* kt, int pw) -> f32x16 {
        f32x16 acc;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.f;
#pragma unroll
        for (int kk = 0; kk < NK; ++kk)
            acc = mma32(kt[perm * RS + 2 * kk + hh], pw ? qf[1][kk] : qf[0][kk], acc);  // no dynamic indexing
        return acc;
    };
    // O^T += V^T W^T for one pathway's tile; w[i] is the weight of key 2i + hh.
    auto pv = [&](const float* vt, const f32x16& w) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const int d = db * 32 + ql;
#pragma unroll
            for (int kk = 0; kk < 16; ++kk) {
                const float a = d < D ? vt[(2 * kk + hh) * RS + d] : 0.f;
                o[db] = mma32(a, w[kk], o[db]);
            }
        }
    };

    const int4* ksum_b = reinterpret_cast<const int4*>(ksum) + (int64_t)b * (Lp / 32);
    const int nsub = (L + kKB - 1) / kKB;
    stage_in(0, 0);
    __syncthreads();
    for (int t = 0; t < nsub; ++t) {
        const int bf = t & 1;
        if (t + 1 < nsub) stage_in(t + 1, bf ^ 1);
        const float* st = smem[bf];
        const int4 sm = ksum_b[t];
        const int kmin = __builtin_amdgcn_readfirstlane(sm.x), kmax = __builtin_amdgcn_readfirstlane(sm.y);
        const int npad = __builtin_amdgcn_readfirstlane(sm.z);
        int mode = 2;  // 0 self, 1 multimer, 2 general, 3 skip
        if (npad == kKB) mode = 3;
        else if (!DENSE && npad == 0) {
            if (kmin == kmax && cq_min == cq_max && kmin == cq_min) mode = 0;
            else if (kmax < cq_min || kmin > cq_max) mode = 1;
        }
        if (mode != 3) {
            f32x16 s;
            uint32_t same = 0;  // bit i: key 2i + hh on the query's chain
            if (mode != 2) {
                const f32x16 acc = qk(st + mode * TILE, mode);
#pragma unroll
                for (int i = 0; i < 16; ++i) s[i] = acc[i] * c;
                same = mode == 0 ? 0xffffu : 0u;
            } else {
                const f32x16 as = qk(st, 0), am = qk(st + TILE, 1);
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int kl = 2 * i + hh;
                    const int ck = scid[bf][kl];
                    bool sm_;
                    if constexpr (DENSE) {
                        const int kg = t * kKB + kl;
                        sm_ = !(kg < L && mrow[(int64_t)kg * p.mask_stride_k] != 0);
                    } else {
                        sm_ = ck == cq;
                    }
                    same |= (uint32_t)sm_ << i;
                    s[i] = ck == kPadChain ? -INFINITY : (sm_ ? as[i] : am[i]) * c;
                }
            }
            float mx = s[0];
#pragma unroll
            for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[i]);
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float m_new = fmaxf(m_run, mx);
            if (m_new > m_run) {  // -inf -> finite, or a larger max
                const float alpha = m_run == -INFINITY ? 0.f : fast_exp2(m_run - m_new);
                l_run *= alpha;
#pragma unroll
                for (int db = 0; db < NDB; ++db)
#pragma unroll
                    for (int i = 0; i < 16; ++i) o[db][i] *= SQRT ? sqrtf(alpha) : alpha;
                m_run = m_new;
            }
            f32x16 w, ws, wm;
            const float mr = m_run == -INFINITY ? 0.f : m_run;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float pr = fast_exp2(s[i] - mr);  // 0 for padded keys
                l_run += pr;
                w[i] = SQRT ? sqrtf(pr) : pr;
                if constexpr (DROP)
                    if (!drop_keep(drow, drop.hi, (uint32_t)(t * kKB + 2 * i + hh), drop.thr)) w[i] = 0.f;
                const bool sm_ = (same >> i) & 1u;
                ws[i] = sm_ ? w[i] : 0.f;
                wm[i] = sm_ ? 0.f : w[i];
            }
            if (mode == 0) pv(st + 2 * TILE, w);
            else if (mode == 1) pv(st + 3 * TILE, w);
            else {
                pv(st + 2 * TILE, ws);
                pv(st + 3 * TILE, wm);
            }
        }
        __syncthreads();
    }

    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const float inv = l_tot > 0.f ? (SQRT ? 1.0f / sqrtf(l_tot) : 1.0f / l_tot) * (DROP ? drop.rkeep : 1.0f) : 0.f;
    if (qvalid) {
        float* orow = (float*)p.out.ptr + b * p.out.stride_b + h * p.out.stride_h + (int64_t)q * p.out.stride_t;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                const int d = db * 32 + 8 * a4 + 4 * hh;
                if (d < D) {
                    float4 v;
                    v.x = o[db][4 * a4 + 0] * inv;
                    v.y = o[db][4 * a4 + 1] * inv;
                    v.z = o[db][4 * a4 + 2] * inv;
                    v.w = o[db][4 * a4 + 3] * inv;
                    *reinterpret_cast<float4*>(orow + d) = v;
                }
            }
        if (p.lse && hh == 0)
            p.lse[((int64_t)b * H + h) * L + q] = l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
    }
}

template <int D, bool ROPE, bool DENSE, bool SQRT, bool DROP>
hipError_t launch32(const mpattn_fwd_params& p, const int* keff, const int* ksum, const int* qsum, int Lp,
                    hipStream_t stream) {
    const float f = p.scale * kLog2e;
    // Q is scaled by scale*log2(e) with fused RoPE (its values are rounded
    // once either way in fp32); otherwise the factor is applied to the logits.
    const bool fused = ROPE;
    const int nqb = (p.L + 127) / 128;
    hipLaunchKernelGGL((fwd32_kernel<D, ROPE, DENSE, SQRT, DROP>), dim3((unsigned)((int64_t)p.B * p.H * nqb)),
                       dim3(256), 0, stream, p, keff, ksum, qsum, Lp, fused ? f : 1.0f, fused ? 1.0f : f,
                       drop_cfg(p.dropout_p, p.dropout_seed));
    return hipGetLastError();
}

template <int D, bool DROP>
hipError_t dispatch32_d(const mpattn_fwd_params& p, const int* keff, const int* ksum, const int* qsum, int Lp,
                        hipStream_t s) {
    const bool rope = p.rope == MPATTN_ROPE_FUSED, dense = p.chain_mask != nullptr, sq = p.sqrt_softmax != 0;
#define MPATTN_L32(R, DN, SQ) return launch32<D, R, DN, SQ, DROP>(p, keff, ksum, qsum, Lp, s)
    if (rope) {
        if (dense) { if (sq) MPATTN_L32(true, true, true); MPATTN_L32(true, true, false); }
        if (sq) MPATTN_L32(true, false, true);
        MPATTN_L32(true, false, false);
    }
    if (dense) { if (sq) MPATTN_L32(false, true, true); MPATTN_L32(false, true, false); }
    if (sq) MPATTN_L32(false, false, true);
    MPATTN_L32(false, false, false);
#undef MPATTN_L32
}

template <int D>
hipError_t dispatch32(const mpattn_fwd_params& p, const int* keff, const int* ksum, const int* qsum, int Lp,
                      hipStream_t s) {
    if (p.dropout_p > 0.f) return dispatch32_d<D, true>(p, keff, ksum, qsum, Lp, s);
    return dispatch32_d<D, false>(p, keff, ksum, qsum, Lp, s);
}

}  // namespace

hipError_t launch_fwd32(const mpattn_fwd_params& p, hipStream_t stream) {
    int64_t o_keff, o_ksum, o_qsum;
    fwd_ws_offsets(p.B, p.H, p.L, p.D, 4, false, &o_keff, &o_ksum, &o_qsum);
    char* w = (char*)p.workspace;
    int* keff = (int*)(w + o_keff);
    int* ksum = (int*)(w + o_ksum);
    int* qsum = (int*)(w + o_qsum);
    const int Lp = (p.L + 63) / 64 * 64;
    hipError_t e = launch_fwd_prep_f32(p, keff, ksum, qsum, Lp, stream);
    if (e != hipSuccess) return e;
    switch (p.D) {
        case 16: return dispatch32<16>(p, keff, ksum, qsum, Lp, stream);
        case 24: return dispatch32<24>(p, keff, ksum, qsum, Lp, stream);
        case 32: return dispatch32<32>(p, keff, ksum, qsum, Lp, stream);
        case 64: return dispatch32<64>(p, keff, ksum, qsum, Lp, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace mpattn
