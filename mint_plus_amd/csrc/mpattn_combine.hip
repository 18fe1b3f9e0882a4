// Materialised-logit combine (forward and backward) on gfx950.
//
// Replaces fused_multimer_combine / fused_multimer_combine_bwd
// (mint_plus/models/kernels/__init__.py:179-242, :247-286): given the two
// (B, H, L, L) logit tensors a caller already holds (pre-softmax, scaled,
// padded keys at -inf), the (B, L, L) "different chain" mask and the two
// (B, H, L, D) value tensors,
//
//   s_ij = mask_ij ? inter_ij : intra_ij
//   P_i  = softmax_j(s_i)                       (fp32; all -inf row -> 0)
//   O_i  = sum_j P_ij (mask_ij ? Vm_j : Vs_j)
//
// Backward: dS_ij = P_ij (dO_i . Vsel_j - Delta_i), Delta_i = dO_i . O_i,
// split into d_intra / d_inter by the mask; dVs_j = sum_i P_ij [!mask] dO_i,
// dVm_j likewise. With dropout (keep mask Z of the fused op's definition,
// r = 1 / (1 - p)): O uses r Z P, dVs / dVm use r Z P, and dO_i . Vsel_j is
// replaced by r Z_ij dO_i . Vsel_j; the softmax and its LSE are undropped.
//
// The op streams 2 L^2 logits per (b, h) against O(L D) other data, so it is
// HBM-bound; the kernels read every logit once per pass with 16-byte loads
// and keep the P.V products on MFMA so the VALU does only the softmax.
//
//   combine_fwd:   one wave per 32 queries, 4 waves per workgroup sharing the
//                  V tiles in LDS. Lane (query c, half h) holds 8 consecutive
//                  keys of its row: exactly the B operand (P^T, k = key) of
//                  the 32x32x16 MFMA, whose accumulator O^T then keeps every
//                  element of a lane on the lane's own query, so the online
//                  softmax rescale is a per-lane multiply. The running max is
//                  lazy: it moves only when a chunk exceeds it by 2^8.
//                  STATS mode writes (lse, Delta = dO . O) instead of O.
//                  16-bit inputs with 16-byte rows take combine_fwd_dma_kernel
//                  instead: the same math on logit / mask / V tiles copied
//                  into an LDS ring with row-contiguous global_load_lds.
//   combine_bwd:   key-stationary; P tiles are recomputed from coalesced
//                  logit loads and transposed through LDS, dV^T = dO^T P and
//                  dW^T = V dO^T on MFMA, then dS = P (dW - Delta) goes out as
//                  both d_logits with coalesced stores.
// fp32 uses the 32x32x2 fp32 MFMA with the same lane-to-query mapping.
#include <math.h>

#include <type_traits>

#include "mpattn_common.h"

namespace mpattn {
namespace {

struct CombineArgs {
    const void *il, *el;              // intra / inter logits
    int64_t il_sb, il_sh, il_st, el_sb, el_sh, el_st;
    const void *vs, *vm;              // values
    int64_t vs_sb, vs_sh, vs_st, vm_sb, vm_sh, vm_st;
    const uint8_t* mask;
    int64_t m_sb, m_sq, m_sk;
    void* out;                        // fwd: O; STATS: unused
    int64_t o_sb, o_sh, o_st;
    const void* go;                   // grad_out (STATS / bwd)
    int64_t g_sb, g_sh, g_st;
    void *dil, *del;                  // d_intra / d_inter logits
    int64_t dil_sb, dil_sh, dil_st, del_sb, del_sh, del_st;
    void *dvs, *dvm;                  // d values
    int64_t dvs_sb, dvs_sh, dvs_st, dvm_sb, dvm_sh, dvm_st;
    float *lse, *delta;               // (B*H*L)
    int B, H, L, D;
    DropCfg drop;
    int drop_on;                      // dropout_p > 0
};

constexpr float kLog2eC = 1.4426950408889634f;
constexpr float kLazy = 8.f;  // log2 headroom before the running max moves

// MFMA operand register of one lane: 8 16-bit elements, or one fp32.
template <typename T> struct OpT { typedef typename Elt<T>::v8 type; };
template <> struct OpT<float> { typedef float type; };

template <typename T> struct CT;
template <> struct CT<bf16_t> { typedef bf16x8 v8; typedef bf16x4 v4; };
template <> struct CT<fp16_t> { typedef fp16x8 v8; typedef fp16x4 v4; };

// N consecutive logits of `row` at key k as fp32; keys >= L read -inf. VEC:
// the row start is 16-byte aligned (k is a multiple of N), so full groups
// use vector loads.
template <typename T, int N, bool VEC>
__device__ __forceinline__ void load_logits(const T* row, int k, int L, float out[N]) {
    if (VEC && k + N <= L) {
        if constexpr (sizeof(T) == 2) {
            if constexpr (N == 8) {
                const typename CT<T>::v8 x = *reinterpret_cast<const typename CT<T>::v8*>(row + k);
#pragma unroll
                for (int j = 0; j < 8; ++j) out[j] = (float)x[j];
            } else {
                const typename CT<T>::v4 x = *reinterpret_cast<const typename CT<T>::v4*>(row + k);
#pragma unroll
                for (int j = 0; j < 4; ++j) out[j] = (float)x[j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < N; j += 4) {
                const f32x4 x = *reinterpret_cast<const f32x4*>(row + k + j);
#pragma unroll
                for (int t = 0; t < 4; ++t) out[j + t] = x[t];
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < N; ++j) out[j] = (k + j < L) ? (float)row[k + j] : -INFINITY;
    }
}

// Bit j set when mask[k + j] is nonzero (keys >= L read 0). VEC: unit key
// stride and 8-byte aligned rows.
template <int N, bool VEC>
__device__ __forceinline__ unsigned load_mask(const uint8_t* row, int64_t sk, int k, int L) {
    unsigned bits = 0;
    if (VEC && k + N <= L) {
        uint64_t x;
        if constexpr (N == 8) x = *reinterpret_cast<const uint64_t*>(row + k);
        else x = *reinterpret_cast<const uint32_t*>(row + k);
#pragma unroll
        for (int j = 0; j < N; ++j) bits |= (((x >> (8 * j)) & 0xff) != 0) << j;
    } else {
#pragma unroll
        for (int j = 0; j < N; ++j)
            if (k + j < L && row[(int64_t)(k + j) * sk]) bits |= 1u << j;
    }
    return bits;
}

// 4 consecutive elements at row[d] as fp32 (d % 4 == 0, d < D, D % 8 == 0).
template <typename T>
__device__ __forceinline__ void load4f(const T* row, int d, float out[4]) {
    if constexpr (sizeof(T) == 2) {
        const typename CT<T>::v4 x = *reinterpret_cast<const typename CT<T>::v4*>(row + d);
#pragma unroll
        for (int j = 0; j < 4; ++j) out[j] = (float)x[j];
    } else {
        const f32x4 x = *reinterpret_cast<const f32x4*>(row + d);
#pragma unroll
        for (int j = 0; j < 4; ++j) out[j] = x[j];
    }
}

template <typename T>
__device__ __forceinline__ void store4(T* row, int d, const float v[4]) {
    if constexpr (sizeof(T) == 2) {
        typename CT<T>::v4 x;
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = (T)v[j];
        *reinterpret_cast<typename CT<T>::v4*>(row + d) = x;
    } else {
        *reinterpret_cast<f32x4*>(row + d) = f32x4{v[0], v[1], v[2], v[3]};
    }
}

// 8 elements [d0, d0 + 8) of a 16-bit row as an MFMA operand; dims >= D and
// invalid rows read 0.
template <typename T>
__device__ __forceinline__ typename CT<T>::v8 load8op(const T* row, int d0, int D, bool valid) {
    typename CT<T>::v8 r;
    if (valid && d0 < D) {
        r = *reinterpret_cast<const typename CT<T>::v8*>(row + d0);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = (T)0.f;
    }
    return r;
}

__device__ __forceinline__ void decode_bh(int bh, int H, int& b, int& h) {
    b = bh / H;
    h = bh - b * H;
}

// ---------------------------------------------------------------------------
// Forward (and the backward's statistics pass).
// ---------------------------------------------------------------------------
template <typename T, int ND, bool VEC, bool STATS, bool DROPK = true>
__global__ __launch_bounds__(256) void combine_fwd_kernel(CombineArgs a) {
    constexpr int KC = 64;               // keys per LDS stage
    constexpr int DP = ND * 32;          // head dim padded to the MFMA tile
    constexpr bool F32 = sizeof(T) == 4;
    constexpr int VT_RS = KC + 8;        // 16-bit: transposed V rows (one per dim)
    constexpr int VF_RS = DP + 4;        // fp32: V rows (one per key)
    constexpr int LDS_ELEMS = F32 ? 2 * KC * VF_RS : 2 * DP * VT_RS;
    __shared__ __align__(16) T lds[LDS_ELEMS];

    const int L = a.L, D = a.D;
    const int nqb = (L + 127) / 128;
    const int bid = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = bid / nqb, qb = bid - bh * nqb;
    int b, h;
    decode_bh(bh, a.H, b, h);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int col = lane & 31, half = lane >> 5;
    const int q = qb * 128 + wave * 32 + col;
    const int qc = min(q, L - 1);

    const T* il_row = (const T*)a.il + b * a.il_sb + h * a.il_sh + (int64_t)qc * a.il_st;
    const T* el_row = (const T*)a.el + b * a.el_sb + h * a.el_sh + (int64_t)qc * a.el_st;
    const uint8_t* m_row = a.mask + b * a.m_sb + (int64_t)qc * a.m_sq;
    const T* vs = (const T*)a.vs + b * a.vs_sb + h * a.vs_sh;
    const T* vm = (const T*)a.vm + b * a.vm_sb + h * a.vm_sh;

    f32x16 acc[ND];
#pragma unroll
    for (int n = 0; n < ND; ++n)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[n][i] = 0.f;
    float mref = -INFINITY, lsum = 0.f;
    const bool dropon = DROPK && a.drop_on != 0;
    const uint32_t drow = dropon ? drop_row(a.drop.lo, (uint32_t)bh, (uint32_t)q) : 0u;

    const int nch = D / 8;  // 8-element chunks per value row
    // 16-bit logits with 16-byte rows: the raw logits and mask bytes of the
    // next 16-key step are loaded while the current step's softmax runs.
    constexpr bool PF = VEC && !F32;
    typedef typename OpT<T>::type rv8;
    struct Raw {
        rv8 i, e;
        uint64_t m;
    };
    auto fetch = [&](int k, Raw& r) {
        if (PF && k + 8 <= L) {
            r.i = *reinterpret_cast<const rv8*>(il_row + k);
            r.e = *reinterpret_cast<const rv8*>(el_row + k);
            r.m = *reinterpret_cast<const uint64_t*>(m_row + k);
        }
    };
    Raw nxt;
    fetch(half * 8, nxt);
    for (int kc = 0; kc < L; kc += KC) {
        __syncthreads();
        // Stage the V tiles of both pathways (rows kc .. kc+KC-1; rows >= L
        // and dims >= D are zero).
        for (int c = tid; c < 2 * KC * (DP / 8); c += 256) {
            const int pw = c / (KC * (DP / 8));
            const int rem = c - pw * KC * (DP / 8);
            const int r = rem / (DP / 8), dc = rem - r * (DP / 8);
            const int key = kc + r;
            float x[8];
            if (key < L && dc < nch) {
                const T* src = (pw ? vm + (int64_t)key * a.vm_st : vs + (int64_t)key * a.vs_st) + dc * 8;
#pragma unroll
                for (int j = 0; j < 8; j += 4) load4f<T>(src, j, x + j);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) x[j] = 0.f;
            }
            if constexpr (F32) {
                float* dst = (float*)lds + pw * KC * VF_RS + r * VF_RS + dc * 8;
#pragma unroll
                for (int j = 0; j < 8; ++j) dst[j] = x[j];
            } else {
                T* dst = lds + pw * DP * VT_RS + (dc * 8) * VT_RS + r;
#pragma unroll
                for (int j = 0; j < 8; ++j) dst[j * VT_RS] = (T)x[j];
            }
        }
        __syncthreads();

#pragma unroll
        for (int ks = 0; ks < KC / 16; ++ks) {
            const int k = kc + ks * 16 + half * 8;
            float si[8], se[8];
            unsigned bits = 0;
            if (PF && k + 8 <= L) {
                const Raw cur = nxt;
                fetch(k + 16, nxt);
                if constexpr (PF) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        si[j] = (float)cur.i[j];
                        se[j] = (float)cur.e[j];
                        bits |= (((cur.m >> (8 * j)) & 0xff) != 0) << j;
                    }
                }
            } else {
                load_logits<T, 8, VEC>(il_row, k, L, si);
                load_logits<T, 8, VEC>(el_row, k, L, se);
                bits = load_mask<8, VEC>(m_row, a.m_sk, k, L);
            }
            float s[8];
            float cm = -INFINITY;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                s[j] = ((bits >> j) & 1 ? se[j] : si[j]) * kLog2eC;
                cm = fmaxf(cm, s[j]);
            }
            cm = fmaxf(cm, __shfl_xor(cm, 32));
            if (__any(cm > mref + kLazy)) {
                const float mn = fmaxf(mref, cm);
                const float f = (mn == -INFINITY) ? 1.f : fast_exp2(mref - mn);
#pragma unroll
                for (int n = 0; n < ND; ++n)
#pragma unroll
                    for (int i = 0; i < 16; ++i) acc[n][i] *= f;
                lsum *= f;
                mref = mn;
            }
            const float mu = (mref == -INFINITY) ? 0.f : mref;
            float pi[8], pe[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float p = fast_exp2(s[j] - mu);
                lsum += p;  // the row sum is over the undropped P
                if (dropon && !drop_keep(drow, a.drop.hi, (uint32_t)(k + j), a.drop.thr)) p = 0.f;
                const bool x = (bits >> j) & 1;
                pi[j] = x ? 0.f : p;
                pe[j] = x ? p : 0.f;
            }
            if constexpr (F32) {
                const float* Vs = (const float*)lds + (ks * 16 + half * 8) * VF_RS + col;
                const float* Vm = Vs + KC * VF_RS;
#pragma unroll
                for (int c = 0; c < 8; ++c)
#pragma unroll
                    for (int n = 0; n < ND; ++n) {
                        acc[n] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[c * VF_RS + n * 32], pi[c],
                                                                      acc[n], 0, 0, 0);
                        acc[n] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vm[c * VF_RS + n * 32], pe[c],
                                                                      acc[n], 0, 0, 0);
                    }
            } else {
                const typename Elt<T>::v8 bi = pack8<T>(pi), be = pack8<T>(pe);
#pragma unroll
                for (int n = 0; n < ND; ++n) {
                    const T* vt = lds + (n * 32 + col) * VT_RS + ks * 16 + half * 8;
                    const typename Elt<T>::v8 as = *reinterpret_cast<const typename Elt<T>::v8*>(vt);
                    const typename Elt<T>::v8 am =
                        *reinterpret_cast<const typename Elt<T>::v8*>(vt + DP * VT_RS);
                    acc[n] = Elt<T>::mma(as, bi, acc[n]);
                    acc[n] = Elt<T>::mma(am, be, acc[n]);
                }
            }
        }
    }

    const float lt = lsum + __shfl_xor(lsum, 32);
    const float inv = lt > 0.f ? (dropon ? a.drop.rkeep : 1.f) / lt : 0.f;
    const int64_t row = (int64_t)bh * L + qc;
    if (a.lse && q < L && half == 0) {
        const float mu = (mref == -INFINITY) ? 0.f : mref;
        a.lse[row] = lt > 0.f ? (mu + __log2f(lt)) * kLn2 : -INFINITY;
    }
    if constexpr (STATS) {
        const T* g = (const T*)a.go + b * a.g_sb + h * a.g_sh + (int64_t)qc * a.g_st;
        float dot = 0.f;
#pragma unroll
        for (int n = 0; n < ND; ++n)
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                const int d = n * 32 + gi * 8 + half * 4;
                if (d < D) {
                    float gg[4];
                    load4f<T>(g, d, gg);
#pragma unroll
                    for (int r = 0; r < 4; ++r) dot += gg[r] * acc[n][gi * 4 + r];
                }
            }
        dot = (dot + __shfl_xor(dot, 32)) * inv;
        if (q < L && half == 0) a.delta[row] = dot;
    } else {
        if (q < L) {
            T* o = (T*)a.out + b * a.o_sb + h * a.o_sh + (int64_t)q * a.o_st;
#pragma unroll
            for (int n = 0; n < ND; ++n)
#pragma unroll
                for (int gi = 0; gi < 4; ++gi) {
                    const int d = n * 32 + gi * 8 + half * 4;
                    if (d < D) {
                        float v[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) v[r] = acc[n][gi * 4 + r] * inv;
                        store4<T>(o, d, v);
                    }
                }
        }
    }
}

// ---------------------------------------------------------------------------
// Forward (and statistics pass) for 16-bit logits with 16-byte rows: the
// logit and mask tiles are copied into LDS with global_load_lds, four lanes
// per 64-byte row segment (row-contiguous reads instead of one 16-byte piece
// of 32 different rows per instruction), in a ring of NB stages of 32 keys
// per wavefront, so each wavefront keeps NB-1 stages of its logits in flight
// without holding them in registers. The V tiles of both pathways (32 keys,
// shared by the workgroup) ride in the same ring, stored row-major with the
// fused kernels' chunk swizzle and read transposed (ds_read_b64_tr_b16) as
// the A operand. Each lane then reads its 8 keys of its own query row from
// LDS (16-byte chunks XOR-swizzled by row: conflict-free) and runs the same
// lazy-max online softmax and MFMA accumulation as combine_fwd_kernel.
// ---------------------------------------------------------------------------
constexpr int kCKC = 32;  // keys per stage
#ifndef MPATTN_COMB_NB
#define MPATTN_COMB_NB 2
#endif
constexpr int kCNB = MPATTN_COMB_NB;  // stages in the ring

template <int D> struct CombTile {
    using TS = TileShape<D>;
    static constexpr int VT = kCKC * TS::RB;          // bytes of one V tile (32 rows)
    static constexpr int VSLOTS = kCKC * TS::NCH;     // 16-byte chunks per V tile
    static constexpr int VINS = (VSLOTS + 63) / 64;   // copy instructions per V tile
    static constexpr int LG = 32 * kCKC * 2;          // one logit tile: 32 rows x 32 keys (16-bit)
    static constexpr int MK = 32 * kCKC;              // mask tile: 32 rows x 32 bytes
    static constexpr int WAVE = 2 * LG + MK;          // per-wave part of a stage
    static constexpr int STAGE = 4 * WAVE + 2 * VT;   // one ring stage of the workgroup
};

template <typename T, int D, bool STATS, bool DROPK>
__global__ __launch_bounds__(256) void combine_fwd_dma_kernel(CombineArgs a) {
    using TS = TileShape<D>;
    using CT_ = CombTile<D>;
    constexpr int ND = (D + 31) / 32;
    typedef typename Elt<T>::v8 v8;
    typedef short s4 __attribute__((ext_vector_type(4)));
    __shared__ __attribute__((aligned(1024))) char smem[kCNB * CT_::STAGE];

    const int L = a.L;
    const int nqb = (L + 127) / 128;
    const int bid = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = bid / nqb, qb = bid - bh * nqb;
    int b, h;
    decode_bh(bh, a.H, b, h);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, half = lane >> 5;
    const int q = qb * 128 + wave * 32 + col;
    const int qc = min(q, L - 1);
    // copy bases: the wave's first (clamped) row; rows past L re-read row L-1
    const int q0c = min(qb * 128 + wave * 32, L - 1);
    const char* il_b = (const char*)((const T*)a.il + b * a.il_sb + h * a.il_sh + (int64_t)q0c * a.il_st);
    const char* el_b = (const char*)((const T*)a.el + b * a.el_sb + h * a.el_sh + (int64_t)q0c * a.el_st);
    const char* m_b = (const char*)(a.mask + b * a.m_sb + (int64_t)q0c * a.m_sq);
    const char* vs_b = (const char*)((const T*)a.vs + b * a.vs_sb + h * a.vs_sh);
    const char* vm_b = (const char*)((const T*)a.vm + b * a.vm_sb + h * a.vm_sh);
    const unsigned il_rs = (unsigned)(a.il_st * 2), el_rs = (unsigned)(a.el_st * 2);
    const unsigned m_rs = (unsigned)a.m_sq;
    const unsigned vs_rs = (unsigned)(a.vs_st * 2), vm_rs = (unsigned)(a.vm_st * 2);

    // Per-lane copy offsets. Logits: instruction j covers rows 16j + lane/4,
    // physical 16-byte chunk lane%4 holding logical chunk (lane%4) ^ swizzle.
    int lrow[2], lchk[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int r = 16 * j + (lane >> 2);
        lrow[j] = min(q0c + r, L - 1) - q0c;
        lchk[j] = (lane & 3) ^ ((r >> 2) & 3);
    }
    const int mrow = min(q0c + (lane >> 1), L - 1) - q0c, mchk = lane & 1;
    const unsigned smem_base = lds_addr(smem);

    // Copy stage t (keys kc = 32 t ..) into ring slot bf; returns the number
    // of copy instructions this wave issued.
    auto issue = [&](int t, int bf) -> int {
        const int kc = t * kCKC;
        const unsigned sb = __builtin_amdgcn_readfirstlane(smem_base + bf * CT_::STAGE);
        const unsigned wb = sb + wave * CT_::WAVE;
        const int m0v = m0_save();
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            // a chunk starting at or past L is read from the row start (its keys are masked)
            const int k0 = kc + 8 * lchk[j];
            const unsigned cb = k0 < L ? (unsigned)k0 * 2u : 0u;
            dma16(il_b, (unsigned)lrow[j] * il_rs + cb, wb + j * 1024);
            dma16(el_b, (unsigned)lrow[j] * el_rs + cb, wb + CT_::LG + j * 1024);
        }
        {
            const int k0 = kc + 16 * mchk;
            dma16(m_b, (unsigned)mrow * m_rs + (k0 < L ? (unsigned)k0 : 0u), wb + 2 * CT_::LG);
        }
        int n = 5;
        // V tiles: instruction i of 2*VINS, spread over the waves
#pragma unroll
        for (int i = wave; i < 2 * CT_::VINS; i += 4) {
            const int ten = i / CT_::VINS, part = i % CT_::VINS;
            const int slot = part * 64 + lane;
            const unsigned ld = __builtin_amdgcn_readfirstlane(sb + 4 * CT_::WAVE + ten * CT_::VT + part * 1024);
            const int r = min(slot, CT_::VSLOTS - 1) / TS::NCH;
            const int cbv = TS::swz(r, slot % TS::NCH) * 16;
            const unsigned vo = (unsigned)min(kc + r, L - 1) * (ten ? vm_rs : vs_rs) + cbv;
            if constexpr (CT_::VSLOTS % 64 == 0) {
                dma16(ten ? vm_b : vs_b, vo, ld);
            } else if (slot < CT_::VSLOTS) {  // (D = 24: the last copy has 32 lanes)
                dma16(ten ? vm_b : vs_b, vo, ld);
            }
            ++n;
        }
        m0_restore(m0v);
        return n;
    };

    // V^T operand (as the fused forward): lane (tg, ti) reads rows
    // 8*(tg>>1) + 4*rr + ti/4 of chunk 8*db + 4*(tg&1) + ti%4 (8-byte halves).
    const int tg = lane >> 4, ti = lane & 15;
    int voffv[ND][2];
#pragma unroll
    for (int db = 0; db < ND; ++db) {
        int e = 8 * db + 4 * (tg & 1) + (ti & 3);
        if (8 * e >= TS::RB) e = ti & 3;
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
            const int row = 8 * (tg >> 1) + 4 * rr + (ti >> 2);
            voffv[db][rr] = row * TS::RB + TS::swz(row, e >> 1) * 16 + (e & 1) * 8;
        }
    }
    auto vop = [&](const char* tile, int cc, int db) -> v8 {
        s4 hv[2];
#pragma unroll
        for (int rr = 0; rr < 2; ++rr)
            hv[rr] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s4*)(tile + 16 * cc * TS::RB + voffv[db][rr]));
        return __builtin_bit_cast(v8, __builtin_shufflevector(hv[0], hv[1], 0, 1, 2, 3, 4, 5, 6, 7));
    };

    f32x16 acc[ND];
#pragma unroll
    for (int n = 0; n < ND; ++n)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[n][i] = 0.f;
    float mref = -INFINITY, lsum = 0.f;
    const bool dropon = DROPK && a.drop_on != 0;
    const uint32_t drow = dropon ? drop_row(a.drop.lo, (uint32_t)bh, (uint32_t)q) : 0u;

    const int nst = (L + kCKC - 1) / kCKC;
    int pend[kCNB];
#pragma unroll
    for (int t = 0; t < kCNB; ++t) pend[t] = 0;
#pragma unroll
    for (int t = 0; t < kCNB - 1; ++t)
        if (t < nst) pend[t] = issue(t, t);
    int bf = 0;
    for (int t = 0; t < nst; ++t) {
        int allow = 0;
#pragma unroll
        for (int k = 1; k < kCNB - 1; ++k) allow += pend[k];
        wait_vm_var(allow);
        stage_barrier();
#pragma unroll
        for (int k = 0; k < kCNB - 1; ++k) pend[k] = pend[k + 1];
        pend[kCNB - 1] = 0;
        if (t + kCNB - 1 < nst) pend[kCNB - 2] = issue(t + kCNB - 1, bf == 0 ? kCNB - 1 : bf - 1);
        const char* sg = smem + bf * CT_::STAGE;
        const char* wb = sg + wave * CT_::WAVE;
        const char* vst = sg + 4 * CT_::WAVE;
        const int kc = t * kCKC;
        // TAIL: the last stage, whose keys past L are masked
        auto stage_steps = [&](auto tail_c) {
            constexpr bool tail = decltype(tail_c)::value;
#pragma unroll
        for (int ks = 0; ks < kCKC / 16; ++ks) {
            const int k = kc + ks * 16 + half * 8;
            const int lc = ks * 2 + half;  // logical 16-byte chunk of the row
            const int pc = lc ^ ((col >> 2) & 3);
            const v8 ri = *reinterpret_cast<const v8*>(wb + col * 64 + pc * 16);
            const v8 re = *reinterpret_cast<const v8*>(wb + CT_::LG + col * 64 + pc * 16);
            const uint2 mw = *reinterpret_cast<const uint2*>(wb + 2 * CT_::LG + col * 32 + ks * 16 + half * 8);
            // Selected raw logits (natural units; the log2(e) factor goes into
            // the exp2 argument) and their max.
            bool x[8];
            float v[8];
            float cm = -INFINITY;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                x[j] = (((j < 4 ? mw.x : mw.y) >> (8 * (j & 3))) & 0xffu) != 0;
                v[j] = x[j] ? (float)re[j] : (float)ri[j];
                if (tail && k + j >= L) v[j] = -INFINITY;
            }
#pragma unroll
            for (int j = 0; j < 8; j += 2) cm = fmaxf(cm, fmaxf(v[j], v[j + 1]));
            cm = fmaxf(cm, __shfl_xor(cm, 32)) * kLog2eC;
            if (__any(cm > mref + kLazy)) {
                const float mn = fmaxf(mref, cm);
                const float f = (mn == -INFINITY) ? 1.f : fast_exp2(mref - mn);
#pragma unroll
                for (int n = 0; n < ND; ++n)
#pragma unroll
                    for (int i = 0; i < 16; ++i) acc[n][i] *= f;
                lsum *= f;
                mref = mn;
            }
            const float mu = (mref == -INFINITY) ? 0.f : mref;
            float pi[8], pe[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float p = fast_exp2(fmaf(v[j], kLog2eC, -mu));
                lsum += p;  // the row sum is over the undropped P
                if (dropon && !drop_keep(drow, a.drop.hi, (uint32_t)(k + j), a.drop.thr)) p = 0.f;
                pi[j] = x[j] ? 0.f : p;
                pe[j] = x[j] ? p : 0.f;
            }
            const v8 bi = pack8<T>(pi), be = pack8<T>(pe);
#pragma unroll
            for (int n = 0; n < ND; ++n) {
                acc[n] = Elt<T>::mma(vop(vst, ks, n), bi, acc[n]);
                acc[n] = Elt<T>::mma(vop(vst + CT_::VT, ks, n), be, acc[n]);
            }
        }
        };
        if (kc + kCKC > L) stage_steps(std::true_type{});
        else stage_steps(std::false_type{});
        bf = bf + 1 == kCNB ? 0 : bf + 1;
    }

    const float lt = lsum + __shfl_xor(lsum, 32);
    const float inv = lt > 0.f ? (dropon ? a.drop.rkeep : 1.f) / lt : 0.f;
    const int64_t row = (int64_t)bh * L + qc;
    if (a.lse && q < L && half == 0) {
        const float mu = (mref == -INFINITY) ? 0.f : mref;
        a.lse[row] = lt > 0.f ? (mu + __log2f(lt)) * kLn2 : -INFINITY;
    }
    if constexpr (STATS) {
        const T* g = (const T*)a.go + b * a.g_sb + h * a.g_sh + (int64_t)qc * a.g_st;
        float dot = 0.f;
#pragma unroll
        for (int n = 0; n < ND; ++n)
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                const int d = n * 32 + gi * 8 + half * 4;
                if (d < D) {
                    float gg[4];
                    load4f<T>(g, d, gg);
#pragma unroll
                    for (int r = 0; r < 4; ++r) dot += gg[r] * acc[n][gi * 4 + r];
                }
            }
        dot = (dot + __shfl_xor(dot, 32)) * inv;
        if (q < L && half == 0) a.delta[row] = dot;
    } else {
        if (q < L) {
            T* o = (T*)a.out + b * a.o_sb + h * a.o_sh + (int64_t)q * a.o_st;
#pragma unroll
            for (int n = 0; n < ND; ++n)
#pragma unroll
                for (int gi = 0; gi < 4; ++gi) {
                    const int d = n * 32 + gi * 8 + half * 4;
                    if (d < D) {
                        float v[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) v[r] = acc[n][gi * 4 + r] * inv;
                        store4<T>(o, d, v);
                    }
                }
        }
    }
}

// 8 consecutive elements of a row from fp32 values (k % 8 == 0, row 16-byte
// aligned).
template <typename T>
__device__ __forceinline__ void store8(T* row, int k, const float v[8]) {
    if constexpr (sizeof(T) == 2) {
        typename CT<T>::v8 x;
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = (T)v[j];
        *reinterpret_cast<typename CT<T>::v8*>(row + k) = x;
    } else {
        *reinterpret_cast<f32x4*>(row + k) = f32x4{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f32x4*>(row + k + 4) = f32x4{v[4], v[5], v[6], v[7]};
    }
}

// ---------------------------------------------------------------------------
// Backward: dV and both d_logits (key-stationary, 64 keys per workgroup).
//
// Per 32-query chunk: every thread loads 8 consecutive keys of one query row
// of both logit tensors (16-byte loads, 8 threads per 128-byte row segment)
// and turns them into P with the row's LSE; P^T and the dO tile go to LDS.
// Wavefront (pathway pw, key half kw) then accumulates dV_pw^T += dO^T P_pw
// over the chunk and computes dW_pw^T = V_pw dO^T for its 32 keys (V rows held
// in registers for the whole kernel), written to LDS as fp32. Each thread
// finally reads dW of its own 8 keys for the selected pathway and writes
// dS = P (dW - Delta) into d_intra or d_inter with coalesced 16-byte stores.
// ---------------------------------------------------------------------------
// Register budget: 4 wavefronts per SIMD for D <= 32 (with the prefetch the
// compiler would otherwise settle at 3; it keeps 8 bytes of scratch), 3 for
// D = 64.
template <typename T, int ND, bool VEC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(ND == 1 ? 4 : 3))) void combine_bwd_kernel(
    CombineArgs a) {
    constexpr bool F32 = sizeof(T) == 4;
    constexpr int DP = ND * 32;
    // 16-bit: P^T [2][64 keys][32 q + 8], dO^T [DP][32 + 8], dO rows [32][DP + 8].
    // fp32:   P   [2][32 q][64 + 4],      dO rows [32][DP + 4].
    // both:   dW  fp32 [2][32 q][64 + 4].
    constexpr int PT_RS = 40, GT_RS = 40, GR_RS = DP + 8;
    constexpr int PF_RS = 68, GF_RS = DP + 4, W_RS = 68;
    constexpr int P_ELEMS = F32 ? 2 * 32 * PF_RS : 2 * 64 * PT_RS;
    constexpr int G_ELEMS = F32 ? 32 * GF_RS : DP * GT_RS + 32 * GR_RS;
    __shared__ __align__(16) T lp[P_ELEMS];
    __shared__ __align__(16) T lg[G_ELEMS];
    __shared__ __align__(16) float lw[2 * 32 * W_RS];
    T* lgr = lg + (F32 ? 0 : DP * GT_RS);  // dO rows

    const int L = a.L, D = a.D;
    const int nkb = (L + 63) / 64;
    const int bid = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = bid / nkb, kb = bid - bh * nkb;
    int b, h;
    decode_bh(bh, a.H, b, h);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int col = lane & 31, half = lane >> 5;
    const int pw = wave >> 1, kw = (wave & 1) * 32;

    const T* il = (const T*)a.il + b * a.il_sb + h * a.il_sh;
    const T* el = (const T*)a.el + b * a.el_sb + h * a.el_sh;
    T* dil = (T*)a.dil + b * a.dil_sb + h * a.dil_sh;
    T* del = (T*)a.del + b * a.del_sb + h * a.del_sh;
    const uint8_t* mk = a.mask + b * a.m_sb;
    const T* g = (const T*)a.go + b * a.g_sb + h * a.g_sh;
    const float* lse = a.lse + (int64_t)bh * L;
    const float* dlt = a.delta + (int64_t)bh * L;

    // A operand of dW^T = V dO^T: this wavefront's 32 V rows (k = head dim).
    const int vkey = kb * 64 + kw + col;
    const bool vkv = vkey < L;
    const T* vrow = pw ? (const T*)a.vm + b * a.vm_sb + h * a.vm_sh + (int64_t)min(vkey, L - 1) * a.vm_st
                       : (const T*)a.vs + b * a.vs_sb + h * a.vs_sh + (int64_t)min(vkey, L - 1) * a.vs_st;
    constexpr int NS16 = ND * 2;
    typename OpT<T>::type vop[F32 ? ND * 16 : NS16];
    if constexpr (F32) {
#pragma unroll
        for (int c = 0; c < ND * 16; ++c) {
            const int d = 2 * c + half;
            vop[c] = (vkv && d < D) ? (float)vrow[d] : 0.f;
        }
    } else {
#pragma unroll
        for (int s = 0; s < NS16; ++s) vop[s] = load8op<T>(vrow, s * 16 + half * 8, D, vkv);
    }

    // Loader role: thread -> (query row tq of the chunk, 8-key group tg).
    const int tq = tid >> 3, tg = tid & 7;
    const int k8 = kb * 64 + tg * 8;

    f32x16 acc[ND];
#pragma unroll
    for (int n = 0; n < ND; ++n)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[n][i] = 0.f;

    const int nch = D / 8;
    const bool dropon = a.drop_on != 0;
    // 16-bit logits with 16-byte rows: the next step's raw logits, mask
    // bytes, LSE and Delta are loaded while the current step runs.
    constexpr bool PF = VEC && !F32;
    typedef typename OpT<T>::type rv8;
    const bool pfk = PF && k8 + 8 <= L;
    rv8 ni, ne;
    uint64_t nm = 0;
    float nl = 0.f, nd = 0.f;
    // The next step's dO chunk of this thread (16-bit: rows of 16-byte
    // multiples; at most one chunk per thread): row q0 + gr, dims 8*gdc..
    const int gr = tid / (DP / 8), gdc = tid % (DP / 8);
    const bool gown = PF && tid < 32 * (DP / 8);
    rv8 ngo{};
    auto fetch = [&](int q) {
        const int qc = min(q, L - 1);
        if (pfk) {
            ni = *reinterpret_cast<const rv8*>(il + (int64_t)qc * a.il_st + k8);
            ne = *reinterpret_cast<const rv8*>(el + (int64_t)qc * a.el_st + k8);
            nm = *reinterpret_cast<const uint64_t*>(mk + (int64_t)qc * a.m_sq + k8);
        }
        nl = lse[qc];
        nd = dlt[qc];
        if constexpr (PF) {
            const int qr = q - tq + gr;  // (q is the step's first row + tq)
            if (gown && qr < L && gdc < nch) ngo = *reinterpret_cast<const rv8*>(g + (int64_t)qr * a.g_st + gdc * 8);
        }
    };
    fetch(tq);
    for (int q0 = 0; q0 < L; q0 += 32) {
        const int qq = q0 + tq;
        const int qc = min(qq, L - 1);
        float p[8];
        unsigned bits = 0, keep = 0xFFu;  // keep: dropout bits of the 8 keys
        float dq;
        __syncthreads();
        {
            float si[8], se[8];
            if (pfk) {
                if constexpr (PF) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        si[j] = (float)ni[j];
                        se[j] = (float)ne[j];
                        bits |= (((nm >> (8 * j)) & 0xff) != 0) << j;
                    }
                }
            } else {
                load_logits<T, 8, VEC>(il + (int64_t)qc * a.il_st, k8, L, si);
                load_logits<T, 8, VEC>(el + (int64_t)qc * a.el_st, k8, L, se);
                bits = load_mask<8, VEC>(mk + (int64_t)qc * a.m_sq, a.m_sk, k8, L);
            }
            const float l = nl;
            dq = nd;
            if constexpr (!PF)
                if (q0 + 32 < L) fetch(qq + 32);
            const bool ok = qq < L && l > -INFINITY;
            const float l2 = ok ? l * kLog2eC : 0.f;
            if (dropon) {
                const uint32_t drow = drop_row(a.drop.lo, (uint32_t)bh, (uint32_t)qq);
                keep = 0;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    keep |= (unsigned)drop_keep(drow, a.drop.hi, (uint32_t)(k8 + j), a.drop.thr) << j;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const bool x = (bits >> j) & 1;
                p[j] = ok ? fast_exp2((x ? se[j] : si[j]) * kLog2eC - l2) : 0.f;
                const float pz = (keep >> j) & 1 ? p[j] : 0.f;  // the dV operand: Z P
                if constexpr (F32) {
                    float* P = (float*)lp;
                    P[tq * PF_RS + tg * 8 + j] = x ? 0.f : pz;
                    P[32 * PF_RS + tq * PF_RS + tg * 8 + j] = x ? pz : 0.f;
                } else {
                    lp[(tg * 8 + j) * PT_RS + tq] = (T)(x ? 0.f : pz);
                    lp[64 * PT_RS + (tg * 8 + j) * PT_RS + tq] = (T)(x ? pz : 0.f);
                }
            }
        }
        // dO rows q0 .. q0+31 (rows >= L and dims >= D are zero); 16-bit:
        // this thread's chunk was loaded with the previous step's fetch.
        const rv8 cgo = ngo;
        if constexpr (PF)
            if (q0 + 32 < L) fetch(qq + 32);
        for (int c = tid; c < 32 * (DP / 8); c += 256) {
            const int r = c / (DP / 8), dc = c - r * (DP / 8);
            const int qr = q0 + r;
            float x[8];
            if (qr < L && dc < nch) {
                if constexpr (PF) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) x[j] = (float)cgo[j];
                } else {
                    const T* src = g + (int64_t)qr * a.g_st + dc * 8;
#pragma unroll
                    for (int j = 0; j < 8; j += 4) load4f<T>(src, j, x + j);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) x[j] = 0.f;
            }
            if constexpr (F32) {
                float* G = (float*)lg + r * GF_RS + dc * 8;
#pragma unroll
                for (int j = 0; j < 8; ++j) G[j] = x[j];
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) lg[(dc * 8 + j) * GT_RS + r] = (T)x[j];
                typename CT<T>::v8 xv;
#pragma unroll
                for (int j = 0; j < 8; ++j) xv[j] = (T)x[j];
                *reinterpret_cast<typename CT<T>::v8*>(lgr + r * GR_RS + dc * 8) = xv;
            }
        }
        __syncthreads();
        f32x16 dw;
#pragma unroll
        for (int i = 0; i < 16; ++i) dw[i] = 0.f;
        if constexpr (F32) {
            const float* P = (const float*)lp + pw * 32 * PF_RS + kw + col;
            const float* G = (const float*)lg + col;
            const float* Gq = (const float*)lg + col * GF_RS;
#pragma unroll 4
            for (int c = 0; c < 16; ++c) {
                const int qr = 2 * c + half;
                const float bp = P[qr * PF_RS];
#pragma unroll
                for (int n = 0; n < ND; ++n)
                    acc[n] = __builtin_amdgcn_mfma_f32_32x32x2f32(G[qr * GF_RS + n * 32], bp, acc[n],
                                                                  0, 0, 0);
            }
#pragma unroll
            for (int c = 0; c < ND * 16; ++c)
                dw = __builtin_amdgcn_mfma_f32_32x32x2f32(vop[c], Gq[2 * c + half], dw, 0, 0, 0);
        } else {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const typename Elt<T>::v8 bp = *reinterpret_cast<const typename Elt<T>::v8*>(
                    lp + pw * 64 * PT_RS + (kw + col) * PT_RS + s * 16 + half * 8);
#pragma unroll
                for (int n = 0; n < ND; ++n) {
                    const typename Elt<T>::v8 ag = *reinterpret_cast<const typename Elt<T>::v8*>(
                        lg + (n * 32 + col) * GT_RS + s * 16 + half * 8);
                    acc[n] = Elt<T>::mma(ag, bp, acc[n]);
                }
            }
#pragma unroll
            for (int s = 0; s < NS16; ++s) {
                const typename Elt<T>::v8 bg = *reinterpret_cast<const typename Elt<T>::v8*>(
                    lgr + col * GR_RS + s * 16 + half * 8);
                dw = Elt<T>::mma(vop[s], bg, dw);
            }
        }
        // dW^T accumulator slot 4*gi + r: key kw + 8*gi + 4*half + r, query col.
#pragma unroll
        for (int gi = 0; gi < 4; ++gi)
            *reinterpret_cast<f32x4*>(lw + pw * 32 * W_RS + col * W_RS + kw + gi * 8 + half * 4) =
                f32x4{dw[gi * 4], dw[gi * 4 + 1], dw[gi * 4 + 2], dw[gi * 4 + 3]};
        __syncthreads();
        if (qq < L) {
            const float* ws = lw + tq * W_RS + tg * 8;
            const float* wm = ws + 32 * W_RS;
            float di[8], de[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const bool x = (bits >> j) & 1;
                float w = x ? wm[j] : ws[j];
                if (dropon) w = (keep >> j) & 1 ? w * a.drop.rkeep : 0.f;
                const float ds = p[j] * (w - dq);
                di[j] = x ? 0.f : ds;
                de[j] = x ? ds : 0.f;
            }
            T* ri = dil + (int64_t)qq * a.dil_st;
            T* re = del + (int64_t)qq * a.del_st;
            if (VEC && k8 + 8 <= L) {
                store8<T>(ri, k8, di);
                store8<T>(re, k8, de);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (k8 + j < L) {
                        ri[k8 + j] = (T)di[j];
                        re[k8 + j] = (T)de[j];
                    }
            }
        }
    }

    const int key = kb * 64 + kw + col;
    if (key < L) {
        T* dv = pw ? (T*)a.dvm + b * a.dvm_sb + h * a.dvm_sh + (int64_t)key * a.dvm_st
                   : (T*)a.dvs + b * a.dvs_sb + h * a.dvs_sh + (int64_t)key * a.dvs_st;
#pragma unroll
        for (int n = 0; n < ND; ++n)
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                const int d = n * 32 + gi * 8 + half * 4;
                if (d < D) {
                    float v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) v[r] = acc[n][gi * 4 + r] * (dropon ? a.drop.rkeep : 1.f);
                    store4<T>(dv, d, v);
                }
            }
    }
}

bool aligned_rows(const void* p, int64_t sb, int64_t sh, int64_t st, int es);

// The DMA-staged forward / statistics pass for 16-bit inputs whose logit,
// mask and value rows are 16-byte aligned (mask bytes unit-strided).
bool dma_ok(const CombineArgs& a) {
    const bool lg = aligned_rows(a.il, a.il_sb, a.il_sh, a.il_st, 2) && aligned_rows(a.el, a.el_sb, a.el_sh, a.el_st, 2);
    const bool mk = a.m_sk == 1 && (uintptr_t)a.mask % 16 == 0 && a.m_sb % 16 == 0 && a.m_sq % 16 == 0;
    const bool v = aligned_rows(a.vs, a.vs_sb, a.vs_sh, a.vs_st, 2) && aligned_rows(a.vm, a.vm_sb, a.vm_sh, a.vm_st, 2);
    return lg && mk && v;
}

template <typename T, int D, bool STATS>
void launch_dma_d(const CombineArgs& a, hipStream_t st) {
    const unsigned grid = (unsigned)(a.B * a.H * ((a.L + 127) / 128));
    if (a.drop_on)
        hipLaunchKernelGGL((combine_fwd_dma_kernel<T, D, STATS, true>), dim3(grid), dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((combine_fwd_dma_kernel<T, D, STATS, false>), dim3(grid), dim3(256), 0, st, a);
}

template <typename T, bool STATS>
void launch_dma(const CombineArgs& a, hipStream_t st) {
    switch (a.D) {
        case 16: launch_dma_d<T, 16, STATS>(a, st); break;
        case 24: launch_dma_d<T, 24, STATS>(a, st); break;
        case 32: launch_dma_d<T, 32, STATS>(a, st); break;
        default: launch_dma_d<T, 64, STATS>(a, st); break;
    }
}

// Delta = dO . O per row from the forward's output, for a backward given
// the forward's LSE (no statistics pass): 8 lanes per row, 8 dims each.
template <typename T>
__global__ __launch_bounds__(256) void combine_delta_kernel(const CombineArgs a) {
    const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t row = item >> 3;  // (b * H + h) * L + q
    const int c = (int)(item & 7);
    const int64_t nrow = (int64_t)a.B * a.H * a.L;
    float dot = 0.f;
    if (row < nrow && c * 8 < a.D) {
        const int q = (int)(row % a.L);
        const int bh = (int)(row / a.L);
        const int b = bh / a.H, h = bh % a.H;
        const T* o = (const T*)a.out + b * a.o_sb + h * a.o_sh + (int64_t)q * a.o_st;
        const T* g = (const T*)a.go + b * a.g_sb + h * a.g_sh + (int64_t)q * a.g_st;
#pragma unroll
        for (int k = 0; k < 8; k += 4) {
            float x[4], y[4];
            load4f<T>(o, c * 8 + k, x);
            load4f<T>(g, c * 8 + k, y);
#pragma unroll
            for (int r = 0; r < 4; ++r) dot += x[r] * y[r];
        }
    }
    dot += __shfl_xor(dot, 4);
    dot += __shfl_xor(dot, 2);
    dot += __shfl_xor(dot, 1);
    if (row < nrow && c == 0) a.delta[row] = dot;
}

// mode 0: forward; 1: backward with its statistics pass; 2: backward given
// the forward's LSE and O (Delta from them, no pass over the logits).
template <typename T, int ND, bool VEC>
hipError_t launch_combine_t(const CombineArgs& a, int mode, hipStream_t st) {
    const int nqb = (a.L + 127) / 128, nkb = (a.L + 63) / 64;
    const int bh = a.B * a.H;
    if (mode == 2) {
        const int64_t nrow = (int64_t)bh * a.L;
        hipLaunchKernelGGL(combine_delta_kernel<T>, dim3((unsigned)((nrow * 8 + 255) / 256)), dim3(256), 0, st, a);
        hipLaunchKernelGGL((combine_bwd_kernel<T, ND, VEC>), dim3(bh * nkb), dim3(256), 0, st, a);
        return hipGetLastError();
    }
    if constexpr (sizeof(T) == 2 && VEC) {
        if (dma_ok(a)) {
            if (mode == 0) {
                launch_dma<T, false>(a, st);
                return hipGetLastError();
            }
            launch_dma<T, true>(a, st);
            hipLaunchKernelGGL((combine_bwd_kernel<T, ND, VEC>), dim3(bh * nkb), dim3(256), 0, st, a);
            return hipGetLastError();
        }
    }
    // Without dropout the forward is instantiated with no dropout code.
    if (mode == 0) {
        if (a.drop_on)
            hipLaunchKernelGGL((combine_fwd_kernel<T, ND, VEC, false, true>), dim3(bh * nqb), dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL((combine_fwd_kernel<T, ND, VEC, false, false>), dim3(bh * nqb), dim3(256), 0, st, a);
    } else {
        if (a.drop_on)
            hipLaunchKernelGGL((combine_fwd_kernel<T, ND, VEC, true, true>), dim3(bh * nqb), dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL((combine_fwd_kernel<T, ND, VEC, true, false>), dim3(bh * nqb), dim3(256), 0, st, a);
        hipLaunchKernelGGL((combine_bwd_kernel<T, ND, VEC>), dim3(bh * nkb), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

template <typename T>
hipError_t launch_combine_d(const CombineArgs& a, bool vec, int mode, hipStream_t st) {
    if (a.D <= 32) return vec ? launch_combine_t<T, 1, true>(a, mode, st) : launch_combine_t<T, 1, false>(a, mode, st);
    return vec ? launch_combine_t<T, 2, true>(a, mode, st) : launch_combine_t<T, 2, false>(a, mode, st);
}

bool aligned_rows(const void* p, int64_t sb, int64_t sh, int64_t st, int es) {
    const int64_t q = 16 / es;
    return (uintptr_t)p % 16 == 0 && sb % q == 0 && sh % q == 0 && st % q == 0;
}

void fill_common(CombineArgs& a, const mpattn_tensor& il, const mpattn_tensor& el,
                 const mpattn_tensor& vs, const mpattn_tensor& vm, const uint8_t* mask, int64_t msb,
                 int64_t msq, int64_t msk, int B, int H, int L, int D) {
    a.il = il.ptr; a.il_sb = il.stride_b; a.il_sh = il.stride_h; a.il_st = il.stride_t;
    a.el = el.ptr; a.el_sb = el.stride_b; a.el_sh = el.stride_h; a.el_st = el.stride_t;
    a.vs = vs.ptr; a.vs_sb = vs.stride_b; a.vs_sh = vs.stride_h; a.vs_st = vs.stride_t;
    a.vm = vm.ptr; a.vm_sb = vm.stride_b; a.vm_sh = vm.stride_h; a.vm_st = vm.stride_t;
    a.mask = mask; a.m_sb = msb; a.m_sq = msq; a.m_sk = msk;
    a.B = B; a.H = H; a.L = L; a.D = D;
}

// Whether the logits and mask admit the vector-load path.
bool vec_ok(const CombineArgs& a, int es) {
    const bool lg = aligned_rows(a.il, a.il_sb, a.il_sh, a.il_st, es) &&
                    aligned_rows(a.el, a.el_sb, a.el_sh, a.el_st, es);
    const bool mk = a.m_sk == 1 && (uintptr_t)a.mask % 8 == 0 && a.m_sb % 8 == 0 && a.m_sq % 8 == 0;
    return lg && mk;
}

}  // namespace

int64_t combine_ws_offset_delta(int B, int H, int L) {
    return (((int64_t)B * H * L * 4) + 255) / 256 * 256;
}

int64_t combine_bwd_workspace_bytes(int B, int H, int L) {
    return 2 * combine_ws_offset_delta(B, H, L);
}

hipError_t launch_combine_fwd(const mpattn_combine_fwd_params& p, float* lse_buf, hipStream_t st) {
    CombineArgs a{};
    fill_common(a, p.intra_logits, p.inter_logits, p.intra_values, p.inter_values, p.chain_mask,
                p.mask_stride_b, p.mask_stride_q, p.mask_stride_k, p.B, p.H, p.L, p.D);
    a.out = (void*)p.out.ptr; a.o_sb = p.out.stride_b; a.o_sh = p.out.stride_h; a.o_st = p.out.stride_t;
    a.lse = lse_buf;
    a.drop = drop_cfg(p.dropout_p, p.dropout_seed);
    a.drop_on = p.dropout_p > 0.f;
    const int es = p.dtype == MPATTN_FP32 ? 4 : 2;
    const bool vec = vec_ok(a, es);
    switch (p.dtype) {
        case MPATTN_BF16: return launch_combine_d<bf16_t>(a, vec, 0, st);
        case MPATTN_FP16: return launch_combine_d<fp16_t>(a, vec, 0, st);
        default: return launch_combine_d<float>(a, vec, 0, st);
    }
}

hipError_t launch_combine_bwd(const mpattn_combine_bwd_params& p, hipStream_t st) {
    CombineArgs a{};
    fill_common(a, p.intra_logits, p.inter_logits, p.intra_values, p.inter_values, p.chain_mask,
                p.mask_stride_b, p.mask_stride_q, p.mask_stride_k, p.B, p.H, p.L, p.D);
    a.go = p.grad_out.ptr; a.g_sb = p.grad_out.stride_b; a.g_sh = p.grad_out.stride_h;
    a.g_st = p.grad_out.stride_t;
    a.dil = (void*)p.d_intra_logits.ptr; a.dil_sb = p.d_intra_logits.stride_b;
    a.dil_sh = p.d_intra_logits.stride_h; a.dil_st = p.d_intra_logits.stride_t;
    a.del = (void*)p.d_inter_logits.ptr; a.del_sb = p.d_inter_logits.stride_b;
    a.del_sh = p.d_inter_logits.stride_h; a.del_st = p.d_inter_logits.stride_t;
    a.dvs = (void*)p.d_intra_values.ptr; a.dvs_sb = p.d_intra_values.stride_b;
    a.dvs_sh = p.d_intra_values.stride_h; a.dvs_st = p.d_intra_values.stride_t;
    a.dvm = (void*)p.d_inter_values.ptr; a.dvm_sb = p.d_inter_values.stride_b;
    a.dvm_sh = p.d_inter_values.stride_h; a.dvm_st = p.d_inter_values.stride_t;
    a.drop = drop_cfg(p.dropout_p, p.dropout_seed);
    a.drop_on = p.dropout_p > 0.f;
    char* ws = (char*)p.workspace;
    a.lse = (float*)ws;
    a.delta = (float*)(ws + combine_ws_offset_delta(p.B, p.H, p.L));
    int mode = 1;
    if (p.lse) {  // the forward's statistics (read only)
        a.lse = const_cast<float*>(p.lse);
        a.out = (void*)p.out.ptr; a.o_sb = p.out.stride_b; a.o_sh = p.out.stride_h; a.o_st = p.out.stride_t;
        mode = 2;
    }
    const int es = p.dtype == MPATTN_FP32 ? 4 : 2;
    // the d_logits stores use the same vector path as the logit loads
    const bool vec = vec_ok(a, es) &&
                     aligned_rows(a.dil, a.dil_sb, a.dil_sh, a.dil_st, es) &&
                     aligned_rows(a.del, a.del_sb, a.del_sh, a.del_st, es);
    switch (p.dtype) {
        case MPATTN_BF16: return launch_combine_d<bf16_t>(a, vec, mode, st);
        case MPATTN_FP16: return launch_combine_d<fp16_t>(a, vec, mode, st);
        default: return launch_combine_d<float>(a, vec, mode, st);
    }
}

}  // namespace mpattn
