// Shared device helpers for the gfx950 multi-pathway attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mpattn.h"

namespace mpattn {

typedef __bf16 bf16_t;
typedef _Float16 fp16_t;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 fp16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 fp16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 fp16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Marks a padded key in the per-tile chain-id staging buffers. Real chain ids
// must be larger than this value.
constexpr int kPadChain = INT32_MIN;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// 16-bit element traits: the 8-wide MFMA operand vector and the
// 32x32x16 MFMA (gfx950) that consumes it.
template <typename T> struct Elt;

template <> struct Elt<bf16_t> {
    typedef bf16x8 v8;
    typedef bf16x4 v4;
    typedef bf16x2 v2;
    static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4 mma16(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    // acc + x[0] + x[1] in fp32 (v_dot2_f32_bf16 against (1, 1)).
    static __device__ __forceinline__ float sum2(v2 x, float acc) {
        const v2 one = {(bf16_t)1.0f, (bf16_t)1.0f};
        return __builtin_amdgcn_fdot2_f32_bf16(x, one, acc, false);
    }
    // acc + x[0]^2 + x[1]^2 in fp32.
    static __device__ __forceinline__ float sq2(v2 x, float acc) {
        return __builtin_amdgcn_fdot2_f32_bf16(x, x, acc, false);
    }
};

template <> struct Elt<fp16_t> {
    typedef fp16x8 v8;
    typedef fp16x4 v4;
    typedef fp16x2 v2;
    static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4 mma16(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ float sum2(v2 x, float acc) {
        const v2 one = {(fp16_t)1.0f, (fp16_t)1.0f};
        return __builtin_amdgcn_fdot2(x, one, acc, false);
    }
    static __device__ __forceinline__ float sq2(v2 x, float acc) {
        return __builtin_amdgcn_fdot2(x, x, acc, false);
    }
};

// fp32 rows, for the kernels that handle every element type alike (the
// backward's prep: Delta, LSE2 and the RoPE-rotated operands).
typedef float f32x8 __attribute__((ext_vector_type(8)));
template <> struct Elt<float> {
    typedef f32x8 v8;
};

__device__ __forceinline__ float fast_exp2(float x) {
    return __builtin_amdgcn_exp2f(x);
}

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup i runs on
// XCD i % 8). Remap so each XCD receives one contiguous range of logical ids:
// neighbouring logical ids (query blocks of the same (b, h)) then share an
// L2 and reuse each other's K/V tiles.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
    constexpr int kXcd = 8;
    const int xcd = bid % kXcd, slot = bid / kXcd;
    const int per = nblocks / kXcd, rem = nblocks % kXcd;
    return xcd * per + (xcd < rem ? xcd : rem) + slot;
}

// Position `slot` of the share of XCD `xcd` -> (row block, b*H + h), for
// nblk_bh row blocks per (b, h) and ngrp whole (b, h) groups per share (the
// share of XCD x is groups [x*ngrp, (x+1)*ngrp), so their shared operands
// stay in that XCD's L2). The share is walked in runs of a few groups whose
// shared operands (`group_bytes` each) fit together in `budget` bytes of
// L2. With `sums` (one int4 {min chain, max chain, #padded, -} per 32 rows
// of each batch row, `nsum` of them valid, `rows32` of them per block),
// inside a run the blocks whose rows span two chains (about twice the work
// per stage; with pad_heavy also those holding padded rows) come first, so
// they overlap the others instead of extending the last round. Results are
// wavefront-uniform.
__device__ inline void order_in_share(int xcd, int slot, int nblk_bh, int ngrp, int H, const int4* sums,
                                      int64_t sums_per_b, int nsum, int rows32, bool pad_heavy,
                                      int64_t group_bytes, int64_t budget, int& blk, int& bh) {
    // run length: a divisor of ngrp, at most `budget` bytes of shared operands
    int run = (int)min<int64_t>(ngrp, max<int64_t>(1, budget / max<int64_t>(group_bytes, 1)));
    while (ngrp % run) --run;
    const int r0 = slot / (run * nblk_bh), in = slot % (run * nblk_bh);
    bh = xcd * ngrp + r0 * run + in % run;
    const int rank = in / run;  // position inside the group
    uint64_t heavy = 0;
    if (sums && nblk_bh <= 64) {
        const int lane = threadIdx.x & 63;
        const int4* sb = sums + (int64_t)(bh / H) * sums_per_b;
        for (int c0 = 0; c0 < nsum; c0 += 64) {
            bool two = false;
            if (c0 + lane < nsum) {
                const int4 v = sb[c0 + lane];
                two = (v.z < 32 && v.x != v.y) || (pad_heavy && v.z > 0);
            }
            uint64_t bits = __builtin_amdgcn_ballot_w64(two);
            while (bits) {
                heavy |= 1ull << ((c0 + __builtin_ctzll(bits)) / rows32);
                bits &= bits - 1;
            }
        }
    }
    const int nh = __builtin_popcountll(heavy);
    if (nblk_bh > 64 || nh == 0) {
        blk = rank;
    } else {
        uint64_t pool = rank < nh ? heavy : ~heavy & (nblk_bh == 64 ? ~0ull : (1ull << nblk_bh) - 1);
        for (int k = rank < nh ? rank : rank - nh; k > 0; --k) pool &= pool - 1;
        blk = __builtin_ctzll(pool);
    }
    blk = __builtin_amdgcn_readfirstlane(blk);
    bh = __builtin_amdgcn_readfirstlane(bh);
}

// Workgroup -> (row block, b*H + h) for a grid of one workgroup per block:
// order_in_share over the XCD shares when the grid splits evenly over the 8
// XCDs (dispatch is round-robin over them), else xcd_remap's order.
// `bid` / `nblk`: the workgroup's index among the `nblk` workgroups of this
// mapping (a grid may host several mappings back to back; the XCD of `bid`
// is then the hardware's one when the mappings before it hold a multiple of
// 8 workgroups, and the mapping is a bijection either way).
__device__ inline void dispatch_order_at(int bid, int nblk, int nblk_bh, int H, const int4* sums,
                                         int64_t sums_per_b, int nsum, int rows32, bool pad_heavy,
                                         int64_t group_bytes, int64_t budget, int& blk, int& bh) {
    constexpr int kXcd = 8;
    const int per = nblk / kXcd;
    if (nblk % kXcd == 0 && per % nblk_bh == 0) {
        order_in_share(bid % kXcd, bid / kXcd, nblk_bh, per / nblk_bh, H, sums, sums_per_b, nsum, rows32,
                       pad_heavy, group_bytes, budget, blk, bh);
    } else {
        const int g = xcd_remap(bid, nblk);
        blk = __builtin_amdgcn_readfirstlane(g % nblk_bh);
        bh = __builtin_amdgcn_readfirstlane(g / nblk_bh);
    }
}

__device__ inline void dispatch_order(int nblk_bh, int H, const int4* sums, int64_t sums_per_b, int nsum,
                                      int rows32, bool pad_heavy, int64_t group_bytes, int64_t budget,
                                      int& blk, int& bh) {
    dispatch_order_at(blockIdx.x, gridDim.x, nblk_bh, H, sums, sums_per_b, nsum, rows32, pad_heavy, group_bytes,
                      budget, blk, bh);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = min(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = max(v, __shfl_xor(v, o));
    return v;
}

// Reductions inside each 32-lane half of a wave.
__device__ __forceinline__ int half_min_i(int v) {
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) v = min(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ int half_max_i(int v) {
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) v = max(v, __shfl_xor(v, o));
    return v;
}

// 8 consecutive elements of a row, widened to fp32. `d0` is a multiple of 8.
template <typename T>
__device__ __forceinline__ void load8f(const T* row, int d0, float out[8]) {
    typedef typename Elt<T>::v8 v8;
    const v8 x = *reinterpret_cast<const v8*>(row + d0);
#pragma unroll
    for (int t = 0; t < 8; ++t) out[t] = (float)x[t];
}

// One element of RoPE's half-split rotation: x*cos - partner*sin for a dim in
// the lower half, x*cos + partner*sin for the upper half, as one fma. Every
// kernel that rotates an operand goes through this, so the forward and the
// backward round the same fp32 values to the same 16-bit operands.
__device__ __forceinline__ float rope_rot(float x, float partner, float c, float s, bool lo) {
    return __builtin_fmaf(x, c, (lo ? -partner : partner) * s);
}

// 8 elements [d0, d0+8) of RoPE(row) * mul at position `pos`, for head dim D
// (half-split layout: dim d pairs with d +- D/2; emb = cat(freqs, freqs)).
// Dims >= D read as 0.
template <typename T, int D>
__device__ __forceinline__ void load8_rot(const T* row, const float* cos_tab,
                                          const float* sin_tab, int pos, int d0,
                                          float mul, bool rope, float out[8]) {
    constexpr int H2 = D / 2;
    if (d0 >= D) {
#pragma unroll
        for (int t = 0; t < 8; ++t) out[t] = 0.f;
        return;
    }
    float x[8];
    load8f<T>(row, d0, x);
    if (!rope) {
#pragma unroll
        for (int t = 0; t < 8; ++t) out[t] = x[t] * mul;
        return;
    }
    const float* cr = cos_tab + (int64_t)pos * H2;
    const float* sr = sin_tab + (int64_t)pos * H2;
    if constexpr (H2 % 8 == 0) {
        // The whole 8-chunk lies on one side of D/2: one partner chunk.
        const bool lo = d0 < H2;
        const int dp = lo ? d0 + H2 : d0 - H2;
        const int fi = lo ? d0 : dp;
        float y[8];
        load8f<T>(row, dp, y);
        const f32x4 c0 = *reinterpret_cast<const f32x4*>(cr + fi);
        const f32x4 c1 = *reinterpret_cast<const f32x4*>(cr + fi + 4);
        const f32x4 s0 = *reinterpret_cast<const f32x4*>(sr + fi);
        const f32x4 s1 = *reinterpret_cast<const f32x4*>(sr + fi + 4);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float c = t < 4 ? c0[t & 3] : c1[t & 3];
            const float s = t < 4 ? s0[t & 3] : s1[t & 3];
            out[t] = rope_rot(x[t], y[t], c, s, lo) * mul;
        }
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int d = d0 + t;
            const bool lo = d < H2;
            const int dp = lo ? d + H2 : d - H2;
            const int fi = lo ? d : dp;
            const float y = (float)row[dp];
            out[t] = rope_rot(x[t], y, cr[fi], sr[fi], lo) * mul;
        }
    }
}

template <typename T>
__device__ __forceinline__ typename Elt<T>::v8 pack8(const float x[8]) {
    typename Elt<T>::v8 r;
#pragma unroll
    for (int t = 0; t < 8; ++t) r[t] = (T)x[t];
    return r;
}

// Attention dropout mask (the definition is in mpattn.h): per-row hash of
// (seed low word, b*H + h, query i), then per element the keep test for key j.
__device__ __forceinline__ uint32_t fmix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x85EBCA6Bu;
    x ^= x >> 13;
    x *= 0xC2B2AE35u;
    x ^= x >> 16;
    return x;
}
__device__ __forceinline__ uint32_t drop_row(uint32_t lo, uint32_t bh, uint32_t i) {
    return fmix32(lo ^ (bh * 0xC2B2AE3Du) ^ (i * 0x9E3779B1u));
}
__device__ __forceinline__ bool drop_keep(uint32_t row, uint32_t hi, uint32_t j, uint32_t thr) {
    return (fmix32(row ^ (j * 0x85EBCA77u + hi)) >> 8) >= thr;
}

// Dropout constants of a call: seed words, the 24-bit drop threshold and the
// keep scale 1 / (1 - p).
struct DropCfg {
    uint32_t lo, hi, thr;
    float rkeep;
};
inline DropCfg drop_cfg(float p, uint64_t seed) {
    DropCfg d;
    d.lo = (uint32_t)seed;
    d.hi = (uint32_t)(seed >> 32);
    d.thr = (uint32_t)((double)p * 16777216.0 + 0.5);
    d.rkeep = p > 0.f ? 1.0f / (1.0f - p) : 1.0f;
    return d;
}

// LDS byte address of a __shared__ object.
__device__ __forceinline__ unsigned lds_addr(const void* ptr) {
    return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void*)ptr;
}

// global -> LDS copy (global_load_lds): lane i writes its `size` bytes at LDS
// address M0 + i*size; the global address is sbase + voff (per lane). Issued
// as inline asm so the compiler does not wait for it before unrelated LDS
// reads; completion is tracked by hand with wait_vm<> and the barrier. M0 is
// saved before a batch of copies and restored after it (m0_save/m0_restore).
__device__ __forceinline__ int m0_save() {
    int v;
    asm volatile("s_mov_b32 %0, m0" : "=s"(v));
    return v;
}
__device__ __forceinline__ void m0_restore(int v) { asm volatile("s_mov_b32 m0, %0" ::"s"(v)); }
__device__ __forceinline__ void dma16(const void* sbase, unsigned voff, unsigned lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :: "v"(voff), "s"(sbase), "s"(lds) : "memory");
}
__device__ __forceinline__ void dma4(const void* sbase, unsigned voff, unsigned lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
                 :: "v"(voff), "s"(sbase), "s"(lds) : "memory");
}

// The same copies with a per-lane 64-bit global address (no scalar base).
__device__ __forceinline__ void dma16v(const void* addr, unsigned lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(addr), "s"(lds) : "memory");
}
__device__ __forceinline__ void dma4v(const void* addr, unsigned lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
                 :: "v"(addr), "s"(lds) : "memory");
}

// Wait until at most N vector-memory instructions of this wave are in flight.
template <int N> __device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// wait_vm<n> for a run-time (wavefront-uniform) n; counts above 15 wait for
// everything, which is always correct.
__device__ __forceinline__ void wait_vm_var(int n) {
    switch (n) {
        case 0: wait_vm<0>(); break;
        case 1: wait_vm<1>(); break;
        case 2: wait_vm<2>(); break;
        case 3: wait_vm<3>(); break;
        case 4: wait_vm<4>(); break;
        case 5: wait_vm<5>(); break;
        case 6: wait_vm<6>(); break;
        case 7: wait_vm<7>(); break;
        case 8: wait_vm<8>(); break;
        case 9: wait_vm<9>(); break;
        case 10: wait_vm<10>(); break;
        case 11: wait_vm<11>(); break;
        case 12: wait_vm<12>(); break;
        case 13: wait_vm<13>(); break;
        case 14: wait_vm<14>(); break;
        case 15: wait_vm<15>(); break;
        default: wait_vm<0>(); break;
    }
}

// Workgroup barrier without the release fence of __syncthreads (which would
// also drain the stages still in flight); LDS reads of this wave complete first.
__device__ __forceinline__ void stage_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// 64-row tiles of 16-bit rows of D elements staged in LDS: rows are stored
// densely (RB bytes each) with their 16-byte chunks XOR-swizzled by row so the
// MFMA operand reads below hit distinct banks. The swizzle repeats every 16
// rows (RP * NCH = 16).
template <int D> struct TileShape {
    static constexpr int RB = D * 2;        // row bytes
    static constexpr int NCH = RB / 16;     // 16-byte chunks per row
    static constexpr int TILE = 64 * RB;    // bytes per 64-row tile
    static constexpr int NI = TILE / 1024;  // global_load_lds wave-instructions per tile
    static constexpr bool POW2 = (NCH & (NCH - 1)) == 0;
    static constexpr int RP = 256 / RB;     // rows per 256-byte bank window
    static __device__ __forceinline__ int swz(int r, int c) {
        if constexpr (POW2) return c ^ ((r / RP) & (NCH - 1));
        return c;
    }
};

// Row of the MFMA row-operand this lane reads for subtile row ql: bits 2 and 3
// swapped, so accumulator slot i of lane half hh is row 16*(i/8) + 8*hh + i%8.
__device__ __forceinline__ int swapped_row(int ql) {
    return (ql & ~12) | ((ql & 4) << 1) | ((ql & 8) >> 1);
}

}  // namespace mpattn
