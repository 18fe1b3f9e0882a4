// Shared by the 16-bit and fp32 backward launches (mpattn_bwd.hip,
// mpattn_bwd32.hip): workspace layout, kernel arguments, and the fp32
// key-stationary / query-stationary kernels' launcher.
#pragma once

#include "mpattn_common.h"

namespace mpattn {

constexpr int kBS = 64;  // rows per LDS stage

inline int rup(int x, int m) { return (x + m - 1) / m * m; }

// Workspace layout (offsets 256-byte aligned), Lp = L rounded up to 64:
//   lse2  f32   [B][H][Lp]   -LSE * log2(e); -inf past L (negated: the dK/dV
//                            kernel starts its S accumulators from it)
//   delta f32   [B][H][Lp]   -(dO . O); 0 past L (negated, likewise for dP)
//   keff  int32 [B][Lp]      key chain id, kPadChain for padded / past L
//   ksum  int32 [B][Lp/32][4] key blocks: min, max chain (valid keys), #padded
//   qcid  int32 [B][Lp]      query chain id (queries past L: 0)
//   qsum  int32 [B][Lp/32][4] query blocks: min, max chain (queries < L)
//   qrot, krot, qmf T [B][H][Lp][D]  fused RoPE only: the forward's MFMA
//                operands, rounded as the forward rounds them: Q_self rotated
//                and multiplied by the logit factor, K_self rotated, Q_multi
//                multiplied by the logit factor (so the logits recomputed here
//                are the ones the forward's LSE was taken over)
struct BwdWs {
    int64_t lse2, delta, keff, ksum, qcid, qsum, qrot, krot, qmf, label, valid, total;
};

inline BwdWs bwd_ws_layout(int B, int H, int L, int D, int esize, bool rope) {
    const int64_t Lp = rup(L, kBS);
    auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
    BwdWs w;
    w.lse2 = 0;
    w.delta = al(w.lse2 + (int64_t)B * H * Lp * 4);
    w.keff = al(w.delta + (int64_t)B * H * Lp * 4);
    w.ksum = al(w.keff + (int64_t)B * Lp * 4);
    w.qcid = al(w.ksum + (int64_t)B * (Lp / 32) * 16);
    w.qsum = al(w.qcid + (int64_t)B * Lp * 4);
    w.qrot = al(w.qsum + (int64_t)B * (Lp / 32) * 16);
    const int64_t rot = rope ? (int64_t)B * H * Lp * D * esize : 0;
    w.krot = al(w.qrot + rot);
    w.qmf = al(w.krot + rot);
    w.label = al(w.qmf + rot);               // dense mask: row labels [B][L]
    w.valid = al(w.label + (int64_t)B * L * 4);  // dense mask: chain partition per batch row, then any row not
    w.total = al(w.valid + (int64_t)(B + 1) * 4);
    return w;
}

struct BwdArgs {
    mpattn_bwd_params p;
    const float* lse2;
    const float* delta;
    const int* keff;
    const int* ksum;
    const int* qcid;
    const int* qsum;
    const void* qrot;
    const void* krot;
    const void* qmf;  // folded Q_multi (fused RoPE)
    float kmul;       // dK factor: scale, or scale / (logit factor) when Q is folded
    int Lp;
    float c;     // logit factor: scale * log2(e), halved for sqrt-softmax (1 when
                 // fused RoPE folds it into Q, as the forward does)
    float lmul;  // LSE factor: log2(e), halved for sqrt-softmax
    float qmul;  // logit factor folded into Q by the prep kernel (fused RoPE)
    DropCfg drop;
    int mvec;  // dense mask rows readable as aligned 8-byte words
    int mdma;  // dense mask tiles copyable to LDS in 16-byte chunks (dK/dV)
    // Dense masks: row labels of the mask and per-batch-row flags (1: the
    // mask is the "different chain" relation of the labels; gate[B] != 0
    // when some row is not). A launch with gate set runs only the rows whose
    // flag != 0 equals gate_want.
    const int* label;
    const int* gate;
    int gate_want;
};

// Row labels of a dense (B, L, L) mask (first key j with mask[b, i, j] == 0)
// and, with verify, valid[b] = 1 exactly when row b of the mask is the
// "different chain" relation of its labels, valid[B] = 1 when some row is
// not (valid holds B + 1 ints; mpattn_fwd.hip).
hipError_t launch_mask_labels(const uint8_t* mask, int64_t msb, int64_t msq, int64_t msk, int B, int L, int* label,
                              int* valid, int vec, bool verify, hipStream_t stream);

// fp32 dK/dV and dQ kernels (mpattn_bwd32.hip), run after the prep kernel
// has filled the workspace that `a` points into.
hipError_t launch_bwd32(const BwdArgs& a, hipStream_t stream);

}  // namespace mpattn
