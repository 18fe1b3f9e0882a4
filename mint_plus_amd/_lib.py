"""ctypes binding of libmpattn.so (C ABI declared in include/mpattn.h).

Torch is used only for device memory and the current HIP stream: every
computation of the op happens in the gfx950 kernels behind this ABI. When the
library is missing, every entry point raises -- there is no CPU fallback.
"""
import ctypes
import os
import threading

import numpy as np
import torch

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG_DIR, "libmpattn.so")

MPATTN_OK = 0
MPATTN_ERR_INVALID = -1
MPATTN_ERR_UNSUPPORTED = -2
MPATTN_ERR_LAUNCH = -3

MPATTN_BF16, MPATTN_FP16, MPATTN_FP32 = 0, 1, 2
MPATTN_ROPE_NONE, MPATTN_ROPE_FUSED = 0, 1

ROPE_BASE = 10000.0
SUPPORTED_HEAD_DIMS = (16, 24, 32, 64)

_DTYPES = {torch.bfloat16: MPATTN_BF16, torch.float16: MPATTN_FP16, torch.float32: MPATTN_FP32}


class MpattnError(RuntimeError):
    """A libmpattn call returned an error code."""

    def __init__(self, code, fn, detail):
        self.code = code
        super().__init__(f"{fn} failed ({code}: {_strerror(code)}): {detail}")


class MpattnUnsupported(MpattnError):
    """Valid request outside what the library implements (MPATTN_ERR_UNSUPPORTED)."""


class Tensor4(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("stride_b", ctypes.c_int64),
                ("stride_h", ctypes.c_int64), ("stride_t", ctypes.c_int64)]


class FwdParams(ctypes.Structure):
    _fields_ = [
        ("q_self", Tensor4), ("k_self", Tensor4), ("v_self", Tensor4),
        ("q_multi", Tensor4), ("k_multi", Tensor4), ("v_multi", Tensor4),
        ("out", Tensor4),
        ("lse", ctypes.c_void_p),
        ("chain_id", ctypes.c_void_p), ("chain_mask", ctypes.c_void_p),
        ("mask_stride_b", ctypes.c_int64), ("mask_stride_q", ctypes.c_int64),
        ("mask_stride_k", ctypes.c_int64),
        ("key_pad", ctypes.c_void_p),
        ("rope_cos", ctypes.c_void_p), ("rope_sin", ctypes.c_void_p),
        ("B", ctypes.c_int32), ("H", ctypes.c_int32), ("L", ctypes.c_int32), ("D", ctypes.c_int32),
        ("dtype", ctypes.c_int32), ("rope", ctypes.c_int32),
        ("scale", ctypes.c_float), ("sqrt_softmax", ctypes.c_int32),
        ("dropout_p", ctypes.c_float),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
        ("dropout_seed", ctypes.c_uint64),
    ]


class BwdParams(ctypes.Structure):
    _fields_ = [
        ("q_self", Tensor4), ("k_self", Tensor4), ("v_self", Tensor4),
        ("q_multi", Tensor4), ("k_multi", Tensor4), ("v_multi", Tensor4),
        ("out", Tensor4), ("grad_out", Tensor4),
        ("lse", ctypes.c_void_p),
        ("dq_self", Tensor4), ("dk_self", Tensor4), ("dv_self", Tensor4),
        ("dq_multi", Tensor4), ("dk_multi", Tensor4), ("dv_multi", Tensor4),
        ("chain_id", ctypes.c_void_p), ("chain_mask", ctypes.c_void_p),
        ("mask_stride_b", ctypes.c_int64), ("mask_stride_q", ctypes.c_int64),
        ("mask_stride_k", ctypes.c_int64),
        ("key_pad", ctypes.c_void_p),
        ("rope_cos", ctypes.c_void_p), ("rope_sin", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
        ("B", ctypes.c_int32), ("H", ctypes.c_int32), ("L", ctypes.c_int32), ("D", ctypes.c_int32),
        ("dtype", ctypes.c_int32), ("rope", ctypes.c_int32),
        ("scale", ctypes.c_float), ("sqrt_softmax", ctypes.c_int32),
        ("dropout_p", ctypes.c_float), ("dropout_seed", ctypes.c_uint64),
    ]


class CombineFwdParams(ctypes.Structure):
    _fields_ = [
        ("intra_logits", Tensor4), ("inter_logits", Tensor4),
        ("intra_values", Tensor4), ("inter_values", Tensor4),
        ("out", Tensor4),
        ("lse", ctypes.c_void_p),
        ("chain_mask", ctypes.c_void_p),
        ("mask_stride_b", ctypes.c_int64), ("mask_stride_q", ctypes.c_int64),
        ("mask_stride_k", ctypes.c_int64),
        ("B", ctypes.c_int32), ("H", ctypes.c_int32), ("L", ctypes.c_int32), ("D", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("dropout_p", ctypes.c_float), ("dropout_seed", ctypes.c_uint64),
    ]


class CombineBwdParams(ctypes.Structure):
    _fields_ = [
        ("intra_logits", Tensor4), ("inter_logits", Tensor4),
        ("intra_values", Tensor4), ("inter_values", Tensor4),
        ("grad_out", Tensor4),
        ("d_intra_logits", Tensor4), ("d_inter_logits", Tensor4),
        ("d_intra_values", Tensor4), ("d_inter_values", Tensor4),
        ("chain_mask", ctypes.c_void_p),
        ("mask_stride_b", ctypes.c_int64), ("mask_stride_q", ctypes.c_int64),
        ("mask_stride_k", ctypes.c_int64),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
        ("B", ctypes.c_int32), ("H", ctypes.c_int32), ("L", ctypes.c_int32), ("D", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("dropout_p", ctypes.c_float), ("dropout_seed", ctypes.c_uint64),
        ("lse", ctypes.c_void_p), ("out", Tensor4),
    ]


# Functions declared in include/mpattn.h, with their ctypes signatures.
EXPORTS = {
    "mpattn_fwd": (ctypes.c_int, [ctypes.POINTER(FwdParams), ctypes.c_void_p]),
    "mpattn_fwd_noalloc": (ctypes.c_int, [ctypes.POINTER(FwdParams), ctypes.c_void_p]),
    "mpattn_bwd": (ctypes.c_int, [ctypes.POINTER(BwdParams), ctypes.c_void_p]),
    "mpattn_fwd_workspace_size": (ctypes.c_int64, [ctypes.c_int32] * 6),
    "mpattn_bwd_workspace_size": (ctypes.c_int64, [ctypes.c_int32] * 4),
    "mpattn_combine_fwd": (ctypes.c_int, [ctypes.POINTER(CombineFwdParams), ctypes.c_void_p]),
    "mpattn_combine_bwd": (ctypes.c_int, [ctypes.POINTER(CombineBwdParams), ctypes.c_void_p]),
    "mpattn_combine_bwd_workspace_size": (ctypes.c_int64, [ctypes.c_int32] * 4),
    "mpattn_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "mpattn_last_error": (ctypes.c_char_p, []),
    "mpattn_version": (ctypes.c_int, []),
}

_lib = None
_lib_lock = threading.Lock()


def load_library(path=LIB_PATH):
    """Load libmpattn.so once; raise if it is not built."""
    global _lib
    with _lib_lock:
        if _lib is None:
            if not os.path.exists(path):
                raise RuntimeError(
                    f"{path} is not built: run `python -m mint_plus_amd.build` "
                    "(or __graft_entry__.build()); there is no fallback path")
            lib = ctypes.CDLL(path)
            for name, (res, args) in EXPORTS.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
        return _lib


def _strerror(code):
    try:
        return load_library().mpattn_strerror(code).decode()
    except Exception:  # library absent: still produce a message
        return "error"


def _check(code, fn):
    if code != MPATTN_OK:
        detail = load_library().mpattn_last_error().decode()
        cls = MpattnUnsupported if code == MPATTN_ERR_UNSUPPORTED else MpattnError
        raise cls(code, fn, detail)


def version():
    return load_library().mpattn_version()


def _t4(t):
    """(B, H, L, D) view with unit head-dim stride -> Tensor4."""
    if t is None:
        return Tensor4(None, 0, 0, 0)
    if t.dim() != 4:
        raise ValueError(f"expected a 4-D (B, H, L, D) tensor, got shape {tuple(t.shape)}")
    if t.stride(3) != 1 and t.shape[3] > 1:
        raise ValueError("head-dim stride must be 1")
    return Tensor4(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))


_rope_cache = {}
_rope_lock = threading.Lock()


def rope_tables(L, D, device):
    """Device cos/sin tables (L, D/2) fp32 of ``t * inv_freq``.

    ``inv_freq = 1 / 10000**(arange(0, D, 2) / D)`` as in
    mint_plus/models/rotary_embedding.py:44, rounded to fp32; the angle is
    the fp32 product ``t * inv_freq`` (rotary_embedding.py:49-50); cos/sin are
    evaluated in fp64 on the host and rounded to fp32 once.

    One table per (D, device) is kept, at the largest length seen so far
    (rounded up to 256 rows); shorter lengths get its first L rows (rows are
    indexed by position, so they are a prefix, and a contiguous view).
    """
    dev = torch.device(device)
    key = (int(D), dev.type, dev.index)
    with _rope_lock:
        hit = _rope_cache.get(key)
        if hit is None or hit[0].shape[0] < L:
            n = (int(L) + 255) // 256 * 256
            inv = (1.0 / ROPE_BASE ** (np.arange(0, D, 2, dtype=np.float64) / D)).astype(np.float32)
            ang = (np.arange(n, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float64)
            cos = torch.from_numpy(np.cos(ang).astype(np.float32)).to(dev)
            sin = torch.from_numpy(np.sin(ang).astype(np.float32)).to(dev)
            hit = (cos, sin)
            _rope_cache[key] = hit
        return hit[0][:L], hit[1][:L]


def _stream_handle(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _selection_args(params, chain_ids, chain_mask, key_pad, B, L, device):
    """Fill chain_id / chain_mask / key_pad fields; returns tensors to keep alive."""
    keep = []
    if chain_ids is not None:
        if tuple(chain_ids.shape) != (B, L):
            raise ValueError(f"chain_ids must be (B, L) = {(B, L)}, got {tuple(chain_ids.shape)}")
        cid = chain_ids.to(device=device, dtype=torch.int32).contiguous()
        keep.append(cid)
        params.chain_id = cid.data_ptr()
    elif chain_mask is not None:
        if tuple(chain_mask.shape) != (B, L, L):
            raise ValueError(f"chain_mask must be (B, L, L) = {(B, L, L)}, got {tuple(chain_mask.shape)}")
        cm = chain_mask
        if cm.dtype != torch.bool and cm.dtype != torch.uint8:
            cm = cm != 0
        cm = cm.to(device)
        keep.append(cm)
        params.chain_mask = cm.data_ptr()
        params.mask_stride_b, params.mask_stride_q, params.mask_stride_k = cm.stride()
    else:
        raise ValueError("one of chain_ids / chain_mask is required")
    if key_pad is not None:
        if tuple(key_pad.shape) != (B, L):
            raise ValueError(f"key_padding_mask must be (B, L) = {(B, L)}, got {tuple(key_pad.shape)}")
        kp = key_pad.to(device=device, dtype=torch.bool).contiguous()
        keep.append(kp)
        params.key_pad = kp.data_ptr()
    return keep


def _common_checks(tensors, names):
    t0 = tensors[0]
    if not t0.is_cuda:
        raise RuntimeError("multi-pathway attention runs on the GPU only (inputs are on the CPU)")
    if t0.dtype not in _DTYPES:
        raise TypeError(f"unsupported dtype {t0.dtype} (bfloat16, float16, float32)")
    for t, n in zip(tensors, names):
        if t.shape != t0.shape:
            raise ValueError(f"{n} has shape {tuple(t.shape)}, expected {tuple(t0.shape)}")
        if t.dtype != t0.dtype:
            raise TypeError(f"{n} has dtype {t.dtype}, expected {t0.dtype}")
        if t.device != t0.device:
            raise ValueError(f"{n} is on {t.device}, expected {t0.device}")


def _check_out(t, shape, like, name):
    """A caller-provided output must match shape, dtype and device and keep
    the ABI's row alignment (it is written in place, so it cannot be copied)."""
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if t.dtype != like.dtype or t.device != like.device:
        raise TypeError(f"{name} must be {like.dtype} on {like.device}")
    if _aligned(t) is not t:
        raise ValueError(f"{name}: rows must be 16-byte aligned with unit head-dim stride")


def _aligned(t):
    """Return t, or a contiguous copy when its layout breaks the ABI's
    16-byte row alignment rule (strides in 16-byte multiples)."""
    q = 16 // t.element_size()
    ok = (t.stride(3) == 1 and t.data_ptr() % 16 == 0
          and all(s % q == 0 for s in t.stride()[:3]))
    return t if ok else t.contiguous()


def mpattn_fwd(q_self, k_self, v_self, q_multi, k_multi, v_multi, *, chain_ids=None,
               chain_mask=None, key_padding_mask=None, rope=False, scale=1.0,
               sqrt_softmax=False, dropout_p=0.0, dropout_seed=0, out=None, need_lse=False,
               lse=None, noalloc=False):
    """Launch the forward kernel on the current stream.

    Returns ``out`` (B, H, L, D) and, if ``need_lse``, the fp32 (B, H, L)
    log-sum-exp (natural units of the scaled logits). With ``dropout_p`` > 0
    the keep mask is a function of ``dropout_seed`` (a 64-bit integer) and the
    element's (b, h, query, key); the LSE is that of the undropped softmax.

    ``noalloc`` calls ``mpattn_fwd_noalloc`` (the workspace is the library's
    static device scratch, nothing is allocated; give ``out`` and, with
    ``need_lse``, ``lse`` to allocate nothing here either).
    """
    ins = [q_self, k_self, v_self, q_multi, k_multi, v_multi]
    names = ["q_self", "k_self", "v_self", "q_multi", "k_multi", "v_multi"]
    _common_checks(ins, names)
    B, H, L, D = q_self.shape
    if D not in SUPPORTED_HEAD_DIMS:
        raise MpattnUnsupported(MPATTN_ERR_UNSUPPORTED, "mpattn_fwd",
                                f"head dim {D} (supported: {SUPPORTED_HEAD_DIMS})")
    ins = [_aligned(t) for t in ins]
    dev = q_self.device
    if out is None:
        out = torch.empty((B, H, L, D), dtype=q_self.dtype, device=dev)
    else:
        _check_out(out, (B, H, L, D), q_self, "out")
    if need_lse and lse is None:
        lse = torch.empty((B, H, L), dtype=torch.float32, device=dev)
    elif need_lse and (tuple(lse.shape) != (B, H, L) or lse.dtype != torch.float32
                       or not lse.is_contiguous() or lse.device != dev):
        raise ValueError(f"lse must be a contiguous fp32 (B, H, L) = {(B, H, L)} tensor on {dev}")
    elif not need_lse:
        lse = None
    p = FwdParams()
    p.q_self, p.k_self, p.v_self, p.q_multi, p.k_multi, p.v_multi = (_t4(t) for t in ins)
    p.out = _t4(out)
    p.lse = lse.data_ptr() if lse is not None else None
    keep = _selection_args(p, chain_ids, chain_mask, key_padding_mask, B, L, dev)
    if rope:
        cos, sin = rope_tables(L, D, dev)
        p.rope_cos, p.rope_sin = cos.data_ptr(), sin.data_ptr()
    p.B, p.H, p.L, p.D = B, H, L, D
    p.dtype = _DTYPES[q_self.dtype]
    p.rope = MPATTN_ROPE_FUSED if rope else MPATTN_ROPE_NONE
    p.scale = float(scale)
    p.sqrt_softmax = 1 if sqrt_softmax else 0
    p.dropout_p = float(dropout_p)
    p.dropout_seed = int(dropout_seed) & 0xFFFFFFFFFFFFFFFF
    lib = load_library()
    if noalloc:
        ws = None
        rc = lib.mpattn_fwd_noalloc(ctypes.byref(p), _stream_handle(dev))
        _check(rc, "mpattn_fwd_noalloc")
    else:
        ws_bytes = lib.mpattn_fwd_workspace_size(B, H, L, D, p.dtype, p.rope)
        if ws_bytes < 0:
            raise MpattnError(MPATTN_ERR_INVALID, "mpattn_fwd_workspace_size", "bad shape")
        # torch's caching allocator returns 512-byte aligned blocks
        ws = torch.empty(max(1, ws_bytes), dtype=torch.uint8, device=dev)
        p.workspace, p.workspace_bytes = ws.data_ptr(), ws_bytes
        rc = lib.mpattn_fwd(ctypes.byref(p), _stream_handle(dev))
        _check(rc, "mpattn_fwd")
    del keep, ins, ws
    return (out, lse) if need_lse else out


def mpattn_bwd(q_self, k_self, v_self, q_multi, k_multi, v_multi, out, lse, grad_out, *,
               chain_ids=None, chain_mask=None, key_padding_mask=None, rope=False, scale=1.0,
               sqrt_softmax=False, dropout_p=0.0, dropout_seed=0, grads=None):
    """Launch the backward kernels; returns (dq_s, dk_s, dv_s, dq_m, dk_m, dv_m).

    ``dropout_p`` / ``dropout_seed`` must be the forward's: the keep mask is
    regenerated from them.

    ``grads`` optionally supplies the six (B, H, L, D) output views (any
    strides the ABI accepts, e.g. slices of one projection-gradient buffer);
    by default they are allocated contiguous.
    """
    ins = [q_self, k_self, v_self, q_multi, k_multi, v_multi, out, grad_out]
    names = ["q_self", "k_self", "v_self", "q_multi", "k_multi", "v_multi", "out", "grad_out"]
    _common_checks(ins, names)
    B, H, L, D = q_self.shape
    if D not in SUPPORTED_HEAD_DIMS:
        raise MpattnUnsupported(MPATTN_ERR_UNSUPPORTED, "mpattn_bwd", f"head dim {D}")
    ins = [_aligned(t) for t in ins]
    dev = q_self.device
    lib = load_library()
    if grads is None:
        grads = [torch.empty((B, H, L, D), dtype=q_self.dtype, device=dev) for _ in range(6)]
    else:
        grads = list(grads)
        if len(grads) != 6:
            raise ValueError("grads must hold six tensors")
        for g, n in zip(grads, ("dq_self", "dk_self", "dv_self", "dq_multi", "dk_multi", "dv_multi")):
            _check_out(g, (B, H, L, D), q_self, n)
    ws_bytes = lib.mpattn_bwd_workspace_size(B, H, L, D)
    if ws_bytes < 0:
        raise MpattnError(MPATTN_ERR_INVALID, "mpattn_bwd_workspace_size", "bad shape")
    ws = torch.empty(max(1, (ws_bytes + 3) // 4), dtype=torch.float32, device=dev)
    lse = lse.to(device=dev, dtype=torch.float32).contiguous()
    p = BwdParams()
    (p.q_self, p.k_self, p.v_self, p.q_multi, p.k_multi, p.v_multi, p.out,
     p.grad_out) = (_t4(t) for t in ins)
    p.lse = lse.data_ptr()
    (p.dq_self, p.dk_self, p.dv_self, p.dq_multi, p.dk_multi, p.dv_multi) = (_t4(g) for g in grads)
    keep = _selection_args(p, chain_ids, chain_mask, key_padding_mask, B, L, dev)
    if rope:
        cos, sin = rope_tables(L, D, dev)
        p.rope_cos, p.rope_sin = cos.data_ptr(), sin.data_ptr()
    p.workspace, p.workspace_bytes = ws.data_ptr(), ws.numel() * ws.element_size()
    p.B, p.H, p.L, p.D = B, H, L, D
    p.dtype = _DTYPES[q_self.dtype]
    p.rope = MPATTN_ROPE_FUSED if rope else MPATTN_ROPE_NONE
    p.scale = float(scale)
    p.sqrt_softmax = 1 if sqrt_softmax else 0
    p.dropout_p = float(dropout_p)
    p.dropout_seed = int(dropout_seed) & 0xFFFFFFFFFFFFFFFF
    rc = lib.mpattn_bwd(ctypes.byref(p), _stream_handle(dev))
    _check(rc, "mpattn_bwd")
    del keep, ins
    return tuple(grads)


def _logits4(t, name, B, H, L):
    """(B, H, L, L) logits view with unit key stride -> Tensor4 (a copy is
    made when the key stride is not 1)."""
    if tuple(t.shape) != (B, H, L, L):
        raise ValueError(f"{name} must be (B, H, L, L) = {(B, H, L, L)}, got {tuple(t.shape)}")
    if t.stride(3) != 1:
        t = t.contiguous()
    return t, Tensor4(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))


def _combine_common(intra_logits, inter_logits, chain_mask, intra_values, inter_values):
    _common_checks([intra_values, inter_values], ["intra_values", "inter_values"])
    B, H, L, D = intra_values.shape
    for t, n in ((intra_logits, "intra_logits"), (inter_logits, "inter_logits")):
        if t.dtype != intra_values.dtype or t.device != intra_values.device:
            raise TypeError(f"{n} must be {intra_values.dtype} on {intra_values.device}")
    if tuple(chain_mask.shape) != (B, L, L):
        raise ValueError(f"chain_mask must be (B, L, L) = {(B, L, L)}, got {tuple(chain_mask.shape)}")
    cm = chain_mask.to(intra_values.device)
    if cm.dtype != torch.bool and cm.dtype != torch.uint8:
        cm = cm != 0
    return B, H, L, D, cm


def mpattn_combine_fwd(intra_logits, inter_logits, chain_mask, intra_values, inter_values, *,
                       dropout_p=0.0, dropout_seed=0, need_lse=False):
    """Launch the materialised-logit combine; returns ``out`` (B, H, L, D)
    (and the fp32 (B, H, L) log-sum-exp when ``need_lse``). Dropout uses the
    fused op's mask definition for ``dropout_seed``."""
    B, H, L, D, cm = _combine_common(intra_logits, inter_logits, chain_mask, intra_values,
                                     inter_values)
    dev = intra_values.device
    vs, vm = _aligned(intra_values), _aligned(inter_values)
    il, til = _logits4(intra_logits, "intra_logits", B, H, L)
    el, tel = _logits4(inter_logits, "inter_logits", B, H, L)
    out = torch.empty((B, H, L, D), dtype=vs.dtype, device=dev)
    lse = torch.empty((B, H, L), dtype=torch.float32, device=dev) if need_lse else None
    p = CombineFwdParams()
    p.intra_logits, p.inter_logits = til, tel
    p.intra_values, p.inter_values, p.out = _t4(vs), _t4(vm), _t4(out)
    p.lse = lse.data_ptr() if lse is not None else None
    p.chain_mask = cm.data_ptr()
    p.mask_stride_b, p.mask_stride_q, p.mask_stride_k = cm.stride()
    p.B, p.H, p.L, p.D = B, H, L, D
    p.dtype = _DTYPES[vs.dtype]
    p.dropout_p = float(dropout_p)
    p.dropout_seed = int(dropout_seed) & 0xFFFFFFFFFFFFFFFF
    rc = load_library().mpattn_combine_fwd(ctypes.byref(p), _stream_handle(dev))
    _check(rc, "mpattn_combine_fwd")
    del il, el, vs, vm, cm
    return (out, lse) if need_lse else out


def mpattn_combine_bwd(intra_logits, inter_logits, chain_mask, intra_values, inter_values,
                       grad_out, *, dropout_p=0.0, dropout_seed=0, lse=None, out=None):
    """Launch the combine backward; returns (d_intra_logits, d_inter_logits,
    d_intra_values, d_inter_values) in the inputs' dtype.

    ``lse`` / ``out``: the forward's fp32 (B, H, L) log-sum-exp and output
    (``mpattn_combine_fwd(..., need_lse=True)``); given both, the row
    statistics come from them instead of a pass over both logit tensors."""
    B, H, L, D, cm = _combine_common(intra_logits, inter_logits, chain_mask, intra_values,
                                     inter_values)
    _common_checks([intra_values, grad_out], ["intra_values", "grad_out"])
    dev = intra_values.device
    vs, vm, go = _aligned(intra_values), _aligned(inter_values), _aligned(grad_out)
    il, til = _logits4(intra_logits, "intra_logits", B, H, L)
    el, tel = _logits4(inter_logits, "inter_logits", B, H, L)
    d_il = torch.empty((B, H, L, L), dtype=vs.dtype, device=dev)
    d_el = torch.empty((B, H, L, L), dtype=vs.dtype, device=dev)
    d_vs = torch.empty((B, H, L, D), dtype=vs.dtype, device=dev)
    d_vm = torch.empty((B, H, L, D), dtype=vs.dtype, device=dev)
    lib = load_library()
    ws_bytes = lib.mpattn_combine_bwd_workspace_size(B, H, L, D)
    if ws_bytes < 0:
        raise MpattnError(MPATTN_ERR_INVALID, "mpattn_combine_bwd_workspace_size", "bad shape")
    ws = torch.empty(max(1, ws_bytes), dtype=torch.uint8, device=dev)
    p = CombineBwdParams()
    p.intra_logits, p.inter_logits = til, tel
    p.intra_values, p.inter_values, p.grad_out = _t4(vs), _t4(vm), _t4(go)
    p.d_intra_logits = Tensor4(d_il.data_ptr(), *d_il.stride()[:3])
    p.d_inter_logits = Tensor4(d_el.data_ptr(), *d_el.stride()[:3])
    p.d_intra_values, p.d_inter_values = _t4(d_vs), _t4(d_vm)
    p.chain_mask = cm.data_ptr()
    p.mask_stride_b, p.mask_stride_q, p.mask_stride_k = cm.stride()
    p.workspace, p.workspace_bytes = ws.data_ptr(), ws.numel()
    p.B, p.H, p.L, p.D = B, H, L, D
    p.dtype = _DTYPES[vs.dtype]
    p.dropout_p = float(dropout_p)
    p.dropout_seed = int(dropout_seed) & 0xFFFFFFFFFFFFFFFF
    if (lse is None) != (out is None):
        raise ValueError("mpattn_combine_bwd: give both lse and out, or neither")
    fo = None
    if lse is not None:
        if lse.dtype != torch.float32 or tuple(lse.shape) != (B, H, L) or not lse.is_contiguous():
            raise ValueError("mpattn_combine_bwd: lse must be a contiguous fp32 (B, H, L) tensor")
        if tuple(out.shape) != (B, H, L, D) or out.dtype != vs.dtype or out.device != dev:
            raise ValueError("mpattn_combine_bwd: out must be the forward's (B, H, L, D) output")
        if lse.device != dev:
            raise ValueError("mpattn_combine_bwd: lse is on another device")
        fo = _aligned(out)
        p.lse, p.out = lse.data_ptr(), _t4(fo)
    rc = lib.mpattn_combine_bwd(ctypes.byref(p), _stream_handle(dev))
    _check(rc, "mpattn_combine_bwd")
    del fo
    del il, el, vs, vm, go, cm, ws
    return d_il, d_el, d_vs, d_vm


def default_scale(D):
    return D ** -0.5 if D > 0 else 1.0


__all__ = ["mpattn_fwd", "mpattn_bwd", "mpattn_combine_fwd", "mpattn_combine_bwd", "load_library", "rope_tables", "version",
           "MpattnError", "MpattnUnsupported", "EXPORTS", "LIB_PATH", "default_scale"]
