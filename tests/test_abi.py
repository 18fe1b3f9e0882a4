"""C-ABI checks that need no GPU: the library loads, exports every function
include/mpattn.h declares with the layout the ctypes binding assumes, and
rejects invalid or unsupported requests before anything is enqueued."""
import ctypes
import os
import re

import pytest
import torch

from mint_plus_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "mpattn.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(mpattn_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libmpattn.so is not built (run __graft_entry__.build())")
    return _lib.load_library()


def test_exports_every_header_function(lib):
    names = header_functions()
    assert "mpattn_fwd" in names and "mpattn_bwd" in names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in mpattn.h but not exported"
        assert n in _lib.EXPORTS, f"{n} has no ctypes signature in _lib.EXPORTS"
    assert set(_lib.EXPORTS) == set(names)


def test_version_and_strings(lib):
    assert lib.mpattn_version() == 6
    assert lib.mpattn_strerror(0) == b"success"
    assert lib.mpattn_strerror(-2) == b"unsupported configuration"
    assert lib.mpattn_strerror(-99) == b"unknown error"


def test_struct_layout_matches_header():
    """Field offsets of the ctypes mirrors follow the C declaration order with
    natural alignment (x86-64 SysV, the layout hipcc's host pass uses)."""
    assert ctypes.sizeof(_lib.Tensor4) == 32
    f = _lib.FwdParams
    assert f.out.offset == 6 * 32 and f.lse.offset == 7 * 32
    assert f.B.offset == f.rope_sin.offset + 8
    assert f.workspace.offset % 8 == 0
    b = _lib.BwdParams
    assert b.grad_out.offset == 7 * 32 and b.lse.offset == 8 * 32
    assert b.dv_multi.offset == 8 * 32 + 8 + 5 * 32


_STRUCTS = {
    "mpattn_fwd_params": _lib.FwdParams,
    "mpattn_bwd_params": _lib.BwdParams,
    "mpattn_combine_fwd_params": _lib.CombineFwdParams,
    "mpattn_combine_bwd_params": _lib.CombineBwdParams,
}


def test_struct_offsets_match_c_compiler(tmp_path):
    """Every field's offset and every struct's size, as the C compiler lays
    out include/mpattn.h, equals the ctypes mirror's."""
    import shutil
    import subprocess
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "mpattn.h"', "int main(void) {"]
    for cname, cls in _STRUCTS.items():
        lines.append(f'printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    inc = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
    subprocess.run([cc, "-std=c99", "-I", inc, str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    got = {}
    for line in out.splitlines():
        cname, field, val = line.split()
        got[(cname, field)] = int(val)
    for cname, cls in _STRUCTS.items():
        assert got[(cname, "sizeof")] == ctypes.sizeof(cls), cname
        for fname, _ in cls._fields_:
            assert got[(cname, fname)] == getattr(cls, fname).offset, (cname, fname)


def test_workspace_sizes(lib):
    assert lib.mpattn_fwd_workspace_size(0, 1, 1, 32, 0, 1) == -1
    assert lib.mpattn_bwd_workspace_size(1, 0, 1, 32) == -1
    a = lib.mpattn_fwd_workspace_size(16, 20, 1024, 32, 0, 1)
    b = lib.mpattn_fwd_workspace_size(16, 20, 1024, 32, 0, 0)
    assert a > b > 0  # fused RoPE stages rotated K_self in the workspace
    assert a >= 16 * 20 * 1024 * 32 * 2
    w = lib.mpattn_bwd_workspace_size(8, 20, 1024, 32)
    assert w >= 2 * 8 * 20 * 1024 * 4  # LSE and Delta rows at least


def _fake(ptr=1 << 20):
    return _lib.Tensor4(ptr, 40960, 2048, 32)


def _fwd_params(**over):
    p = _lib.FwdParams()
    for n in ("q_self", "k_self", "v_self", "q_multi", "k_multi", "v_multi", "out"):
        setattr(p, n, _fake())
    p.chain_id = 1 << 21
    p.rope_cos = p.rope_sin = 1 << 22
    p.B, p.H, p.L, p.D = 2, 20, 64, 32
    p.dtype, p.rope, p.scale = _lib.MPATTN_BF16, _lib.MPATTN_ROPE_FUSED, 32 ** -0.5
    p.workspace, p.workspace_bytes = 1 << 24, 1 << 30
    for k, v in over.items():
        setattr(p, k, v)
    return p


# Each case fails validation, so nothing reaches the HIP runtime.
FWD_CASES = [
    (dict(D=48), _lib.MPATTN_ERR_UNSUPPORTED, "head dim"),
    (dict(L=0), _lib.MPATTN_ERR_INVALID, "must be >= 1"),
    (dict(dtype=7), _lib.MPATTN_ERR_INVALID, "dtype"),
    (dict(rope=5), _lib.MPATTN_ERR_INVALID, "rope"),
    (dict(scale=0.0), _lib.MPATTN_ERR_INVALID, "scale"),
    (dict(scale=float("nan")), _lib.MPATTN_ERR_INVALID, "scale"),
    (dict(chain_mask=1 << 23), _lib.MPATTN_ERR_INVALID, "exactly one"),
    (dict(chain_id=None), _lib.MPATTN_ERR_INVALID, "exactly one"),
    (dict(rope_cos=None), _lib.MPATTN_ERR_INVALID, "rope tables"),
    (dict(dropout_p=-0.1), _lib.MPATTN_ERR_INVALID, "dropout"),
    (dict(dropout_p=1.0), _lib.MPATTN_ERR_INVALID, "dropout"),
    (dict(dropout_p=float("nan")), _lib.MPATTN_ERR_INVALID, "dropout"),
    (dict(q_self=_lib.Tensor4(None, 0, 0, 32)), _lib.MPATTN_ERR_INVALID, "null"),
    (dict(k_self=_lib.Tensor4((1 << 20) + 8, 40960, 2048, 32)), _lib.MPATTN_ERR_UNSUPPORTED, "aligned"),
    (dict(v_multi=_lib.Tensor4(1 << 20, 40960, 2048, 36)), _lib.MPATTN_ERR_UNSUPPORTED, "multiples"),
    (dict(workspace_bytes=16), _lib.MPATTN_ERR_INVALID, "workspace"),
    (dict(workspace=(1 << 24) + 16), _lib.MPATTN_ERR_INVALID, "workspace"),
    # grids past 2^32 work-items: 24 per padded row, and a dense mask's checks
    (dict(B=1 << 16, H=64, L=1024), _lib.MPATTN_ERR_UNSUPPORTED, "too large for one launch"),
    (dict(chain_id=None, chain_mask=1 << 23, B=64, H=1, L=1 << 16), _lib.MPATTN_ERR_UNSUPPORTED,
     "too large for one launch"),
]


@pytest.mark.parametrize("over,code,msg", FWD_CASES)
def test_fwd_validation(lib, over, code, msg):
    p = _fwd_params(**over)
    rc = lib.mpattn_fwd(ctypes.byref(p), None)
    assert rc == code
    assert msg in lib.mpattn_last_error().decode()


def test_null_params(lib):
    assert lib.mpattn_fwd(None, None) == _lib.MPATTN_ERR_INVALID
    assert lib.mpattn_bwd(None, None) == _lib.MPATTN_ERR_INVALID


def test_bwd_validation(lib):
    p = _lib.BwdParams()
    for n in ("q_self", "k_self", "v_self", "q_multi", "k_multi", "v_multi", "out", "grad_out",
              "dq_self", "dk_self", "dv_self", "dq_multi", "dk_multi", "dv_multi"):
        setattr(p, n, _fake())
    p.chain_id = 1 << 21
    p.B, p.H, p.L, p.D = 2, 20, 64, 32
    p.dtype, p.rope, p.scale = _lib.MPATTN_BF16, _lib.MPATTN_ROPE_NONE, 1.0
    p.workspace = 1 << 24
    # lse missing
    assert lib.mpattn_bwd(ctypes.byref(p), None) == _lib.MPATTN_ERR_INVALID
    assert "lse" in lib.mpattn_last_error().decode()
    p.lse = 1 << 25
    p.D = 40
    assert lib.mpattn_bwd(ctypes.byref(p), None) == _lib.MPATTN_ERR_UNSUPPORTED
    p.D = 32
    # workspace missing, undersized, misaligned
    assert lib.mpattn_bwd(ctypes.byref(p), None) == _lib.MPATTN_ERR_INVALID
    assert "workspace" in lib.mpattn_last_error().decode()
    need = lib.mpattn_bwd_workspace_size(2, 20, 64, 32)
    p.workspace_bytes = need - 1
    assert lib.mpattn_bwd(ctypes.byref(p), None) == _lib.MPATTN_ERR_INVALID
    assert "workspace" in lib.mpattn_last_error().decode()
    p.workspace, p.workspace_bytes = (1 << 24) + 8, need
    assert lib.mpattn_bwd(ctypes.byref(p), None) == _lib.MPATTN_ERR_INVALID
    p.workspace = 1 << 24


def _bwd_params(**over):
    p = _lib.BwdParams()
    for n in ("q_self", "k_self", "v_self", "q_multi", "k_multi", "v_multi", "out", "grad_out",
              "dq_self", "dk_self", "dv_self", "dq_multi", "dk_multi", "dv_multi"):
        setattr(p, n, _fake())
    p.chain_id = 1 << 21
    p.lse = 1 << 25
    p.B, p.H, p.L, p.D = 2, 20, 64, 32
    p.dtype, p.rope, p.scale = _lib.MPATTN_BF16, _lib.MPATTN_ROPE_NONE, 1.0
    p.workspace, p.workspace_bytes = 1 << 24, 1 << 40
    for k, v in over.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("name", ["q_self", "grad_out", "out", "dk_multi", "dv_self"])
def test_bwd_rejects_rows_past_32bit_offsets(lib, name):
    """Every one of the 14 backward tensors: a row stride that puts row L-1
    past 2^31 bytes from the (b, h) base is refused (the DMA offsets are
    32-bit), before anything is enqueued."""
    L = 64
    stride_t = (1 << 31) // (L * 2) + 8
    p = _bwd_params(**{name: _lib.Tensor4(1 << 20, 0, 0, stride_t)})
    assert lib.mpattn_bwd(ctypes.byref(p), None) == _lib.MPATTN_ERR_UNSUPPORTED
    assert "32-bit row offsets" in lib.mpattn_last_error().decode()
    assert name in lib.mpattn_last_error().decode()


def test_bwd_rejects_grid_past_32bit_work_items(lib):
    """dK/dV and dQ run as one grid of 4 B H ceil(L/128) workgroups and the
    prep at up to 20 threads per row: shapes whose launches would pass 2^32
    work-items are refused before anything is enqueued."""
    p = _bwd_params(B=1 << 16, H=64, L=1024)
    assert lib.mpattn_bwd(ctypes.byref(p), None) == _lib.MPATTN_ERR_UNSUPPORTED
    assert "too large for one launch" in lib.mpattn_last_error().decode()
    # 4096 * 44 rows of 1024: 24 work-items per row pass 2^32
    p = _bwd_params(B=1 << 12, H=44, L=1024)
    assert lib.mpattn_bwd(ctypes.byref(p), None) == _lib.MPATTN_ERR_UNSUPPORTED
    assert "too large for one launch" in lib.mpattn_last_error().decode()


def test_bwd_rejects_dense_mask_past_32bit_offsets(lib):
    L = 64
    p = _bwd_params(chain_id=None, chain_mask=1 << 23, mask_stride_b=0,
                    mask_stride_q=(1 << 31) // L + 16, mask_stride_k=1)
    assert lib.mpattn_bwd(ctypes.byref(p), None) == _lib.MPATTN_ERR_UNSUPPORTED
    assert "chain_mask" in lib.mpattn_last_error().decode()


def test_python_api_rejects_cpu_tensors():
    """No CPU fallback: host tensors are refused, never computed."""
    import mint_plus_amd as m
    x = torch.zeros(1, 2, 16, 32, dtype=torch.bfloat16)
    cid = torch.zeros(1, 16, dtype=torch.int32)
    with pytest.raises((RuntimeError, AssertionError, ValueError)):
        m.fused_multi_pathway_attention(x, x, x, x, x, x, None, chain_ids=cid, training=False)


def test_python_api_shape_asserts():
    """Shape mismatches raise AssertionError as in the reference wrapper."""
    import mint_plus_amd as m
    x = torch.zeros(1, 2, 16, 32, dtype=torch.bfloat16)
    y = torch.zeros(1, 2, 17, 32, dtype=torch.bfloat16)
    mask = torch.zeros(1, 16, 16, dtype=torch.bool)
    with pytest.raises(AssertionError):
        m.fused_multi_pathway_attention(x, y, x, x, x, x, mask, training=False)
    with pytest.raises(AssertionError):
        m.fused_multi_pathway_attention(x, x, x, x, x, x, mask[:, :8], training=False)


def _combine_fwd_params(**over):
    p = _lib.CombineFwdParams()
    p.intra_logits = p.inter_logits = _lib.Tensor4(1 << 26, 64 * 64 * 20, 64 * 64, 64)
    for n in ("intra_values", "inter_values", "out"):
        setattr(p, n, _fake())
    p.chain_mask = 1 << 21
    p.mask_stride_b, p.mask_stride_q, p.mask_stride_k = 64 * 64, 64, 1
    p.B, p.H, p.L, p.D = 2, 20, 64, 32
    p.dtype = _lib.MPATTN_BF16
    for k, v in over.items():
        setattr(p, k, v)
    return p


COMBINE_CASES = [
    (dict(D=12), _lib.MPATTN_ERR_UNSUPPORTED, "head dim"),
    (dict(D=72), _lib.MPATTN_ERR_UNSUPPORTED, "head dim"),
    (dict(B=0), _lib.MPATTN_ERR_INVALID, "must be >= 1"),
    (dict(dtype=3), _lib.MPATTN_ERR_INVALID, "dtype"),
    (dict(chain_mask=None), _lib.MPATTN_ERR_INVALID, "chain_mask"),
    (dict(mask_stride_k=-1), _lib.MPATTN_ERR_UNSUPPORTED, "negative"),
    (dict(dropout_p=1.0), _lib.MPATTN_ERR_INVALID, "dropout"),
    (dict(dropout_p=-0.5), _lib.MPATTN_ERR_INVALID, "dropout"),
    (dict(intra_logits=_lib.Tensor4(None, 0, 0, 64)), _lib.MPATTN_ERR_INVALID, "intra_logits"),
    (dict(out=_lib.Tensor4((1 << 20) + 4, 40960, 2048, 32)), _lib.MPATTN_ERR_UNSUPPORTED, "aligned"),
]


@pytest.mark.parametrize("over,code,msg", COMBINE_CASES)
def test_combine_fwd_validation(lib, over, code, msg):
    p = _combine_fwd_params(**over)
    assert lib.mpattn_combine_fwd(ctypes.byref(p), None) == code
    assert msg in lib.mpattn_last_error().decode()


def test_combine_bwd_validation(lib):
    assert lib.mpattn_combine_bwd(None, None) == _lib.MPATTN_ERR_INVALID
    p = _lib.CombineBwdParams()
    lg = _lib.Tensor4(1 << 26, 64 * 64 * 20, 64 * 64, 64)
    p.intra_logits = p.inter_logits = p.d_intra_logits = p.d_inter_logits = lg
    for n in ("intra_values", "inter_values", "grad_out", "d_intra_values", "d_inter_values"):
        setattr(p, n, _fake())
    p.chain_mask = 1 << 21
    p.mask_stride_b, p.mask_stride_q, p.mask_stride_k = 64 * 64, 64, 1
    p.B, p.H, p.L, p.D = 2, 20, 64, 32
    p.dtype = _lib.MPATTN_FP32
    # workspace missing
    assert lib.mpattn_combine_bwd(ctypes.byref(p), None) == _lib.MPATTN_ERR_INVALID
    assert "workspace" in lib.mpattn_last_error().decode()
    p.workspace = (1 << 24) + 128
    p.workspace_bytes = 1 << 30
    assert lib.mpattn_combine_bwd(ctypes.byref(p), None) == _lib.MPATTN_ERR_INVALID
    p.workspace = 1 << 24
    p.workspace_bytes = lib.mpattn_combine_bwd_workspace_size(2, 20, 64, 32) - 1
    assert lib.mpattn_combine_bwd(ctypes.byref(p), None) == _lib.MPATTN_ERR_INVALID
    assert "need" in lib.mpattn_last_error().decode()
    p.workspace_bytes = 1 << 30
    p.dropout_p = 1.5
    assert lib.mpattn_combine_bwd(ctypes.byref(p), None) == _lib.MPATTN_ERR_INVALID
    assert "dropout" in lib.mpattn_last_error().decode()


def test_combine_workspace_size(lib):
    assert lib.mpattn_combine_bwd_workspace_size(0, 1, 1, 32) == -1
    w = lib.mpattn_combine_bwd_workspace_size(16, 20, 1024, 32)
    assert w >= 2 * 16 * 20 * 1024 * 4 and w % 256 == 0


def test_combine_struct_layout():
    f = _lib.CombineFwdParams
    assert f.out.offset == 4 * 32 and f.lse.offset == 5 * 32
    assert f.B.offset == f.mask_stride_k.offset + 8
    b = _lib.CombineBwdParams
    assert b.d_inter_values.offset == 8 * 32 and b.chain_mask.offset == 9 * 32
    assert b.workspace_bytes.offset == b.workspace.offset + 8
    assert b.B.offset == b.workspace_bytes.offset + 8


def test_combine_python_rejects_non_bool_mask():
    """As the reference wrapper (kernels/__init__.py:203): the mask must be bool."""
    import mint_plus_amd as m
    x = torch.zeros(1, 2, 16, 32)
    lg = torch.zeros(1, 2, 16, 16)
    with pytest.raises(AssertionError):
        m.fused_multimer_combine(lg, lg, torch.zeros(1, 16, 16, dtype=torch.int32), x, x)


def test_resolve_dropout():
    """Dropout arguments: off outside training, p in [0, 1), the seed drawn
    from torch's CPU generator when not given."""
    from mint_plus_amd.kernels.multi_pathway_attention import _resolve_dropout
    assert _resolve_dropout(0.5, False) == (0.0, 0)
    assert _resolve_dropout(0.0, True) == (0.0, 0)
    assert _resolve_dropout(0.25, True, 7) == (0.25, 7)
    assert _resolve_dropout(0.25, True, -1) == (0.25, (1 << 64) - 1)
    for bad in (-0.1, 1.0, 1.5, float("nan")):
        with pytest.raises(ValueError):
            _resolve_dropout(bad, True)
    torch.manual_seed(3)
    a = _resolve_dropout(0.1, True)
    torch.manual_seed(3)
    b = _resolve_dropout(0.1, True)
    c = _resolve_dropout(0.1, True)
    assert a == b and a != c


def test_fwd_noalloc_rejects_shapes_beyond_scratch(lib):
    """mpattn_fwd_noalloc validates like mpattn_fwd, then refuses a shape
    whose workspace exceeds the static scratch, before touching the device."""
    limit = 48 << 20
    p = _fwd_params(B=8, H=40, L=2048, D=64)
    need = lib.mpattn_fwd_workspace_size(8, 40, 2048, 64, _lib.MPATTN_BF16, _lib.MPATTN_ROPE_FUSED)
    assert need > limit
    assert lib.mpattn_fwd_noalloc(ctypes.byref(p), None) == _lib.MPATTN_ERR_UNSUPPORTED
    msg = lib.mpattn_last_error().decode()
    assert "static scratch" in msg and str(need) in msg and str(limit) in msg
    p = _fwd_params(D=48)
    assert lib.mpattn_fwd_noalloc(ctypes.byref(p), None) == _lib.MPATTN_ERR_UNSUPPORTED
    assert "head dim" in lib.mpattn_last_error().decode()
    assert lib.mpattn_fwd_noalloc(None, None) == _lib.MPATTN_ERR_INVALID
