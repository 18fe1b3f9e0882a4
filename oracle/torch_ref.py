"""Chunked torch restatement of the oracle -- TEST INFRASTRUCTURE ONLY.

Same math as ``oracle/mpattn_oracle.py`` (which cites the reference lines it
follows), written with torch ops so parity at the benchmark shapes
(B=16, H=20, L=1024) can run on the GPU in fp32 or fp64 one batch element at
a time. ``tests/test_oracle.py`` pins it to the float64 numpy oracle.
Only tests, ``smoke()`` and ``bench.py``'s CPU-baseline leg use it.
"""
import numpy as np
import torch


def rope_tables(L, D, device, dtype=torch.float64):
    inv = (1.0 / 10000.0 ** (np.arange(0, D, 2, dtype=np.float64) / D)).astype(np.float32)
    ang = (np.arange(L, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float64)
    return (torch.from_numpy(np.cos(ang)).to(device=device, dtype=dtype),
            torch.from_numpy(np.sin(ang)).to(device=device, dtype=dtype))


def apply_rope(x, cos, sin):
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)


def forward(qs, ks, vs, qm, km, vm, chain_ids=None, chain_mask=None, key_pad=None, rope=False,
            scale=1.0, sqrt_softmax=False, dtype=torch.float32, chunk=1):
    """Reference forward; inputs (B, H, L, D) tensors. Returns (out, lse) in ``dtype``."""
    B, H, L, D = qs.shape
    dev = qs.device
    outs, lses = [], []
    if rope:
        cos, sin = rope_tables(L, D, dev, dtype)
    for b0 in range(0, B, chunk):
        sl = slice(b0, min(B, b0 + chunk))
        q1, k1, v1 = (t[sl].to(dtype) for t in (qs, ks, vs))
        q2, k2, v2 = (t[sl].to(dtype) for t in (qm, km, vm))
        if rope:
            q1, k1 = apply_rope(q1, cos, sin), apply_rope(k1, cos, sin)
        s_self = scale * torch.matmul(q1, k1.transpose(-1, -2).contiguous())
        s_multi = scale * torch.matmul(q2, k2.transpose(-1, -2).contiguous())
        if chain_mask is not None:
            cross = chain_mask[sl].to(dev).bool()
        else:
            c = chain_ids[sl].to(dev)
            cross = c[:, :, None] != c[:, None, :]
        s = torch.where(cross[:, None], s_multi, s_self)
        del s_self, s_multi
        if key_pad is not None:
            s = s.masked_fill(key_pad[sl].to(dev).bool()[:, None, None, :], float("-inf"))
        m = s.amax(dim=-1, keepdim=True)
        dead = ~torch.isfinite(m)
        m = torch.where(dead, torch.zeros_like(m), m)
        e = torch.exp(s - m)
        del s
        l = e.sum(dim=-1, keepdim=True)
        p = torch.where(l > 0, e / torch.where(l > 0, l, torch.ones_like(l)), torch.zeros_like(e))
        del e
        w = p.sqrt() if sqrt_softmax else p
        out = torch.matmul(w.masked_fill(cross[:, None], 0.0), v1) + \
            torch.matmul(w.masked_fill(~cross[:, None], 0.0), v2)
        lse = torch.where(l[..., 0] > 0, m[..., 0] + torch.log(torch.where(l[..., 0] > 0, l[..., 0],
                                                                           torch.ones_like(l[..., 0]))),
                          torch.full_like(l[..., 0], float("-inf")))
        outs.append(out)
        lses.append(lse)
    return torch.cat(outs), torch.cat(lses)
