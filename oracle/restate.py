"""numpy restatement of the reference's hot-path rows -- TEST INFRASTRUCTURE ONLY.

Each function restates the arithmetic of one CpuDevice row of olibartfast/nert
and cites the file:line it follows. The reference accumulates every dot product
in double and rounds once to float32; a float32 x float32 product is exact in
double, so a float64 matmul of the float32 operands differs from the reference
only in the order of its double additions (relative 1e-16), which the final
float32 rounding almost always absorbs. That makes these restatements usable at
full BASELINE sizes where the reference's naive loops would take minutes.

Every function here is pinned by tests/test_oracle.py against the reference
library (oracle/_ref) and the reference's own known-answer values.
"""

from __future__ import annotations

import numpy as np


def gemm(a: np.ndarray, b: np.ndarray, c: np.ndarray | None = None, trans_a: int = 0, trans_b: int = 0,
         alpha: float = 1.0, beta: float = 1.0) -> np.ndarray:
    """src/kernels/gemm.cpp:119-136: y = alpha*op(A)op(B) + beta*C, in double, rounded once."""
    A = a.astype(np.float64)
    B = b.astype(np.float64)
    if trans_a:
        A = A.T
    if trans_b:
        B = B.T
    y = np.float64(np.float32(alpha)) * (A @ B)
    if c is not None:
        y = y + np.float64(np.float32(beta)) * c.astype(np.float64)
    return y.astype(np.float32)


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """src/kernels/mat_mul.cpp:94-168: NumPy matmul semantics (1-D promotion,
    batch broadcast), double accumulation, one rounding."""
    return np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(np.float32)


def _pads(auto_pad: str, in_sp, k, d, s, pads):
    """src/kernels/conv.cpp:78-119."""
    r = len(in_sp)
    if auto_pad == "VALID":
        return [0] * r, [0] * r
    if auto_pad in ("SAME_UPPER", "SAME_LOWER"):
        pb, pe = [], []
        for i in range(r):
            out = (in_sp[i] + s[i] - 1) // s[i]
            eff = d[i] * (k[i] - 1) + 1
            total = max(0, (out - 1) * s[i] + eff - in_sp[i])
            if auto_pad == "SAME_UPPER":
                pb.append(total // 2)
                pe.append(total - total // 2)
            else:
                pe.append(total // 2)
                pb.append(total - total // 2)
        return pb, pe
    if not pads:
        return [0] * r, [0] * r
    return list(pads[:r]), list(pads[r:])


def conv(x: np.ndarray, w: np.ndarray, bias: np.ndarray | None = None, strides=None, dilations=None, pads=None,
         group: int = 1, auto_pad: str = "NOTSET") -> np.ndarray:
    """src/kernels/conv.cpp:138-295: ONNX cross-correlation, 1-3 spatial axes,
    groups, strides, dilations, pads; bias + sum of products in double, one
    rounding. Restated as per-tap shifted products (im2col order does not
    matter for a double sum)."""
    sp = x.ndim - 2
    strides = list(strides) if strides else [1] * sp
    dilations = list(dilations) if dilations else [1] * sp
    in_sp = list(x.shape[2:])
    k = list(w.shape[2:])
    pb, pe = _pads(auto_pad, in_sp, k, dilations, strides, pads or [])
    out_sp = [(in_sp[i] + pb[i] + pe[i] - (dilations[i] * (k[i] - 1) + 1)) // strides[i] + 1 for i in range(sp)]
    n, c = x.shape[:2]
    m = w.shape[0]
    cg, mg = c // group, m // group
    xp = np.zeros([n, c] + [in_sp[i] + pb[i] + pe[i] + dilations[i] * k[i] for i in range(sp)], np.float64)
    xp[(slice(None), slice(None)) + tuple(slice(pb[i], pb[i] + in_sp[i]) for i in range(sp))] = x
    y = np.zeros([n, m] + out_sp, np.float64)
    w64 = w.astype(np.float64)
    for g in range(group):
        xg = xp[:, g * cg:(g + 1) * cg]
        wg = w64[g * mg:(g + 1) * mg]
        for tap in np.ndindex(*k):
            sl = tuple(slice(tap[i] * dilations[i], tap[i] * dilations[i] + strides[i] * (out_sp[i] - 1) + 1,
                             strides[i]) for i in range(sp))
            patch = xg[(slice(None), slice(None)) + sl]  # [n, cg, *out]
            wt = wg[(slice(None), slice(None)) + tap]     # [mg, cg]
            y[:, g * mg:(g + 1) * mg] += np.einsum("nc...,mc->nm...", patch, wt)
    if bias is not None:
        y += bias.astype(np.float64).reshape([1, m] + [1] * sp)
    return y.astype(np.float32)
