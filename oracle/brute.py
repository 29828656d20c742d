"""numpy float64 scalar loops over tiny inputs — TEST INFRASTRUCTURE.

These pin ``oracle.eager`` independently of torch: every quantity is built
element by element from the closed forms of the reference
(kernels.py:1328-1365 norms, :2053-2084 attention, :2592-2601 quantiser).
Only ``tests/`` use this module.  Inputs must be small (pure-Python loops).
"""
from __future__ import annotations

import math

import numpy as np

EPS = 1e-12


def squareplus(a: float) -> float:
    return 0.5 * (a + math.sqrt(a * a + 4.0))


def family_weights(x: np.ndarray, alpha: float, theta: float, power: int) -> np.ndarray:
    out = np.empty(x.shape, dtype=np.float64)
    for idx in np.ndindex(x.shape):
        out[idx] = squareplus(alpha * (float(x[idx]) - theta)) ** power
    return out


def norm_rowwise(x: np.ndarray, alpha=2.0, theta=0.5, power=2) -> np.ndarray:
    """y_ij / (sum_j y_ij + EPS) over the last axis."""
    x = np.asarray(x, dtype=np.float64)
    y = family_weights(x, alpha, theta, power)
    out = np.empty_like(y)
    for idx in np.ndindex(x.shape[:-1]):
        s = 0.0
        for j in range(x.shape[-1]):
            s += y[idx + (j,)]
        for j in range(x.shape[-1]):
            out[idx + (j,)] = y[idx + (j,)] / (s + EPS)
    return out


def norm_causal(x: np.ndarray, alpha=2.0, theta=0.5, power=2) -> np.ndarray:
    """Causal: row i of each [L, L] matrix normalises over j <= i, zeros above."""
    x = np.asarray(x, dtype=np.float64)
    L = x.shape[-1]
    out = np.zeros_like(x)
    for idx in np.ndindex(x.shape[:-2]):
        for i in range(L):
            ys = [squareplus(alpha * (float(x[idx + (i, j)]) - theta)) ** power for j in range(i + 1)]
            s = sum(ys) + EPS
            for j in range(i + 1):
                out[idx + (i, j)] = ys[j] / s
    return out


def fd_grad(f, x: np.ndarray, dy: np.ndarray, h: float = 1e-6) -> np.ndarray:
    """Central finite differences of sum(f(x) * dy) with respect to x."""
    x = np.asarray(x, dtype=np.float64).copy()
    g = np.zeros_like(x)
    for idx in np.ndindex(x.shape):
        old = x[idx]
        x[idx] = old + h
        fp = float((f(x) * dy).sum())
        x[idx] = old - h
        fm = float((f(x) * dy).sum())
        x[idx] = old
        g[idx] = (fp - fm) / (2 * h)
    return g


def attention(q, k, v, scale=None, window_size=0) -> np.ndarray:
    """O[b,h,i] = sum_{j<=i, i-j<W} y_ij V[b,h//G,j] / (sum y + EPS), scalar loops."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = np.zeros((B, Hq, T, D))
    for b in range(B):
        for h in range(Hq):
            hk = h // G
            for i in range(T):
                ws = []
                for j in range(i + 1):
                    if window_size > 0 and i - j >= window_size:
                        ws.append(0.0)
                        continue
                    s = 0.0
                    for d in range(D):
                        s += q[b, h, i, d] * k[b, hk, j, d]
                    ws.append(squareplus(2.0 * s * scale - 1.0) ** 2)
                tot = sum(ws) + EPS
                for j, w in enumerate(ws):
                    out[b, h, i] += (w / tot) * v[b, hk, j]
    return out


def e4m3fn_grid() -> np.ndarray:
    """All finite non-negative float8_e4m3fn values, from the format definition.

    e4m3fn (OCP): 1 sign, 4 exponent (bias 7), 3 mantissa bits; no infinities;
    only S.1111.111 is NaN, so the largest finite value is 1.75 * 2^8 = 448.
    Returned as (code, value) pairs for codes 0..126.
    """
    vals = []
    for code in range(0x7F):
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0:
            val = (m / 8.0) * 2.0 ** (1 - 7)
        else:
            val = (1.0 + m / 8.0) * 2.0 ** (e - 7)
        vals.append((code, val))
    return np.array(vals, dtype=np.float64)


def e4m3fn_round(x: float) -> int:
    """Round-to-nearest-even of a finite |x| <= 448 onto e4m3fn; returns the 8-bit code."""
    grid = e4m3fn_grid()
    sign = 0x80 if (x < 0 or (x == 0 and math.copysign(1.0, x) < 0)) else 0
    ax = abs(x)
    vals = grid[:, 1]
    i = int(np.searchsorted(vals, ax))
    if i == 0:
        code = 0
    elif i >= len(vals):
        code = int(grid[-1, 0])
    else:
        lo, hi = vals[i - 1], vals[i]
        if ax == hi:
            code = int(grid[i, 0])
        elif ax - lo < hi - ax:
            code = int(grid[i - 1, 0])
        elif ax - lo > hi - ax:
            code = int(grid[i, 0])
        else:  # tie: even mantissa
            code = int(grid[i - 1, 0]) if int(grid[i - 1, 0]) % 2 == 0 else int(grid[i, 0])
    return sign | code


def rope(x: np.ndarray, base: float = 10000.0) -> np.ndarray:
    """Rotate-half RoPE of x [..., T, D] as a complex rotation: the pair
    (x[d], x[d + D/2]) is z = x[d] + i x[d + D/2], multiplied by
    exp(i t base^(-2d/D)) at position t (float64)."""
    x = np.asarray(x, dtype=np.float64)
    T, D = x.shape[-2], x.shape[-1]
    h = D // 2
    out = np.empty_like(x)
    for idx in np.ndindex(x.shape[:-2]):
        for t in range(T):
            for d in range(h):
                ang = t * base ** (-2.0 * d / D)
                z = complex(x[idx + (t, d)], x[idx + (t, d + h)]) * complex(math.cos(ang), math.sin(ang))
                out[idx + (t, d)] = z.real
                out[idx + (t, d + h)] = z.imag
    return out


def softmax(x: np.ndarray) -> np.ndarray:
    """exp(x_j - max) / sum over the last axis, element by element."""
    x = np.asarray(x, dtype=np.float64)
    out = np.empty_like(x)
    for idx in np.ndindex(x.shape[:-1]):
        row = [float(v) for v in x[idx]]
        m = max(row)
        e = [math.exp(v - m) for v in row]
        s = sum(e)
        for j, v in enumerate(e):
            out[idx + (j,)] = v / s
    return out
