"""torch-CPU restatement of the reference's eager formulas — TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may use this module, as the checker or as the timed CPU baseline.  The
product never imports it.

All citations are ``path:line`` into the reference (NoSelection/smooth-attn).
Each function says what pins it ("pinned by: …"); the pins live in
``tests/test_oracle.py`` and compare against ``oracle.brute`` (numpy float64
scalar loops), closed forms, invariants, finite differences and torch autograd.

Numerics follow the reference's eager path: inputs are upcast with ``.float()``
(fp32 math) unless a float64 tensor is passed in, in which case everything
stays float64 (used for tight fixtures).
"""
from __future__ import annotations

import math

import torch

# kernels.py:57
EPS = 1e-12
# kernels.py:24
SUPPORTED_POWERS = (1, 2, 3)
# kernels.py:2597 (largest finite float8_e4m3fn)
FP8_MAX = 448.0


def _work_dtype(t: torch.Tensor) -> torch.dtype:
    return torch.float64 if t.dtype == torch.float64 else torch.float32


def squareplus(a: torch.Tensor) -> torch.Tensor:
    """squareplus(a) = (a + sqrt(a^2 + 4)) / 2 — kernels.py:1328-1329.

    pinned by: sp(0)=1, sp(a)*sp(-a)=1, sp(a)-sp(-a)=a, brute.squareplus.
    """
    return 0.5 * (a + torch.sqrt(a * a + 4.0))


def family_weights(x: torch.Tensor, alpha: float, theta: float, power: int) -> torch.Tensor:
    """y = squareplus(alpha*(x-theta))^power by repeated products — kernels.py:1338-1343.

    pinned by: brute.family_weights (float64 loops).
    """
    if power not in SUPPORTED_POWERS:
        raise ValueError(f"power must be one of {SUPPORTED_POWERS}, got {power}")
    y = squareplus(alpha * (x - theta))
    if power == 2:
        y = y * y
    elif power == 3:
        y = y * y * y
    return y


def causal_mask(seq_len: int) -> torch.Tensor:
    """Strict upper triangle (True = masked) — kernels.py:226-233."""
    return torch.triu(torch.ones(seq_len, seq_len, dtype=torch.bool), diagonal=1)


def softplus_norm_eager(x, alpha=2.0, theta=0.5, power=2):
    """Row-wise normalisation y / (sum_row y + EPS) — kernels.py:1332-1346.

    pinned by: brute.norm_rowwise on tiny rows; constant row -> 1/L; rows sum to 1.
    """
    x = x.to(_work_dtype(x))
    y = family_weights(x, alpha, theta, power)
    return y / (y.sum(dim=-1, keepdim=True) + EPS)


def softplus_norm_causal_eager(x, alpha=2.0, theta=0.5, power=2):
    """Causal normalisation over j <= i, exact zeros above — kernels.py:1349-1365.

    pinned by: brute.norm_causal; row 0 = e0; constant row -> 1/(i+1) on the
    visible prefix; strict upper triangle exactly 0; rows sum to 1.
    """
    x = x.to(_work_dtype(x))
    y = family_weights(x, alpha, theta, power)
    y = y.masked_fill(causal_mask(x.shape[-1]), 0.0)
    return y / (y.sum(dim=-1, keepdim=True) + EPS)


def softplus_norm_causal_cpu_path(x, alpha=2.0, theta=0.5, power=2):
    """The reference's CPU path ``implementation="eager"`` — kernels.py:1418-1419.

    ``softplus_norm_causal_eager(x.float()).to(x.dtype)``: fp32 math, result in
    the input dtype.  This is what bench.py times as the CPU baseline.
    """
    return softplus_norm_causal_eager(x.float(), alpha, theta, power).to(x.dtype)


def softmax_eager(x):
    """Row-wise softmax in the work dtype — the comparison baseline of
    kernels.py:534-562 (F.softmax over the last dim).

    pinned by: brute.softmax (float64 loops); rows sum to 1; invariance under
    a per-row shift.
    """
    return torch.softmax(x.to(_work_dtype(x)), dim=-1)


def softmax_causal_eager(x):
    """Causal softmax: strict upper triangle masked to -inf, then softmax —
    kernels.py:1368-1370 (and the kernel :852-884, which writes 0 there).

    pinned by: brute.softmax on each visible prefix; exact zeros above the
    diagonal; row 0 is e0.
    """
    xw = x.to(_work_dtype(x))
    return torch.softmax(xw.masked_fill(causal_mask(x.shape[-1]), float("-inf")), dim=-1)


def softplus_norm_backward(x, dy, alpha=2.0, theta=0.5, power=2, *, causal=True):
    """Closed-form gradient of the (causal or row-wise) normalisation.

    Restates the fused backward formula of kernels.py:711-739 (generic family)
    and :771-789 (default family), which the reference checks against autograd
    of the eager forward (tests/test_training_api.py:63-78):

        a = alpha (x - theta),  s = a^2 + 4,  sp = (a + sqrt s)/2
        y = sp^p (masked),      S = sum y + EPS,  P = y / S
        dydx = alpha p sp^(p-1) * (1 + a / sqrt s)/2   (masked)
        dx = dydx / S * (dy - sum_j dy_j P_j)          (masked)

    The row-wise variant has no reference kernel (the reference row-wise API
    has no autograd, kernels.py:985-1031); its gradient is autograd of
    ``softplus_norm_eager`` (kernels.py:1332-1346), which this formula equals.

    pinned by: torch autograd of the eager forward in float64; central finite
    differences (brute.fd_grad); dy constant along a row -> dx ~ 0.
    """
    wd = _work_dtype(x)
    x = x.to(wd)
    g = dy.to(wd)
    a = alpha * (x - theta)
    s = a * a + 4.0
    rs = torch.sqrt(s)
    sp = 0.5 * (a + rs)
    if power == 1:
        y, dydx = sp, alpha * (0.5 * (1.0 + a / rs))
    elif power == 2:
        y, dydx = sp * sp, alpha * 2.0 * sp * (0.5 * (1.0 + a / rs))
    elif power == 3:
        y, dydx = sp * sp * sp, alpha * 3.0 * sp * sp * (0.5 * (1.0 + a / rs))
    else:
        raise ValueError(f"power must be one of {SUPPORTED_POWERS}, got {power}")
    if causal:
        m = causal_mask(x.shape[-1])
        y = y.masked_fill(m, 0.0)
        dydx = dydx.masked_fill(m, 0.0)
        g = g.masked_fill(m, 0.0)
    S = y.sum(dim=-1, keepdim=True) + EPS
    P = y / S
    dot = (g * P).sum(dim=-1, keepdim=True)
    dx = dydx / S * (g - dot)
    if causal:
        dx = dx.masked_fill(causal_mask(x.shape[-1]), 0.0)
    return dx


def _expand_kv(t: torch.Tensor, n_q_heads: int) -> torch.Tensor:
    """GQA head expansion, query head h reads KV head h // G — kernels.py:2060-2064."""
    B, Hkv, T, D = t.shape
    if Hkv == n_q_heads:
        return t
    g = n_q_heads // Hkv
    return t.unsqueeze(2).expand(B, Hkv, g, T, D).reshape(B, n_q_heads, T, D)


def flash_attention_eager(q, k, v, *, scale=None, window_size=0, return_row_sums=False,
                          score_scale=None):
    """Materialised squareplus attention — kernels.py:2053-2084.

    O_i = sum_{j<=i, i-j<W} y_ij V_j / (sum_j y_ij + EPS),
    y = squareplus(2 s - 1)^2, s = scale * q_i . k_j.

    Returns the fp32 (or fp64 for fp64 inputs) output without the final cast
    the reference applies (``.to(q.dtype)``, :2084); callers cast when needed.
    With ``return_row_sums`` also returns sum_j y_ij + EPS, which is what the
    fused kernels store as row sums (s_acc starts at 1e-12, :1584, :1629-1631).
    ``score_scale`` overrides ``scale`` as the full multiplier on q.k (the fp8
    path folds dequantisation scales into it).  Computed one (b, h) slice at a
    time so that large shapes fit in host memory.

    pinned by: brute.attention on tiny shapes; T=1 -> O=V0; identical V rows ->
    O=V; W>=T equals full causal; W=1 -> O_i=V_i; GQA = repeat_interleave;
    equals softplus_norm_causal_eager(scale q k^T) @ V.
    """
    B, Hq, T, D = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    mult = scale if score_scale is None else score_scale
    wd = _work_dtype(q)
    k = _expand_kv(k, Hq)
    v = _expand_kv(v, Hq)
    out = torch.empty(B, Hq, T, D, dtype=wd)
    rows = torch.empty(B, Hq, T, dtype=wd)
    cm = causal_mask(T)
    if window_size > 0:
        pos = torch.arange(T)
        cm = cm | ((pos[:, None] - pos[None, :]) >= window_size)
    for b in range(B):
        for h in range(Hq):
            s = (q[b, h].to(wd) @ k[b, h].to(wd).transpose(0, 1)) * mult
            a = 2.0 * s - 1.0
            sp = 0.5 * (a + torch.sqrt(a * a + 4.0))
            y = (sp * sp).masked_fill(cm, 0.0)
            S = y.sum(dim=-1, keepdim=True) + EPS
            out[b, h] = (y / S) @ v[b, h].to(wd)
            rows[b, h] = S[:, 0]
    if return_row_sums:
        return out, rows
    return out


def flash_attention_grads(q, k, v, do, *, scale=None, window_size=0):
    """(dq, dk, dv) by autograd of the eager attention in fp32/fp64.

    This is the reference's own backward check (tests/test_training_api.py:
    147-158): autograd through ``sp2norm_flash_attention_eager`` with the
    upstream gradient.  pinned by: central finite differences on tiny shapes.
    """
    wd = _work_dtype(q)
    qr = q.detach().to(wd).requires_grad_(True)
    kr = k.detach().to(wd).requires_grad_(True)
    vr = v.detach().to(wd).requires_grad_(True)
    B, Hq, T, D = q.shape
    sc = scale if scale is not None else 1.0 / math.sqrt(D)
    ke = _expand_kv(kr, Hq)
    ve = _expand_kv(vr, Hq)
    s = torch.matmul(qr, ke.transpose(-2, -1)) * sc
    a = 2.0 * s - 1.0
    sp = 0.5 * (a + torch.sqrt(a * a + 4.0))
    cm = causal_mask(T)
    if window_size > 0:
        pos = torch.arange(T)
        cm = cm | ((pos[:, None] - pos[None, :]) >= window_size)
    y = (sp * sp).masked_fill(cm, 0.0)
    o = torch.matmul(y / (y.sum(-1, keepdim=True) + EPS), ve)
    (o * do.to(wd)).sum().backward()
    return qr.grad, kr.grad, vr.grad


def flash_attention_bwd(q, k, v, o, do, *, scale=None, window_size=0):
    """(dq, dk, dv) by the reference backward's own formula, given the
    forward output ``o`` — kernels.py:1667-1784 (dQ; delta = rowsum(dO * O)
    from the stored O, :1722-1727) and :1787-1909 (dK, dV summed over the
    GQA group):
        R = sum_j y_ij + EPS, P = y / R, dP = dO V^T,
        dS = (dP - delta) / R * 4 sp sp' scale,  sp' = (1 + a / sqrt(a^2 + 4)) / 2,
        dQ = dS K, dK = dS^T Q, dV = P^T dO.
    Work dtype float64 for float64 inputs.  With ``o`` taken from a forward
    that rounded P (the fused kernels do), delta carries that rounding, as it
    does in the reference; this matters where the true gradient vanishes
    (one visible key: dQ = dK = 0 up to that rounding).

    pinned by: equals flash_attention_grads (autograd) when ``o`` is the
    exact eager output, causal / window / GQA (tests/test_oracle.py).
    """
    wd = _work_dtype(q)
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    sc = scale if scale is not None else 1.0 / math.sqrt(D)
    qf, kf, vf, of, dof = (t.detach().to(wd) for t in (q, k, v, o, do))
    ke = _expand_kv(kf, Hq)
    ve = _expand_kv(vf, Hq)
    cm = causal_mask(T)
    if window_size > 0:
        pos = torch.arange(T)
        cm = cm | ((pos[:, None] - pos[None, :]) >= window_size)
    s = torch.matmul(qf, ke.transpose(-2, -1)) * sc
    a = 2.0 * s - 1.0
    r4 = torch.sqrt(a * a + 4.0)
    sp = 0.5 * (a + r4)
    y = (sp * sp).masked_fill(cm, 0.0)
    R = y.sum(-1, keepdim=True) + EPS
    P = y / R
    dP = torch.matmul(dof, ve.transpose(-2, -1))
    delta = (dof * of).sum(-1, keepdim=True)
    dS = ((dP - delta) / R * 4.0 * sp * (0.5 * (1.0 + a / r4)) * sc).masked_fill(cm, 0.0)
    dq = torch.matmul(dS, ke)
    dk = torch.matmul(dS.transpose(-2, -1), qf).view(B, Hkv, G, T, D).sum(2)
    dv = torch.matmul(P.transpose(-2, -1), dof).view(B, Hkv, G, T, D).sum(2)
    return dq, dk, dv


def rope_cos_sin(dim, seq_len, base=10000.0, dtype=torch.float32):
    """cos / sin tables [seq_len, dim/2] — kernels.py:2093-2101 (fp32 math,
    as the reference).

    pinned by: cos(t * base^(-2i/dim)) / sin(...) evaluated in float64.
    """
    inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2).float() / dim))
    t = torch.arange(seq_len, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    return freqs.cos().to(dtype), freqs.sin().to(dtype)


def apply_rope(x, cos, sin):
    """Rotate-half RoPE over the last dim, position = index along dim -2 —
    the reference test's ``apply_rope_eager`` (tests/test_rope_proj.py:15-30):
    x * [cos, cos] + [-x2, x1] * [sin, sin].

    pinned by: complex multiplication (x_a + i x_b) e^{i theta} (brute.rope);
    identity at position 0; pairwise norms preserved; dot products of rotated
    vectors depend only on the position difference.
    """
    T, D = x.shape[-2], x.shape[-1]
    c = cos[:T].to(x.dtype)
    s = sin[:T].to(x.dtype)
    cf = torch.cat([c, c], dim=-1)
    sf = torch.cat([s, s], dim=-1)
    x1 = x[..., : D // 2]
    x2 = x[..., D // 2:]
    return x * cf + torch.cat([-x2, x1], dim=-1) * sf


def rope_flash_attention_eager(q, k, v, cos, sin, *, scale=None, window_size=0, round_to=torch.bfloat16):
    """The reference test's oracle for the RoPE forward
    (tests/test_rope_proj.py:46-63): rotate q and k in fp32, round them to
    ``round_to`` (None keeps them), then eager attention in the work dtype.

    pinned by: apply_rope and flash_attention_eager (each pinned).
    """
    wd = _work_dtype(q)
    qr = apply_rope(q.to(wd), cos.to(wd), sin.to(wd))
    kr = apply_rope(k.to(wd), cos.to(wd), sin.to(wd))
    if round_to is not None:
        qr = qr.to(round_to).to(wd)
        kr = kr.to(round_to).to(wd)
    return flash_attention_eager(qr, kr, v.to(wd), scale=scale, window_size=window_size)


def rope_proj_eager(q, k, v, w_o, cos, sin, *, scale=None, window_size=0, round_to=torch.bfloat16):
    """RoPE attention then sum_h O_h W_o[h] -> [B, T, D_model] — the
    reference test's projection oracle (tests/test_rope_proj.py:117-146).

    pinned by: equals one matmul of O in [B, T, H*D] order with W_o
    reshaped to [H*D, D_model].
    """
    o = rope_flash_attention_eager(q, k, v, cos, sin, scale=scale, window_size=window_size, round_to=round_to)
    B, H, T, D = o.shape
    out = torch.zeros(B, T, w_o.shape[2], dtype=o.dtype)
    for h in range(H):
        out += o[:, h] @ w_o[h].to(o.dtype)
    return out


def quantize_to_fp8(x: torch.Tensor):
    """Per-tensor absmax e4m3fn quantiser — kernels.py:2592-2601.

    scale = max(amax|x| / 448, 1e-12); x8 = e4m3fn(clamp(x / scale, +-448)).
    Returns (x8, scale) with scale as a 0-d float32 tensor (the reference
    returns ``scale.item()``, the same fp32 value as a Python float).

    pinned by: brute.e4m3fn_round (nearest-even over the enumerated e4m3fn
    grid) bit-exactly, and the dequantisation error bound |x - x8*s| <= ulp/2.
    """
    xf = x.detach().float()
    amax = xf.abs().amax()
    scale = (amax / FP8_MAX).clamp(min=1e-12)
    xs = (xf / scale).clamp(-FP8_MAX, FP8_MAX)
    return xs.to(torch.float8_e4m3fn), scale


def fp8_flash_attention_eager(q8, k8, v, q_scale, k_scale, v_scale, attn_scale, *,
                              window_size=0, return_row_sums=False):
    """Dequantised restatement of the fp8 fused forward — kernels.py:2498-2589.

    scores = (q8 . k8) * q_scale * k_scale * attn_scale   (:2534, :2565)
    O = sum y * (v * v_scale) / (sum y + EPS)            (:2579-2581)
    ``v`` may be fp8 (the reference entry point, :2666) or bf16 (v_scale = 1).
    Evaluated in float64 on the exactly dequantised codes.

    pinned by: reduces to flash_attention_eager on dequantised inputs (the
    function is exactly that composition); tests check the composition against
    brute.attention.
    """
    qd = q8.double()
    kd = k8.double()
    vd = v.double() * float(v_scale)
    mult = float(q_scale) * float(k_scale) * float(attn_scale)
    return flash_attention_eager(qd, kd, vd, score_scale=mult, window_size=window_size,
                                 return_row_sums=return_row_sums)


def paged_decode_eager(q, k_cache, v_cache, block_table, context_lens, *, scale=None):
    """Single-token decode through a block table.

    Gathers each sequence's first ``ctx`` tokens page by page
    (``K[t] = k_cache[block_table[b, t // P], h // G, t % P]``, the addressing of
    kernels.py:2733-2743) and applies the decode reference of
    tests/test_paged_long_context.py:39-65 (and test_paged_attention.py:76-109):
    scores = scale q.K, y = squareplus(2 s - 1)^2, O = y/(sum y + 1e-12) @ V.
    Returns fp32 [B, Hq, D] (the reference casts to bf16 at the end).

    pinned by: equals the last row of flash_attention_eager on the gathered
    sequence; shuffled tables equal sequential ones; ctx=1 -> O=V0; results
    independent of page size.
    """
    B, Hq, _, D = q.shape
    _, Hkv, P, _ = k_cache.shape
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    wd = _work_dtype(q)
    out = torch.empty(B, Hq, D, dtype=wd)
    for b in range(B):
        n = int(context_lens[b])
        npg = (n + P - 1) // P
        pages = block_table[b, :npg].long()
        kk = k_cache[pages].to(wd).permute(1, 0, 2, 3).reshape(Hkv, npg * P, D)[:, :n]
        vv = v_cache[pages].to(wd).permute(1, 0, 2, 3).reshape(Hkv, npg * P, D)[:, :n]
        for h in range(Hq):
            s = (kk[h // G] @ q[b, h, 0].to(wd)) * scale
            a = 2.0 * s - 1.0
            sp = 0.5 * (a + torch.sqrt(a * a + 4.0))
            y = sp * sp
            out[b, h] = (y / (y.sum() + EPS)) @ vv[h // G]
    return out
