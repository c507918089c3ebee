"""Independent statements of the operation used to pin the C oracle (not the oracle itself).

* `conv1d_fwd`: the textbook form, a grouped torch F.conv1d over concat(initial_states | zeros, x),
  in float64 (reference README.md:7, causal_conv1d.py:1-9).
* `shifted_fwd`: a shifted-sum form with sequence-equality masks, for seq_idx (README.md:44-46,
  causal_conv1d.py:17-25 and :129-138), also float64 and differentiable.
* `brute_fwd` / `brute_bwd`: per-element pure-Python loops over the definition, for tiny shapes.

Backward values come from torch autograd of the float64 forms.
"""

import math

import torch
import torch.nn.functional as F


def _pre(x, init, P):
    B, _, D = x.shape
    if init is None:
        return torch.zeros(B, P, D, dtype=x.dtype)
    return init.to(x.dtype)


def conv1d_fwd(x, w, bias=None, init=None, silu=False):
    """act(F.conv1d(concat(init|0, x), groups=D) + bias) and final = concat(init|0, x)[:, T:]."""
    B, T, D = x.shape
    P = w.shape[1] - 1
    xx = torch.cat([_pre(x, init, P), x], dim=1)
    z = F.conv1d(xx.transpose(1, 2), w[:, None, :], bias, groups=D).transpose(1, 2)
    out = z * torch.sigmoid(z) if silu else z
    return out, xx[:, T:]


def shifted_fwd(x, w, bias=None, seq=None, init=None, silu=False):
    """z[t] = w[P] x[t] + sum_k [s(t-P+k) == s(t)] w[k] xx[t-P+k] (+ bias), z = 0 where s(t) < 0."""
    B, T, D = x.shape
    W = w.shape[1]
    P = W - 1
    xx = torch.cat([_pre(x, init, P), x], dim=1)
    z = w[:, P] * x
    if seq is not None:
        s0 = seq[:, :1] if init is not None else torch.full((B, 1), -1, dtype=seq.dtype)
        s_ext = torch.cat([s0.expand(B, P), seq], dim=1)
    for k in range(P):
        term = w[:, k] * xx[:, k:k + T]
        if seq is not None:
            term = term * (s_ext[:, k:k + T] == seq)[..., None].to(x.dtype)
        z = z + term
    if bias is not None:
        z = z + bias
    if seq is not None:
        z = z * (seq >= 0)[..., None].to(x.dtype)
    out = z * torch.sigmoid(z) if silu else z
    return out, xx[:, T:]


def autograd_bwd(fwd_fn, x, w, dout, bias=None, init=None, dfinal=None, silu=False, seq=None):
    """(dx, dweight, dbias, dinit) of <out, dout> + <final, dfinal> through fwd_fn, in float64."""
    x = x.detach().double().requires_grad_(True)
    w = w.detach().double().requires_grad_(True)
    b = None if bias is None else bias.detach().double().requires_grad_(True)
    i = None if init is None else init.detach().double().requires_grad_(True)
    if seq is None:
        out, fin = fwd_fn(x, w, b, init=i, silu=silu)
    else:
        out, fin = fwd_fn(x, w, b, seq=seq, init=i, silu=silu)
    loss = (out * dout.double()).sum()
    if dfinal is not None:
        loss = loss + (fin * dfinal.double()).sum()
    grads = torch.autograd.grad(loss, [t for t in (x, w, b, i) if t is not None], allow_unused=True)
    it = iter(grads)
    gx = next(it)
    gw = next(it)
    gb = next(it) if b is not None else None
    gi = next(it) if i is not None else None
    if gi is None and i is not None:
        gi = torch.zeros_like(i)
    return gx, gw, gb, gi


def _sig(z):
    return 1.0 / (1.0 + math.exp(-z)) if z > -700 else 0.0


def brute_fwd(x, w, bias=None, seq=None, init=None, silu=False):
    """Nested lists in, nested lists out; definition applied element by element."""
    B, T, D = len(x), len(x[0]) if x else 0, len(w)
    W = len(w[0])
    P = W - 1

    def xx(b, t, d):
        if 0 <= t < T:
            return x[b][t][d]
        if -P <= t < 0 and init is not None:
            return init[b][t + P][d]
        return 0.0

    def s(b, t):
        if t >= T:
            return -1
        if t < 0:
            return seq[b][0] if init is not None else -1
        return seq[b][t]

    out = [[[0.0] * D for _ in range(T)] for _ in range(B)]
    for b in range(B):
        for t in range(T):
            for d in range(D):
                z = 0.0
                for k in range(W):
                    r = t - P + k
                    if seq is None or s(b, r) == s(b, t):
                        z += w[d][k] * xx(b, r, d)
                if bias is not None:
                    z += bias[d]
                if seq is not None and s(b, t) < 0:
                    z = 0.0
                out[b][t][d] = z * _sig(z) if silu else z
    return out


def brute_bwd(x, w, dout, bias=None, seq=None, init=None, silu=False, dfinal=None):
    """(dx, dweight, dbias, dinit) by the chain rule written out per element."""
    B, T, D = len(x), len(x[0]) if x else 0, len(w)
    W = len(w[0])
    P = W - 1

    def xx(b, t, d):
        if 0 <= t < T:
            return x[b][t][d]
        if -P <= t < 0 and init is not None:
            return init[b][t + P][d]
        return 0.0

    def s(b, t):
        if t >= T:
            return -1
        if t < 0:
            return seq[b][0] if init is not None else -1
        return seq[b][t]

    def m(b, r, t):
        return seq is None or s(b, r) == s(b, t)

    g = [[[0.0] * D for _ in range(T)] for _ in range(B)]
    for b in range(B):
        for t in range(T):
            for d in range(D):
                if seq is not None and s(b, t) < 0:
                    continue
                gv = dout[b][t][d]
                if silu:
                    z = sum(w[d][k] * xx(b, t - P + k, d) for k in range(W) if m(b, t - P + k, t))
                    if bias is not None:
                        z += bias[d]
                    sg = _sig(z)
                    gv *= sg * (1 + z * (1 - sg))
                g[b][t][d] = gv
    # d/d xx[r] of sum_t g[t] * w[t-r+P... ]: xx[r] feeds out[r + j] through w[P - j].
    dxx = {}
    for b in range(B):
        for r in range(-P, T):
            for d in range(D):
                v = 0.0
                for j in range(W):
                    t = r + j
                    if 0 <= t < T and m(b, r, t):
                        v += w[d][P - j] * g[b][t][d]
                if dfinal is not None and 0 <= r - (T - P) < P:
                    v += dfinal[b][r - (T - P)][d]
                dxx[(b, r, d)] = v
    dx = [[[dxx[(b, t, d)] for d in range(D)] for t in range(T)] for b in range(B)]
    dinit = [[[dxx[(b, r - P, d)] for d in range(D)] for r in range(P)] for b in range(B)]
    dw = [[0.0] * W for _ in range(D)]
    db = [0.0] * D
    for b in range(B):
        for t in range(T):
            for d in range(D):
                for k in range(W):
                    if m(b, t - P + k, t):
                        dw[d][k] += g[b][t][d] * xx(b, t - P + k, d)
                db[d] += g[b][t][d]
    return dx, dw, db, dinit
