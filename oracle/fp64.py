"""Float64 numpy formulation of the AttnRes read, written from the math (TEST INFRASTRUCTURE).

Independent of torch and of ``attnres_oracle``: forward *and* closed-form
backward are spelled out here, so that comparing this module with autograd
through the eager restatement pins both (a dropped term, a sign, a head/source
index swap or a transposed operand in either one makes them disagree).

Shapes use the flattened token axis ``n = B*T``:

* values ``[S, n, D]``; LR keys ``[S, n, R]``; heads ``H`` split ``D`` and
  ``R`` into contiguous chunks ``dh = D/H`` and ``rh = R/H``.
* static LR query ``[H, rh]``; per-token query ``[n, H, rh]``; base query ``[D]``.
* bias ``[S]`` (added to the logit of every token/head of that source).

The math (reference semantics, ``attnres_ops.py:4163-4192`` for LR,
``:2176-2190`` for base; backward as in ``:449-746``)::

    khat_{s,h}  = k_{s,h} / sqrt(mean(k_{s,h}^2) + eps)        (if key_norm)
    logit_{s,h} = scale * <khat_{s,h}, q_h> + bias_s
    p_{s,h}     = softmax_s(logit_{., h})
    out_h       = sum_s p_{s,h} v_{s,h}

    dW_{s,h}    = <g_h, v_{s,h}>
    dlogit      = p (dW - sum_s p dW)
    dv_{s,h}    = p_{s,h} g_h                       (+ key path for base)
    dkhat       = scale * dlogit * q_h
    dk          = inv_rms * (dkhat - khat * <dkhat, khat> / rh)
    dq_h        = sum_{tokens, s} scale * dlogit * khat
    dbias_s     = sum_{tokens, h} dlogit
"""

from __future__ import annotations

import numpy as np


def _softmax0(x: np.ndarray) -> np.ndarray:
    m = x.max(axis=0, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=0, keepdims=True)


def _rms(x: np.ndarray, eps: float) -> np.ndarray:
    return 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


# ---------------------------------------------------------------- LR read

def lr_forward(values, keys, query, H, scale, key_norm, bias=None, eps=np.finfo(np.float64).eps,
               normalize_output=False):
    """Returns (out [n,D], p [S,n,H], aux dict)."""
    v = np.asarray(values, np.float64)
    k = np.asarray(keys, np.float64)
    q = np.asarray(query, np.float64)
    S, n, D = v.shape
    R = k.shape[-1]
    dh, rh = D // H, R // H
    v4 = v.reshape(S, n, H, dh)
    k4 = k.reshape(S, n, H, rh)
    inv = _rms(k4, eps) if key_norm else np.ones((S, n, H, 1))
    kh = k4 * inv
    if q.ndim == 2:
        logits = scale * np.einsum("snhr,hr->snh", kh, q)
    else:
        logits = scale * np.einsum("snhr,nhr->snh", kh, q.reshape(n, H, rh))
    if bias is not None:
        logits = logits + np.asarray(bias, np.float64).reshape(S, 1, 1)
    p = _softmax0(logits)
    out = np.einsum("snh,snhd->nhd", p, v4).reshape(n, D)
    out_inv = None
    pre = out
    if normalize_output:
        out_inv = _rms(out, eps)
        out = out * out_inv
    return out, p, dict(inv=inv, kh=kh, v4=v4, pre=pre, out_inv=out_inv)


def lr_backward(values, keys, query, H, scale, key_norm, grad_out, bias=None,
                eps=np.finfo(np.float64).eps, normalize_output=False):
    """Closed-form gradients.  Returns dict(dv [S,n,D], dk [S,n,R], dq, dbias [S])."""
    v = np.asarray(values, np.float64)
    k = np.asarray(keys, np.float64)
    q = np.asarray(query, np.float64)
    S, n, D = v.shape
    R = k.shape[-1]
    dh, rh = D // H, R // H
    out, p, aux = lr_forward(v, k, q, H, scale, key_norm, bias, eps, normalize_output)
    g = np.asarray(grad_out, np.float64).reshape(n, D)
    if normalize_output:
        y = out
        g = aux["out_inv"] * (g - y * np.mean(g * y, axis=-1, keepdims=True))
    g3 = g.reshape(n, H, dh)
    dW = np.einsum("nhd,snhd->snh", g3, aux["v4"])
    dlogit = p * (dW - np.sum(p * dW, axis=0, keepdims=True))
    dv = (p[..., None] * g3[None]).reshape(S, n, D)
    kh = aux["kh"]
    if q.ndim == 2:
        qb = np.broadcast_to(q[None, None], (S, n, H, rh))
    else:
        qb = np.broadcast_to(q.reshape(1, n, H, rh), (S, n, H, rh))
    dkh = scale * dlogit[..., None] * qb
    if key_norm:
        dk = aux["inv"] * (dkh - kh * np.mean(dkh * kh, axis=-1, keepdims=True))
    else:
        dk = dkh
    dq_tok = np.einsum("snh,snhr->nhr", scale * dlogit, kh)
    dq = dq_tok.sum(axis=0) if q.ndim == 2 else dq_tok.reshape(q.shape)
    dbias = dlogit.sum(axis=(1, 2))
    return dict(dv=dv, dk=dk.reshape(S, n, R), dq=dq, dbias=dbias, p=p, dlogit=dlogit)


# ---------------------------------------------------------------- base read

def base_forward(values, query, key_norm, bias=None, eps=np.finfo(np.float64).eps, normalize_output=False):
    """Returns (out [n,D], p [S,n], aux)."""
    v = np.asarray(values, np.float64)
    q = np.asarray(query, np.float64)
    inv = _rms(v, eps) if key_norm else np.ones(v.shape[:-1] + (1,))
    kh = v * inv
    logits = np.einsum("snd,d->sn", kh, q)
    if bias is not None:
        logits = logits + np.asarray(bias, np.float64).reshape(-1, 1)
    p = _softmax0(logits)
    out = np.einsum("sn,snd->nd", p, v)
    out_inv = None
    if normalize_output:
        out_inv = _rms(out, eps)
        out = out * out_inv
    return out, p, dict(inv=inv, kh=kh, out_inv=out_inv)


def base_backward(values, query, key_norm, grad_out, bias=None, eps=np.finfo(np.float64).eps,
                  normalize_output=False):
    v = np.asarray(values, np.float64)
    q = np.asarray(query, np.float64)
    S, n, D = v.shape
    out, p, aux = base_forward(v, q, key_norm, bias, eps, normalize_output)
    g = np.asarray(grad_out, np.float64).reshape(n, D)
    if normalize_output:
        y = out
        g = aux["out_inv"] * (g - y * np.mean(g * y, axis=-1, keepdims=True))
    dW = np.einsum("nd,snd->sn", g, v)
    dlogit = p * (dW - np.sum(p * dW, axis=0, keepdims=True))
    dkh = dlogit[..., None] * q[None, None, :]
    kh = aux["kh"]
    if key_norm:
        dkey = aux["inv"] * (dkh - kh * np.mean(dkh * kh, axis=-1, keepdims=True))
    else:
        dkey = dkh
    dv = p[..., None] * g[None] + dkey
    dq = np.einsum("sn,snd->d", dlogit, kh)
    dbias = dlogit.sum(axis=1)
    return dict(dv=dv, dq=dq, dbias=dbias, p=p, dlogit=dlogit)


# ---------------------------------------------------------------- average read

def average_forward(values, normalize_output=False, eps=np.finfo(np.float64).eps):
    v = np.asarray(values, np.float64)
    out = v.mean(axis=0)
    if normalize_output:
        out = out * _rms(out, eps)
    return out


# ---------------------------------------------------------------- brute force (tiny inputs)

def lr_forward_loops(values, keys, query, H, scale, key_norm, bias=None, eps=np.finfo(np.float64).eps):
    """Token-by-token, head-by-head, element-by-element loops (tiny sizes only).

    Used to pin the vectorised ``lr_forward`` itself.
    """
    import math
    v = np.asarray(values, np.float64)
    k = np.asarray(keys, np.float64)
    q = np.asarray(query, np.float64)
    S, n, D = v.shape
    R = k.shape[-1]
    dh, rh = D // H, R // H
    out = np.zeros((n, D))
    for t in range(n):
        for h in range(H):
            logits = []
            for s in range(S):
                seg = [k[s, t, h * rh + j] for j in range(rh)]
                if key_norm:
                    ms = sum(x * x for x in seg) / rh
                    r = 1.0 / math.sqrt(ms + eps)
                    seg = [x * r for x in seg]
                qq = q[h] if q.ndim == 2 else q.reshape(n, H, rh)[t, h]
                lg = scale * sum(seg[j] * qq[j] for j in range(rh))
                if bias is not None:
                    lg += float(bias[s])
                logits.append(lg)
            m = max(logits)
            ex = [math.exp(x - m) for x in logits]
            z = sum(ex)
            for d in range(dh):
                out[t, h * dh + d] = sum(ex[s] / z * v[s, t, h * dh + d] for s in range(S))
    return out
