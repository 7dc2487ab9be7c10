"""Dequantize-then-matmul references for the decode GEMVs (TEST ORACLE ONLY).

The reference computes decode attention in transformers' eager path over the
dense K/V that ``cache.py`` returns (TF/models/llama/modeling_llama.py:179-215):
``repeat_kv`` maps query head h to KV head ``h // n_rep``; logits are
``matmul(q, K^T) * head_dim**-0.5``; ``softmax(logits, dtype=float32)`` is cast
to the query dtype; the output is ``matmul(p, V)``.  The functions here do the
same linear algebra in float64 over fp32-dequantized K/V so that a HIP result
can be compared against it with a relative tolerance.
"""
from __future__ import annotations

import numpy as np


def _rep(x, n_rep):
    return np.repeat(x, n_rep, axis=1) if n_rep > 1 else x


def qk_logits(q, kdeq, scale):
    """q [B,Hq,D], kdeq [B,Hkv,T,D] -> float64 [B,Hq,T] = scale * q . k."""
    B, Hq, D = q.shape
    n_rep = Hq // kdeq.shape[1]
    k = _rep(kdeq.astype(np.float64), n_rep)
    return np.einsum("bhd,bhtd->bht", q.astype(np.float64), k) * scale


def av_out(p, vdeq):
    """p [B,Hq,T], vdeq [B,Hkv,T,D] -> float64 [B,Hq,D]."""
    n_rep = p.shape[1] // vdeq.shape[1]
    v = _rep(vdeq.astype(np.float64), n_rep)
    return np.einsum("bht,bhtd->bhd", p.astype(np.float64), v)


def softmax(x, axis=-1):
    m = x.max(axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=axis, keepdims=True)


def decode_attention(q, k_dense, v_dense, scale, p_dtype=np.float16):
    """Full decode step over dense K/V [B,Hkv,T,D]: logits -> fp32 softmax ->
    cast to ``p_dtype`` (the reference casts to the query dtype) -> p.V."""
    logits = qk_logits(q, k_dense, scale)
    p = softmax(logits.astype(np.float32).astype(np.float64))
    if p_dtype is not None:
        p = p.astype(np.float32).astype(p_dtype).astype(np.float64)
    return av_out(p, v_dense)


def qk_factored(q, codes, scale, zero, group, out_scale):
    """Factored form  sum_g s_g * (sum_{i in g} q_i c_i) + z_g * sum_{i in g} q_i
    over channel-dim groups; codes int [B,Hkv,T,D], scale/zero [B,Hkv,T,D/G]
    (zero None for sym codes stored signed).  A different computation from
    dequantize-then-matmul, used to cross-check ``qk_logits``."""
    B, Hq, D = q.shape
    Hkv = codes.shape[1]
    n_rep = Hq // Hkv
    T = codes.shape[2]
    ng = D // group
    qg = q.astype(np.float64).reshape(B, Hq, ng, group)
    cg = _rep(codes.astype(np.float64), n_rep).reshape(B, Hq, T, ng, group)
    dot = np.einsum("bhgi,bhtgi->bhtg", qg, cg)
    out = dot * _rep(scale.astype(np.float64), n_rep)
    if zero is not None:
        out = out + _rep(zero.astype(np.float64), n_rep) * qg.sum(-1)[:, :, None, :]
    return out.sum(-1) * out_scale


def av_factored(p, codes, scale, zero, group):
    """sum_g s[g,d] * sum_{t in g} p_t c[t,d] + z[g,d] * sum_{t in g} p_t."""
    B, Hq, T = p.shape
    Hkv, D = codes.shape[1], codes.shape[3]
    n_rep = Hq // Hkv
    ng = T // group
    pg = p.astype(np.float64).reshape(B, Hq, ng, group)
    cg = _rep(codes.astype(np.float64), n_rep).reshape(B, Hq, ng, group, D)
    dot = np.einsum("bhgt,bhgtd->bhgd", pg, cg)
    out = dot * _rep(scale.astype(np.float64), n_rep)
    if zero is not None:
        out = out + _rep(zero.astype(np.float64), n_rep) * pg.sum(-1)[..., None]
    return out.sum(2)


def rel_err(got, ref):
    """max |got - ref| / max |ref| (the tolerance metric used by the parity tests)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))
