"""Pin the attention oracle (oracle/attn_ref.py) independently of itself.

Every QK^T, attn.V and decode-attention GPU parity test takes its expected
values from attn_ref, so attn_ref is checked here against three things that
do not share its code:

* transformers' own eager attention (``repeat_kv`` + ``eager_attention_forward``,
  TF/models/llama/modeling_llama.py:179-215), which is what the reference runs
  over the dense K/V that cache.py returns (cache.py:235-281, 395);
* float64 brute-force loops written index by index on tiny shapes, with the
  GQA mapping spelled out as ``kv = h // n_rep``;
* the factored group sums (qk_factored / av_factored) over quantized codes,
  which reach the same values by a different order of operations.

The KV heads always carry distinct data, so an ``h % Hkv`` head mapping, a
missing ``head_dim ** -0.5``, a softmax over the wrong axis or a dropped zero
point term changes the result.  ``test_checks_catch_planted_mistakes`` plants
each of those mistakes in a copy of the oracle (on the CPU) and asserts that
the same checks reject it.
"""
import math

import numpy as np
import pytest
import torch
from transformers.models.llama import modeling_llama as TF

from oracle import attn_ref as A
from oracle import quant_ref as Q


class _Module(torch.nn.Module):
    """The attributes eager_attention_forward reads from the attention module."""

    def __init__(self, n_rep):
        super().__init__()
        self.num_key_value_groups = n_rep
        self.training = False


def _inputs(B, Hq, Hkv, T, D, seed, dtype=np.float32):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Hq, D)).astype(dtype)
    # per-head offsets make every KV head's data distinct even at tiny T
    k = (rng.standard_normal((B, Hkv, T, D)) + np.arange(Hkv)[None, :, None, None] * 0.5).astype(dtype)
    v = (rng.standard_normal((B, Hkv, T, D)) - np.arange(Hkv)[None, :, None, None] * 0.75).astype(dtype)
    return q, k, v


def _tf_eager(q, k, v, scale, torch_dtype):
    """transformers' eager attention for one query token: (out [B,Hq,D], p [B,Hq,T])."""
    n_rep = q.shape[1] // k.shape[1]
    qt = torch.from_numpy(q).to(torch_dtype)[:, :, None, :]
    kt = torch.from_numpy(k).to(torch_dtype)
    vt = torch.from_numpy(v).to(torch_dtype)
    out, w = TF.eager_attention_forward(_Module(n_rep), qt, kt, vt, None, scaling=scale)
    return out[:, 0].double().numpy(), w[:, :, 0].double().numpy()  # out is [B, 1, Hq, D]


def _loops_logits(q, k, scale):
    B, Hq, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    n_rep = Hq // Hkv
    out = np.zeros((B, Hq, T))
    for b in range(B):
        for h in range(Hq):
            kv = h // n_rep
            for t in range(T):
                acc = 0.0
                for d in range(D):
                    acc += float(q[b, h, d]) * float(k[b, kv, t, d])
                out[b, h, t] = acc * scale
    return out


def _loops_av(p, v):
    B, Hq, T = p.shape
    Hkv, D = v.shape[1], v.shape[3]
    n_rep = Hq // Hkv
    out = np.zeros((B, Hq, D))
    for b in range(B):
        for h in range(Hq):
            kv = h // n_rep
            for d in range(D):
                acc = 0.0
                for t in range(T):
                    acc += float(p[b, h, t]) * float(v[b, kv, t, d])
                out[b, h, d] = acc
    return out


def _loops_softmax(x):
    out = np.zeros_like(x, dtype=np.float64)
    for idx in np.ndindex(x.shape[:-1]):
        row = [float(a) for a in x[idx]]
        m = max(row)
        e = [math.exp(a - m) for a in row]
        s = sum(e)
        out[idx] = [a / s for a in e]
    return out


# --------------------------------------------------------------------------------------------
# the checks (shared by the tests and by the planted-mistake test)

def check_against_tf(oracle, B, Hq, Hkv, T, D, seed):
    """attn_ref's softmax(qk_logits), av_out and decode_attention vs transformers' eager attention on fp64
    tensors (its softmax runs in fp32 whatever the input dtype, so p agrees to fp32 rounding)."""
    q, k, v = _inputs(B, Hq, Hkv, T, D, seed, np.float64)
    scale = D ** -0.5
    ref_out, ref_p = _tf_eager(q, k, v, scale, torch.float64)
    p = oracle.softmax(oracle.qk_logits(q, k, scale))
    np.testing.assert_allclose(p, ref_p, rtol=2e-6, atol=1e-9)
    np.testing.assert_allclose(oracle.av_out(ref_p, v), ref_out, rtol=1e-10, atol=1e-12)
    assert A.rel_err(oracle.decode_attention(q, k, v, scale, p_dtype=None), ref_out) < 2e-6


def check_against_loops(oracle, B, Hq, Hkv, T, D, seed):
    q, k, v = _inputs(B, Hq, Hkv, T, D, seed)
    scale = D ** -0.5
    lg = _loops_logits(q, k, scale)
    np.testing.assert_allclose(oracle.qk_logits(q, k, scale), lg, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.softmax(lg), _loops_softmax(lg), rtol=1e-12, atol=1e-15)
    p = _loops_softmax(lg)
    np.testing.assert_allclose(oracle.av_out(p, v), _loops_av(p, v), rtol=1e-12, atol=1e-12)


def check_factored(oracle, B, Hq, Hkv, T, D, G, bits, mode, seed):
    """qk_factored / av_factored on quantized codes vs qk_logits / av_out on the dequantized tensors."""
    _, k, v = _inputs(B, Hq, Hkv, T, D, seed, np.float16)
    rng = np.random.default_rng(seed + 1)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    p = rng.random((B, Hq, T))
    p = (p / p.sum(-1, keepdims=True)).astype(np.float16)
    scale = D ** -0.5
    if mode == "asym":
        ck, sk, zk = Q.quantize_channeldim_asym(k, G, bits)
        cv, sv, zv = Q.quantize_tokendim_asym(v, G, bits)
        kd = Q.dequantize_channeldim_asym(ck, sk, zk, G)
        vd = Q.dequantize_tokendim_asym(cv, sv, zv, G)
    else:
        ck, sk, gk = Q.quantize_channeldim_sym(k, G, bits)
        cv, sv, gv = Q.quantize_tokendim_sym(v, G, bits)
        kd = Q.dequantize_channeldim_sym(ck, sk, gk, G)
        vd = Q.dequantize_tokendim_sym(cv, sv, gv, G)
        ck = ck * gk.astype(np.int64)  # signed codes, no zero point
        cv = cv * gv.astype(np.int64)
        zk = zv = None
    lf = oracle.qk_factored(q, ck, sk, zk, G, scale)
    ld = oracle.qk_logits(q, kd, scale)
    assert A.rel_err(lf, ld) < 1e-6, A.rel_err(lf, ld)
    of = oracle.av_factored(p, cv, sv, zv, G)
    od = oracle.av_out(p, vd)
    assert A.rel_err(of, od) < 1e-6, A.rel_err(of, od)


# --------------------------------------------------------------------------------------------

@pytest.mark.parametrize("Hq,Hkv", [(4, 4), (4, 2), (8, 2), (8, 1), (16, 2)])
@pytest.mark.parametrize("T,D", [(7, 16), (64, 64), (130, 128)])
def test_against_transformers_eager(Hq, Hkv, T, D):
    check_against_tf(A, 2, Hq, Hkv, T, D, seed=Hq * 100 + Hkv * 10 + T)


def test_decode_attention_fp16_probabilities_match_transformers_fp16():
    """The reference casts the fp32 softmax to the query dtype (fp16) before p.V
    (modeling_llama.py:208); attn_ref's p_dtype=float16 reproduces that cast."""
    B, Hq, Hkv, T, D = 2, 8, 2, 96, 64
    q, k, v = _inputs(B, Hq, Hkv, T, D, 7, np.float16)
    scale = D ** -0.5
    _, ref_p = _tf_eager(q, k, v, scale, torch.float32)  # fp32 eager: p before the fp16 cast
    logits32 = A.qk_logits(q, k, scale).astype(np.float32)
    p16 = A.softmax(logits32.astype(np.float64)).astype(np.float32).astype(np.float16)
    tf16 = ref_p.astype(np.float32).astype(np.float16)
    # the oracle's float64 softmax and torch's fp32 one round to the same fp16
    # except, rarely, one ulp apart next to a rounding tie
    ulp = np.spacing(np.maximum(np.abs(p16), np.abs(tf16)).astype(np.float16)).astype(np.float32)
    diff = np.abs(p16.astype(np.float32) - tf16.astype(np.float32))
    assert np.all(diff <= ulp) and np.count_nonzero(diff) <= p16.size // 100
    out = A.decode_attention(q, k, v, scale, p_dtype=np.float16)
    ref = A.av_out(p16.astype(np.float64), v)
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)
    # and the fp16 eager path of transformers itself, within fp16 matmul rounding
    ref16, _ = _tf_eager(q, k, v, scale, torch.float16)
    assert A.rel_err(out, ref16) < 2e-3


@pytest.mark.parametrize("Hq,Hkv,T,D", [(4, 2, 5, 8), (8, 2, 9, 16), (6, 3, 4, 4)])
def test_against_float64_loops(Hq, Hkv, T, D):
    check_against_loops(A, 2, Hq, Hkv, T, D, seed=T * 13 + D)


@pytest.mark.parametrize("mode", ["asym", "sym"])
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("G", [32, 64])
def test_factored_forms_match_dequantize_then_matmul(mode, bits, G):
    check_factored(A, 2, 8, 2, 128, 128, G, bits, mode, seed=bits * 10 + G)


def test_rel_err_metric():
    """rel_err is max|got - ref| / max|ref| (normwise), the metric every parity tolerance uses."""
    ref = np.array([1.0, -4.0, 0.001])
    got = np.array([1.0, -4.0, 0.003])
    assert A.rel_err(got, ref) == pytest.approx(0.002 / 4.0)
    assert A.rel_err(ref, ref) == 0.0


# --------------------------------------------------------------------------------------------
# planted mistakes: each broken oracle must fail at least one of the checks above

class _Broken:
    """A copy of attn_ref with one function replaced."""

    def __init__(self, **over):
        for name in ("qk_logits", "av_out", "softmax", "decode_attention", "qk_factored", "av_factored"):
            setattr(self, name, over.get(name, getattr(A, name)))
        if "qk_logits" in over or "softmax" in over or "av_out" in over:
            me = self

            def decode_attention(q, k, v, scale, p_dtype=np.float16):
                p = me.softmax(me.qk_logits(q, k, scale))
                if p_dtype is not None:
                    p = p.astype(np.float32).astype(p_dtype).astype(np.float64)
                return me.av_out(p, v)
            if "decode_attention" not in over:
                self.decode_attention = decode_attention


def _tile_rep(x, n_rep):
    return np.tile(x, (1, n_rep, 1, 1))  # head h -> KV head h % Hkv


def _qk_mod_heads(q, kdeq, scale):
    k = _tile_rep(kdeq.astype(np.float64), q.shape[1] // kdeq.shape[1])
    return np.einsum("bhd,bhtd->bht", q.astype(np.float64), k) * scale


def _qk_no_scale(q, kdeq, scale):
    return A.qk_logits(q, kdeq, 1.0)


def _av_mod_heads(p, vdeq):
    v = _tile_rep(vdeq.astype(np.float64), p.shape[1] // vdeq.shape[1])
    return np.einsum("bht,bhtd->bhd", p.astype(np.float64), v)


def _softmax_wrong_axis(x, axis=-1):
    return A.softmax(x, axis=1)


def _qk_factored_no_zero(q, codes, scale, zero, group, out_scale):
    return A.qk_factored(q, codes, scale, None, group, out_scale)


def _av_factored_no_zero(p, codes, scale, zero, group):
    return A.av_factored(p, codes, scale, None, group)


@pytest.mark.parametrize("over,check", [
    ({"qk_logits": _qk_mod_heads}, "tf"),
    ({"qk_logits": _qk_mod_heads}, "loops"),
    ({"qk_logits": _qk_no_scale}, "tf"),
    ({"qk_logits": _qk_no_scale}, "loops"),
    ({"av_out": _av_mod_heads}, "tf"),
    ({"av_out": _av_mod_heads}, "loops"),
    ({"softmax": _softmax_wrong_axis}, "tf"),
    ({"softmax": _softmax_wrong_axis}, "loops"),
    ({"qk_factored": _qk_factored_no_zero}, "factored"),
    ({"av_factored": _av_factored_no_zero}, "factored"),
])
def test_checks_catch_planted_mistakes(over, check):
    broken = _Broken(**over)
    with pytest.raises(AssertionError):
        if check == "tf":
            check_against_tf(broken, 2, 8, 2, 33, 16, seed=5)
        elif check == "loops":
            check_against_loops(broken, 2, 8, 2, 6, 8, seed=5)
        else:
            check_factored(broken, 2, 8, 2, 64, 64, 32, 4, "asym", seed=5)
