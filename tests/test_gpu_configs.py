"""GPU parity at BASELINE.json's configurations 0-3, each at its own shape.

Every check goes through the C ABI (innerq_amd.quant / ops / cache) and
compares with the CPU oracle:

* config 0 -- the HIP quantizer on the config's exact input reproduces the
  SHA-256 digests the live reference quant.py wrote (tests/golden/
  quant_golden.npz, ``cfg0_*``), through the reference-format API and through
  a packed store; the round-trip error is bounded by half a quantization step;
* config 1 -- the QK^T GEMV at B=1, 32/8 heads, T=8192, 4-bit asym G=32
  against the oracle's float64 logits over the oracle's dequantization;
* config 2 -- the attn.V GEMV at B=8, T=32768, 2-bit G=64, asym and sym, p the
  fp16 softmax of N(0, 2) logits: every (batch, KV head) against fp32 attn.V
  over the library's dequantization, and sampled heads end to end against the
  oracle (codes bit-exact, output within 1e-3);
* config 3 -- a full decode step of the drop-in cache (3-bit K and V, B=16,
  T=16384, G=32, a 128-token fp16 window, 6 outlier channels per head x8):
  quantize-on-append of the new token (codes bit-exact to the oracle), then
  attend() against fp32 attention over the cache's fp32 dequantized K and V
  (get_keys_deq / get_values_deq), and sampled heads against the oracle.

Tolerances: codes, scales and zero points bit-exact; GEMV and attention
outputs within 1e-3 in the max-normwise metric max|got-ref| / max|ref|
(oracle.attn_ref.rel_err).
"""
import hashlib

import numpy as np
import pytest
import torch

from innerq_amd import cache as C
from innerq_amd import ops
from innerq_amd import quant as IQ
from innerq_amd import synth
from oracle import attn_ref as A
from oracle import quant_ref as Q

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-3


def _sha(a):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), dtype=np.uint8)


def _np(t):
    return t.detach().cpu().numpy()


def _relerr_t(got, ref):
    return ((got.double() - ref.double()).abs().max() / ref.double().abs().max()).item()


# ------------------------------------------------------------------------------------------
# config 0: [1,8,4096,128] fp16 K and V, 4 outlier channels per head x10, 4-bit asym G=32
# ------------------------------------------------------------------------------------------
CFG0 = dict(B=1, H=8, T=4096, D=128, G=32, bits=4)


def _cfg0_inputs():
    c = CFG0
    k = synth.kv_tensor(c["B"], c["H"], c["T"], c["D"], seed=0, n_out=4, factor=10.0)
    v = synth.kv_tensor(c["B"], c["H"], c["T"], c["D"], seed=1, n_out=4, factor=10.0)
    return k, v


def test_config0_quantize_api_matches_reference_digests(quant_golden):
    """quantize_channeldim_asym (K) / quantize_tokendim_asym (V) of the drop-in
    API on the GPU: codes, scales and zero points hash to the digests the live
    reference wrote for this exact input; dequantize round-trips within half a
    step (s/2 plus one fp16 rounding of the fp32 result)."""
    k, v = _cfg0_inputs()
    G, bits = CFG0["G"], CFG0["bits"]
    for name, x, qf, df in (("k", k, IQ.quantize_channeldim_asym, IQ.dequantize_channeldim_asym),
                            ("v", v, IQ.quantize_tokendim_asym, IQ.dequantize_tokendim_asym)):
        xt = torch.from_numpy(x).to(DEV)
        c, s, z = qf(xt, G, bits)
        for part, arr in (("codes", _np(c).astype(np.int32)), ("scale", _np(s).view(np.uint16)),
                          ("zero", _np(z).view(np.uint16))):
            np.testing.assert_array_equal(_sha(arr), quant_golden[f"cfg0_{name}_{part}_sha256"],
                                          err_msg=f"config 0 {name} {part}")
        d = _np(df(c, s, z, G))
        step = _np(s).astype(np.float32)
        step = np.repeat(step, G, axis=-1) if name == "k" else np.repeat(step, G, axis=-2)
        err = np.abs(d - x.astype(np.float32))
        # half a step, plus the fp16 roundings of x - mn and of the quotient
        # (<= L * s * 2^-10 with L = 15) and of s itself
        assert np.all(err <= 0.6 * step + 1e-6)
        print(f"config 0 {name}: packed-code digests equal, max abs round-trip error {err.max():.4f}")


def test_config0_packed_store_matches_reference_digests(quant_golden):
    """The same input through quantize-on-append into packed stores: the codes,
    scales and zero points unpacked from the stores hash to the reference's
    digests, and the packed bytes equal the oracle's packing of them."""
    k, v = _cfg0_inputs()
    c0 = CFG0
    G, bits = c0["G"], c0["bits"]
    for name, x, axis in (("k", k, "channel"), ("v", v, "token")):
        st = ops.PackedStore(axis, c0["B"], c0["H"], c0["D"], G, bits, "asymmetric", DEV, t_cap=c0["T"])
        # appended in pieces, as a prefill followed by flushes would
        for a, b in ((0, 2048), (2048, 4032), (4032, 4096)):
            st.append(torch.from_numpy(x[:, :, a:b].copy()).to(DEV))
        c, s, z = ops.unpack_store(st)
        for part, arr in (("codes", _np(c).astype(np.int32)), ("scale", _np(s).view(np.uint16)),
                          ("zero", _np(z).view(np.uint16))):
            np.testing.assert_array_equal(_sha(arr), quant_golden[f"cfg0_{name}_{part}_sha256"],
                                          err_msg=f"config 0 store {name} {part}")
        rc, rs, rz = (Q.quantize_channeldim_asym if axis == "channel" else Q.quantize_tokendim_asym)(x, G, bits)
        build = Q.build_k_store if axis == "channel" else Q.build_v_store
        ref_words, ref_meta = build(rc, rs, rz, bits, G, "asymmetric", tcap=st.t_cap)
        np.testing.assert_array_equal(_np(st.codes).view(np.uint32).ravel(), ref_words.ravel())
        np.testing.assert_array_equal(_np(st.meta).view(np.uint16).ravel(), ref_meta.ravel())


# ------------------------------------------------------------------------------------------
# config 1: QK^T GEMV, B=1, 32 query / 8 KV heads, T=8192, D=128, 4-bit asym G=32
# ------------------------------------------------------------------------------------------
def test_config1_qk_gemv():
    B, Hkv, nrep, T, D, G = 1, 8, 4, 8192, 128, 32
    k = synth.kv_tensor(B, Hkv, T, D, seed=10, n_out=4, factor=10.0)
    q = synth.normal((B, Hkv * nrep, D), seed=11).astype(np.float16)
    st = ops.PackedStore("channel", B, Hkv, D, G, 4, "asymmetric", DEV, t_cap=T)
    st.append(torch.from_numpy(k).to(DEV))
    got = _np(ops.qk_gemv(torch.from_numpy(q).to(DEV), st, D ** -0.5))
    c, s, z = Q.quantize_channeldim_asym(k, G, 4)
    ref = A.qk_logits(q, Q.dequantize_channeldim_asym(c, s, z, G), D ** -0.5)
    assert got.shape == (1, 32, 8192) and got.dtype == np.float32
    err = A.rel_err(got, ref)
    print(f"config 1 QK^T: max-normwise error {err:.2e}")
    assert err < TOL


# ------------------------------------------------------------------------------------------
# config 2: attn.V GEMV, B=8, 32/8 heads, T=32768, D=128, 2-bit G=64 along tokens
# ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("mode", ["asymmetric", "symmetric"])
def test_config2_av_gemv(mode):
    B, Hkv, nrep, T, D, G, bits = 8, 8, 4, 32768, 128, 64, 2
    gen = torch.Generator(device=DEV).manual_seed(20 if mode == "asymmetric" else 21)
    v = torch.randn(B, Hkv, T, D, generator=gen, device=DEV)
    ch = torch.randperm(D, generator=torch.Generator().manual_seed(22))[:4].to(DEV)
    v[..., ch] *= 10.0
    v = v.to(torch.float16)
    p = torch.softmax(torch.randn(B, Hkv * nrep, T, generator=gen, device=DEV) * 2.0, dim=-1).to(torch.float16)
    st = ops.PackedStore("token", B, Hkv, D, G, bits, mode, DEV, t_cap=T)
    st.append(v)
    got16 = ops.av_gemv(p, st)
    got32 = ops.av_gemv(p, st, out32=torch.empty(B, Hkv * nrep, D, device=DEV))
    assert got16.shape == (8, 32, 128) and got16.dtype == torch.float16
    # every head: fp32 attn.V over the library's dequantization (bit-exact to the oracle's elsewhere)
    vd = st.dequant(dtype=torch.float32)
    ref = torch.matmul(p.float().view(B, Hkv, nrep, T), vd).view(B, Hkv * nrep, D)
    del vd
    e32, e16 = _relerr_t(got32, ref), _relerr_t(got16.float(), ref)
    # sampled (batch, KV head)s end to end through the oracle: codes, then output
    pn = _np(p)
    gc, gs, _ = ops.unpack_store(st)
    for b, h in ((0, 0), (3, 5), (7, 7)):
        x = _np(v[b:b + 1, h:h + 1])
        qf = Q.quantize_tokendim_asym if mode == "asymmetric" else Q.quantize_tokendim_sym
        dq = Q.dequantize_tokendim_asym if mode == "asymmetric" else Q.dequantize_tokendim_sym
        rc, rs, rz = qf(x, G, bits)
        np.testing.assert_array_equal(_np(gc[b:b + 1, h:h + 1]), rc)
        np.testing.assert_array_equal(_np(gs[b:b + 1, h:h + 1]).view(np.uint16), rs.view(np.uint16))
        o = A.av_out(pn[b:b + 1, h * nrep:(h + 1) * nrep], dq(rc, rs, rz, G))
        assert A.rel_err(_np(got32[b:b + 1, h * nrep:(h + 1) * nrep]), o) < TOL
    print(f"config 2 attn.V {mode}: max-normwise error fp32 out {e32:.2e}, fp16 out {e16:.2e}")
    assert e32 < TOL and e16 < TOL


# ------------------------------------------------------------------------------------------
# config 3: full decode step of the drop-in cache, 3-bit K and V, B=16, T=16384, G=32,
# a 128-token fp16 window, 5% (6 of 128) outlier channels per head scaled x8
# ------------------------------------------------------------------------------------------
CFG3 = dict(k_bits=3, v_bits=3, key_group_size=32, value_group_size=32, key_w_recent=128, value_w_recent=128,
            key_w_sink=0, value_w_sink=0, key_flush_size=1, value_flush_size=32, key_normalize=False,
            key_quantize_over_token=False, value_quantize_over_token=True)


class _Cfg:
    def __init__(self, **kw):
        self.__dict__.update(kw)


@pytest.mark.parametrize("mode", ["symmetric", "asymmetric"])
def test_config3_decode_step(mode):
    B, Hkv, nrep, T, D, G = 16, 8, 4, 16384, 128, 32
    cfg = _Cfg(**CFG3, key_quantize_mode=mode, value_quantize_mode=mode)
    gen = torch.Generator(device=DEV).manual_seed(30 if mode == "symmetric" else 31)

    def kv(n):
        x = torch.randn(B, Hkv, n, D, generator=gen, device=DEV)
        for h in range(Hkv):
            ch = torch.randperm(D, generator=torch.Generator().manual_seed(40 + h))[:6].to(DEV)
            x[:, h, :, ch] *= 8.0
        return x.to(torch.float16)

    k, v = kv(T + 1), kv(T + 1)
    q = torch.randn(B, Hkv * nrep, 1, D, generator=gen, device=DEV).to(torch.float16)
    layer = C.InnerqDynamicLayer(cfg, 0)
    layer.update(k[:, :, :T], v[:, :, :T])            # prefill: 16256 packed + 128 recent
    assert layer._kq.length == T - 128 and layer._vq.length == T - 128
    # the decode step: the new token joins the window, K flushes its oldest token
    # (quantize-on-append of one token per sequence), V its oldest 32
    layer.append(k[:, :, T:], v[:, :, T:])
    assert layer._kq.length == T - 127 and layer.keys_recent.shape[2] == 128
    assert layer._vq.length == T - 96 and layer.values_recent.shape[2] == 97
    got = layer.attend(q, D ** -0.5)[:, :, 0]
    # the appended token's codes: bit-exact to the oracle
    qk = Q.quantize_channeldim_sym if mode == "symmetric" else Q.quantize_channeldim_asym
    x_new = _np(k[:, :, T - 128:T - 127])
    rc, rs, rz = qk(x_new, G, 3)
    gc, gs, gz = ops.unpack_store(layer._kq.store, T - 128, 1)
    np.testing.assert_array_equal(_np(gc), rc)
    np.testing.assert_array_equal(_np(gs).view(np.uint16), rs.view(np.uint16))
    if mode == "asymmetric":
        np.testing.assert_array_equal(_np(gz).view(np.uint16), rz.view(np.uint16))
    # every head: dequantize-then-matmul in fp32 over the reference's fp32 dense K and V
    # (get_keys_deq / get_values_deq, cache.py:235-276: [sink | fp32 dequantized | recent])
    K = layer.get_keys_deq()
    assert K.shape == (B, Hkv, T + 1, D) and K.dtype == torch.float32
    lg = torch.matmul(q[:, :, 0].float().view(B, Hkv, nrep, D), K.transpose(-1, -2).contiguous())
    del K
    pr = torch.softmax(lg * D ** -0.5, dim=-1)
    ref = torch.matmul(pr, layer.get_values_deq()).view(B, Hkv * nrep, D)
    del lg, pr
    err = _relerr_t(got.float(), ref)
    # sampled (batch, KV head)s end to end through the oracle
    qv = Q.quantize_tokendim_sym if mode == "symmetric" else Q.quantize_tokendim_asym
    dk = Q.dequantize_channeldim_sym if mode == "symmetric" else Q.dequantize_channeldim_asym
    dv = Q.dequantize_tokendim_sym if mode == "symmetric" else Q.dequantize_tokendim_asym
    nk, nv = T - 127, T - 96
    for b, h in ((0, 0), (9, 3), (15, 7)):
        kx, vx = _np(k[b:b + 1, h:h + 1]), _np(v[b:b + 1, h:h + 1])
        kd = np.concatenate([dk(*qk(kx[:, :, :nk], G, 3), G), kx[:, :, nk:].astype(np.float32)], axis=2)
        vd = np.concatenate([dv(*qv(vx[:, :, :nv], G, 3), G), vx[:, :, nv:].astype(np.float32)], axis=2)
        qh = _np(q[b:b + 1, h * nrep:(h + 1) * nrep, 0])
        o = A.decode_attention(qh, kd, vd, D ** -0.5, p_dtype=None)
        assert A.rel_err(_np(got[b:b + 1, h * nrep:(h + 1) * nrep]).astype(np.float64), o) < TOL
    print(f"config 3 decode step {mode}: max-normwise error {err:.2e}")
    assert err < TOL
