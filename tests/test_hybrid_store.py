"""Hybrid quantization (quant.py:133-176) as one packed store.

A hybrid store keeps, per group, the representation the reference's mask
selects: the (b-1)-bit asym codes with {scale, zero}, or the b-bit sym codes
(offset binary) with {scale | 0x8000, 0}; the flag is bit 15 of the scale half
and is tested as a bit.  CPU: the host-side split of a raw unpack into
quant.py's dicts.  GPU: the quantize kernel's masks and dequantized values
against the live reference's golden vectors, the selected codes against the
oracle, and the attn.V GEMV / decode attention over hybrid V against float64
attention over the oracle's dequantized values (max-relative error 1e-3).
"""
import hashlib

import numpy as np
import pytest
import torch

from innerq_amd import _lib, ops, synth
from oracle import attn_ref as A
from oracle import quant_ref as Q

DEV = "cuda:0"
TOL = 1e-3
BITS = [2, 3, 4]


def _sha(a):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), dtype=np.uint8)


def _expand(mask, group, axis):
    return np.repeat(mask, group, axis=-1 if axis == "channel" else 2)


def _raw_of(c, s, z, bits, group, axis):
    """The raw unpack of a hybrid store holding the oracle's hybrid quantization
    (c, s, z dicts): fields, scale half (flag = bit 15), zero half."""
    mask = s["mask"]
    el = _expand(mask, group, axis)
    signed = np.where(c["nozp"] == Q.INT32_MIN, 0, c["nozp"]) * z["nozp"].astype(np.int32)
    zp = np.where(c["zp"] == Q.INT32_MIN, 0, c["zp"])
    fields = np.where(el, signed + (1 << (bits - 1)), zp).astype(np.int32)
    sc = np.where(mask, s["nozp"].view(np.uint16) | 0x8000, s["zp"].view(np.uint16) & 0x7FFF).astype(np.uint16)
    zero = np.where(mask, np.uint16(0), z["zp"].view(np.uint16)).astype(np.uint16)
    return fields, sc, zero


def _check_selected(c, s, z, oc, os_, oz, group, axis):
    """The dicts of a hybrid store hold the oracle's selected half exactly (a NaN
    code as 0, a sym sign only where the code is nonzero) and zeros elsewhere."""
    mask = os_["mask"]
    el = _expand(mask, group, axis)
    np.testing.assert_array_equal(s["mask"], mask)
    np.testing.assert_array_equal(c["zp"], np.where(el | (oc["zp"] == Q.INT32_MIN), 0, oc["zp"]))
    np.testing.assert_array_equal(c["nozp"], np.where(el & (oc["nozp"] != Q.INT32_MIN), oc["nozp"], 0))
    np.testing.assert_array_equal(s["zp"].view(np.uint16), np.where(mask, 0, os_["zp"].view(np.uint16)))
    np.testing.assert_array_equal(s["nozp"].view(np.uint16), np.where(mask, os_["nozp"].view(np.uint16), 0))
    np.testing.assert_array_equal(z["zp"].view(np.uint16), np.where(mask, 0, oz["zp"].view(np.uint16)))
    nz = el & (oc["nozp"] != 0)
    np.testing.assert_array_equal(z["nozp"][nz], oz["nozp"][nz])
    assert np.all(z["nozp"][~nz] == 0)


# ----------------------------------------------------------------------------
# CPU: host logic
# ----------------------------------------------------------------------------
@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("bits", BITS)
def test_split_hybrid_recovers_the_selected_half(quant_golden, axis, bits):
    x = quant_golden["x"].view(np.float16)
    oc, os_, oz = getattr(Q, f"quantize_{axis}dim_hybrid")(x, 32, bits)
    np.testing.assert_array_equal(os_["mask"], quant_golden[f"{axis}_hybrid_b{bits}_g32_mask"])
    fields, sc, zero = _raw_of(oc, os_, oz, bits, 32, axis)
    c, s, z = ops.split_hybrid(torch.from_numpy(fields), torch.from_numpy(sc.view(np.int16)).view(torch.float16),
                               torch.from_numpy(zero.view(np.int16)).view(torch.float16), bits, 32, axis)
    c = {k: v.numpy() for k, v in c.items()}
    s = {k: v.numpy() for k, v in s.items()}
    z = {k: v.numpy() for k, v in z.items()}
    _check_selected(c, s, z, oc, os_, oz, 32, axis)
    # the reference's dequantize_hybrid over the split dicts gives the reference's values
    d = getattr(Q, f"dequantize_{axis}dim_hybrid")(c, s, z, 32).astype(np.float32)
    np.testing.assert_array_equal(_sha(d + np.float32(0.0)), quant_golden[f"{axis}_hybrid_b{bits}_g32_deq_pz_sha256"])


def test_split_hybrid_flag_is_a_bit():
    """A flagged -0.0 scale (0x8000) is a sym group: -0.0 < 0 is false, the bit is set."""
    fields = torch.full((1, 1, 1, 32), 2, dtype=torch.int32)  # 2-bit offset binary: signed 0
    fields[0, 0, 0, 0] = 3                                    # signed +1
    for raw, want in ((0x8000, True), (0x0000, False), (0xBC00, True), (0x3C00, False)):
        sc = torch.tensor([[[[raw - 0x10000 if raw & 0x8000 else raw]]]], dtype=torch.int16).view(torch.float16)
        zero = torch.tensor([[[[0x3C00]]]], dtype=torch.int16).view(torch.float16)
        c, s, z = ops.split_hybrid(fields, sc, zero, 2, 32, "channel")
        assert bool(s["mask"].item()) is want
        if want:
            assert s["nozp"].item() == abs(sc.float().item()) and s["zp"].item() == 0.0
            assert c["nozp"][0, 0, 0, 0].item() == 1 and c["nozp"][0, 0, 0, 1].item() == 0
            assert z["nozp"][0, 0, 0, 0].item() == 1.0 and z["zp"].item() == 0.0
        else:
            assert s["zp"].item() == sc.float().item() and z["zp"].item() == 1.0
            assert torch.equal(c["zp"], fields) and int(c["nozp"].abs().sum()) == 0


# ----------------------------------------------------------------------------
# GPU: the quantize kernel, the reads, the GEMV and the decode step
# ----------------------------------------------------------------------------
def _f16t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _mixed_v(B, H, T, D, seed):
    """V with outlier channels and 48 columns offset by +6: groups of both kinds
    at every bit width (Gaussian columns alone pick sym at 2 bits)."""
    v = synth.kv_tensor(B, H, T, D, seed=seed, n_out=3, factor=8.0).astype(np.float32)
    v[..., :48] += 6.0
    return v.astype(np.float16)


def _store(x, axis, bits, G=32):
    B, H, _, D = x.shape
    st = ops.PackedStore(axis, B, H, D, G, bits, "hybrid", DEV)
    st.append(_f16t(x))
    return st


@pytest.mark.gpu
@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("bits", BITS)
def test_hybrid_store_matches_reference(quant_golden, axis, bits):
    """Masks equal the live reference's; the store's dequantized values equal
    dequantize_hybrid's (golden digest, -0.0 read as +0.0); the selected codes,
    scales, zero points and signs equal the oracle's."""
    x = quant_golden["x"].view(np.float16)
    st = _store(x, axis, bits)
    c, s, z = ops.unpack_store(st)
    key = f"{axis}_hybrid_b{bits}_g32"
    np.testing.assert_array_equal(s["mask"].cpu().numpy(), quant_golden[key + "_mask"])
    d = st.dequant(dtype=torch.float32).cpu().numpy()
    np.testing.assert_array_equal(_sha(d + np.float32(0.0)), quant_golden[key + "_deq_pz_sha256"])
    oc, os_, oz = getattr(Q, f"quantize_{axis}dim_hybrid")(x, 32, bits)
    _check_selected({k: v.cpu().numpy() for k, v in c.items()}, {k: v.cpu().numpy() for k, v in s.items()},
                    {k: v.cpu().numpy() for k, v in z.items()}, oc, os_, oz, 32, axis)
    # meta words: flagged groups carry no zero point
    mw = st.meta.view(torch.int32).cpu().numpy().astype(np.uint32)
    flagged = (mw & 0x8000) != 0
    assert flagged.any() and (~flagged).any()
    assert np.all(mw[flagged] >> 16 == 0)
    # fp16 dequant: the fp32 values rounded once
    np.testing.assert_array_equal(st.dequant().cpu().numpy(), d.astype(np.float16))


@pytest.mark.gpu
@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("G", [32, 64, 128])
@pytest.mark.parametrize("nrep", [1, 4])
def test_hybrid_av_gemv_parity(bits, G, nrep):
    B, Hkv, D = 2, 2, 128
    T = 6 * G
    vx = _mixed_v(B, Hkv, T, D, seed=bits * 7 + G + nrep)
    st = _store(vx, "token", bits, G)
    c, s, z = Q.quantize_tokendim_hybrid(vx, G, bits)
    assert 0 < s["mask"].mean() < 1
    vdeq = Q.dequantize_tokendim_hybrid(c, s, z, G)
    np.testing.assert_array_equal(st.dequant(dtype=torch.float32).cpu().numpy() + np.float32(0),
                                  vdeq.astype(np.float32) + np.float32(0))
    logits = synth.normal((B, Hkv * nrep, T), seed=G + bits, std=2.0).astype(np.float64)
    p = A.softmax(logits).astype(np.float16)
    got = ops.av_gemv(_f16t(p), st).cpu().numpy().astype(np.float64)
    assert A.rel_err(got, A.av_out(p, vdeq)) < TOL


@pytest.mark.gpu
@pytest.mark.parametrize("kmode", ["symmetric", "asymmetric"])
@pytest.mark.parametrize("vbits", [2, 4])
def test_hybrid_decode_attention_segments(kmode, vbits):
    """[sink | packed | recent] K and V with hybrid V (the innerq_hybrid preset's
    layout: 3-bit K, group 32, 32 sinks, a recent window)."""
    B, Hkv, nrep, D, G = 2, 2, 4, 128, 32
    ks, kq, kr = 32, 1280 - 32 - 96, 96
    vs, vq, vr = 32, 1280 - 32 - 64, 64
    T = ks + kq + kr
    kx = synth.kv_tensor(B, Hkv, T, D, seed=31, n_out=4, factor=8.0)
    vx = _mixed_v(B, Hkv, T, D, seed=32)
    kst = ops.PackedStore("channel", B, Hkv, D, G, 3, kmode, DEV)
    kst.append(_f16t(kx[:, :, ks:ks + kq]))
    vst = _store(vx[:, :, vs:vs + vq], "token", vbits, G)
    q = synth.normal((B, Hkv * nrep, D), seed=33).astype(np.float16)
    kxt, vxt = _f16t(kx), _f16t(vx)
    got = ops.decode_attention(_f16t(q), kxt[:, :, :ks], kst, kxt[:, :, ks + kq:], vxt[:, :, :vs], vst,
                               vxt[:, :, vs + vq:], D ** -0.5).cpu().numpy().astype(np.float64)
    qk = Q.quantize_channeldim_sym if kmode == "symmetric" else Q.quantize_channeldim_asym
    dk = Q.dequantize_channeldim_sym if kmode == "symmetric" else Q.dequantize_channeldim_asym
    kd = np.concatenate([kx[:, :, :ks].astype(np.float32), dk(*qk(kx[:, :, ks:ks + kq], G, 3), G),
                         kx[:, :, ks + kq:].astype(np.float32)], axis=2)
    vd = np.concatenate([vx[:, :, :vs].astype(np.float32),
                         Q.dequantize_tokendim_hybrid(*Q.quantize_tokendim_hybrid(vx[:, :, vs:vs + vq], G, vbits), G),
                         vx[:, :, vs + vq:].astype(np.float32)], axis=2)
    assert A.rel_err(got, A.decode_attention(q, kd, vd, D ** -0.5, p_dtype=None)) < TOL


@pytest.mark.gpu
@pytest.mark.parametrize("vmode", ["asymmetric", "symmetric", "hybrid"])
@pytest.mark.parametrize("kbits,G", [(2, 32), (3, 32), (4, 32), (3, 64)])
def test_hybrid_k_decode_attention_segments(vmode, kbits, G):
    """[sink | packed | recent] with a hybrid K store (key_quantize_mode='hybrid',
    cache.py:92-98; K groups of both kinds): the fused kernel reads each K group
    as its flag says, the dense kernel the K rows packed in K only."""
    B, Hkv, nrep, D = 2, 2, 4, 128
    ks, kq, kr = 32, 1280 - 32 - 96, 96
    T = ks + kq + kr
    vs = 32
    vq = (T - vs - 64) // G * G
    vr = T - vs - vq
    kx = _mixed_v(B, Hkv, T, D, seed=41 + kbits + G)
    vx = _mixed_v(B, Hkv, T, D, seed=42)
    kst = _store(kx[:, :, ks:ks + kq], "channel", kbits, G)
    kc, ksc, kz = Q.quantize_channeldim_hybrid(kx[:, :, ks:ks + kq], G, kbits)
    assert 0 < ksc["mask"].mean() < 1
    kdq = Q.dequantize_channeldim_hybrid(kc, ksc, kz, G)
    np.testing.assert_array_equal(kst.dequant(dtype=torch.float32).cpu().numpy() + np.float32(0),
                                  kdq.astype(np.float32) + np.float32(0))
    vpart = vx[:, :, vs:vs + vq]
    if vmode == "hybrid":
        vst = _store(vpart, "token", 2, G)
        vdq = Q.dequantize_tokendim_hybrid(*Q.quantize_tokendim_hybrid(vpart, G, 2), G)
    else:
        vst = ops.PackedStore("token", B, Hkv, D, G, 4, vmode, DEV)
        vst.append(_f16t(vpart))
        qv = Q.quantize_tokendim_sym if vmode == "symmetric" else Q.quantize_tokendim_asym
        dv = Q.dequantize_tokendim_sym if vmode == "symmetric" else Q.dequantize_tokendim_asym
        vdq = dv(*qv(vpart, G, 4), G)
    q = synth.normal((B, Hkv * nrep, D), seed=43).astype(np.float16)
    kxt, vxt = _f16t(kx), _f16t(vx)
    got = ops.decode_attention(_f16t(q), kxt[:, :, :ks], kst, kxt[:, :, ks + kq:], vxt[:, :, :vs], vst,
                               vxt[:, :, vs + vq:], D ** -0.5).cpu().numpy().astype(np.float64)
    kd = np.concatenate([kx[:, :, :ks].astype(np.float32), kdq, kx[:, :, ks + kq:].astype(np.float32)], axis=2)
    vd = np.concatenate([vx[:, :, :vs].astype(np.float32), vdq, vx[:, :, vs + vq:].astype(np.float32)], axis=2)
    assert A.rel_err(got, A.decode_attention(q, kd, vd, D ** -0.5, p_dtype=None)) < TOL


@pytest.mark.gpu
def test_hybrid_k_needs_one_group_size():
    """A hybrid K store is read by the fused kernel only, which takes K and V of
    one group size: K groups of 32 with V groups of 64 are refused (no launch)."""
    B, Hkv, D, T = 1, 2, 128, 256
    kx = _mixed_v(B, Hkv, T, D, seed=44)
    kst = _store(kx, "channel", 3, 32)
    vst = ops.PackedStore("token", B, Hkv, D, 64, 4, "symmetric", DEV)
    vst.append(_f16t(kx))
    q = synth.normal((B, Hkv * 4, D), seed=45).astype(np.float16)
    with pytest.raises(_lib.IQError) as e:
        ops.decode_attention(_f16t(q), None, kst, None, None, vst, None, D ** -0.5)
    assert e.value.status == -7  # IQ_ERR_MODE


@pytest.mark.gpu
def test_hybrid_decode_attention_full_size():
    """The benchmark's shapes (B=8, 32 query / 8 KV heads, D=128, 32768 tokens)
    with 3-bit sym K and 2-bit hybrid V, all packed; three calls in a row.
    Reference: fp32 attention over K/V dequantized by the library (bit-exact
    to the oracle above), query heads grouped per KV head."""
    B, Hkv, nrep, D, T = 8, 8, 4, 128, 32768
    gen = torch.Generator(device=DEV).manual_seed(5)
    k = torch.randn(B, Hkv, T, D, generator=gen, device=DEV).to(torch.float16)
    v = torch.randn(B, Hkv, T, D, generator=gen, device=DEV).to(torch.float16)
    k[..., :4] *= 10
    v[..., :48] += 6  # columns with an offset: asym groups at 2 bits
    q = torch.randn(B, Hkv * nrep, D, generator=gen, device=DEV).to(torch.float16)
    kst = ops.PackedStore("channel", B, Hkv, D, 32, 3, "symmetric", DEV, t_cap=T)
    vst = ops.PackedStore("token", B, Hkv, D, 32, 2, "hybrid", DEV, t_cap=T)
    kst.append(k)
    vst.append(v)
    mask = ops.unpack_store(vst, 0, 4096)[1]["mask"]
    assert 0.0 < mask.float().mean().item() < 1.0
    kd, vd = kst.dequant(dtype=torch.float32), vst.dequant(dtype=torch.float32)
    lg = torch.matmul(q.float().view(B, Hkv, nrep, D), kd.transpose(-1, -2).contiguous()) * D ** -0.5
    ref = torch.matmul(torch.softmax(lg, dim=-1), vd).view(B, Hkv * nrep, D)
    del kd, vd, lg
    for _ in range(3):
        got = ops.decode_attention(q, None, kst, None, None, vst, None, D ** -0.5)
        torch.cuda.synchronize()
        assert ((got.float() - ref).abs().max() / ref.abs().max()).item() < TOL


@pytest.mark.gpu
@pytest.mark.parametrize("axis", ["channel", "token"])
def test_hybrid_store_wire_round_trip(axis):
    """to_bytes / from_bytes keep the flag bits: the loaded store dequantizes and
    keeps appending exactly like the original."""
    x = _mixed_v(1, 2, 256, 128, seed=41)
    st = _store(x[:, :, :160], axis, 2)
    back = ops.PackedStore.from_bytes(st.to_bytes(), DEV)
    assert back.mode == st.mode and back.length == 160
    assert torch.equal(back.dequant(dtype=torch.float32), st.dequant(dtype=torch.float32))
    for s in (st, back):
        s.append(_f16t(x[:, :, 160:]))
    assert torch.equal(back.dequant(dtype=torch.float32), st.dequant(dtype=torch.float32))


@pytest.mark.gpu
@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("bits", BITS)
def test_hybrid_exact_ties_keep_asym(hybrid_ties, axis, bits):
    """Groups whose two L1 errors tie exactly (the live reference's masks:
    all False, quant.py:144 compares strictly) through every hybrid path: the
    quant.py-API functional hybrid (iq_hybrid_mask), a hybrid store's append
    (one thread per group) and a window flush (one lane per element)."""
    from innerq_amd import quant as IQ
    x = hybrid_ties[f"{axis}_b{bits}_x"].view(np.float16)
    want = hybrid_ties[f"{axis}_b{bits}_mask"]
    xt = _f16t(x)
    qa, qs = getattr(IQ, f"quantize_{axis}dim_asym"), getattr(IQ, f"quantize_{axis}dim_sym")
    da, ds = getattr(IQ, f"dequantize_{axis}dim_asym"), getattr(IQ, f"dequantize_{axis}dim_sym")
    _, s, _ = IQ.quantize_hybrid(qa, qs, da, ds)(xt, 32, bits)
    np.testing.assert_array_equal(s["mask"].cpu().numpy(), want)
    # the store's flags (bit 15 of each unit's scale): none set
    st = _store(x, axis, bits)
    assert not ops.unpack_store(st)[1]["mask"].cpu().numpy().any()
    # a window flush of the same tokens
    w = ops.RecentWindow(xt[:, :, :1])
    ws = ops.PackedStore(axis, 1, 1, x.shape[3], 32, bits, "hybrid", DEV)
    n = x.shape[2]
    if axis == "channel":
        ops.window_append(w, xt[:, :, 1:], n, ws, None, None, None, 0, None)
    else:
        ops.window_append(None, None, 0, None, None, w, xt[:, :, 1:], n, ws)
    torch.cuda.synchronize()
    assert not ops.unpack_store(ws)[1]["mask"].cpu().numpy().any()
    np.testing.assert_array_equal(ws.codes.cpu().numpy(), st.codes.cpu().numpy())
