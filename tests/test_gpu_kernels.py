"""GPU parity of the HIP kernels (through the C ABI) against the CPU oracle.

Bars: packed bytes, codes, scales and zero points bit-exact; dense dequantized
values bit-exact (fp16, up to the sign of zero for sym); QK^T logits and
attn.V outputs within 1e-3 of the float64 dequantize-then-matmul oracle in
the max-relative metric  max|got-ref| / max|ref|.
"""
import numpy as np
import pytest
import torch

from innerq_amd import ops, synth
from oracle import attn_ref as A
from oracle import quant_ref as Q

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-3
MODES = ["asymmetric", "symmetric"]


def f16t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


_MODE_TAG = {"asymmetric": "asym", "symmetric": "sym", "hybrid": "hybrid"}


def oracle_q(x, bits, G, mode, axis):
    fn = getattr(Q, f"quantize_{axis}dim_{_MODE_TAG[mode]}")
    return fn(x, G, bits)


def oracle_deq(c, s, z, G, mode, axis):
    fn = getattr(Q, f"dequantize_{axis}dim_{_MODE_TAG[mode]}")
    return fn(c, s, z, G)


def special_input(B, H, T, D, seed):
    x = synth.kv_tensor(B, H, T, D, seed=seed, n_out=3, factor=10.0).astype(np.float32)
    x[0, 0, 3, :] = 0.5                          # constant channel-dim groups
    x[0, 0, :32, 5] = -2.0                       # a constant token-dim group
    x[0, H - 1, 7, :32] = np.arange(32) % 4 - 2  # ties
    x[0, H - 1, 8, :] = 0.0
    return x.astype(np.float16)


# ----------------------------------------------------------------------------
# quantize-on-append (A1, A2, A5)
# ----------------------------------------------------------------------------
@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("G", [32, 64, 128])
def test_quantize_dense_bit_exact(axis, mode, bits, G):
    x = special_input(2, 3, 128, 128, seed=bits * 10 + G)
    c, s, z = ops.quantize_dense(f16t(x), G, bits, mode, axis)
    rc, rs, rz = oracle_q(x, bits, G, mode, axis)
    np.testing.assert_array_equal(c.cpu().numpy(), rc)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint16), rs.view(np.uint16))
    np.testing.assert_array_equal(z.cpu().numpy().view(np.uint16), rz.view(np.uint16))


def test_quantize_dense_matches_reference_golden(quant_golden):
    g = quant_golden
    x = g["x"].view(np.float16)
    for axis in ("channel", "token"):
        for mode, tag in (("asymmetric", "asym"), ("symmetric", "sym")):
            for bits in (2, 3, 4):
                for G in (32, 64):
                    c, s, z = ops.quantize_dense(f16t(x), G, bits, mode, axis)
                    key = f"{axis}_{tag}_b{bits}_g{G}"
                    cc = c.cpu().numpy()
                    cc = np.where(cc == -2147483648, -128, cc).astype(np.int8)
                    np.testing.assert_array_equal(cc, g[key + "_codes"], err_msg=key)
                    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint16), g[key + "_scale"], err_msg=key)
                    np.testing.assert_array_equal(z.cpu().numpy().view(np.uint16),
                                                  g[key + ("_zero" if tag == "asym" else "_signs")], err_msg=key)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("G", [32, 64])
def test_k_store_append_bit_exact(mode, bits, G):
    """quantize-on-append in pieces (prefill, single tokens, a burst) == oracle store bytes"""
    B, H, T, D = 2, 2, 200, 128
    x = special_input(B, H, T, D, seed=bits + G)
    st = ops.PackedStore("channel", B, H, D, G, bits, mode, DEV)
    xt = f16t(x)
    for a, b in ((0, 130), (130, 131), (131, 132), (132, 200)):
        st.append(xt[:, :, a:b])
    assert st.length == T
    c, s, z = oracle_q(x, bits, G, mode, "channel")
    cw, meta = Q.build_k_store(c, s, z, bits, G, mode, tcap=st.t_cap)
    nblk = -(-T // 64)
    got_c = st.codes.cpu().numpy().view(np.uint32).reshape(cw.shape)
    got_m = st.meta.cpu().numpy().view(np.uint16).reshape(meta.shape)
    # rows past T in the last block are unspecified
    gc, rc = Q.k_store_to_codes(got_c, got_m, T, bits, G, mode), Q.k_store_to_codes(cw, meta, T, bits, G, mode)
    np.testing.assert_array_equal(gc[0], rc[0])
    np.testing.assert_array_equal(gc[1].view(np.uint16), rc[1].view(np.uint16))
    if mode == "asymmetric":
        np.testing.assert_array_equal(gc[2].view(np.uint16), rc[2].view(np.uint16))
    np.testing.assert_array_equal(got_c[:, :, :nblk - 1], cw[:, :, :nblk - 1])


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("G", [32, 64])
def test_v_store_append_bit_exact(mode, bits, G):
    B, H, T, D = 2, 2, 4 * G, 128
    x = special_input(B, H, T, D, seed=3 * bits + G)
    st = ops.PackedStore("token", B, H, D, G, bits, mode, DEV)
    xt = f16t(x)
    st.append(xt[:, :, :G])
    st.append(xt[:, :, G:4 * G])
    c, s, z = oracle_q(x, bits, G, mode, "token")
    cw, meta = Q.build_v_store(c, s, z, bits, G, mode, tcap=st.t_cap)
    np.testing.assert_array_equal(st.codes.cpu().numpy().view(np.uint32).reshape(cw.shape)[:, :, :T // G],
                                  cw[:, :, :T // G])
    np.testing.assert_array_equal(st.meta.cpu().numpy().view(np.uint16).reshape(meta.shape)[:, :, :T // G],
                                  meta[:, :, :T // G])


# ----------------------------------------------------------------------------
# dense read path (A3, A4, A10)
# ----------------------------------------------------------------------------
@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_store_dequant_bit_exact(axis, mode, bits):
    B, H, T, D, G = 1, 3, 192, 128, 32
    x = special_input(B, H, T, D, seed=40 + bits)
    st = ops.PackedStore(axis, B, H, D, G, bits, mode, DEV)
    st.append(f16t(x))
    c, s, z = oracle_q(x, bits, G, mode, axis)
    ref = oracle_deq(c, s, z, G, mode, axis)
    got32 = st.dequant(dtype=torch.float32).cpu().numpy()
    np.testing.assert_array_equal(got32, ref)  # value equality (+0 == -0)
    got16 = st.dequant().cpu().numpy()
    np.testing.assert_array_equal(got16, ref.astype(np.float16))
    # a strided sub-range
    out = torch.zeros(B, H, 300, D, dtype=torch.float16, device=DEV)
    st.dequant(64, 96, out=out[:, :, 10:106])
    np.testing.assert_array_equal(out[:, :, 10:106].cpu().numpy(), ref[:, :, 64:160].astype(np.float16))


@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("mode", MODES)
def test_dequantize_dense_api(axis, mode):
    x = special_input(1, 2, 64, 128, seed=77)
    c, s, z = oracle_q(x, 4, 32, mode, axis)
    ref = oracle_deq(c, s, z, 32, mode, axis)
    got = ops.dequantize_dense(torch.from_numpy(c).to(DEV), f16t(s), f16t(z), 32, mode, axis).cpu().numpy()
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("D,T,layout", [
    (128, 32768, "contiguous"),  # a prefill's prompt: the row kernel, 16-byte loads
    (128, 4099, "token_stride"),  # every other token of a longer tensor, rows past a multiple of the lanes
    (64, 1, "contiguous"),
    (64, 777, "unaligned"),  # rows not 16-byte aligned: element loads
    (96, 300, "contiguous"),  # head_dim outside {64, 128}: one thread per channel
])
def test_key_norm_factor_matches_numpy(D, T, layout):
    """sqrt(max_t |k|) per (batch, head, channel) rounded to fp16 (cache.py:121-126),
    bit for bit against numpy's float32 square root of the fp16 maxima, with an
    infinity and a NaN planted (torch's and numpy's max propagate NaN)."""
    B, H = 2, 3
    x = synth.kv_tensor(B, H, 2 * T + 1, D + 1, seed=D + T, n_out=3, factor=9.0).astype(np.float16)
    view = {"token_stride": np.s_[:, :, 1::2, :D], "unaligned": np.s_[:, :, :T, 1:]}.get(layout, np.s_[:, :, T + 1:, :D])
    kn = x[view]  # a numpy view: the planted values land in x
    kn[0, 1, min(5, T - 1), 7] = np.inf
    kn[1, 2, T - 1, 3] = np.nan
    k = f16t(x)[view]
    if layout == "contiguous":
        k = k.contiguous()
    got = ops.key_norm_factor(k).cpu().numpy()
    ref = np.sqrt(np.abs(kn).astype(np.float32).max(axis=2, keepdims=True)).astype(np.float16)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(got[ok].view(np.uint16), ref[ok].view(np.uint16))


def test_key_normalized_store_dequant():
    B, H, T, D, G = 1, 2, 128, 128, 32
    x = special_input(B, H, T, D, seed=5)
    norm = np.sqrt(np.abs(x).max(axis=-2, keepdims=True).astype(np.float32)).astype(np.float16)
    xn = (x.astype(np.float32) / norm.astype(np.float32)).astype(np.float16)
    st = ops.PackedStore("channel", B, H, D, G, 3, "symmetric", DEV)
    st.append(f16t(x), norm=f16t(norm))
    c, s, sg = Q.quantize_channeldim_sym(xn, G, 3)
    ref = Q.dequantize_channeldim_sym(c, s, sg, G) * norm.astype(np.float32)
    got = st.dequant(norm=f16t(norm), dtype=torch.float32).cpu().numpy()
    np.testing.assert_array_equal(got, ref)


# ----------------------------------------------------------------------------
# GEMVs (A6, A8)
# ----------------------------------------------------------------------------
def build_k(B, Hkv, T, D, G, bits, mode, seed):
    x = synth.kv_tensor(B, Hkv, T, D, seed=seed, n_out=4, factor=10.0)
    st = ops.PackedStore("channel", B, Hkv, D, G, bits, mode, DEV)
    st.append(f16t(x))
    c, s, z = oracle_q(x, bits, G, mode, "channel")
    return st, oracle_deq(c, s, z, G, mode, "channel")


def build_v(B, Hkv, T, D, G, bits, mode, seed):
    x = synth.kv_tensor(B, Hkv, T, D, seed=seed, n_out=4, factor=10.0)
    st = ops.PackedStore("token", B, Hkv, D, G, bits, mode, DEV)
    st.append(f16t(x))
    c, s, z = oracle_q(x, bits, G, mode, "token")
    return st, oracle_deq(c, s, z, G, mode, "token")


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("G", [32, 64, 128])
@pytest.mark.parametrize("nrep", [1, 4])
def test_qk_gemv_parity(mode, bits, G, nrep):
    B, Hkv, T, D = 2, 2, 333, 128
    st, kdeq = build_k(B, Hkv, T, D, G, bits, mode, seed=bits * 7 + G + nrep)
    q = synth.normal((B, Hkv * nrep, D), seed=99 + G).astype(np.float16)
    scale = D ** -0.5
    got = ops.qk_gemv(f16t(q), st, scale).cpu().numpy()
    ref = A.qk_logits(q, kdeq, scale)
    assert A.rel_err(got, ref) < TOL


@pytest.mark.parametrize("nrep", [2, 8])
@pytest.mark.parametrize("D", [64, 128])
def test_qk_gemv_shapes(nrep, D):
    B, Hkv, T = 3, 1, 64 * 5 + 17
    st, kdeq = build_k(B, Hkv, T, D, 32, 4, "asymmetric", seed=nrep + D)
    q = synth.normal((B, Hkv * nrep, D), seed=3).astype(np.float16)
    got = ops.qk_gemv(f16t(q), st, 1.0).cpu().numpy()
    assert A.rel_err(got, A.qk_logits(q, kdeq, 1.0)) < TOL
    # sub-range starting at a block boundary, written into a strided output
    out = torch.full((B, Hkv * nrep, 400), 7.0, device=DEV)
    ops.qk_gemv(f16t(q), st, 1.0, t0=128, T=T - 128, out=out[:, :, 5:5 + T - 128])
    o = out.cpu().numpy()
    assert A.rel_err(o[:, :, 5:5 + T - 128], A.qk_logits(q, kdeq[:, :, 128:], 1.0)) < TOL
    assert np.all(o[:, :, :5] == 7.0) and np.all(o[:, :, 5 + T - 128:] == 7.0)


# The normalization is folded into the query as hi/lo fp16 rows (n_rep query
# heads become 2*n_rep matrix-core rows): every n_rep exercises another row
# layout (n_rep 1, 2: one 4-row block; 4: two blocks; 8: four).
@pytest.mark.parametrize("nrep,G", [(1, 32), (2, 128), (4, 32), (8, 64)])
def test_qk_gemv_key_norm_folded(nrep, G):
    B, Hkv, T, D = 1, 2, 256, 128
    x = synth.kv_tensor(B, Hkv, T, D, seed=11, n_out=4, factor=8.0)
    norm = np.sqrt(np.abs(x).max(axis=-2, keepdims=True).astype(np.float32)).astype(np.float16)
    st = ops.PackedStore("channel", B, Hkv, D, G, 3, "symmetric", DEV)
    st.append(f16t(x), norm=f16t(norm))
    xn = (x.astype(np.float32) / norm.astype(np.float32)).astype(np.float16)
    c, s, sg = Q.quantize_channeldim_sym(xn, G, 3)
    kdeq = Q.dequantize_channeldim_sym(c, s, sg, G) * norm.astype(np.float32)
    q = synth.normal((B, Hkv * nrep, D), seed=12).astype(np.float16)
    got = ops.qk_gemv(f16t(q), st, D ** -0.5, norm=f16t(norm)).cpu().numpy()
    assert A.rel_err(got, A.qk_logits(q, kdeq, D ** -0.5)) < TOL


@pytest.mark.parametrize("bits,G,mode,norm", [(4, 32, "asymmetric", False), (2, 64, "symmetric", True),
                                              (3, 128, "asymmetric", False)])
def test_qk_gemv_many_runs(bits, G, mode, norm):
    """A long range over several (batch, KV head)s: the persistent kernel's shares
    cut every head into several runs, each building its own query records.
    Reference: fp32 q . K over the store's own dequantization (dequant is
    bit-exact to the oracle in the tests above) times the normalization."""
    B, Hkv, nrep, D, T = 2, 4, 4, 128, 16384 + 64 * 5 + 9
    gen = torch.Generator(device=DEV).manual_seed(bits * G + norm)
    x = torch.randn(B, Hkv, T, D, generator=gen, device=DEV).to(torch.float16)
    nrm = (torch.rand(B, Hkv, 1, D, generator=gen, device=DEV) + 0.5).to(torch.float16) if norm else None
    st = ops.PackedStore("channel", B, Hkv, D, G, bits, mode, DEV, t_cap=T)
    st.append(x, norm=nrm)
    kd = st.dequant(norm=nrm, dtype=torch.float32)
    q = torch.randn(B, Hkv * nrep, D, generator=gen, device=DEV).to(torch.float16)
    got = ops.qk_gemv(q, st, D ** -0.5, norm=nrm)
    ref = torch.matmul(q.float().view(B, Hkv, nrep, D), kd.transpose(-1, -2).contiguous())
    ref = ref.view(B, Hkv * nrep, T) * D ** -0.5
    assert A.rel_err(got.cpu().numpy(), ref.cpu().numpy()) < TOL


@pytest.mark.parametrize("axis,bits,mode,n0,n1", [("channel", 4, "asymmetric", 150, 50),
                                                  ("token", 3, "symmetric", 128, 64)])
def test_store_wire_round_trip(axis, bits, mode, n0, n1):
    """A store written to the wire format and read back onto the device (a
    partial last K block included) dequantizes bit for bit like the original,
    decodes the same, and keeps appending like it."""
    B, H, D, G = 2, 2, 128, 32
    x = torch.randn(B, H, n0 + n1, D, generator=torch.Generator(device=DEV).manual_seed(bits), device=DEV).half()
    st = ops.PackedStore(axis, B, H, D, G, bits, mode, DEV)
    st.append(x[:, :, :n0])
    back = ops.PackedStore.from_bytes(st.to_bytes(), DEV)
    assert back.length == n0
    assert torch.equal(back.dequant(dtype=torch.float32), st.dequant(dtype=torch.float32))
    st.append(x[:, :, n0:])
    back.append(x[:, :, n0:])
    assert torch.equal(back.dequant(dtype=torch.float32), st.dequant(dtype=torch.float32))
    if axis == "channel":
        q = torch.randn(B, 4 * H, D, device=DEV).half()
        assert torch.equal(ops.qk_gemv(q, back, 0.1), ops.qk_gemv(q, st, 0.1))


def peaked_p(B, Hq, T, seed, std=2.0):
    logits = synth.normal((B, Hq, T), seed=seed, std=std).astype(np.float64)
    return A.softmax(logits).astype(np.float16)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("G", [32, 64, 128])
@pytest.mark.parametrize("nrep", [1, 4])
def test_av_gemv_parity(mode, bits, G, nrep):
    B, Hkv, D = 2, 2, 128
    T = 6 * G
    st, vdeq = build_v(B, Hkv, T, D, G, bits, mode, seed=bits * 5 + G + nrep)
    p = peaked_p(B, Hkv * nrep, T, seed=G + bits)
    got = ops.av_gemv(f16t(p), st).cpu().numpy().astype(np.float64)
    ref = A.av_out(p, vdeq)
    assert A.rel_err(got, ref) < TOL


@pytest.mark.parametrize("nrep", [2, 8])
@pytest.mark.parametrize("D", [64, 128])
def test_av_gemv_shapes_and_accumulate(nrep, D):
    B, Hkv, G = 2, 1, 32
    T = 3000 - 3000 % G
    st, vdeq = build_v(B, Hkv, T, D, G, 4, "asymmetric", seed=nrep * D)
    p = peaked_p(B, Hkv * nrep, T, seed=4)
    o32 = torch.ones(B, Hkv * nrep, D, device=DEV)
    o16 = torch.empty(B, Hkv * nrep, D, dtype=torch.float16, device=DEV)
    ops.av_gemv(f16t(p[:, :, G:T - G]), st, t0=G, T=T - 2 * G, out=o16, out32=o32, accumulate=True)
    ref = A.av_out(p[:, :, G:T - G], vdeq[:, :, G:T - G]) + 1.0
    assert A.rel_err(o32.cpu().numpy(), ref) < TOL
    assert A.rel_err(o16.cpu().numpy().astype(np.float64), ref) < 2e-3


@pytest.mark.parametrize("bits,G,mode,B,Hkv,T", [(2, 64, "asymmetric", 2, 4, 16384),
                                                  (4, 32, "symmetric", 2, 4, 16384),
                                                  # one head of 37 splits: a run per workgroup,
                                                  # the combine's rounds of eight end short
                                                  (2, 64, "asymmetric", 1, 1, 37 * 256)])
def test_av_gemv_many_runs(bits, G, mode, B, Hkv, T):
    """A long range over many (batch, KV head)s: the persistent kernel's shares cut the
    heads into several runs each, whose partials the combine sums.  Reference: fp32
    p @ V over V unpacked by the library (unpack is bit-exact to the oracle elsewhere)."""
    nrep, D = 4, 128
    gen = torch.Generator(device=DEV).manual_seed(bits * G)
    x = torch.randn(B, Hkv, T, D, generator=gen, device=DEV).to(torch.float16)
    st = ops.PackedStore("token", B, Hkv, D, G, bits, mode, DEV, t_cap=T)
    st.append(x)
    vd = ops.dequantize_dense(*ops.unpack_store(st), G, mode, "token")
    p = torch.softmax(torch.randn(B, Hkv * nrep, T, generator=gen, device=DEV) * 2.0, dim=-1).to(torch.float16)
    got = ops.av_gemv(p, st, out32=torch.empty(B, Hkv * nrep, D, device=DEV))
    ref = torch.matmul(p.float().view(B, Hkv, nrep, T), vd).view(B, Hkv * nrep, D)
    err = ((got - ref).abs().max() / ref.abs().max()).item()
    assert err < TOL


def test_av_gemv_linearity():
    """p -> p.V is linear: AV(p1 + p2) == AV(p1) + AV(p2) (size-independent property)"""
    B, Hkv, T, D, G = 1, 2, 4096, 128, 64
    st, _ = build_v(B, Hkv, T, D, G, 2, "asymmetric", seed=8)
    p1 = peaked_p(B, Hkv * 4, T, seed=1).astype(np.float32) / 2
    p2 = peaked_p(B, Hkv * 4, T, seed=2).astype(np.float32) / 2
    a = ops.av_gemv(f16t(p1.astype(np.float16)), st, out32=torch.empty(B, 8, D, device=DEV)).cpu().numpy()
    b = ops.av_gemv(f16t(p2.astype(np.float16)), st, out32=torch.empty(B, 8, D, device=DEV)).cpu().numpy()
    c = ops.av_gemv(f16t((p1.astype(np.float16).astype(np.float32) + p2.astype(np.float16).astype(np.float32))
                         .astype(np.float16)), st, out32=torch.empty(B, 8, D, device=DEV)).cpu().numpy()
    assert A.rel_err(c, a + b) < 2e-3


# ----------------------------------------------------------------------------
# decode step (A9 + segments)
# ----------------------------------------------------------------------------
@pytest.mark.parametrize("kb,vb,kmode,vmode", [(4, 4, "asymmetric", "asymmetric"), (3, 3, "symmetric", "symmetric"),
                                               (2, 4, "asymmetric", "symmetric")])
def test_decode_attention_segments(kb, vb, kmode, vmode):
    B, Hkv, nrep, D, G = 2, 2, 4, 128, 32
    ks, kq, kr = 32, 640 - 32 - 96, 96        # K: flush 1 keeps the recent window full
    vs, vq, vr = 32, 640 - 32 - 64, 64        # V: flush 32 drains it
    T = ks + kq + kr
    kx = synth.kv_tensor(B, Hkv, T, D, seed=21, n_out=4, factor=8.0)
    vx = synth.kv_tensor(B, Hkv, T, D, seed=22, n_out=4, factor=8.0)
    kst = ops.PackedStore("channel", B, Hkv, D, G, kb, kmode, DEV)
    kst.append(f16t(kx[:, :, ks:ks + kq]))
    vst = ops.PackedStore("token", B, Hkv, D, G, vb, vmode, DEV)
    vst.append(f16t(vx[:, :, vs:vs + vq]))
    q = synth.normal((B, Hkv * nrep, D), seed=23).astype(np.float16)
    kxt, vxt = f16t(kx), f16t(vx)
    got = ops.decode_attention(f16t(q), kxt[:, :, :ks], kst, kxt[:, :, ks + kq:], vxt[:, :, :vs], vst,
                               vxt[:, :, vs + vq:], D ** -0.5).cpu().numpy().astype(np.float64)
    c, s, z = oracle_q(kx[:, :, ks:ks + kq], kb, G, kmode, "channel")
    kd = np.concatenate([kx[:, :, :ks].astype(np.float32), oracle_deq(c, s, z, G, kmode, "channel"),
                         kx[:, :, ks + kq:].astype(np.float32)], axis=2)
    c, s, z = oracle_q(vx[:, :, vs:vs + vq], vb, G, vmode, "token")
    vd = np.concatenate([vx[:, :, :vs].astype(np.float32), oracle_deq(c, s, z, G, vmode, "token"),
                         vx[:, :, vs + vq:].astype(np.float32)], axis=2)
    ref = A.decode_attention(q, kd, vd, D ** -0.5, p_dtype=None)
    assert A.rel_err(got, ref) < TOL


def test_decode_attention_all_quantized_and_all_dense():
    B, Hkv, nrep, D, G, T = 1, 2, 4, 128, 32, 512
    kx = synth.kv_tensor(B, Hkv, T, D, seed=31)
    vx = synth.kv_tensor(B, Hkv, T, D, seed=32)
    q = synth.normal((B, Hkv * nrep, D), seed=33).astype(np.float16)
    kst = ops.PackedStore("channel", B, Hkv, D, G, 4, "asymmetric", DEV)
    vst = ops.PackedStore("token", B, Hkv, D, G, 4, "asymmetric", DEV)
    kst.append(f16t(kx))
    vst.append(f16t(vx))
    got = ops.decode_attention(f16t(q), None, kst, None, None, vst, None, D ** -0.5).cpu().numpy()
    c, s, z = Q.quantize_channeldim_asym(kx, G, 4)
    kd = Q.dequantize_channeldim_asym(c, s, z, G)
    c, s, z = Q.quantize_tokendim_asym(vx, G, 4)
    vd = Q.dequantize_tokendim_asym(c, s, z, G)
    assert A.rel_err(got.astype(np.float64), A.decode_attention(q, kd, vd, D ** -0.5, None)) < TOL
    # fp16 only (no quantized segments): exactly the eager attention over fp16 K/V
    got = ops.decode_attention(f16t(q), f16t(kx), None, None, f16t(vx), None, None, D ** -0.5).cpu().numpy()
    ref = A.decode_attention(q, kx.astype(np.float32), vx.astype(np.float32), D ** -0.5, None)
    assert A.rel_err(got.astype(np.float64), ref) < TOL


def _decode_case(B, Hkv, nrep, D, kseg, vseg, kfmt, vfmt, seed, norm=False):
    """kseg/vseg = (sink, packed, recent) token counts; fmt = (bits, group, mode)."""
    T = sum(kseg)
    assert sum(vseg) == T
    kx = synth.kv_tensor(B, Hkv, T, D, seed=seed, n_out=4, factor=8.0)
    vx = synth.kv_tensor(B, Hkv, T, D, seed=seed + 1, n_out=4, factor=8.0)
    q = synth.normal((B, Hkv * nrep, D), seed=seed + 2).astype(np.float16)
    ks, kq, kr = kseg
    vs, vq, vr = vseg
    kb, kg, km = kfmt
    vb, vg, vm = vfmt
    nrm = None
    kpart = kx[:, :, ks:ks + kq]
    if norm:
        nrm = np.sqrt(np.abs(kpart).max(axis=-2, keepdims=True).astype(np.float32)).astype(np.float16)
    kst = ops.PackedStore("channel", B, Hkv, D, kg, kb, km, DEV)
    kst.append(f16t(kpart), norm=None if nrm is None else f16t(nrm))
    vst = ops.PackedStore("token", B, Hkv, D, vg, vb, vm, DEV)
    vst.append(f16t(vx[:, :, vs:vs + vq]))
    kxt, vxt = f16t(kx), f16t(vx)
    got = ops.decode_attention(f16t(q), kxt[:, :, :ks] if ks else None, kst if kq else None,
                               kxt[:, :, ks + kq:] if kr else None, vxt[:, :, :vs] if vs else None,
                               vst if vq else None, vxt[:, :, vs + vq:] if vr else None, D ** -0.5,
                               norm=None if nrm is None else f16t(nrm)).cpu().numpy().astype(np.float64)
    kin = kpart if nrm is None else (kpart.astype(np.float32) / nrm.astype(np.float32)).astype(np.float16)
    c, s, z = oracle_q(kin, kb, kg, km, "channel")
    kd = oracle_deq(c, s, z, kg, km, "channel")
    if nrm is not None:
        kd = kd * nrm.astype(np.float32)
    kd = np.concatenate([kx[:, :, :ks].astype(np.float32), kd, kx[:, :, ks + kq:].astype(np.float32)], axis=2)
    c, s, z = oracle_q(vx[:, :, vs:vs + vq], vb, vg, vm, "token")
    vd = np.concatenate([vx[:, :, :vs].astype(np.float32), oracle_deq(c, s, z, vg, vm, "token"),
                         vx[:, :, vs + vq:].astype(np.float32)], axis=2)
    ref = A.decode_attention(q, kd, vd, D ** -0.5, p_dtype=None)
    return A.rel_err(got, ref)


@pytest.mark.parametrize("kseg,vseg", [
    ((4, 64 * 20, 100), (0, 32 * 41, 72)),      # different sinks, V drained, fused range shifted
    ((32, 64 * 9, 96), (32, 32 * 19, 64)),      # innerq preset shape, partial last split
    ((0, 64 * 3, 7), (0, 32 * 4, 71)),          # K packed past V's packed range
    ((3, 0, 200), (3, 64, 136)),                # no packed K: everything dense
])
def test_decode_attention_fused_and_dense_ranges(kseg, vseg):
    err = _decode_case(2, 2, 4, 128, kseg, vseg, (4, 32, "asymmetric"), (4, 32, "asymmetric"), seed=sum(kseg))
    assert err < TOL


# fp16 windows of up to 256 tokens next to the fused range (K and V laid out
# alike) are attended after the fused kernel by the merging dense kernel: two
# halves of the window side by side, then the merge with the fused runs'
# partials; 257 tokens take the dense slices and the combine.  Odd and one-token
# windows (an empty half), sinks and recents together, 8 query heads per KV
# head (two output elements per thread at D = 128), D = 64, and a long packed
# range (32 fused runs per head, more than the merging kernel preloads: the
# window then takes the dense slices, launched after the fused kernel, and the
# combine).
@pytest.mark.parametrize("seg,nrep,D", [
    ((0, 64 * 8, 1), 4, 128),
    ((0, 64 * 128, 100), 4, 128),
    ((16, 64 * 8, 17), 8, 128),
    ((0, 64 * 6, 255), 2, 64),
    ((128, 64 * 6, 128), 8, 128),
    ((1, 64 * 6, 256), 4, 128),
])
def test_decode_attention_window_after_fused_kernel(seg, nrep, D):
    err = _decode_case(2, 2, nrep, D, seg, seg, (4, 32, "asymmetric"), (4, 32, "asymmetric"), seed=sum(seg) + nrep)
    assert err < TOL


def test_decode_attention_past_the_split_slot_limit():
    """300,096 tokens in one call (1,173 splits of 256, past the 1,024 split slots
    a combine over every slot holds): the fused path's combine reads only the live
    slots (one run per workgroup here, plus the window's slices)."""
    seg = (0, 300032, 64)
    err = _decode_case(1, 1, 4, 128, seg, seg, (4, 32, "asymmetric"), (4, 32, "asymmetric"), seed=41)
    assert err < TOL


@pytest.mark.parametrize("kfmt,vfmt", [((3, 32, "symmetric"), (3, 32, "symmetric")),
                                       ((2, 64, "asymmetric"), (4, 64, "symmetric")),
                                       ((4, 128, "asymmetric"), (2, 128, "asymmetric")),
                                       # different group sizes: the unfused QK^T / attn.V kernels
                                       ((4, 32, "asymmetric"), (4, 64, "symmetric")),
                                       ((2, 128, "symmetric"), (3, 32, "asymmetric"))])
def test_decode_attention_formats_and_norm(kfmt, vfmt):
    G = max(kfmt[1], vfmt[1])
    kseg = (32, 64 * 24, 96)
    vq = (64 * 24 + 96) // G * G - G
    vseg = (32, vq, 64 * 24 + 96 - vq)
    err = _decode_case(1, 2, 4, 128, kseg, vseg, kfmt, vfmt, seed=5, norm=True)
    assert err < TOL


@pytest.mark.parametrize("nrep,D", [(1, 128), (8, 64), (2, 128)])
def test_decode_attention_gqa_shapes(nrep, D):
    err = _decode_case(2, 2, nrep, D, (0, 64 * 17, 128), (0, 32 * 34, 128), (4, 32, "asymmetric"),
                       (4, 32, "asymmetric"), seed=nrep * D)
    assert err < TOL


@pytest.mark.parametrize("nrep,D,R", [(8, 64, 72), (1, 128, 200), (4, 128, 1000)])
def test_decode_attention_dense_window_unaligned(nrep, D, R):
    """Recent windows given as views whose rows are not 16-byte aligned (odd token
    stride, base two bytes in): the dense gather's element-wise path; R = 1000 runs
    several 64-token chunks per dense slice."""
    B, Hkv, G = 2, 2, 32
    Tq = 64 * 6
    T = Tq + R
    kx = synth.kv_tensor(B, Hkv, T, D, seed=71 + R, n_out=4, factor=8.0)
    vx = synth.kv_tensor(B, Hkv, T, D, seed=72 + R, n_out=4, factor=8.0)
    q = synth.normal((B, Hkv * nrep, D), seed=73).astype(np.float16)
    kst = ops.PackedStore("channel", B, Hkv, D, G, 4, "asymmetric", DEV)
    vst = ops.PackedStore("token", B, Hkv, D, G, 4, "asymmetric", DEV)
    kst.append(f16t(kx[:, :, :Tq]))
    vst.append(f16t(vx[:, :, :Tq]))

    def unaligned(x):
        buf = torch.zeros(B, Hkv, R, D + 1, dtype=torch.float16, device=DEV)
        buf[..., 1:] = f16t(x)
        return buf[..., 1:]

    kr, vr = unaligned(kx[:, :, Tq:]), unaligned(vx[:, :, Tq:])
    assert kr.stride(2) % 8 and kr.data_ptr() % 16
    got = ops.decode_attention(f16t(q), None, kst, kr, None, vst, vr, D ** -0.5).cpu().numpy().astype(np.float64)
    c, s, z = oracle_q(kx[:, :, :Tq], 4, G, "asymmetric", "channel")
    kd = np.concatenate([oracle_deq(c, s, z, G, "asymmetric", "channel"), kx[:, :, Tq:].astype(np.float32)], axis=2)
    c, s, z = oracle_q(vx[:, :, :Tq], 4, G, "asymmetric", "token")
    vd = np.concatenate([oracle_deq(c, s, z, G, "asymmetric", "token"), vx[:, :, Tq:].astype(np.float32)], axis=2)
    assert A.rel_err(got, A.decode_attention(q, kd, vd, D ** -0.5, p_dtype=None)) < TOL


def _decode_inputs(B, Hkv, nrep, D, Tq, R, bits, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    k = torch.randn(B, Hkv, Tq + R, D, generator=gen, device=DEV).to(torch.float16)
    v = torch.randn(B, Hkv, Tq + R, D, generator=gen, device=DEV).to(torch.float16)
    q = torch.randn(B, Hkv * nrep, D, generator=gen, device=DEV).to(torch.float16)
    kst = ops.PackedStore("channel", B, Hkv, D, 32, bits, "asymmetric", DEV, t_cap=Tq)
    vst = ops.PackedStore("token", B, Hkv, D, 32, bits, "asymmetric", DEV, t_cap=Tq)
    kst.append(k[:, :, :Tq])
    vst.append(v[:, :, :Tq])
    kd = torch.cat([ops.dequantize_dense(*ops.unpack_store(kst), 32, "asymmetric", "channel"),
                    k[:, :, Tq:].float()], dim=2)
    vd = torch.cat([ops.dequantize_dense(*ops.unpack_store(vst), 32, "asymmetric", "token"),
                    v[:, :, Tq:].float()], dim=2)
    lg = torch.matmul(q.float().view(B, Hkv, nrep, D), kd.transpose(-1, -2).contiguous()) * D ** -0.5
    ref = torch.matmul(torch.softmax(lg, dim=-1), vd).view(B, Hkv * nrep, D)
    return q, kst, vst, k[:, :, Tq:], v[:, :, Tq:], ref


def test_decode_attention_long_range_repeated():
    """A long range over 8 (batch, KV head)s (several workgroups per head, a dense
    window), three calls in a row on one workspace.  Reference: fp32 attention over
    K/V dequantized by the library (unpack is bit-exact to the oracle elsewhere)."""
    q, kst, vst, kr, vr, ref = _decode_inputs(2, 4, 4, 128, 16384, 64, 4, seed=91)
    for _ in range(3):
        got = ops.decode_attention(q, None, kst, kr, None, vst, vr, 128 ** -0.5)
        torch.cuda.synchronize()
        assert ((got.float() - ref).abs().max() / ref.abs().max()).item() < TOL


@pytest.mark.parametrize("kbits,vbits,R", [(4, 4, 0), (2, 4, 128)])
def test_decode_attention_full_size(kbits, vbits, R):
    """The benchmark's shapes at full size: B=8, 32 query / 8 KV heads, D=128,
    32768 tokens, asym G=32; 4-bit K and V all packed (the headline step) and
    2-bit K / 4-bit V with a 128-token fp16 window (one layer of config 4).
    Reference: fp32 attention over K/V dequantized by the library (unpack is
    bit-exact to the oracle elsewhere), query heads grouped per KV head, and
    three sampled heads end to end through the oracle."""
    B, Hkv, nrep, D, T = 8, 8, 4, 128, 32768
    Tq = T - R
    gen = torch.Generator(device=DEV).manual_seed(kbits * 10 + vbits + R)
    k = torch.randn(B, Hkv, T, D, generator=gen, device=DEV).to(torch.float16)
    v = torch.randn(B, Hkv, T, D, generator=gen, device=DEV).to(torch.float16)
    k[..., :4] *= 10  # outlier channels, as in the benchmark's data
    q = torch.randn(B, Hkv * nrep, D, generator=gen, device=DEV).to(torch.float16)
    kst = ops.PackedStore("channel", B, Hkv, D, 32, kbits, "asymmetric", DEV, t_cap=Tq)
    vst = ops.PackedStore("token", B, Hkv, D, 32, vbits, "asymmetric", DEV, t_cap=Tq)
    kst.append(k[:, :, :Tq])
    vst.append(v[:, :, :Tq])
    kr = k[:, :, Tq:] if R else None
    vr = v[:, :, Tq:] if R else None
    got = ops.decode_attention(q, None, kst, kr, None, vst, vr, D ** -0.5).float()
    kd = torch.cat([kst.dequant(dtype=torch.float32), k[:, :, Tq:].float()], dim=2)
    lg = torch.matmul(q.float().view(B, Hkv, nrep, D), kd.transpose(-1, -2).contiguous()) * D ** -0.5
    del kd
    vd = torch.cat([vst.dequant(dtype=torch.float32), v[:, :, Tq:].float()], dim=2)
    ref = torch.matmul(torch.softmax(lg, dim=-1), vd).view(B, Hkv * nrep, D)
    del vd, lg
    assert ((got - ref).abs().max() / ref.abs().max()).item() < TOL
    # sampled (batch, KV head)s end to end through the oracle: its quantization
    # of the same tokens, dequantization and float64 attention
    for b, h in ((0, 0), (5, 3), (7, 7)):
        kx, vx = k[b:b + 1, h:h + 1].cpu().numpy(), v[b:b + 1, h:h + 1].cpu().numpy()
        kq = oracle_deq(*oracle_q(kx[:, :, :Tq], kbits, 32, "asymmetric", "channel"), 32, "asymmetric", "channel")
        vq = oracle_deq(*oracle_q(vx[:, :, :Tq], vbits, 32, "asymmetric", "token"), 32, "asymmetric", "token")
        kd = np.concatenate([kq, kx[:, :, Tq:].astype(np.float32)], axis=2)
        vd = np.concatenate([vq, vx[:, :, Tq:].astype(np.float32)], axis=2)
        qh = q[b:b + 1, h * nrep:(h + 1) * nrep].cpu().numpy()
        o = A.decode_attention(qh, kd, vd, D ** -0.5, p_dtype=None)
        assert A.rel_err(got[b:b + 1, h * nrep:(h + 1) * nrep].cpu().numpy().astype(np.float64), o) < TOL


@pytest.mark.parametrize("B,Hkv,nrep,T", [(10, 10, 1, 768 + 40), (3, 8, 2, 4096 + 40)])
def test_decode_attention_shares_straddle_heads(B, Hkv, nrep, T):
    """More splits than workgroups, not a multiple of them: shares of one or two
    splits cross (batch, KV head) boundaries (two runs in one workgroup), dealt
    to the XCDs in contiguous eighths of the list."""
    q, kst, vst, kr, vr, ref = _decode_inputs(B, Hkv, nrep, 64, T - 40, 40, 4, seed=B * Hkv + T)
    got = ops.decode_attention(q, None, kst, kr, None, vst, vr, 64 ** -0.5)
    assert ((got.float() - ref).abs().max() / ref.abs().max()).item() < TOL


def test_decode_attention_graph_replay():
    """The decode step captured in a HIP graph and replayed several times (eager
    work between replays): every replay equals the eager result."""
    q, kst, vst, kr, vr, ref = _decode_inputs(2, 4, 4, 128, 8192, 64, 4, seed=92)
    side = torch.cuda.Stream()
    out = torch.empty(2, 16, 128, dtype=torch.float16, device=DEV)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on the capture stream: its workspace exists before capture
        ops.decode_attention(q, None, kst, kr, None, vst, vr, 128 ** -0.5, out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    eager = out.clone()
    assert ((eager.float() - ref).abs().max() / ref.abs().max()).item() < TOL
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        ops.decode_attention(q, None, kst, kr, None, vst, vr, 128 ** -0.5, out=out)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert ((out.float() - eager.float()).abs().max() / eager.float().abs().max()).item() < 1e-5
        ops.decode_attention(q, None, kst, kr, None, vst, vr, 128 ** -0.5)  # eager work between replays
        torch.cuda.synchronize()


# K and V of one bit width and group size take the fused split kernel (one
# workgroup runs QK^T, the split softmax and attn.V); sym/asym may differ.
@pytest.mark.parametrize("fmt,nrep,D", [
    ((2, 2, 32, "asymmetric", "asymmetric"), 4, 128),
    ((2, 2, 64, "symmetric", "asymmetric"), 8, 128),
    ((3, 3, 64, "asymmetric", "symmetric"), 2, 64),
    ((3, 3, 128, "asymmetric", "asymmetric"), 1, 128),
    ((4, 4, 64, "asymmetric", "symmetric"), 4, 64),
    ((4, 4, 128, "symmetric", "symmetric"), 4, 128),
    # K and V of different bit widths (one group size)
    ((2, 4, 32, "asymmetric", "asymmetric"), 4, 128),
    ((4, 2, 32, "symmetric", "asymmetric"), 8, 128),
    ((3, 4, 64, "asymmetric", "symmetric"), 4, 64),
    ((2, 3, 128, "symmetric", "symmetric"), 2, 128),
    ((4, 3, 32, "asymmetric", "asymmetric"), 1, 64),
])
def test_decode_attention_fused_formats(fmt, nrep, D):
    kbits, vbits, G, km, vm = fmt
    kseg = (16, 64 * 21, 80)
    vq = (64 * 21 + 80) // G * G - G
    vseg = (16, vq, 64 * 21 + 80 - vq)
    err = _decode_case(2, 2, nrep, D, kseg, vseg, (kbits, G, km), (vbits, G, vm), seed=kbits * G + nrep + vbits,
                       norm=True)
    assert err < TOL


# Windows attended after the fused kernel by the merging dense kernel: at the
# BASELINE decode shapes (groups of 32, D = 128, four query heads per KV head)
# with every store-mode instance of the fused kernel (asym, sym, mixed, hybrid
# V), key normalization, rows packed in only one of K and V (three sections)
# and windows of one chunk or two per section; then eight query heads per KV
# head with packed rows (two sections), and D = 64 (two token subgroups per
# wave in attn.V).
@pytest.mark.parametrize("kfmt,vfmt,kseg,vseg,norm,nrep,D", [
    ((2, 32, "asymmetric"), (4, 32, "asymmetric"), (0, 64 * 20, 128), (0, 64 * 20, 128), False, 4, 128),
    ((3, 32, "symmetric"), (3, 32, "symmetric"), (0, 64 * 20, 128), (0, 64 * 20, 128), False, 4, 128),
    ((3, 32, "symmetric"), (4, 32, "asymmetric"), (5, 64 * 12, 60), (5, 64 * 12, 60), False, 4, 128),
    ((3, 32, "symmetric"), (3, 32, "symmetric"), (32, 64 * 9 + 20, 76), (32, 64 * 9, 96), True, 4, 128),
    ((3, 32, "symmetric"), (2, 32, "hybrid"), (32, 64 * 9 + 20, 76), (32, 64 * 9, 96), True, 4, 128),
    ((4, 32, "asymmetric"), (4, 32, "asymmetric"), (7, 64 * 10, 193), (7, 64 * 10, 193), False, 4, 128),
    ((2, 32, "asymmetric"), (2, 32, "symmetric"), (32, 64 * 9 + 20, 150), (32, 64 * 9, 170), True, 4, 128),
    ((3, 32, "symmetric"), (3, 32, "symmetric"), (32, 64 * 9 + 20, 76), (32, 64 * 9, 96), True, 8, 128),
    ((4, 32, "asymmetric"), (4, 32, "asymmetric"), (16, 64 * 9 + 20, 120), (16, 64 * 9, 140), False, 2, 64),
    ((2, 32, "asymmetric"), (4, 32, "asymmetric"), (3, 64 * 8, 200), (3, 64 * 8, 200), False, 1, 64),
])
def test_decode_attention_window_formats(kfmt, vfmt, kseg, vseg, norm, nrep, D):
    print(f"window formats: K {kfmt} V {vfmt} segments {kseg} {vseg} norm={norm} nrep={nrep} D={D}", flush=True)
    err = _decode_case(2, 2, nrep, D, kseg, vseg, kfmt, vfmt, seed=sum(kseg) + kfmt[0] * 7 + vfmt[0] + nrep, norm=norm)
    assert err < TOL


@pytest.mark.parametrize("fused", [True, False])
def test_decode_stages_equal_decode_attention(fused):
    """iq_decode_attention_splits + _combine give decode_attention's output: bit for
    bit on the unfused path (different group sizes); with the fused kernel (K and
    V of one group size, here of different bit widths) decode_attention attends
    the 40-token window after the fused kernel and merges in the same kernel,
    whose window sections and softmax denominator are summed in another order
    than the combine's, so the two fp16 outputs agree to fp32 rounding that can
    cross an fp16 rounding boundary (a unit or two in the last place): within
    the decode tolerance, 1e-3 max-normwise."""
    B, Hkv, nrep, D = 2, 2, 4, 128
    kg, vg = (32, 32) if fused else (32, 64)
    T = 64 * 12 + 40
    kx = synth.kv_tensor(B, Hkv, T, D, seed=61)
    vx = synth.kv_tensor(B, Hkv, T, D, seed=62)
    kst = ops.PackedStore("channel", B, Hkv, D, kg, 2, "asymmetric", DEV)
    vst = ops.PackedStore("token", B, Hkv, D, vg, 4, "asymmetric", DEV)
    kst.append(f16t(kx[:, :, :768]))
    vst.append(f16t(vx[:, :, :768]))
    kr, vr = f16t(kx[:, :, 768:]), f16t(vx[:, :, 768:])
    q = f16t(synth.normal((B, Hkv * nrep, D), seed=63).astype(np.float16))
    ref = ops.decode_attention(q, None, kst, kr, None, vst, vr, D ** -0.5).cpu().numpy()
    ns = ops.decode_attention_splits(q, None, kst, kr, None, vst, vr, D ** -0.5)
    assert ns == 3 + 2  # three 256-token splits of the packed range + the 40 dense tokens in two slices
    got = ops.decode_attention_combine(ns, B, Hkv * nrep, T, D, DEV).cpu().numpy()
    if fused:
        assert A.rel_err(got.astype(np.float64), ref.astype(np.float64)) < TOL
    else:
        np.testing.assert_array_equal(got.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("kbits,vbits,R", [(4, 4, 0), (2, 4, 0), (4, 4, 128)])
def test_decode_live_stages_equal_decode_attention(kbits, vbits, R):
    """iq_decode_attention_splits_live + _combine_live against decode_attention and
    against fp32 attention over the library's dequantized K and V, at the headline
    shape (B=8, 32/8 heads, 32k tokens): the split stage launches the step's own
    fused kernel (live slots, the same grid: the 4/4-bit paired partition, the
    plain one for 2/4-bit).  The fused kernel's waves claim token blocks
    dynamically and round p to fp16 against their own running max, so two runs
    of it agree to that rounding (the decode tolerance, 1e-3), not bit for bit.
    With a 128-token window decode_attention merges it after the fused kernel,
    while the stages take dense slices and the combine."""
    B, Hkv, nrep, D, T, G = 8, 8, 4, 128, 32768, 32
    print(f"live stages: kbits={kbits} vbits={vbits} R={R}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(kbits * 10 + vbits + R)
    Tq = T - R
    kst = ops.PackedStore("channel", B, Hkv, D, G, kbits, "asymmetric", DEV, t_cap=Tq)
    vst = ops.PackedStore("token", B, Hkv, D, G, vbits, "asymmetric", DEV, t_cap=Tq)
    k = torch.randn(B, Hkv, T, D, generator=gen, device=DEV).to(torch.float16)
    v = torch.randn(B, Hkv, T, D, generator=gen, device=DEV).to(torch.float16)
    kst.append(k[:, :, :Tq])
    vst.append(v[:, :, :Tq])
    kr = k[:, :, Tq:] if R else None
    vr = v[:, :, Tq:] if R else None
    q = torch.randn(B, Hkv * nrep, D, generator=gen, device=DEV).to(torch.float16)
    kd = torch.cat([kst.dequant(dtype=torch.float32), k[:, :, Tq:].float()], dim=2)
    lg = torch.matmul(q.float().view(B, Hkv, nrep, D), kd.transpose(-1, -2).contiguous()) * D ** -0.5
    del kd
    vd = torch.cat([vst.dequant(dtype=torch.float32), v[:, :, Tq:].float()], dim=2)
    ref32 = torch.matmul(torch.softmax(lg, dim=-1), vd).view(B, Hkv * nrep, D)
    del vd, lg
    ref = ops.decode_attention(q, None, kst, kr, None, vst, vr, D ** -0.5)
    plan = ops.decode_attention_splits_live(q, None, kst, kr, None, vst, vr, D ** -0.5)
    assert plan.grid > 0 and plan.nsf == -(-Tq // 256) and plan.nrep == nrep
    assert plan.pair_e0 == (68 if kbits == vbits == 4 else 0)
    assert (plan.nsplit > plan.nsf) == (R > 0)  # the window's dense slices
    got = ops.decode_attention_combine_live(plan, B, Hkv * nrep, T, D, DEV)
    torch.cuda.synchronize()

    def err(a, b):
        return ((a.float() - b.float()).abs().max() / b.float().abs().max()).item()
    print(f"  vs decode_attention {err(got, ref):.2e}, vs fp32 {err(got, ref32):.2e}, "
          f"decode_attention vs fp32 {err(ref, ref32):.2e}", flush=True)
    assert err(got, ref32) < TOL and err(ref, ref32) < TOL and err(got, ref) < TOL
