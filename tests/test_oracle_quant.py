"""Pin the CPU oracle (oracle/quant_ref.py) against the live reference's golden
vectors, closed-form known answers, exhaustive fp16 checks and brute force."""
import hashlib

import numpy as np
import pytest

from oracle import quant_ref as Q


def _sha(a):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), dtype=np.uint8)


def _codes8(c):
    c = np.where(c == Q.INT32_MIN, -128, c)
    return c.astype(np.int8)


@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("mode", ["asym", "sym"])
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("G", [32, 64])
def test_quantize_matches_reference_golden(quant_golden, axis, mode, bits, G):
    g = quant_golden
    x = g["x"].view(np.float16)
    fn = getattr(Q, f"quantize_{axis}dim_{mode}")
    c, s, z = fn(x, G, bits)
    key = f"{axis}_{mode}_b{bits}_g{G}"
    np.testing.assert_array_equal(_codes8(c), g[key + "_codes"])
    np.testing.assert_array_equal(s.view(np.uint16), g[key + "_scale"])
    np.testing.assert_array_equal(z.view(np.uint16), g[key + ("_zero" if mode == "asym" else "_signs")])


@pytest.mark.parametrize("axis", ["channel", "token"])
def test_dequantize_matches_reference_golden(quant_golden, axis):
    x = quant_golden["x"].view(np.float16)
    c, s, z = getattr(Q, f"quantize_{axis}dim_asym")(x, 32, 4)
    d = getattr(Q, f"dequantize_{axis}dim_asym")(c, s, z, 32)
    np.testing.assert_array_equal(_sha(d.astype(np.float32)), quant_golden[f"{axis}_asym_b4_g32_deq_sha256"])
    c, s, sg = getattr(Q, f"quantize_{axis}dim_sym")(x, 32, 3)
    d = getattr(Q, f"dequantize_{axis}dim_sym")(c, s, sg, 32)
    np.testing.assert_array_equal(_sha(d.astype(np.float32)), quant_golden[f"{axis}_sym_b3_g32_deq_sha256"])


@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_hybrid_matches_reference_golden(quant_golden, axis, bits):
    x = quant_golden["x"].view(np.float16)
    qf = getattr(Q, f"quantize_{axis}dim_hybrid")
    df = getattr(Q, f"dequantize_{axis}dim_hybrid")
    c, s, z = qf(x, 32, bits)
    key = f"{axis}_hybrid_b{bits}_g32"
    np.testing.assert_array_equal(s["mask"], quant_golden[key + "_mask"])
    assert 0 < s["mask"].mean() < 1  # both representations occur in the fixture
    d = df(c, s, z, 32).astype(np.float32)
    np.testing.assert_array_equal(_sha(d), quant_golden[key + "_deq_sha256"])
    np.testing.assert_array_equal(_sha(d + np.float32(0.0)), quant_golden[key + "_deq_pz_sha256"])


@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_hybrid_exact_ties_keep_asym(hybrid_ties, axis, bits):
    """Groups whose two L1 errors tie exactly (every term and sum exact in fp32,
    so every summation order agrees): the reference's strict comparison
    (quant.py:144) keeps the asym codes, and so does the oracle."""
    x = hybrid_ties[f"{axis}_b{bits}_x"].view(np.float16)
    _, s, _ = getattr(Q, f"quantize_{axis}dim_hybrid")(x, 32, bits)
    want = hybrid_ties[f"{axis}_b{bits}_mask"]
    assert not want.any()
    np.testing.assert_array_equal(s["mask"], want)


def test_config0_digests(quant_golden):
    """Config 0: [1,8,4096,128] 4-bit asym G=32, K along D, V along T."""
    from innerq_amd import synth
    k0 = synth.kv_tensor(1, 8, 4096, 128, seed=0, n_out=4, factor=10.0)
    v0 = synth.kv_tensor(1, 8, 4096, 128, seed=1, n_out=4, factor=10.0)
    for name, t, fn in (("k", k0, Q.quantize_channeldim_asym), ("v", v0, Q.quantize_tokendim_asym)):
        c, s, z = fn(t, 32, 4)
        for part, arr in (("codes", c.astype(np.int32)), ("scale", s.view(np.uint16)), ("zero", z.view(np.uint16))):
            np.testing.assert_array_equal(_sha(arr), quant_golden[f"cfg0_{name}_{part}_sha256"], err_msg=f"{name} {part}")


def test_division_paths_agree_exhaustively():
    """x/L == x*(1/L) after fp16 rounding for every finite fp16 x (CPU vs CUDA torch paths)."""
    x = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16)
    for L in (1, 3, 7, 15):
        a = (x.astype(np.float32) / np.float32(L)).astype(np.float16)
        b = (x.astype(np.float32) * (np.float32(1) / np.float32(L))).astype(np.float16)
        c = (x.astype(np.float64) / L).astype(np.float16)
        np.testing.assert_array_equal(a.view(np.uint16), b.view(np.uint16))
        np.testing.assert_array_equal(a.view(np.uint16), c.view(np.uint16))


def test_closed_form_ramp_4bit():
    x = (np.arange(32) % 16).astype(np.float16).reshape(1, 1, 1, 32)
    c, s, z = Q.quantize_channeldim_asym(x, 32, 4)
    assert s.item() == 1.0 and z.item() == 0.0
    np.testing.assert_array_equal(c.ravel(), np.arange(32) % 16)


def test_closed_form_benchmark_pattern():
    """speedtest/benchmark_quantization.cu:427-444 host pattern x = i%4 - 2."""
    x = (np.arange(32) % 4 - 2).astype(np.float16).reshape(1, 1, 1, 32)
    c, s, z = Q.quantize_channeldim_asym(x, 32, 2)
    assert s.item() == 1.0 and z.item() == -2.0
    np.testing.assert_array_equal(c.ravel(), np.arange(32) % 4)
    c, s, sg = Q.quantize_channeldim_sym(x, 32, 2)
    # |x|/2 in {1, .5, 0, .5} -> half-to-even -> {1, 0, 0, 0}
    assert s.item() == 2.0
    np.testing.assert_array_equal(c.ravel(), np.tile([1, 0, 0, 0], 8))
    np.testing.assert_array_equal(sg.ravel(), np.tile([-1, -1, 0, 1], 8).astype(np.float16))


def test_constant_group_is_nan_int_min():
    x = np.full((1, 1, 1, 32), 0.75, np.float16)
    c, s, z = Q.quantize_channeldim_asym(x, 32, 4)
    assert s.item() == 0.0 and np.all(c == Q.INT32_MIN)
    assert np.all(Q.stored_codes(c, 4) == 0)
    d = Q.dequantize_channeldim_asym(np.zeros_like(c), s, z, 32)
    assert np.all(d == np.float32(0.75))


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_invariants_random(bits):
    from innerq_amd import synth
    x = synth.kv_tensor(2, 3, 64, 128, seed=bits, n_out=3, factor=10.0)
    c, s, z = Q.quantize_channeldim_asym(x, 32, bits)
    L = 2 ** bits - 1
    assert c.min() >= 0 and c.max() <= L
    g = x.reshape(2, 3, 64, 4, 32).astype(np.float32)
    cg = c.reshape(2, 3, 64, 4, 32)
    # min maps to 0, max maps to L
    np.testing.assert_array_equal(cg[np.arange(2)[:, None, None, None], np.arange(3)[None, :, None, None],
                                     np.arange(64)[None, None, :, None], np.arange(4)[None, None, None, :],
                                     g.argmin(-1)], 0)
    assert np.all(cg.max(-1) == L)
    d = Q.dequantize_channeldim_asym(c, s, z, 32).reshape(g.shape)
    err = np.abs(d - g)
    # half a step plus the fp16 rounding of (x - mn) and of the scale
    bound = s.astype(np.float32)[..., None] * 0.5 + np.abs(g) * 2 ** -10 + 2 ** -14
    assert np.all(err <= bound + np.abs(g - z.astype(np.float32)[..., None]) * 2 ** -10)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("G", [32, 64, 128])
def test_pack_unpack_bijection(bits, G):
    """every value at every lane position survives pack -> unpack; fields do not overlap"""
    vals = np.arange(1 << bits, dtype=np.uint32)
    for v in vals:
        for pos in range(G):
            f = np.zeros((1, G), np.uint32)
            f[0, pos] = v
            w = Q.pack_groups(f, bits)
            assert int(sum(bin(int(x)).count("1") for x in w.ravel())) == bin(int(v)).count("1")
            np.testing.assert_array_equal(Q.unpack_groups(w, bits, G), f.astype(np.int32))
    rng = np.random.default_rng(bits * 1000 + G)
    f = rng.integers(0, 1 << bits, size=(50, G), dtype=np.uint32)
    np.testing.assert_array_equal(Q.unpack_groups(Q.pack_groups(f, bits), bits, G), f.astype(np.int32))


def test_pack_3bit_straddle_positions():
    """codes 10 and 21 straddle words 0/1 and 1/2 (bits 30..32 and 63..65)"""
    f = np.zeros((1, 32), np.uint32)
    f[0, 10] = 0b101
    f[0, 21] = 0b011
    w = Q.pack_groups(f, 3)[0]
    assert w[0] == (0b01 << 30) and w[1] == (0b1 | (0b1 << 31)) and w[2] == 0b01
    # sym: offset binary (u = signed + 4 at 3 bits), straddling fields included
    f = np.zeros((1, 32), np.int64)
    f[0, 10] = -3
    f[0, 21] = 3
    wp = Q.pack_groups((f + 4).astype(np.uint32), 3)
    w = wp[0]
    assert w[0] >> 30 == 0b01 and w[1] & 1 == 0 and (w[1] >> 31, w[2] & 3) == (1, 0b11)
    np.testing.assert_array_equal(Q.unpack_groups(wp, 3, 32, signed=True)[0], f[0])
    np.testing.assert_array_equal(Q.stored_codes(np.abs(f), 3, np.sign(f)), (f + 4).astype(np.uint32))


@pytest.mark.parametrize("mode", ["asymmetric", "symmetric"])
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_store_layout_roundtrip(mode, bits):
    from innerq_amd import synth
    x = synth.kv_tensor(2, 2, 96, 128, seed=7, n_out=2, factor=10.0)
    if mode == "asymmetric":
        c, s, z = Q.quantize_channeldim_asym(x, 32, bits)
        cw, meta = Q.build_k_store(c, s, z, bits, 32, mode)
        c2, s2, z2 = Q.k_store_to_codes(cw, meta, 96, bits, 32, mode)
        np.testing.assert_array_equal(c2, c)
        np.testing.assert_array_equal(z2.view(np.uint16), z.view(np.uint16))
    else:
        c, s, sg = Q.quantize_channeldim_sym(x, 32, bits)
        cw, meta = Q.build_k_store(c, s, sg, bits, 32, mode)
        c2, s2, z2 = Q.k_store_to_codes(cw, meta, 96, bits, 32, mode)
        np.testing.assert_array_equal(c2, c * sg.astype(np.int64))
        assert z2 is None
    np.testing.assert_array_equal(s2.view(np.uint16), s.view(np.uint16))
    assert cw.shape == (2, 2, 2, 4, 64, bits)
    # V
    if mode == "asymmetric":
        c, s, z = Q.quantize_tokendim_asym(x, 32, bits)
        cw, meta = Q.build_v_store(c, s, z, bits, 32, mode)
        c2, s2, z2 = Q.v_store_to_codes(cw, meta, 96, bits, 32, mode)
        np.testing.assert_array_equal(c2, c)
    else:
        c, s, sg = Q.quantize_tokendim_sym(x, 32, bits)
        cw, meta = Q.build_v_store(c, s, sg, bits, 32, mode)
        c2, s2, z2 = Q.v_store_to_codes(cw, meta, 96, bits, 32, mode)
        np.testing.assert_array_equal(c2, c * sg.astype(np.int64))
    np.testing.assert_array_equal(s2.view(np.uint16), s.view(np.uint16))


def test_qmode_from_str():
    assert Q.qmode_from_str(" Asymmetric ") == "asymmetric"
    with pytest.raises(ValueError):
        Q.qmode_from_str("asym")
