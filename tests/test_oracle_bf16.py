"""Pin the oracle's bf16 path (oracle/quant_ref.py with act="bf16") against the
live reference run on bf16 tensors (tests/golden/bf16_golden.npz: quant.py on
the quant_golden input cast to bf16), and check that the fp16 rounding rule
does not pass for it (the bf16 fixture tells the two apart)."""
import hashlib
import os

import numpy as np
import pytest

from oracle import quant_ref as Q

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "bf16_golden.npz")


@pytest.fixture(scope="module")
def g():
    return np.load(GOLDEN)


def _sha(a):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), dtype=np.uint8)


def _codes8(c):
    return np.where(c == Q.INT32_MIN, -128, c).astype(np.int8)


def _x(g):
    return Q.bf16_from_bits(g["x"]).reshape(1, 2, 64, 128)


def test_bf16_rounding_known_answers():
    # ties to even at the bf16 ulp, overflow, NaN, the largest finite value
    one_ulp = np.float32(2.0 ** -7)
    assert Q.round_bf16(np.float32(1.0) + one_ulp / 2) == np.float32(1.0)            # tie -> even (down)
    assert Q.round_bf16(np.float32(1.0) + 3 * one_ulp / 2) == np.float32(1.0) + 2 * one_ulp  # tie -> even (up)
    assert Q.round_bf16(np.float32(1.0) + one_ulp * 0.51) == np.float32(1.0) + one_ulp
    assert np.isinf(Q.round_bf16(np.float32(3.4e38)))
    assert Q.bf16_bits(np.float32(np.nan)) == 0x7FC0
    assert Q.bf16_bits(Q.bf16_from_bits(np.uint16(0x7F7F))) == 0x7F7F


@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("mode", ["asym", "sym"])
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("G", [32, 64])
def test_bf16_quantize_matches_reference_golden(g, axis, mode, bits, G):
    c, s, z = getattr(Q, f"quantize_{axis}dim_{mode}")(_x(g), G, bits, act="bf16")
    key = f"{axis}_{mode}_b{bits}_g{G}"
    np.testing.assert_array_equal(_codes8(c), g[key + "_codes"])
    np.testing.assert_array_equal(Q.bf16_bits(s), g[key + "_scale"])
    np.testing.assert_array_equal(Q.bf16_bits(z), g[key + ("_zero" if mode == "asym" else "_signs")])


@pytest.mark.parametrize("axis", ["channel", "token"])
def test_bf16_fixture_rejects_fp16_rounding(g, axis):
    # the same input quantized with fp16 rounding (the planted mistake) misses
    # the bf16 reference: some scale differs
    c, s, z = getattr(Q, f"quantize_{axis}dim_asym")(_x(g), 32, 4, act="f16")
    assert not np.array_equal(Q.bf16_bits(s.astype(np.float32)), g[f"{axis}_asym_b4_g32_scale"])


@pytest.mark.parametrize("axis", ["channel", "token"])
def test_bf16_dequantize_matches_reference_golden(g, axis):
    x = _x(g)
    c, s, z = getattr(Q, f"quantize_{axis}dim_asym")(x, 32, 4, act="bf16")
    d = getattr(Q, f"dequantize_{axis}dim_asym")(c, s, z, 32)
    np.testing.assert_array_equal(_sha(d.astype(np.float32)), g[f"{axis}_asym_b4_g32_deq_sha256"])
    c, s, sg = getattr(Q, f"quantize_{axis}dim_sym")(x, 32, 3, act="bf16")
    d = getattr(Q, f"dequantize_{axis}dim_sym")(c, s, sg, 32)
    np.testing.assert_array_equal(_sha(d.astype(np.float32) + np.float32(0.0)),
                                  g[f"{axis}_sym_b3_g32_deq_pz_sha256"])


@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_bf16_hybrid_matches_reference_golden(g, axis, bits):
    c, s, z = getattr(Q, f"quantize_{axis}dim_hybrid")(_x(g), 32, bits, act="bf16")
    key = f"{axis}_hybrid_b{bits}_g32"
    np.testing.assert_array_equal(s["mask"], g[key + "_mask"])
    d = getattr(Q, f"dequantize_{axis}dim_hybrid")(c, s, z, 32).astype(np.float32)
    np.testing.assert_array_equal(_sha(d + np.float32(0.0)), g[key + "_deq_pz_sha256"])
