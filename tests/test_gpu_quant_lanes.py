"""The two K quantizers agree bit for bit: one lane per value (quant_k_lane_kernel
and the window append's group items, used for calls of at most 65,536 groups:
a decode step's tokens) and one thread per group (quant_k_kernel, larger calls:
a prompt).  Same tokens quantized in one large call and in small calls, on
inputs with the groups where the two could part: signed zeros at the minimum,
constant groups (scale 0, NaN codes), NaN and infinity, exact rounding ties,
fp16 subnormals.  The small calls are also checked against the oracle in
test_gpu_kernels (random data)."""
import numpy as np
import pytest
import torch

from innerq_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
N_TOK = 4160  # 8 heads x 4160 tokens: > 65,536 groups of 32 and of 64 -> one thread per group
CHUNK = 64    # 8 x 64 x (128 / G) groups -> one lane per value


def adversarial(H, T, D, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((1, H, T, D)).astype(np.float32)
    x[0, 0, 0, :] = np.where(np.arange(D) % 2 == 0, 0.0, -0.0)       # zeros of both signs only
    x[0, 0, 1, :] = 1.5                                               # constant groups
    x[0, 0, 2, 5] = np.nan                                            # NaN in group 0
    x[0, 0, 2, 40] = np.inf                                           # infinity in group 1
    x[0, 0, 3, :32] = np.arange(32) % 16 + 0.5                        # ties at 4-bit scale 1
    x[0, 0, 3, 32:64] = (np.arange(32) % 4) - 2                       # the 2-bit tie pattern
    x[0, 0, 4, :] = np.abs(x[0, 0, 4, :])
    x[0, 0, 4, ::7] = -0.0                                            # minimum -0 among positives
    x[0, 0, 5, :] = -0.0                                              # negative zeros only
    x[0, 0, 6, :] = rng.standard_normal(D) * 1e-6                     # fp16 subnormals
    x[0, 1, 7, :] = np.where(np.arange(D) % 3 == 0, -0.0, 0.0) + (np.arange(D) % 5 == 0) * 2.0
    return x.astype(np.float16)


def store_bytes(st):
    n = st.length // 64
    bh = st.B * st.H
    return (st.codes.view(bh, st.t_cap // 64, -1)[:, :n].cpu().numpy(),
            st.meta.view(bh, st.t_cap // 64, -1)[:, :n].cpu().numpy())


@pytest.mark.parametrize("mode,bits", [("asymmetric", 1), ("asymmetric", 2), ("asymmetric", 3), ("asymmetric", 4),
                                       ("symmetric", 2), ("symmetric", 3), ("symmetric", 4)])
@pytest.mark.parametrize("G", [32, 64])
@pytest.mark.parametrize("norm", [False, True])
def test_lane_and_thread_quantizers_agree(mode, bits, G, norm):
    H, D = 8, 128
    x = torch.from_numpy(adversarial(H, N_TOK, D, seed=bits * G)).to(DEV)
    nf = ops.key_norm_factor(x[:, :, 8:200]) if norm else None
    big = ops.PackedStore("channel", 1, H, D, G, bits, mode, DEV)
    big.append(x, norm=nf)
    small = ops.PackedStore("channel", 1, H, D, G, bits, mode, DEV)
    for t in range(0, N_TOK, CHUNK):
        small.append(x[:, :, t:t + CHUNK], norm=nf)
    bc, bm = store_bytes(big)
    sc, sm = store_bytes(small)
    np.testing.assert_array_equal(sc, bc)
    np.testing.assert_array_equal(sm, bm)


@pytest.mark.parametrize("mode", ["asymmetric", "symmetric"])
@pytest.mark.parametrize("bits,G", [(2, 32), (3, 64), (4, 32)])
def test_lane_and_thread_reference_outputs_agree(mode, bits, G):
    # quant.py-format outputs (codes, scale, zero | signs) of a small call equal
    # the same rows of a large call
    x = torch.from_numpy(adversarial(8, N_TOK, 128, seed=7 * bits + G)).to(DEV)
    cb, sb, zb = ops.quantize_dense(x, G, bits, mode, "channel")
    cs, ss, zs = ops.quantize_dense(x[:, :, :CHUNK].contiguous(), G, bits, mode, "channel")
    assert torch.equal(cs, cb[:, :, :CHUNK])
    assert torch.equal(ss.view(torch.int16), sb[:, :, :CHUNK].contiguous().view(torch.int16))
    assert torch.equal(zs.view(torch.int16), zb[:, :, :CHUNK].contiguous().view(torch.int16))
