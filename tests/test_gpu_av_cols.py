"""GPU parity of the attn.V GEMV's column-slice path (iq_av_gemv where its
B * Hkv * D/32 workgroups fill the device: one workgroup per (batch, KV head,
32 output columns) over the whole token range, no split-T partials, no
combine launch), through the C ABI.

References: fp32 p @ V over V dequantized by the library (PackedStore.dequant,
bit-exact to the oracle in test_gpu_kernels / test_hybrid_store) for every
head, and the float64 oracle (quantize -> dequantize -> p @ V) for the whole
output at a smaller token count.  Bar: 1e-3 in the max-relative metric
max|got - ref| / max|ref| (the decode GEMV tolerance).  The split-T path (the
same data in a store of fewer heads, which does not fill the device) gives
the same result to fp32 summation order.
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


def _err(got, ref):
    return ((got.double() - ref.double()).abs().max() / ref.double().abs().max()).item()


def _case(B, Hkv, nrep, D, T, G, bits, mode, seed, t0=0):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(B, Hkv, t0 + T, D, generator=gen, device=DEV)
    x[..., :: max(1, D // 4)] *= 8.0  # outlier channels
    x = x.to(torch.float16)
    st = ops.PackedStore("token", B, Hkv, D, G, bits, mode, DEV, t_cap=t0 + T)
    st.append(x)
    p = torch.softmax(torch.randn(B, Hkv * nrep, T, generator=gen, device=DEV) * 2.0, dim=-1).to(torch.float16)
    vd = st.dequant(dtype=torch.float32)[:, :, t0:]
    ref = torch.matmul(p.float().view(B, Hkv, nrep, T), vd).view(B, Hkv * nrep, D)
    return st, p, ref


# every (bits, group, mode) at 4 query heads per KV head; an odd group count
# leaves the last wave step partly past the range
@pytest.mark.parametrize("mode", ["asymmetric", "symmetric", "hybrid"])
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("G", [32, 64, 128])
def test_av_cols_parity(mode, bits, G):
    B, Hkv, nrep, D = 8, 8, 4, 128
    T = 7 * G
    print(f"av cols: bits={bits} G={G} mode={mode} B={B} Hkv={Hkv} T={T}", flush=True)
    st, p, ref = _case(B, Hkv, nrep, D, T, G, bits, mode, seed=bits * 100 + G)
    got = ops.av_gemv(p, st, out32=torch.empty(B, Hkv * nrep, D, device=DEV))
    assert _err(got, ref) < TOL


# query heads per KV head and head_dim (D = 64: two slices per head)
@pytest.mark.parametrize("nrep,D,G,bits", [(1, 128, 64, 2), (2, 128, 32, 4), (8, 128, 64, 2), (8, 128, 128, 4),
                                           (8, 128, 128, 3), (4, 64, 32, 3), (8, 64, 64, 4), (1, 64, 32, 2)])
def test_av_cols_shapes(nrep, D, G, bits):
    Hkv = 8
    B = 8 if D == 128 else 16
    T = 4096 + 3 * G
    print(f"av cols shapes: nrep={nrep} D={D} G={G} bits={bits} B={B}", flush=True)
    st, p, ref = _case(B, Hkv, nrep, D, T, G, bits, "asymmetric", seed=nrep * D + G)
    got = ops.av_gemv(p, st, out32=torch.empty(B, Hkv * nrep, D, device=DEV))
    assert _err(got, ref) < TOL


def test_av_cols_offset_range_and_accumulate():
    """A range that starts inside the store (t0), fp32 accumulate and the fp16
    output together, on strided probabilities (a 16-byte aligned slice)."""
    B, Hkv, nrep, D, G, T, t0 = 8, 8, 4, 128, 64, 64 * 37, 128
    st, p, ref = _case(B, Hkv, nrep, D, T, G, 2, "asymmetric", seed=5, t0=t0)
    wide = torch.zeros(B, Hkv * nrep, T + 64, dtype=torch.float16, device=DEV)
    wide[:, :, 64:] = p
    pv = wide[:, :, 64:]
    o32 = torch.ones(B, Hkv * nrep, D, device=DEV)
    o16 = torch.empty(B, Hkv * nrep, D, dtype=torch.float16, device=DEV)
    ops.av_gemv(pv, st, t0=t0, T=T, out=o16, out32=o32, accumulate=True)
    assert _err(o32, ref + 1.0) < TOL
    assert _err(o16.float(), ref + 1.0) < 2e-3


def test_av_cols_unaligned_probabilities_take_the_split_path():
    """Probability rows that are not 16-byte aligned are not read by the column
    kernel; the call still gives the right result (the split-T path)."""
    B, Hkv, nrep, D, G, T = 8, 8, 4, 128, 32, 32 * 40
    st, p, ref = _case(B, Hkv, nrep, D, T, G, 4, "symmetric", seed=6)
    wide = torch.zeros(B, Hkv * nrep, T + 1, dtype=torch.float16, device=DEV)
    wide[:, :, 1:] = p
    got = ops.av_gemv(wide[:, :, 1:], st, out32=torch.empty(B, Hkv * nrep, D, device=DEV))
    assert _err(got, ref) < TOL


def test_av_cols_equals_split_path():
    """The same two sequences through the column path (a store of 8 sequences)
    and through the split-T path (a store of just those 2): equal to fp32
    summation order."""
    B, Hkv, nrep, D, G, T = 8, 8, 4, 128, 64, 8192
    st, p, ref = _case(B, Hkv, nrep, D, T, G, 2, "asymmetric", seed=7)
    got = ops.av_gemv(p, st, out32=torch.empty(B, Hkv * nrep, D, device=DEV))
    gen = torch.Generator(device=DEV).manual_seed(7)
    x = torch.randn(B, Hkv, T, D, generator=gen, device=DEV)
    x[..., :: D // 4] *= 8.0
    x = x.to(torch.float16)
    small = ops.PackedStore("token", 2, Hkv, D, G, 2, "asymmetric", DEV, t_cap=T)
    small.append(x[:2].contiguous())
    part = ops.av_gemv(p[:2].contiguous(), small, out32=torch.empty(2, Hkv * nrep, D, device=DEV))
    assert _err(got[:2], part) < 1e-5
    assert _err(got, ref) < TOL


def test_av_cols_oracle():
    """End to end against the float64 oracle: the oracle's quantization (bit-exact
    to the store's), dequantization and p @ V."""
    B, Hkv, nrep, D, G, T, bits = 8, 8, 4, 128, 64, 64 * 9, 2
    x = synth.kv_tensor(B, Hkv, T, D, seed=11, n_out=4, factor=10.0)
    st = ops.PackedStore("token", B, Hkv, D, G, bits, "asymmetric", DEV)
    st.append(torch.from_numpy(x).to(DEV))
    c, s, z = Q.quantize_tokendim_asym(x, G, bits)
    vdeq = Q.dequantize_tokendim_asym(c, s, z, G)
    logits = synth.normal((B, Hkv * nrep, T), seed=12, std=2.0).astype(np.float64)
    p = A.softmax(logits).astype(np.float16)
    got = ops.av_gemv(torch.from_numpy(p).to(DEV), st).cpu().numpy().astype(np.float64)
    assert A.rel_err(got, A.av_out(p, vdeq)) < TOL
