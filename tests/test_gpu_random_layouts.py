"""Seeded random layouts through the drop-in cache and the decode entry point,
each against float64 attention over the layer's own dequantized K and V
(get_keys_deq / get_values_deq, bit-exact to the oracle elsewhere): bit
widths, modes (asym / sym / hybrid for either role), groups, head_dim,
query heads per KV head, sinks, windows, flush sizes, key normalization,
fp16 and bf16, left padding, sliding windows with the fix, and K and V of
different group sizes (the unfused path).  Each case prints its layout first.
Tolerance: 1e-3 max-normwise (fp16); bf16 outputs add their own rounding
(2^-8)."""
import random

import numpy as np
import pytest
import torch

from innerq_amd import cache as C
from innerq_amd import ops
from oracle import attn_ref as A

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


class Cfg:
    def __init__(self, **kw):
        self.__dict__.update(kw)


def _check(layer, q, D, pads, s0, tol):
    B = q.shape[0]
    out = layer.attend(q, D ** -0.5, pads)[:, :, 0].float().cpu().numpy().astype(np.float64)
    K = layer.get_keys_deq().float().cpu().numpy()[:, :, s0:]
    V = layer.get_values_deq().float().cpu().numpy()[:, :, s0:]
    qn = q[:, :, 0].float().cpu().numpy()
    for b in range(B):
        p = pads[b] if pads else 0
        ref = A.decode_attention(qn[b:b + 1], K[b:b + 1, :, p:], V[b:b + 1, :, p:], D ** -0.5, None)
        e = A.rel_err(out[b:b + 1], ref)
        assert e < tol, f"sequence {b}: {e:.2e}"


@pytest.mark.parametrize("case", range(24))
def test_random_cache_layout(case):
    rng = random.Random(1000 + case)
    D = rng.choice([64, 128])
    G = rng.choice([g for g in (32, 64, 128) if g <= D])
    vf = rng.choice([G, 2 * G])
    cfg = Cfg(k_bits=rng.choice([2, 3, 4]), v_bits=rng.choice([2, 3, 4]), key_flush_size=rng.choice([1, 1, 32]),
              value_flush_size=vf, key_group_size=G, value_group_size=G, key_w_recent=rng.choice([0, 16, 96, 130]),
              value_w_recent=rng.choice([vf, vf + 40, max(vf, 200)]), key_w_sink=rng.choice([0, 4, 32]),
              value_w_sink=rng.choice([0, 4, 32]), key_normalize=rng.random() < 0.5, key_quantize_over_token=False,
              value_quantize_over_token=True, key_quantize_mode=rng.choice(["asymmetric", "symmetric", "hybrid"]),
              value_quantize_mode=rng.choice(["asymmetric", "symmetric", "hybrid"]))
    B, Hkv, nrep = rng.choice([1, 2, 3]), rng.choice([1, 2, 4]), rng.choice([1, 2, 4, 8])
    dtype = torch.bfloat16 if rng.random() < 0.2 else torch.float16
    prefill, steps = rng.choice([1, 50, 300, 700, 1500]), rng.choice([1, 5, 40])
    print(f"case {case}: B={B} Hkv={Hkv} nrep={nrep} D={D} {dtype} T={prefill}+{steps} {cfg.__dict__}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(case)
    kx = torch.randn(B, Hkv, prefill + steps, D, generator=gen, device=DEV)
    vx = torch.randn(B, Hkv, prefill + steps, D, generator=gen, device=DEV)
    kx[..., ::max(1, D // 8)] *= 6.0
    vx[..., :20] += 3.0
    kx, vx = kx.to(dtype), vx.to(dtype)
    layer = C.InnerqDynamicLayer(cfg, 0)
    layer.update(kx[:, :, :prefill], vx[:, :, :prefill])
    for s in range(steps):
        layer.append(kx[:, :, prefill + s:prefill + s + 1], vx[:, :, prefill + s:prefill + s + 1])
    assert layer._fused_refusal() is None
    q = torch.randn(B, Hkv * nrep, 1, D, generator=gen, device=DEV).to(dtype)
    n = layer.attend_length()
    pads = [rng.randrange(0, max(1, n // 2)) for _ in range(B)] if B > 1 and rng.random() < 0.4 else None
    _check(layer, q, D, pads, 0, 1e-3 if dtype == torch.float16 else 1e-3 + 2.0 ** -8)


@pytest.mark.parametrize("case", range(12))
def test_random_sliding_layout(case):
    rng = random.Random(2000 + case)
    D, G = rng.choice([64, 128]), 32
    w = rng.choice([40, 64, 100, 300])
    cfg = Cfg(k_bits=rng.choice([2, 3, 4]), v_bits=rng.choice([2, 3, 4]), key_flush_size=1, value_flush_size=32,
              key_group_size=G, value_group_size=G, key_w_recent=rng.choice([16, 32]),
              value_w_recent=rng.choice([32, 64]), key_w_sink=rng.choice([0, 4]), value_w_sink=rng.choice([0, 4]),
              key_normalize=rng.random() < 0.5, key_quantize_over_token=False, value_quantize_over_token=True,
              key_quantize_mode=rng.choice(["asymmetric", "symmetric"]),
              value_quantize_mode=rng.choice(["asymmetric", "symmetric", "hybrid"]), fix_sliding_window=True)
    B, Hkv, nrep = rng.choice([1, 2, 3]), rng.choice([1, 2]), rng.choice([1, 4])
    prefill, steps = rng.choice([20, 80, 400]), rng.choice([1, 30, 120])
    print(f"case {case}: w={w} B={B} Hkv={Hkv} nrep={nrep} D={D} T={prefill}+{steps} {cfg.__dict__}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(100 + case)
    kx = torch.randn(B, Hkv, prefill + steps, D, generator=gen, device=DEV).half()
    vx = torch.randn(B, Hkv, prefill + steps, D, generator=gen, device=DEV).half()
    layer = C.InnerqDynamicSlidingWindowLayer(cfg, 0, w)
    layer.update(kx[:, :, :prefill], vx[:, :, :prefill])
    for s in range(steps):
        layer.append(kx[:, :, prefill + s:prefill + s + 1], vx[:, :, prefill + s:prefill + s + 1])
    n = layer.attend_length()
    pads = [rng.randrange(0, n) for _ in range(B)] if B > 1 and rng.random() < 0.5 else None
    q = torch.randn(B, Hkv * nrep, 1, D, generator=gen, device=DEV).half()
    _check(layer, q, D, pads, layer._attend_start(), 1e-3)


@pytest.mark.parametrize("case", range(12))
def test_random_unfused_layout(case):
    """K and V of different group sizes: the unfused split kernels, with random
    sink / packed / recent lengths."""
    rng = random.Random(3000 + case)
    D = rng.choice([64, 128])
    gk, gv = rng.sample([32, 64, 128], 2) if D == 128 else rng.sample([32, 64], 2)
    B, Hkv, nrep = rng.choice([1, 2]), rng.choice([1, 2, 4]), rng.choice([1, 2, 4, 8])
    ns, nr = rng.choice([0, 3, 32]), rng.choice([0, 5, 64])
    nq = 64 * max(gk, gv) // 32 * rng.choice([1, 3, 9])
    T = ns + nq + nr
    kb, vb = rng.choice([2, 3, 4]), rng.choice([2, 3, 4])
    km, vm = rng.choice(["asymmetric", "symmetric"]), rng.choice(["asymmetric", "symmetric", "hybrid"])
    print(f"case {case}: D={D} gk={gk} gv={gv} B={B} Hkv={Hkv} nrep={nrep} sink={ns} packed={nq} recent={nr} "
          f"K{kb} {km} V{vb} {vm}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(500 + case)
    kx = torch.randn(B, Hkv, T, D, generator=gen, device=DEV).half()
    vx = torch.randn(B, Hkv, T, D, generator=gen, device=DEV).half()
    kst = ops.PackedStore("channel", B, Hkv, D, gk, kb, km, DEV)
    kst.append(kx[:, :, ns:ns + nq])
    vst = ops.PackedStore("token", B, Hkv, D, gv, vb, vm, DEV)
    vst.append(vx[:, :, ns:ns + nq])
    q = torch.randn(B, Hkv * nrep, D, generator=gen, device=DEV).half()
    out = ops.decode_attention(q, kx[:, :, :ns] if ns else None, kst, kx[:, :, ns + nq:] if nr else None,
                               vx[:, :, :ns] if ns else None, vst, vx[:, :, ns + nq:] if nr else None, D ** -0.5)
    K = torch.cat([kx[:, :, :ns].float(), kst.dequant(dtype=torch.float32), kx[:, :, ns + nq:].float()], dim=2)
    V = torch.cat([vx[:, :, :ns].float(), vst.dequant(dtype=torch.float32), vx[:, :, ns + nq:].float()], dim=2)
    ref = A.decode_attention(q.float().cpu().numpy(), K.cpu().numpy(), V.cpu().numpy(), D ** -0.5, None)
    assert A.rel_err(out.float().cpu().numpy().astype(np.float64), ref) < 1e-3
