"""The reference's cache presets (innerq_base, innerq_small, innerq_hybrid;
scripts/run_lmeval.sh:94-153) at the config-4 shape on the GPU, through the
drop-in cache: a layer prefilled with 32k tokens (32 fp16 sinks, 32640 packed,
96 recent per role), then three decode steps of append() (the new token joins
the windows, K flushes its oldest token, V its oldest 32 each step until its
window drains to 3) and attend() over [sinks | packed | windows].  That step
runs the fused kernel's key-normalized instances (hi/lo query rows) over 3-bit
sym K and 3-bit sym / 2-bit sym / 2-bit hybrid V, and the merging dense kernel
over a window whose V rows are partly packed.  "hybrid_k" is innerq_hybrid with
3-bit hybrid K as well (key_quantize_mode='hybrid', which the reference accepts,
cache.py:92-98, and no preset uses).

References:
* every head: fp32 attention over the layer's fp32 [sink | dequantized (times
  the key normalization factor) | recent] K and V (get_keys_deq /
  get_values_deq, the reference's read path cache.py:235-276);
* three sampled (batch, KV head)s end to end through the numpy cache oracle
  (oracle.cache_ref.CacheLayerRef fed the same tokens: its quantization,
  dequantization and state machine) and float64 attention: the layer's
  dequantized keys and values bit-exact to the oracle's (up to the sign of
  zero), the attention output within 1e-3 (max-normwise).
"""
import numpy as np
import pytest
import torch

from innerq_amd import cache as C
from innerq_amd import presets
from oracle import attn_ref as A
from oracle import cache_ref as CR

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-3


def _np(t):
    return t.detach().cpu().numpy()


def _err(got, ref):
    return ((got.double() - ref.double()).abs().max() / ref.double().abs().max()).item()


def _config(name):
    """A preset's config; "hybrid_k": innerq_hybrid with hybrid keys as well
    (key_quantize_mode='hybrid', cache.py:92-98; no reference preset uses it)."""
    if name == "hybrid_k":
        return presets.preset_config("innerq_hybrid", key_quantize_mode="hybrid")
    return presets.preset_config(name)


@pytest.mark.parametrize("name", ["innerq_base", "innerq_small", "innerq_hybrid", "hybrid_k"])
def test_preset_decode_full_size(name):
    B, Hkv, nrep, T, D, steps = 8, 8, 4, 32768, 128, 3
    print(f"preset {name}: B={B} Hkv={Hkv} T={T}", flush=True)
    cfg = _config(name)
    gen = torch.Generator(device=DEV).manual_seed(sum(map(ord, name)))

    def kv(n):
        x = torch.randn(B, Hkv, n, D, generator=gen, device=DEV)
        x[..., :: D // 4] *= 8.0
        return x.to(torch.float16)

    k, v = kv(T + steps), kv(T + steps)
    q = torch.randn(B, Hkv * nrep, 1, D, generator=gen, device=DEV).to(torch.float16)
    layer = C.InnerqDynamicLayer(cfg, 0)
    layer.update(k[:, :, :T], v[:, :, :T])
    for i in range(steps):
        layer.append(k[:, :, T + i:T + i + 1], v[:, :, T + i:T + i + 1])
    assert layer._kq.length == T - 128 + steps and layer.keys_recent.shape[2] == 96
    assert layer._vq.length == T + steps - 32 - 3 and layer.values_recent.shape[2] == 3
    assert layer.fused_decode_ready(k[:, :, :1])
    got = layer.attend(q, D ** -0.5)[:, :, 0]
    torch.cuda.synchronize()

    K = layer.get_keys_deq()
    lg = torch.matmul(q[:, :, 0].float().view(B, Hkv, nrep, D), K.transpose(-1, -2).contiguous()) * D ** -0.5
    kdev = K
    del K
    pr = torch.softmax(lg, dim=-1)
    del lg
    V = layer.get_values_deq()
    ref = torch.matmul(pr, V).view(B, Hkv * nrep, D)
    del pr
    err = _err(got.float(), ref)
    print(f"  every head vs fp32 attention over the layer's dequantization: {err:.2e}", flush=True)
    assert err < TOL

    for b, h in ((0, 0), (3, 5), (7, 7)):
        ref_layer = CR.CacheLayerRef(cfg)
        ref_layer.update(_np(k[b:b + 1, h:h + 1, :T]), _np(v[b:b + 1, h:h + 1, :T]))
        for i in range(steps):
            ref_layer.update(_np(k[b:b + 1, h:h + 1, T + i:T + i + 1]), _np(v[b:b + 1, h:h + 1, T + i:T + i + 1]))
        kd = np.concatenate([ref_layer.keys_sink.astype(np.float32),
                             ref_layer.kdq(*ref_layer.keys_q, 32) * ref_layer.norm.astype(np.float32),
                             ref_layer.keys_recent.astype(np.float32)], axis=2)
        vd = np.concatenate([ref_layer.values_sink.astype(np.float32),
                             ref_layer.vdq(*ref_layer.values_q, 32),
                             ref_layer.values_recent.astype(np.float32)], axis=2)
        # the layer's read path equals the oracle's values (-0.0 and +0.0 alike)
        np.testing.assert_array_equal(_np(kdev[b:b + 1, h:h + 1]) + np.float32(0), kd + np.float32(0))
        np.testing.assert_array_equal(_np(V[b:b + 1, h:h + 1]) + np.float32(0), vd + np.float32(0))
        qh = _np(q[b:b + 1, h * nrep:(h + 1) * nrep, 0])
        o = A.decode_attention(qh, kd, vd, D ** -0.5, p_dtype=None)
        e = A.rel_err(_np(got[b:b + 1, h * nrep:(h + 1) * nrep]).astype(np.float64), o)
        print(f"  head ({b}, {h}) vs the oracle: {e:.2e}", flush=True)
        assert e < TOL


@pytest.mark.parametrize("name", ["innerq_base", "innerq_hybrid", "hybrid_k"])
def test_preset_decode_full_size_bf16(name):
    """The same decode step of a bf16 layer (the model in bf16, LongBench/pred.py:240):
    every head against fp32 attention over the layer's fp32 dequantized K and V
    (the bf16 read path is pinned to the reference's by tests/test_gpu_bf16.py);
    the output is the bf16 rounding of the fp32 result, so the bar is 1e-3
    max-normwise beyond that rounding (2^-8 |ref| elementwise)."""
    B, Hkv, nrep, T, D, steps = 8, 8, 4, 32768, 128, 3
    print(f"preset {name} bf16: B={B} Hkv={Hkv} T={T}", flush=True)
    cfg = _config(name)
    gen = torch.Generator(device=DEV).manual_seed(7 + sum(map(ord, name)))

    def kv(n):
        x = torch.randn(B, Hkv, n, D, generator=gen, device=DEV)
        x[..., :: D // 4] *= 8.0
        return x.to(torch.bfloat16)

    k, v = kv(T + steps), kv(T + steps)
    q = torch.randn(B, Hkv * nrep, 1, D, generator=gen, device=DEV).to(torch.bfloat16)
    layer = C.InnerqDynamicLayer(cfg, 0)
    layer.update(k[:, :, :T], v[:, :, :T])
    for i in range(steps):
        layer.append(k[:, :, T + i:T + i + 1], v[:, :, T + i:T + i + 1])
    got = layer.attend(q, D ** -0.5)[:, :, 0]
    assert got.dtype == torch.bfloat16
    K = layer.get_keys_deq()
    lg = torch.matmul(q[:, :, 0].float().view(B, Hkv, nrep, D), K.transpose(-1, -2).contiguous()) * D ** -0.5
    del K
    pr = torch.softmax(lg, dim=-1)
    del lg
    ref = torch.matmul(pr, layer.get_values_deq()).view(B, Hkv * nrep, D)
    g, r = got.double(), ref.double()
    excess = ((g - r).abs() - 2.0 ** -8 * r.abs()).max().item() / r.abs().max().item()
    print(f"  max-normwise {((g - r).abs().max() / r.abs().max()).item():.2e}, beyond the bf16 rounding "
          f"{excess:.2e}", flush=True)
    assert excess <= TOL
