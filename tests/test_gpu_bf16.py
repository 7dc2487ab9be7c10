"""bf16 activations through the drop-in (a bf16 model's cache, as LongBench/pred.py:240
loads the InnerQ model): quant.py's functions, packed stores and the cache layer
on bf16 tensors against the live reference run on the same bf16 tensors
(tests/golden/bf16_golden.npz) and the bf16 oracle pinned to it.

Codes, bf16 scales, zero points and signs bit-exact; dequantized values and the
K / V that update() returns at every step of two reference traces value-exact
(-0.0 read as +0.0, which a packed sym field does not keep).

The decode path on bf16 layers (attend(), decode_attention) against fp32
attention over the layer's fp32 dequantized K and V (get_keys_deq /
get_values_deq, pinned to the reference by the traces here) or the stores'
dequant(): the kernels compute in fp32 and round the output once to bf16, so
the bar is |got - ref| <= 1e-3 max|ref| + 2^-8 |ref| elementwise (the decode
tolerance plus that rounding).  The GEMVs take fp16 stores only."""
import hashlib
import os

import numpy as np
import pytest
import torch

from innerq_amd import cache as C
from innerq_amd import ops
from innerq_amd import quant as IQ
from innerq_amd import synth
from oracle import quant_ref as Q
from tests.test_oracle_cache import PRESETS, Cfg

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "bf16_golden.npz")


@pytest.fixture(scope="module")
def g():
    return np.load(GOLDEN)


def _sha(a):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), dtype=np.uint8)


def _codes8(c):
    return np.where(c == Q.INT32_MIN, -128, c).astype(np.int8)


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _x(g):
    u = torch.from_numpy(g["x"].astype(np.int16)).view(torch.bfloat16).reshape(1, 2, 64, 128)
    return u.to(DEV)


@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("mode", ["asym", "sym"])
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("G", [32, 64])
def test_bf16_quantize_api_matches_reference(g, axis, mode, bits, G):
    c, s, z = getattr(IQ, f"quantize_{axis}dim_{mode}")(_x(g), G, bits)
    assert s.dtype == torch.bfloat16 and z.dtype == torch.bfloat16
    key = f"{axis}_{mode}_b{bits}_g{G}"
    np.testing.assert_array_equal(_codes8(c.cpu().numpy()), g[key + "_codes"])
    np.testing.assert_array_equal(_bits(s), g[key + "_scale"])
    np.testing.assert_array_equal(_bits(z), g[key + ("_zero" if mode == "asym" else "_signs")])


@pytest.mark.parametrize("axis", ["channel", "token"])
def test_bf16_dequantize_api_matches_reference(g, axis):
    x = _x(g)
    c, s, z = getattr(IQ, f"quantize_{axis}dim_asym")(x, 32, 4)
    d = getattr(IQ, f"dequantize_{axis}dim_asym")(c, s, z, 32)
    np.testing.assert_array_equal(_sha(d.cpu().numpy()), g[f"{axis}_asym_b4_g32_deq_sha256"])
    c, s, sg = getattr(IQ, f"quantize_{axis}dim_sym")(x, 32, 3)
    d = getattr(IQ, f"dequantize_{axis}dim_sym")(c, s, sg, 32)
    np.testing.assert_array_equal(_sha(d.cpu().numpy() + np.float32(0.0)), g[f"{axis}_sym_b3_g32_deq_pz_sha256"])
    # op_dtype bf16: one bf16 rounding per op, as torch computes it
    d16 = getattr(IQ, f"dequantize_{axis}dim_sym")(c, s, sg, 32, op_dtype=torch.bfloat16)
    ref = (c.cpu().to(torch.bfloat16) * (s.cpu().repeat_interleave(32, dim=-1 if axis == "channel" else -2))
           * sg.cpu())
    assert torch.equal(d16.cpu(), ref)


@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_bf16_hybrid_api_matches_reference(g, axis, bits):
    qa, qs = getattr(IQ, f"quantize_{axis}dim_asym"), getattr(IQ, f"quantize_{axis}dim_sym")
    da, ds = getattr(IQ, f"dequantize_{axis}dim_asym"), getattr(IQ, f"dequantize_{axis}dim_sym")
    c, s, z = IQ.quantize_hybrid(qa, qs, da, ds)(_x(g), 32, bits)
    key = f"{axis}_hybrid_b{bits}_g32"
    np.testing.assert_array_equal(s["mask"].cpu().numpy(), g[key + "_mask"])
    d = IQ.dequantize_hybrid(da, ds)(c, s, z, 32)
    np.testing.assert_array_equal(_sha(d.cpu().numpy() + np.float32(0.0)), g[key + "_deq_pz_sha256"])


@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("mode", ["asymmetric", "symmetric", "hybrid"])
@pytest.mark.parametrize("bits,G", [(2, 32), (3, 64), (4, 128), (3, 32)])
def test_bf16_store_round_trip_matches_oracle(axis, mode, bits, G):
    # packed stores of bf16 tokens: appended in two calls (lane and thread
    # kernels alike), unpacked to quant.py's tensors and dequantized, against
    # the bf16 oracle
    B, H, T, D = 2, 3, 256, 128
    x = synth.kv_tensor(B, H, T, D, seed=bits * G + len(mode), n_out=3, factor=8.0).astype(np.float32)
    x[0, 0, 3, :] = 0.0                       # constant groups
    xb = Q.round_bf16(x)
    xt = torch.from_numpy(xb).to(torch.bfloat16).to(DEV)
    st = ops.PackedStore(axis, B, H, D, G, bits, mode, DEV, dtype=torch.bfloat16)
    st.append(xt[:, :, :128])
    st.append(xt[:, :, 128:])
    qf = getattr(Q, f"quantize_{axis}dim_{ {'asymmetric': 'asym', 'symmetric': 'sym', 'hybrid': 'hybrid'}[mode] }")
    dq = getattr(Q, f"dequantize_{axis}dim_{ {'asymmetric': 'asym', 'symmetric': 'sym', 'hybrid': 'hybrid'}[mode] }")
    rc, rs, rz = qf(xb, G, bits, act="bf16")
    ref = dq(rc, rs, rz, G).astype(np.float32)
    got = st.dequant(dtype=torch.float32).cpu().numpy()
    np.testing.assert_array_equal(got, ref)
    got16 = st.dequant().cpu()
    assert got16.dtype == torch.bfloat16
    assert torch.equal(got16, torch.from_numpy(ref).to(torch.bfloat16))
    if mode != "hybrid":
        c, s, z = ops.unpack_store(st)
        rcz = np.where(rc == Q.INT32_MIN, 0, rc)   # a NaN code (constant group) is stored as field 0
        np.testing.assert_array_equal(c.cpu().numpy(), np.abs(rcz))
        np.testing.assert_array_equal(_bits(s), Q.bf16_bits(rs))
        if mode == "asymmetric":
            np.testing.assert_array_equal(_bits(z), Q.bf16_bits(rz))
    # the wire format keeps the dtype
    back = ops.PackedStore.from_bytes(st.to_bytes(), DEV)
    assert back.dtype == torch.bfloat16
    assert torch.equal(back.dequant(dtype=torch.float32), st.dequant(dtype=torch.float32))


def test_bf16_key_norm_factor():
    k = torch.from_numpy(Q.round_bf16(synth.kv_tensor(2, 3, 100, 64, seed=5, n_out=2, factor=9.0))).to(
        torch.bfloat16).to(DEV)
    f = ops.key_norm_factor(k)
    assert f.dtype == torch.bfloat16
    ref = Q.round_bf16(np.sqrt(np.abs(k.float().cpu().numpy()).max(axis=2, keepdims=True)))
    np.testing.assert_array_equal(f.float().cpu().numpy(), ref)


BF16_PRESETS = ("innerq_base", "hybrid_v")


@pytest.mark.parametrize("name", BF16_PRESETS)
def test_bf16_cache_update_matches_reference_trace(g, name):
    """update() on bf16 K/V returns the reference's K and V at every step (values;
    bf16 throughout), with the reference's recent-window lengths."""
    seed, B, H, D, prefill, steps = (int(v) for v in g[f"{name}_seed"])
    kx = synth.kv_tensor(B, H, prefill + steps, D, seed=seed, n_out=2, factor=8.0)
    vx = synth.kv_tensor(B, H, prefill + steps, D, seed=seed + 1, n_out=2, factor=8.0)
    kt = torch.from_numpy(kx).to(torch.bfloat16).to(DEV)
    vt = torch.from_numpy(vx).to(torch.bfloat16).to(DEV)
    layer = C.InnerqDynamicLayer(Cfg(**PRESETS[name]), 0)

    def pz(K, V):
        return _sha(np.concatenate([K.float().cpu().numpy().ravel(), V.float().cpu().numpy().ravel()])
                    + np.float32(0.0))

    K, V = layer.update(kt[:, :, :prefill].clone(), vt[:, :, :prefill].clone())
    np.testing.assert_array_equal(pz(K, V), g[f"{name}_step0_pz_sha256"])
    for s in range(steps):
        K, V = layer.update(kt[:, :, prefill + s:prefill + s + 1].clone(), vt[:, :, prefill + s:prefill + s + 1].clone())
        assert K.dtype == torch.bfloat16 and V.dtype == torch.bfloat16
        np.testing.assert_array_equal(pz(K, V), g[f"{name}_step{s + 1}_pz_sha256"], err_msg=f"step {s + 1}")
        assert (K.shape[-2], V.shape[-2], layer.keys_recent.shape[-2], layer.values_recent.shape[-2]) == \
            tuple(g[f"{name}_len{s + 1}"])
    last_k = torch.from_numpy(g[f"{name}_step{steps}_k"].astype(np.int16)).view(torch.bfloat16)
    assert torch.equal(K.cpu().float(), last_k.reshape(K.shape).float())
    assert layer.fused_decode_ready(kt[:, :, :1])   # bf16 layers decode on the fused path too


def test_gemvs_refuse_bf16_stores_and_mixed_dtypes():
    st = ops.PackedStore("channel", 1, 2, 64, 32, 4, "asymmetric", DEV, dtype=torch.bfloat16)
    st.append(torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16, device=DEV))
    q = torch.zeros(1, 2, 64, dtype=torch.float16, device=DEV)
    with pytest.raises(TypeError):
        ops.qk_gemv(q, st, 0.125)
    vs = ops.PackedStore("token", 1, 2, 64, 32, 4, "asymmetric", DEV, dtype=torch.bfloat16)
    vs.append(torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(TypeError):   # an fp16 query over bf16 stores
        ops.decode_attention(q, None, st, None, None, vs, None, 0.125)
    with pytest.raises(TypeError):   # fp16 tokens into a bf16 store
        st.append(torch.zeros(1, 2, 64, 64, dtype=torch.float16, device=DEV))
    with pytest.raises(ops._lib.IQError):  # the split stage alone cannot tell its combine the output's dtype
        ops.decode_attention_splits(q.bfloat16(), None, st, None, None, vs, None, 0.125)


def _check_bf16(got, ref, what=""):
    g, r = got.double(), ref.double()
    excess = ((g - r).abs() - 2.0 ** -8 * r.abs()).max().item() / r.abs().max().item()
    print(f"  {what}: max-normwise {((g - r).abs().max() / r.abs().max()).item():.2e}, "
          f"beyond the bf16 rounding {excess:.2e}", flush=True)
    assert excess <= 1e-3


def _attn32(q, K, V, scale):
    B, Hq, D = q.shape
    Hkv = K.shape[1]
    lg = torch.matmul(q.float().view(B, Hkv, Hq // Hkv, D), K.float().transpose(-1, -2).contiguous()) * scale
    return torch.matmul(torch.softmax(lg, dim=-1), V.float()).view(B, Hq, D)


@pytest.mark.parametrize("name", BF16_PRESETS + ("asym4_nosink", "mixed_k2v4_flush32"))
def test_bf16_attend_every_decode_step(name):
    """A bf16 layer decodes through attend() (the fused kernel over the packed
    range, the merging dense kernel over sinks and windows) at every step of 40
    decode steps after a 300-token prefill, across V flushes."""
    B, H, nrep, D, prefill, steps = 2, 2, 4, 128, 300, 40
    kt = torch.from_numpy(synth.kv_tensor(B, H, prefill + steps, D, seed=81, n_out=2, factor=8.0)).to(
        torch.bfloat16).to(DEV)
    vt = torch.from_numpy(synth.kv_tensor(B, H, prefill + steps, D, seed=82, n_out=2, factor=8.0)).to(
        torch.bfloat16).to(DEV)
    q = torch.randn(B, H * nrep, 1, D, generator=torch.Generator(device=DEV).manual_seed(83), device=DEV).to(
        torch.bfloat16)
    layer = C.InnerqDynamicLayer(Cfg(**PRESETS[name]), 0)
    layer.update(kt[:, :, :prefill], vt[:, :, :prefill])
    print(f"bf16 attend: {name}", flush=True)
    for s in range(steps):
        tok = slice(prefill + s, prefill + s + 1)
        assert layer.fused_decode_ready(kt[:, :, tok])
        layer.append(kt[:, :, tok], vt[:, :, tok])
        got = layer.attend(q, D ** -0.5)[:, :, 0]
        assert got.dtype == torch.bfloat16
        ref = _attn32(q[:, :, 0], layer.get_keys_deq(), layer.get_values_deq(), D ** -0.5)
        if s % 13 == 0 or s == steps - 1:
            _check_bf16(got, ref, f"step {s + 1}")
        else:
            g, r = got.double(), ref.double()
            assert ((g - r).abs() - 2.0 ** -8 * r.abs()).max().item() <= 1e-3 * r.abs().max().item()


# (K bits, V bits, group, K mode, V mode, key normalization) x (query heads per KV head, head_dim),
# groups no wider than head_dim
_BF16_FMTS = [(4, 4, 32, "asymmetric", "asymmetric", False), (3, 3, 32, "symmetric", "symmetric", True),
              (2, 4, 64, "asymmetric", "symmetric", False), (3, 2, 32, "symmetric", "hybrid", True),
              (4, 3, 128, "symmetric", "asymmetric", True)]


@pytest.mark.parametrize("fmt,nrep,D", [(f, r, d) for f in _BF16_FMTS for r, d in ((4, 128), (8, 64), (1, 128))
                                        if f[2] <= d])
def test_bf16_decode_attention_formats(fmt, nrep, D):
    """decode_attention on bf16 stores with bf16 sinks and recent windows, over K / V
    formats, GQA ratios and head_dim, against fp32 attention over the stores'
    dequantization (bit-exact to the bf16 oracle: test_bf16_store_round_trip_*)."""
    kb, vb, G, km, vm, norm = fmt
    B, Hkv, ns, nq, nr = 2, 2, 16, 64 * 20, 48
    gen = torch.Generator(device=DEV).manual_seed(kb * 10 + vb + G + nrep)

    def x(n):
        t = torch.randn(B, Hkv, n, D, generator=gen, device=DEV)
        t[..., ::D // 4] *= 6.0
        return t.to(torch.bfloat16)

    k, v = x(ns + nq + nr), x(ns + nq + nr)
    q = torch.randn(B, Hkv * nrep, D, generator=gen, device=DEV).to(torch.bfloat16)
    f = ops.key_norm_factor(k[:, :, ns:ns + nq]) if norm else None
    kst = ops.PackedStore("channel", B, Hkv, D, G, kb, km, DEV, dtype=torch.bfloat16)
    vst = ops.PackedStore("token", B, Hkv, D, G, vb, vm, DEV, dtype=torch.bfloat16)
    kst.append(k[:, :, ns:ns + nq], norm=f)
    vst.append(v[:, :, ns:ns + nq])
    got = ops.decode_attention(q, k[:, :, :ns], kst, k[:, :, ns + nq:], v[:, :, :ns], vst, v[:, :, ns + nq:],
                               D ** -0.5, norm=f)
    kd = kst.dequant(dtype=torch.float32, norm=f)
    K = torch.cat([k[:, :, :ns].float(), kd, k[:, :, ns + nq:].float()], dim=2)
    V = torch.cat([v[:, :, :ns].float(), vst.dequant(dtype=torch.float32), v[:, :, ns + nq:].float()], dim=2)
    _check_bf16(got, _attn32(q, K, V, D ** -0.5), f"fmt {fmt} nrep {nrep} D {D}")


def test_bf16_decode_attention_oracle():
    """End to end through the bf16 oracle: its quantization of the bf16 tokens
    (bit-exact to the store's), its dequantization and float64 attention."""
    from oracle import attn_ref as A
    B, Hkv, nrep, D, G, T = 2, 2, 4, 128, 32, 64 * 12
    kx = Q.round_bf16(synth.kv_tensor(B, Hkv, T, D, seed=91, n_out=2, factor=8.0))
    vx = Q.round_bf16(synth.kv_tensor(B, Hkv, T, D, seed=92, n_out=2, factor=8.0))
    qx = Q.round_bf16(synth.normal((B, Hkv * nrep, D), seed=93))
    bf = lambda a: torch.from_numpy(a).to(torch.bfloat16).to(DEV)  # noqa: E731
    kst = ops.PackedStore("channel", B, Hkv, D, G, 3, "symmetric", DEV, dtype=torch.bfloat16)
    vst = ops.PackedStore("token", B, Hkv, D, G, 4, "asymmetric", DEV, dtype=torch.bfloat16)
    kst.append(bf(kx))
    vst.append(bf(vx))
    got = ops.decode_attention(bf(qx), None, kst, None, None, vst, None, D ** -0.5)
    kd = Q.dequantize_channeldim_sym(*Q.quantize_channeldim_sym(kx, G, 3, act="bf16"), G)
    vd = Q.dequantize_tokendim_asym(*Q.quantize_tokendim_asym(vx, G, 4, act="bf16"), G)
    ref = A.decode_attention(qx, kd, vd, D ** -0.5, p_dtype=None)
    _check_bf16(got.float().cpu(), torch.from_numpy(ref), "oracle")


def test_bf16_llama_generates_through_the_drop_in(monkeypatch):
    """A random 2-layer Llama loaded in bf16 (as LongBench/pred.py:240 loads the
    InnerQ model) generates on the hook's cache: every layer quantizes bf16 K/V,
    the registered fused attention hands the prefill to sdpa and every decode
    step to attend() on the packed cache, and the step scores match the eager
    reference path on the same cache type within bf16 tolerance."""
    from transformers import LlamaConfig
    from innerq_amd.models import InnerqLlamaForCausalLM
    cfg = LlamaConfig(num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2, hidden_size=512,
                      intermediate_size=256, vocab_size=64, max_position_embeddings=512)
    for k, v in PRESETS["innerq_base"].items():
        setattr(cfg, k, v)
    torch.manual_seed(0)
    model = InnerqLlamaForCausalLM(cfg).to(device=DEV, dtype=torch.bfloat16).eval()
    calls = [0]
    orig = C.InnerqDynamicLayer.attend

    def attend(self, *a, **kw):
        calls[0] += 1
        return orig(self, *a, **kw)

    monkeypatch.setattr(C.InnerqDynamicLayer, "attend", attend)
    ids = torch.randint(0, 64, (1, 150), generator=torch.Generator(device=DEV).manual_seed(3), device=DEV)
    outs = {}
    for attn in ("eager", "innerq_fused"):
        model.config._attn_implementation = attn
        with torch.no_grad():
            outs[attn] = model.generate(ids, max_new_tokens=6, do_sample=False, output_scores=True,
                                        return_dict_in_generate=True)
        assert outs[attn].sequences.shape == (1, 156)
    ref = torch.stack(outs["eager"].scores).float()
    got = torch.stack(outs["innerq_fused"].scores).float()
    assert ((got - ref).abs().max() / ref.abs().max()).item() < 3e-2
    assert calls[0] == 2 * 5  # two layers, five decode steps after the prefill's token
