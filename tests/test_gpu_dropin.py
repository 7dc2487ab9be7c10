"""GPU parity of the drop-in API (innerq_amd.quant / innerq_amd.cache) against
the live reference's golden fixtures (tests/golden/*.npz).

quant: codes, scales, zero points, signs, dequantized values and hybrid masks
bit-exact.  cache: the fp16 K and V that update() returns at every step of the
reference traces bit-exact (SHA-256 per step), and the recent-window lengths
equal.  attend(): the fused decode attention over the packed cache within 1e-3
(max-relative) of float64 attention over update()'s dense K and V.
"""
import hashlib

import numpy as np
import pytest
import torch

from innerq_amd import cache as C
from innerq_amd import quant as IQ
from innerq_amd import synth
from oracle import attn_ref as A
from oracle import quant_ref as Q
from tests.test_oracle_cache import AXES_PRESETS, PRESETS, Cfg, golden_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _sha(a):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), dtype=np.uint8)


def _codes8(c):
    c = np.where(c == Q.INT32_MIN, -128, c)
    return c.astype(np.int8)


def _x(g):
    return torch.from_numpy(g["x"].view(np.float16).copy()).to(DEV)


@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("mode", ["asym", "sym"])
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("G", [32, 64])
def test_quantize_api_matches_reference(quant_golden, axis, mode, bits, G):
    g = quant_golden
    c, s, z = getattr(IQ, f"quantize_{axis}dim_{mode}")(_x(g), G, bits)
    assert c.dtype == torch.int32 and s.dtype == torch.float16 and z.dtype == torch.float16
    key = f"{axis}_{mode}_b{bits}_g{G}"
    np.testing.assert_array_equal(_codes8(c.cpu().numpy()), g[key + "_codes"])
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint16), g[key + "_scale"])
    np.testing.assert_array_equal(z.cpu().numpy().view(np.uint16), g[key + ("_zero" if mode == "asym" else "_signs")])


@pytest.mark.parametrize("axis", ["channel", "token"])
def test_dequantize_api_matches_reference(quant_golden, axis):
    g = quant_golden
    x = _x(g)
    c, s, z = getattr(IQ, f"quantize_{axis}dim_asym")(x, 32, 4)
    d = getattr(IQ, f"dequantize_{axis}dim_asym")(c, s, z, 32)
    assert d.dtype == torch.float32
    np.testing.assert_array_equal(_sha(d.cpu().numpy()), g[f"{axis}_asym_b4_g32_deq_sha256"])
    c, s, sg = getattr(IQ, f"quantize_{axis}dim_sym")(x, 32, 3)
    d = getattr(IQ, f"dequantize_{axis}dim_sym")(c, s, sg, 32)
    np.testing.assert_array_equal(_sha(d.cpu().numpy()), g[f"{axis}_sym_b3_g32_deq_sha256"])


@pytest.mark.parametrize("axis", ["channel", "token"])
@pytest.mark.parametrize("bits", [3, 4])
def test_hybrid_api_matches_reference(quant_golden, axis, bits):
    g = quant_golden
    qa, qs = getattr(IQ, f"quantize_{axis}dim_asym"), getattr(IQ, f"quantize_{axis}dim_sym")
    da, ds = getattr(IQ, f"dequantize_{axis}dim_asym"), getattr(IQ, f"dequantize_{axis}dim_sym")
    c, s, z = IQ.quantize_hybrid(qa, qs, da, ds)(_x(g), 32, bits)
    key = f"{axis}_hybrid_b{bits}_g32"
    assert set(c) == {"zp", "nozp"} and set(s) == {"zp", "nozp", "mask"} and set(z) == {"zp", "nozp"}
    np.testing.assert_array_equal(s["mask"].cpu().numpy(), g[key + "_mask"])
    d = IQ.dequantize_hybrid(da, ds)(c, s, z, 32)
    np.testing.assert_array_equal(_sha(d.cpu().numpy()), g[key + "_deq_sha256"])


def test_quant_api_errors():
    x = torch.zeros(1, 2, 64, 96, dtype=torch.float16, device=DEV)
    with pytest.raises(AssertionError):        # 96 % 64 != 0, as quant.py:61
        IQ.quantize_channeldim_asym(x, 64, 4)
    with pytest.raises(ValueError):
        IQ.quantize_channeldim_asym(x, 32, 5)
    with pytest.raises(TypeError):
        IQ.quantize_channeldim_asym(x.float(), 32, 4)


def _sha16(k, v):
    return _sha(np.concatenate([k.view(np.uint16).ravel(), v.view(np.uint16).ravel()]))


def _np(t):
    return t.cpu().numpy()


@pytest.mark.parametrize("name", list(PRESETS))
def test_cache_update_matches_reference_trace(cache_golden, name):
    """update() returns the reference's K and V at every step: equal values to the
    oracle's (pinned bit-exact to the reference traces) and to the reference's
    last-step arrays.  Values, not bits: the packed sym format does not keep the
    sign of a zero code, so the reference's -0.0 comes back as +0.0."""
    _check_update_trace(cache_golden, name, PRESETS[name])


@pytest.mark.parametrize("name", list(AXES_PRESETS))
def test_cache_update_matches_axes_trace(axes_golden, name):
    """The same with keys grouped along tokens and values along head_dim (the
    KIVI presets, scripts/run_lmeval.sh:54-93; sym keys with hybrid values):
    token-axis K stores flushed 32 tokens at a time, channel-axis V stores one
    token at a time.  These layers decode through update()'s dense K/V (the
    fused attend() reads K grouped along head_dim only and says so)."""
    _check_update_trace(axes_golden, name, AXES_PRESETS[name])
    layer = C.InnerqDynamicLayer(Cfg(**AXES_PRESETS[name]), 0)
    x = torch.zeros(1, 2, 200, 64, dtype=torch.float16, device=DEV)
    layer.update(x, x)
    assert not layer.fused_decode_ready(x[:, :, :1])
    with pytest.raises(NotImplementedError):
        layer.attend(torch.zeros(1, 2, 1, 64, dtype=torch.float16, device=DEV), 0.125)


def _check_update_trace(g, name, cfg):
    from oracle import cache_ref
    kx, vx, prefill, steps = golden_inputs(g, name)
    kt, vt = torch.from_numpy(kx).to(DEV), torch.from_numpy(vx).to(DEV)
    layer = C.InnerqDynamicLayer(Cfg(**cfg), 0)
    ref = cache_ref.CacheLayerRef(Cfg(**cfg))
    K, V = layer.update(kt[:, :, :prefill].clone(), vt[:, :, :prefill].clone())
    Kr, Vr = ref.update(kx[:, :, :prefill], vx[:, :, :prefill])
    np.testing.assert_array_equal(_sha16(_np(K), _np(V)), g[f"{name}_step0_sha256"])
    for s in range(steps):
        K, V = layer.update(kt[:, :, prefill + s:prefill + s + 1].clone(), vt[:, :, prefill + s:prefill + s + 1].clone())
        Kr, Vr = ref.update(kx[:, :, prefill + s:prefill + s + 1], vx[:, :, prefill + s:prefill + s + 1])
        k, v = _np(K), _np(V)
        assert k.dtype == np.float16 and v.dtype == np.float16
        np.testing.assert_array_equal(k, Kr, err_msg=f"K step {s + 1}")
        np.testing.assert_array_equal(v, Vr, err_msg=f"V step {s + 1}")
        if s == steps - 1:
            np.testing.assert_array_equal(k, g[f"{name}_step{s + 1}_k"].view(np.float16))
            np.testing.assert_array_equal(v, g[f"{name}_step{s + 1}_v"].view(np.float16))
        assert (k.shape[-2], v.shape[-2], layer.keys_recent.shape[-2], layer.values_recent.shape[-2]) == \
            tuple(g[f"{name}_len{s + 1}"])
    assert layer.get_seq_length() == prefill + steps


@pytest.mark.parametrize("name", list(PRESETS))
@pytest.mark.parametrize("nrep", [1, 4])
def test_cache_attend_matches_dense_attention(cache_golden, name, nrep):
    """append() + attend() (fused, packed) within 1e-3 of float64 attention over the
    fp32 dequantize-then-matmul K and V (get_keys_deq / get_values_deq, cache.py:235-271)."""
    g = cache_golden
    kx, vx, prefill, steps = golden_inputs(g, name)
    kt, vt = torch.from_numpy(kx).to(DEV), torch.from_numpy(vx).to(DEV)
    layer = C.InnerqDynamicLayer(Cfg(**PRESETS[name]), 0)
    layer.append(kt[:, :, :prefill].clone(), vt[:, :, :prefill].clone())
    B, H, _, D = kx.shape
    for s in range(steps):
        layer.append(kt[:, :, prefill + s:prefill + s + 1].clone(), vt[:, :, prefill + s:prefill + s + 1].clone())
        if s % 23 == 5 or s == steps - 1:
            q = synth.normal((B, H * nrep, D), seed=s + 7 * nrep).astype(np.float16)
            out = layer.attend(torch.from_numpy(q).to(DEV)[:, :, None], D ** -0.5)
            assert out.shape == (B, H * nrep, 1, D) and out.dtype == torch.float16
            K, V = layer.get_keys_deq(), layer.get_values_deq()
            ref = A.decode_attention(q, _np(K.float()), _np(V.float()), D ** -0.5, None)
            assert A.rel_err(_np(out[:, :, 0]).astype(np.float64), ref) < 1e-3, f"step {s + 1}"


@pytest.mark.parametrize("name", ["innerq_base", "innerq_hybrid"])
@pytest.mark.parametrize("pads", [(0, 37, 300, 0), (5, 5, 700, 690)])
@pytest.mark.parametrize("norm", [True, False])
def test_cache_attend_with_padding(name, pads, norm):
    """attend() with a padding mask's hidden prefix per sequence (left padding):
    sequence b attends to tokens [pads[b], T) only, the batch split into runs of
    one start (one decode call each, over batch views of the stores); starts in
    the sinks, the packed range and the recent window.  Each sequence within 1e-3
    of float64 attention over its own tokens of the layer's dequantized K and V."""
    from innerq_amd import presets
    B, H, nrep, D, T = 4, 2, 4, 128, 760
    layer = C.InnerqDynamicLayer(presets.preset_config(name, key_normalize=norm), 0)
    kx = synth.kv_tensor(B, H, T + 3, D, seed=61, n_out=4, factor=8.0)
    vx = synth.kv_tensor(B, H, T + 3, D, seed=62, n_out=4, factor=8.0)
    kt, vt = torch.from_numpy(kx).to(DEV), torch.from_numpy(vx).to(DEV)
    layer.update(kt[:, :, :T], vt[:, :, :T])
    for i in range(3):
        layer.append(kt[:, :, T + i:T + i + 1], vt[:, :, T + i:T + i + 1])
    q = synth.normal((B, H * nrep, D), seed=63).astype(np.float16)
    out = layer.attend(torch.from_numpy(q).to(DEV)[:, :, None], D ** -0.5, pads=list(pads))[:, :, 0]
    K, V = _np(layer.get_keys_deq().float()), _np(layer.get_values_deq().float())
    for b, p in enumerate(pads):
        ref = A.decode_attention(q[b:b + 1], K[b:b + 1, :, p:], V[b:b + 1, :, p:], D ** -0.5, None)
        assert A.rel_err(_np(out[b:b + 1]).astype(np.float64), ref) < 1e-3, f"sequence {b}, pad {p}"
    with pytest.raises(ValueError):
        layer.attend(torch.from_numpy(q).to(DEV)[:, :, None], D ** -0.5, pads=[0, 0, 0, T + 3])


def test_cache_state_views_match_quantizer():
    """keys_q / keys_scale_factor / keys_zp_sign and values_* unpack to quant.py's tensors."""
    cfg = Cfg(k_bits=4, v_bits=3, key_flush_size=1, value_flush_size=64, key_group_size=32, value_group_size=64,
              key_w_recent=8, value_w_recent=64, key_quantize_mode="asymmetric", value_quantize_mode="symmetric")
    kx = synth.kv_tensor(1, 2, 200, 64, seed=3, n_out=2, factor=8.0)
    vx = synth.kv_tensor(1, 2, 200, 64, seed=4, n_out=2, factor=8.0)
    layer = C.InnerqDynamicLayer(cfg, 0)
    layer.update(torch.from_numpy(kx).to(DEV), torch.from_numpy(vx).to(DEV))
    nk = layer.keys_q.shape[2]
    nv = layer.values_q.shape[2]
    assert nk == 200 - 8 and nv == 192  # V keeps 8 recent: (200 - 8) % 64 == 0
    c, s, z = Q.quantize_channeldim_asym(kx[:, :, :nk], 32, 4)
    np.testing.assert_array_equal(_np(layer.keys_q), c)
    np.testing.assert_array_equal(_np(layer.keys_scale_factor).view(np.uint16), s.view(np.uint16))
    np.testing.assert_array_equal(_np(layer.keys_zp_sign).view(np.uint16), z.view(np.uint16))
    c, s, sg = Q.quantize_tokendim_sym(vx[:, :, :nv], 64, 3)
    np.testing.assert_array_equal(_np(layer.values_q), c)
    np.testing.assert_array_equal(_np(layer.values_scale_factor).view(np.uint16), s.view(np.uint16))
    got = _np(layer.values_zp_sign)
    nz = c != 0   # the packed form keeps the sign of non-zero codes only
    np.testing.assert_array_equal(got[nz], sg[nz])
    assert np.all(got[~nz] == 0)


def test_dynamic_cache_from_llama_config():
    from transformers import LlamaConfig
    cfg = LlamaConfig(num_hidden_layers=3, num_attention_heads=8, num_key_value_heads=2, hidden_size=512,
                      intermediate_size=64, vocab_size=32)
    for k, v in PRESETS["asym4_nosink"].items():
        setattr(cfg, k, v)
    cache = C.DynamicCache(config=cfg)
    assert len(cache.layers) == 3 and all(isinstance(l, C.InnerqDynamicLayer) for l in cache.layers)
    k = torch.randn(1, 2, 100, 64, dtype=torch.float16, device=DEV)
    v = torch.randn(1, 2, 100, 64, dtype=torch.float16, device=DEV)
    K, V = cache.update(k, v, 1)
    assert K is k and V is v
    K, V = cache.update(k[:, :, :1], v[:, :, :1], 1)
    assert K.shape == (1, 2, 101, 64) and cache.get_seq_length(1) == 101


def _tiny_llama(preset):
    from transformers import LlamaConfig
    from innerq_amd.models import InnerqLlamaForCausalLM
    cfg = LlamaConfig(num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2, hidden_size=512,
                      intermediate_size=256, vocab_size=64, max_position_embeddings=512)
    for k, v in {**PRESETS, **AXES_PRESETS}[preset].items():
        setattr(cfg, k, v)
    torch.manual_seed(0)
    return InnerqLlamaForCausalLM(cfg).to(device=DEV, dtype=torch.float16).eval()


def _count_attend(monkeypatch):
    calls = [0]
    orig = C.InnerqDynamicLayer.attend

    def attend(self, *a, **kw):
        calls[0] += 1
        return orig(self, *a, **kw)

    monkeypatch.setattr(C.InnerqDynamicLayer, "attend", attend)
    return calls


@pytest.mark.parametrize("preset", ["innerq_base", "mixed_k2v4_flush32", "hybrid_v"])
def test_fused_attention_in_llama_matches_reference_path(preset, monkeypatch):
    """A random 2-layer Llama (8 query / 2 KV heads, head_dim 64) on the drop-in
    cache, teacher-forced through 40 decode steps after a 200-token prefill:
    logits with attn_implementation="innerq_fused" (attend() over the packed
    cache, hybrid V included) against the
    reference's path (update() dequantizes the cache, eager attention), same
    weights and tokens."""
    model = _tiny_llama(preset)
    gen = torch.Generator(device=DEV).manual_seed(7)
    ids = torch.randint(0, 64, (2, 200), generator=gen, device=DEV)
    dec = torch.randint(0, 64, (2, 40), generator=gen, device=DEV)
    logits = {}
    calls = _count_attend(monkeypatch)
    for attn in ("eager", "innerq_fused"):
        model.config._attn_implementation = attn
        cache = C.DynamicCache(config=model.config)
        assert cache.fused_decode == (attn == "innerq_fused")
        steps = []
        with torch.no_grad():
            model(ids, past_key_values=cache, use_cache=True)
            for t in range(dec.shape[1]):
                steps.append(model(dec[:, t:t + 1], past_key_values=cache, use_cache=True).logits[:, -1].float())
        assert cache.get_seq_length() == 240
        logits[attn] = torch.stack(steps)
    ref, got = logits["eager"], logits["innerq_fused"]
    assert ((got - ref).abs().max() / ref.abs().max()).item() < 2e-2
    # every decode step of both layers went through attend()
    assert calls[0] == 2 * dec.shape[1]


def test_kivi_llama_under_fused_attention_takes_the_dense_path(monkeypatch):
    """A Llama whose cache groups keys along tokens (the kivi_sink preset) under
    attn_implementation="innerq_fused": the cache hands its dequantized K/V to
    sdpa at every step (attend() never runs), and the logits match the
    reference's path (eager attention over the same dequantized K/V)."""
    model = _tiny_llama("kivi_sink")
    gen = torch.Generator(device=DEV).manual_seed(5)
    ids = torch.randint(0, 64, (2, 200), generator=gen, device=DEV)
    dec = torch.randint(0, 64, (2, 20), generator=gen, device=DEV)
    calls = _count_attend(monkeypatch)
    logits = {}
    for attn in ("eager", "innerq_fused"):
        model.config._attn_implementation = attn
        cache = C.DynamicCache(config=model.config)
        steps = []
        with torch.no_grad():
            model(ids, past_key_values=cache, use_cache=True)
            for t in range(dec.shape[1]):
                steps.append(model(dec[:, t:t + 1], past_key_values=cache, use_cache=True).logits[:, -1].float())
        assert cache.get_seq_length() == 220
        logits[attn] = torch.stack(steps)
    ref, got = logits["eager"], logits["innerq_fused"]
    assert ((got - ref).abs().max() / ref.abs().max()).item() < 1e-2
    assert calls[0] == 0


def test_fused_attention_padded_batch(monkeypatch):
    """A left-padded batch (pads 0, 17 and 60 of a 150-token prefill; the mask
    hides each sequence's prefix) teacher-forced through 12 decode steps: every
    decode step of both layers goes through attend() with per-sequence start
    tokens, and the logits match those of the reference's path with sdpa (same
    prefill: both run it through sdpa with the mask) on every sequence."""
    model = _tiny_llama("innerq_base")
    gen = torch.Generator(device=DEV).manual_seed(11)
    B, T0, steps = 3, 150, 12
    ids = torch.randint(0, 64, (B, T0), generator=gen, device=DEV)
    dec = torch.randint(0, 64, (B, steps), generator=gen, device=DEV)
    mask = torch.ones(B, T0 + steps, dtype=torch.long, device=DEV)
    for b, p in enumerate((0, 17, 60)):
        mask[b, :p] = 0
    logits = {}
    calls = _count_attend(monkeypatch)
    for attn in ("sdpa", "innerq_fused"):
        model.config._attn_implementation = attn
        cache = C.DynamicCache(config=model.config)
        out = []
        with torch.no_grad():
            model(ids, attention_mask=mask[:, :T0], past_key_values=cache, use_cache=True)
            for t in range(steps):
                out.append(model(dec[:, t:t + 1], attention_mask=mask[:, :T0 + t + 1], past_key_values=cache,
                                 use_cache=True).logits[:, -1].float())
        logits[attn] = torch.stack(out)
    ref, got = logits["sdpa"], logits["innerq_fused"]
    assert torch.isfinite(got).all()
    assert ((got - ref).abs().max() / ref.abs().max()).item() < 2e-2
    assert calls[0] == 2 * steps


def test_fused_attention_generate(monkeypatch):
    """generate() on the hooked model with attn_implementation="innerq_fused":
    the hook's cache decodes in fused mode; the step scores match those of the
    reference's path for a short greedy continuation."""
    model = _tiny_llama("asym4_nosink")
    ids = torch.randint(0, 64, (1, 150), generator=torch.Generator(device=DEV).manual_seed(3), device=DEV)
    outs = {}
    calls = _count_attend(monkeypatch)
    for attn in ("eager", "innerq_fused"):
        model.config._attn_implementation = attn
        with torch.no_grad():
            outs[attn] = model.generate(ids, max_new_tokens=6, do_sample=False, output_scores=True,
                                        return_dict_in_generate=True)
        assert outs[attn].sequences.shape == (1, 156)
    ref = torch.stack(outs["eager"].scores).float()
    got = torch.stack(outs["innerq_fused"].scores).float()
    assert ((got - ref).abs().max() / ref.abs().max()).item() < 2e-2
    assert calls[0] == 2 * 5  # the 5 decode steps after the prefill, both layers


def test_fused_cache_follows_an_attention_switch():
    """A cache built while the model ran "innerq_fused" stays correct when the
    model switches attention mid-generation: update() reads the model's
    current attn_implementation on every call, so a step under sdpa gets the
    dense K and V (the reference's behaviour, from the very first such step)
    and a step under innerq_fused attends over the packed cache.  Every step's
    logits match a cache that only ever ran the reference's path."""
    model = _tiny_llama("asym4_nosink")
    gen = torch.Generator(device=DEV).manual_seed(5)
    ids = torch.randint(0, 64, (1, 150), generator=gen, device=DEV)
    dec = torch.randint(0, 64, (1, 8), generator=gen, device=DEV)
    plan = ["sdpa", "sdpa", "innerq_fused", "sdpa", "innerq_fused", "innerq_fused", "sdpa", "innerq_fused"]
    logits = {}
    for run in ("reference", "switching"):
        model.config._attn_implementation = "eager" if run == "reference" else "innerq_fused"
        cache = C.DynamicCache(config=model.config)
        steps = []
        with torch.no_grad():
            model(ids, past_key_values=cache, use_cache=True)
            for t, attn in enumerate(plan):
                if run == "switching":
                    model.config._attn_implementation = attn
                    assert cache.fused_decode == (attn == "innerq_fused")
                steps.append(model(dec[:, t:t + 1], past_key_values=cache, use_cache=True).logits[:, -1].float())
        assert cache.get_seq_length() == 150 + len(plan)
        logits[run] = torch.stack(steps)
    ref, got = logits["reference"], logits["switching"]
    err = ((got - ref).abs().amax(dim=(1, 2)) / ref.abs().amax(dim=(1, 2)))
    assert err.max().item() < 2e-2, err.tolist()


# ------------------------------------------------------------------------------------------
# sliding-window layer (cache.py:421-461)
from tests.test_oracle_cache import SLIDING, _shape_row, sliding_inputs  # noqa: E402


@pytest.fixture(scope="module")
def sliding_golden():
    import os
    from tests.conftest import GOLDEN
    return np.load(os.path.join(GOLDEN, "sliding_golden.npz"))


@pytest.mark.parametrize("name", list(SLIDING))
def test_sliding_layer_matches_reference_trace(sliding_golden, name):
    """The drop-in sliding layer without the fix reproduces the live reference's
    trace call by call: shapes (a single token, rank 3, once the past exceeds
    the window), recent-window lengths and mask sizes equal to the trace; K/V
    equal in value to the oracle's (pinned bit-exact to the trace) and, for the
    asym preset, in bytes to the trace.  (Values, not bits, for sym: the packed
    sym format does not keep the sign of a zero code.)"""
    from oracle import cache_ref
    g = sliding_golden
    kx, vx, w, prefill, steps = sliding_inputs(g, name)
    layer = C.InnerqDynamicSlidingWindowLayer(Cfg(**SLIDING[name]), 0, w)
    ref = cache_ref.SlidingLayerRef(Cfg(**SLIDING[name]), w)
    kt, vt = torch.from_numpy(kx).to(DEV), torch.from_numpy(vx).to(DEV)
    for s in range(steps + 1):
        lo, hi = (0, prefill) if s == 0 else (prefill + s - 1, prefill + s)
        mask = layer.get_mask_sizes(torch.arange(hi - lo)) if s else (0, 0)
        K, V = layer.update(kt[:, :, lo:hi], vt[:, :, lo:hi])
        Kr, Vr = ref.update(kx[:, :, lo:hi], vx[:, :, lo:hi])
        K, V = K.cpu().numpy(), V.cpu().numpy()
        np.testing.assert_array_equal(_shape_row(K, V), g[f"{name}_step{s}_shape"], err_msg=f"step {s}")
        np.testing.assert_array_equal(K, Kr, err_msg=f"K step {s}")
        np.testing.assert_array_equal(V, Vr, err_msg=f"V step {s}")
        if SLIDING[name]["key_quantize_mode"] == "asymmetric":
            b = np.concatenate([K.view(np.uint16).ravel(), V.view(np.uint16).ravel()])
            np.testing.assert_array_equal(_sha(b), g[f"{name}_step{s}_sha256"], err_msg=f"step {s}")
        state = [layer.keys_recent.shape[-2], layer.values_recent.shape[-2], layer.cumulative_length, *mask]
        np.testing.assert_array_equal(state, g[f"{name}_step{s}_state"], err_msg=f"step {s}")


@pytest.mark.parametrize("name", list(SLIDING))
def test_sliding_layer_fix_matches_oracle(name):
    """fix_sliding_window = True: K/V equal to the oracle's fixed layer at every
    call (values: sym zero codes come back as +0.0), as long as
    get_mask_sizes() announces."""
    from oracle import cache_ref
    cfg = Cfg(**SLIDING[name], fix_sliding_window=True)
    kx = synth.kv_tensor(1, 2, 140, 64, seed=9, n_out=2, factor=8.0)
    vx = synth.kv_tensor(1, 2, 140, 64, seed=10, n_out=2, factor=8.0)
    w = 96
    ref = cache_ref.SlidingLayerRef(cfg, w, fix=True)
    layer = C.InnerqDynamicSlidingWindowLayer(cfg, 0, w)
    kt, vt = torch.from_numpy(kx).to(DEV), torch.from_numpy(vx).to(DEV)
    for s in range(61):
        lo, hi = (0, 80) if s == 0 else (79 + s, 80 + s)
        kv_len, kv_off = layer.get_mask_sizes(hi - lo)
        assert (kv_len, kv_off) == ref.get_mask_sizes(hi - lo)
        K, V = layer.update(kt[:, :, lo:hi], vt[:, :, lo:hi])
        Kr, Vr = ref.update(kx[:, :, lo:hi], vx[:, :, lo:hi])
        assert K.shape[-2] == kv_len
        np.testing.assert_array_equal(K.cpu().numpy(), Kr, err_msg=f"step {s}")
        np.testing.assert_array_equal(V.cpu().numpy(), Vr, err_msg=f"step {s}")


@pytest.mark.parametrize("name", list(SLIDING))
def test_sliding_attend_matches_oracle(name):
    """fix_sliding_window = True: attend() (the fused decode path over the last
    min(T, w) tokens, read packed from a store offset that need not align with a
    K block or V group) at every step from 80 to 140 tokens with w = 96, against
    float64 attention over the oracle's fixed sliding layer's window (its fp32
    [sink | dequantized (times the key factor) | recent] tokens, the last
    min(T, w) of them): within 1e-3."""
    from oracle import attn_ref as A
    from oracle import cache_ref
    cfg = Cfg(**SLIDING[name], fix_sliding_window=True)
    B, H, nrep, D, w = 2, 2, 4, 128, 96
    kx = synth.kv_tensor(B, H, 140, D, seed=19, n_out=2, factor=8.0)
    vx = synth.kv_tensor(B, H, 140, D, seed=20, n_out=2, factor=8.0)
    qx = synth.normal((B, H * nrep, D), seed=21).astype(np.float16)
    ref = cache_ref.SlidingLayerRef(cfg, w, fix=True)
    layer = C.InnerqDynamicSlidingWindowLayer(cfg, 0, w)
    kt, vt, qt = torch.from_numpy(kx).to(DEV), torch.from_numpy(vx).to(DEV), torch.from_numpy(qx).to(DEV)
    layer.update(kt[:, :, :80], vt[:, :, :80])
    ref.update(kx[:, :, :80], vx[:, :, :80])
    worst = 0.0
    for t in range(80, 140):
        assert layer.fused_decode_ready(kt[:, :, t:t + 1])
        layer.append(kt[:, :, t:t + 1], vt[:, :, t:t + 1])
        ref.update(kx[:, :, t:t + 1], vx[:, :, t:t + 1])
        got = layer.attend(qt[:, :, None], D ** -0.5)[:, :, 0].cpu().numpy().astype(np.float64)
        kd = [ref.keys_sink.astype(np.float32)]
        if ref.keys_q is not None:
            d = ref.kdq(*ref.keys_q, ref.key_group_size)
            kd.append(d * ref.norm.astype(np.float32) if ref.key_normalize else d)
        kd.append(ref.keys_recent.astype(np.float32))
        vd = [ref.values_sink.astype(np.float32)]
        if ref.values_q is not None:
            vd.append(ref.vdq(*ref.values_q, ref.value_group_size))
        vd.append(ref.values_recent.astype(np.float32))
        n = min(t + 1, w)
        K = np.concatenate(kd, axis=2)[:, :, -n:]
        V = np.concatenate(vd, axis=2)[:, :, -n:]
        e = A.rel_err(got, A.decode_attention(qx, K, V, D ** -0.5, p_dtype=None))
        worst = max(worst, e)
        assert e < 1e-3, f"T={t + 1}: {e:.2e}"
    print(f"sliding {name}: worst {worst:.2e} over T = 81..140 (w = {w})")


def _tiny_mistral(preset, window=48):
    from transformers import MistralConfig
    from innerq_amd.models import InnerqMistralForCausalLM
    cfg = MistralConfig(num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2, hidden_size=512,
                        intermediate_size=256, vocab_size=64, max_position_embeddings=512, sliding_window=window)
    for k, v in preset.items():
        setattr(cfg, k, v)
    cfg.fix_sliding_window = True
    cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    return InnerqMistralForCausalLM(cfg).to(device=DEV, dtype=torch.float16).eval()


def _decode(model, cache, ids, dec):
    steps = []
    with torch.no_grad():
        model(ids, past_key_values=cache, use_cache=True)
        for t in range(dec.shape[1]):
            steps.append(model(dec[:, t:t + 1], past_key_values=cache, use_cache=True).logits[:, -1].float())
    return torch.stack(steps)


def test_mistral_decodes_past_the_window_with_the_fix():
    """A random 2-layer Mistral (sliding window 48) on the drop-in cache with
    fix_sliding_window = True decodes 30 steps past its window (the reference's
    layer cannot: its K/V lose the token axis).  With quantization off (16-bit
    K and V) the window is exactly transformers' own sliding cache's: logits
    equal to fp16 rounding; with 4-bit K and V the steps run and stay finite."""
    from transformers import DynamicCache as HFCache
    gen = torch.Generator(device=DEV).manual_seed(3)
    ids = torch.randint(0, 64, (1, 40), generator=gen, device=DEV)
    dec = torch.randint(0, 64, (1, 30), generator=gen, device=DEV)
    model = _tiny_mistral(dict(SLIDING["sliding_asym4"], k_bits=16, v_bits=16))
    cache = C.DynamicCache(config=model.config)
    assert all(isinstance(l, C.InnerqDynamicSlidingWindowLayer) for l in cache.layers)
    got = _decode(model, cache, ids, dec)
    ref = _decode(model, HFCache(config=model.config), ids, dec)
    assert ((got - ref).abs().max() / ref.abs().max()).item() < 1e-3
    model = _tiny_mistral(SLIDING["sliding_asym4"])
    cache = C.DynamicCache(config=model.config)
    got = _decode(model, cache, ids, dec)
    assert torch.isfinite(got).all() and cache.get_seq_length() == 70


def test_mistral_decodes_past_the_window_through_attend(monkeypatch):
    """The same Mistral with 4-bit K and V and the fix, now under the fused
    attention: every decode step of both (sliding) layers goes through attend()
    over the last w tokens, read packed, and the step logits match the eager
    path on the same cache type (the dense window update() returns)."""
    gen = torch.Generator(device=DEV).manual_seed(3)
    ids = torch.randint(0, 64, (1, 40), generator=gen, device=DEV)
    dec = torch.randint(0, 64, (1, 30), generator=gen, device=DEV)
    model = _tiny_mistral(SLIDING["sliding_sym3_sinks"])
    ref = _decode(model, C.DynamicCache(config=model.config), ids, dec)
    calls = [0]
    orig = C.InnerqDynamicSlidingWindowLayer.attend

    def attend(self, *a, **kw):
        calls[0] += 1
        return orig(self, *a, **kw)

    monkeypatch.setattr(C.InnerqDynamicSlidingWindowLayer, "attend", attend)
    model.config._attn_implementation = "innerq_fused"
    got = _decode(model, C.DynamicCache(config=model.config), ids, dec)
    assert calls[0] == 2 * 30
    err = ((got - ref).abs().max() / ref.abs().max()).item()
    print(f"mistral fused vs eager past the window: {err:.2e}")
    assert err < 2e-2


def test_mistral_padded_batch_through_attend(monkeypatch):
    """A left-padded batch (pads 0 and 10 of a 40-token prefill) on the Mistral
    with the fix, under the fused attention: every decode step of both sliding
    layers goes through attend(), with per-sequence starts while the window
    still covers the padding and none once it has slid past; the step logits
    match the sdpa path on the same cache type with the same mask."""
    gen = torch.Generator(device=DEV).manual_seed(5)
    B, T0, steps = 2, 40, 30
    ids = torch.randint(0, 64, (B, T0), generator=gen, device=DEV)
    dec = torch.randint(0, 64, (B, steps), generator=gen, device=DEV)
    mask = torch.ones(B, T0 + steps, dtype=torch.long, device=DEV)
    mask[1, :10] = 0
    model = _tiny_mistral(SLIDING["sliding_sym3_sinks"])
    calls = [0]
    orig = C.InnerqDynamicSlidingWindowLayer.attend

    def attend(self, *a, **kw):
        calls[0] += 1
        return orig(self, *a, **kw)

    monkeypatch.setattr(C.InnerqDynamicSlidingWindowLayer, "attend", attend)
    logits = {}
    for attn in ("sdpa", "innerq_fused"):
        model.config._attn_implementation = attn
        cache = C.DynamicCache(config=model.config)
        out = []
        with torch.no_grad():
            model(ids, attention_mask=mask[:, :T0], past_key_values=cache, use_cache=True)
            for t in range(steps):
                out.append(model(dec[:, t:t + 1], attention_mask=mask[:, :T0 + t + 1], past_key_values=cache,
                                 use_cache=True).logits[:, -1].float())
        logits[attn] = torch.stack(out)
    assert calls[0] == 2 * steps
    ref, got = logits["sdpa"], logits["innerq_fused"]
    assert torch.isfinite(got).all()
    err = ((got - ref).abs().max() / ref.abs().max()).item()
    print(f"mistral padded fused vs sdpa: {err:.2e}")
    assert err < 2e-2


_ROW_LAYOUTS = {
    # K flushed token by token, V by groups of 64 (group 64 rows, differing sinks)
    "k1_v64_g64_sinks": dict(k_bits=3, v_bits=4, key_flush_size=1, value_flush_size=64, key_group_size=64,
                             value_group_size=64, key_w_recent=50, value_w_recent=80, key_w_sink=16,
                             value_w_sink=8, key_normalize=True, key_quantize_over_token=False,
                             value_quantize_over_token=True, key_quantize_mode="hybrid",
                             value_quantize_mode="asymmetric"),
    # V flushed ahead of K (K by groups of 32 tokens, V every group)
    "k32_v32_vahead": dict(k_bits=4, v_bits=2, key_flush_size=32, value_flush_size=32, key_group_size=32,
                           value_group_size=32, key_w_recent=90, value_w_recent=20, key_w_sink=0,
                           value_w_sink=4, key_normalize=False, key_quantize_over_token=False,
                           value_quantize_over_token=True, key_quantize_mode="asymmetric",
                           value_quantize_mode="hybrid"),
    # groups of 128: no dequantized rows (the packed-row path)
    "g128": dict(k_bits=4, v_bits=4, key_flush_size=1, value_flush_size=128, key_group_size=128,
                 value_group_size=128, key_w_recent=32, value_w_recent=100, key_w_sink=0, value_w_sink=0,
                 key_normalize=False, key_quantize_over_token=False, value_quantize_over_token=True,
                 key_quantize_mode="symmetric", value_quantize_mode="symmetric"),
}


@pytest.mark.parametrize("name", list(_ROW_LAYOUTS))
def test_attend_with_dequantized_window_rows(name):
    """attend() over 150 decode steps of layouts where one role's store runs
    ahead of the other's (its tokens still in the other role's window): the
    windows' dequantized rows end both packed segments at one V group boundary
    (K ahead, V ahead, groups of 64, sinks of different lengths, hybrid
    stores), or, for groups of 128, the window kernel decodes the packed rows.
    Every 7th step within 1e-3 of float64 attention over the layer's
    dequantized K and V."""
    cfg = Cfg(**_ROW_LAYOUTS[name])
    B, H, nrep, D, prefill, steps = 2, 2, 4, 128, 600, 150
    kx = synth.kv_tensor(B, H, prefill + steps, D, seed=91, n_out=2, factor=8.0)
    vx = synth.kv_tensor(B, H, prefill + steps, D, seed=92, n_out=2, factor=8.0)
    vx[..., :40] += 4.0  # offset columns: hybrid groups of both kinds
    kt, vt = torch.from_numpy(kx).to(DEV), torch.from_numpy(vx).to(DEV)
    layer = C.InnerqDynamicLayer(cfg, 0)
    layer.update(kt[:, :, :prefill], vt[:, :, :prefill])
    used = 0
    for s in range(steps):
        layer.append(kt[:, :, prefill + s:prefill + s + 1], vt[:, :, prefill + s:prefill + s + 1])
        e = layer._packed_end()
        if e is not None:  # the rows past e are read from the windows' kept rows (as _attend_from decides)
            nk = layer.keys_sink.shape[-2] + layer._kq.length - e
            nv = layer.values_sink.shape[-2] + layer._vq.length - e
            used += int((nk or nv) and nk <= layer._kwin.shadow and nv <= layer._vwin.shadow)
        if s % 7 == 3:
            q = synth.normal((B, H * nrep, D), seed=s).astype(np.float16)
            out = layer.attend(torch.from_numpy(q).to(DEV)[:, :, None], D ** -0.5)[:, :, 0]
            ref = A.decode_attention(q, _np(layer.get_keys_deq().float()), _np(layer.get_values_deq().float()),
                                     D ** -0.5, None)
            assert A.rel_err(_np(out).astype(np.float64), ref) < 1e-3, f"step {s + 1}"
    if name == "g128":
        assert layer._kwin.deq_rows is False and used == 0
    else:
        assert layer._kwin.deq_rows and layer._vwin.deq_rows and used > steps // 2


def test_reference_helper_methods_drive_the_same_state():
    """The reference's prefill / decode helpers (cache.py:121-133, 212-224,
    309-381) called one by one, as the reference's add_to_cache does, leave the
    layer in the state update() reaches: equal dense K/V at every step; and
    normalize_keys / unnormalize_keys return the keys divided / multiplied by
    the factor as the reference's methods do."""
    from innerq_amd import presets
    cfg = presets.preset_config("innerq_hybrid")
    B, H, D, prefill, steps = 2, 2, 128, 300, 40
    kx = torch.from_numpy(synth.kv_tensor(B, H, prefill + steps, D, seed=71, n_out=2, factor=8.0)).to(DEV)
    vx = torch.from_numpy(synth.kv_tensor(B, H, prefill + steps, D, seed=72, n_out=2, factor=8.0)).to(DEV)
    a, b = C.InnerqDynamicLayer(cfg, 0), C.InnerqDynamicLayer(cfg, 0)
    a.update(kx[:, :, :prefill], vx[:, :, :prefill])
    b.dtype, b.device = kx.dtype, kx.device
    k, v = b.initialize_sinks(kx[:, :, :prefill], vx[:, :, :prefill])
    k, v = b.initialize_recents(k, v)
    b.initial_quantization(k, v)
    b.is_initialized = True
    b.cumulative_length = prefill
    for s in range(steps):
        tok = slice(prefill + s, prefill + s + 1)
        ka, va = a.update(kx[:, :, tok], vx[:, :, tok])
        b.cumulative_length += 1
        kf, vf = b.update_recents(kx[:, :, tok], vx[:, :, tok])
        if kf.numel():
            (b.quantize_new_keys if b._kq is not None else b.initialize_keys_q)(kf)
        if vf.numel():
            (b.quantize_new_values if b._vq is not None else b.initialize_values_q)(vf)
        kb, vb = b.get_deq_tensors()
        assert torch.equal(ka, kb) and torch.equal(va, vb), f"step {s + 1}"
    n = a.key_normalization_factor
    x = kx[:, :, :5]
    assert torch.equal(a.normalize_keys(x), x / n)
    assert torch.equal(a.unnormalize_keys(x), x * n)
