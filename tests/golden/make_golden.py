"""Write golden vectors from the live reference (run in the build container only).

Imports mthcom/innerq's ``src/innerq/quant.py`` and ``src/innerq/cache.py`` by
file path (``import innerq`` itself pulls in lm_eval, which is absent) and
records small input/output vectors as ``.npz`` fixtures next to this script.
The reference never travels: only these data files are committed, and the
tests read them, never the reference.

Fixtures
--------
quant_golden.npz    quantize_{channeldim,tokendim}_{asym,sym} outputs for
                    bits 2/3/4, group 32/64 on a [1,2,64,128] fp16 input with
                    outlier channels, constant groups and rounding ties; the
                    hybrid quantizer for bits 2/3/4 (masks, digests of the
                    dequantized values, also with -0.0 read as +0.0);
                    config-0 SHA-256 digests.
cache_golden.npz    InnerqDynamicLayer.update() traces: prefill + decode steps
                    for several presets (inputs regenerated from the stored
                    seed with innerq_amd.synth); full dense K/V of the last
                    decode call, SHA-256 of every call's K/V bytes,
                    and the recent-window lengths after every call.
bf16_golden.npz     the same quantizers on the quant_golden input cast to bf16
                    (codes, bf16 scale / zero / sign bits; hybrid masks;
                    dequantization digests) and update() traces of two presets
                    on bf16 K/V (a bf16 model's cache: LongBench/pred.py:240).
sliding_golden.npz  InnerqDynamicSlidingWindowLayer.update() traces
                    (cache.py:421-461) across the window boundary: per call the
                    shapes and SHA-256 of the returned K/V (a single token, the
                    dimension dropped, once the past exceeds the window: the
                    reference indexes [:, :, -w, :]), the recent-window lengths
                    and get_mask_sizes() before the call.

axes_golden.npz     update() traces, as in cache_golden.npz, of layers with keys
                    grouped along tokens and values along head_dim (the KIVI
                    presets of scripts/run_lmeval.sh:54-93, and sym keys with
                    hybrid values on those axes).
hybrid_ties.npz     groups whose two hybrid L1 errors tie exactly (the
                    comparison quant.py:144 makes is strict) and the
                    reference's masks for them.

Usage:  python tests/golden/make_golden.py [/root/reference] [--sliding-only | --bf16-only | --ties-only | --axes-only]
"""
from __future__ import annotations

import hashlib
import importlib.util
import os
import sys
import types

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from innerq_amd import synth  # noqa: E402


def load_reference(root):
    pkg_dir = os.path.join(root, "src", "innerq")
    pkg = types.ModuleType("_innerq_reference")
    pkg.__path__ = [pkg_dir]
    sys.modules["_innerq_reference"] = pkg
    mods = {}
    for name in ("quant", "cache"):
        spec = importlib.util.spec_from_file_location(f"_innerq_reference.{name}",
                                                      os.path.join(pkg_dir, f"{name}.py"))
        mod = importlib.util.module_from_spec(spec)
        sys.modules[spec.name] = mod
        spec.loader.exec_module(mod)
        mods[name] = mod
    return mods["quant"], mods["cache"]


def f16(a):
    return a.detach().cpu().numpy().astype(np.float16).view(np.uint16)


def codes8(a):
    c = a.detach().cpu().numpy().astype(np.int64)
    assert np.all(((c > -128) & (c < 128)) | (c == -2147483648)), "unexpected code"
    c = np.where(c == -2147483648, -128, c)   # INT32_MIN sentinel
    return c.astype(np.int8)


def digest(arr):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(arr).tobytes()).digest(), dtype=np.uint8)


def quant_input():
    x = synth.kv_tensor(1, 2, 64, 128, seed=1234, n_out=4, factor=10.0).astype(np.float32)
    # constant groups (channel-dim group 0 of token 5; token-dim group of channel 7)
    x[0, 0, 5, 0:32] = 0.75
    x[0, 1, 0:32, 7] = -1.5
    # exact ties: ramp with known halves
    x[0, 0, 9, 32:64] = np.arange(32) % 4 - 2.0
    x[0, 1, 11, 64:96] = (np.arange(32) % 16) * 0.5
    return x.astype(np.float16)


SLIDING_PRESETS = {
    "sliding_asym4": dict(k_bits=4, v_bits=4, key_flush_size=1, value_flush_size=32, key_group_size=32,
                          value_group_size=32, key_w_recent=32, value_w_recent=64, key_w_sink=0, value_w_sink=0,
                          key_normalize=False, key_quantize_over_token=False, value_quantize_over_token=True,
                          key_quantize_mode="asymmetric", value_quantize_mode="asymmetric"),
    "sliding_sym3_sinks": dict(k_bits=3, v_bits=3, key_flush_size=1, value_flush_size=32, key_group_size=32,
                               value_group_size=32, key_w_recent=40, value_w_recent=40, key_w_sink=8,
                               value_w_sink=8, key_normalize=True, key_quantize_over_token=False,
                               value_quantize_over_token=True, key_quantize_mode="symmetric",
                               value_quantize_mode="symmetric"),
}
SLIDING = dict(B=1, H=2, D=64, window=96, prefill=80, steps=40)


def sliding_traces(cache):
    """Traces of the reference sliding-window layer across its window."""
    class Layer(cache.InnerqDynamicSlidingWindowLayer):
        def get_max_length(self):   # abstract in the installed transformers
            return self.sliding_window

    class Cfg:
        pass

    out = {}
    B, H, D, w, prefill, steps = (SLIDING[k] for k in ("B", "H", "D", "window", "prefill", "steps"))
    for name, kw in SLIDING_PRESETS.items():
        cfg = Cfg()
        for k, v in kw.items():
            setattr(cfg, k, v)
        layer = Layer(cfg, 0, w)
        seed = sum(map(ord, name))
        kx = synth.kv_tensor(B, H, prefill + steps, D, seed=seed, n_out=2, factor=8.0)
        vx = synth.kv_tensor(B, H, prefill + steps, D, seed=seed + 1, n_out=2, factor=8.0)
        out[f"{name}_seed"] = np.array([seed, B, H, D, w, prefill, steps])
        kt, vt = torch.from_numpy(kx), torch.from_numpy(vx)
        for s in range(steps + 1):
            lo, hi = (0, prefill) if s == 0 else (prefill + s - 1, prefill + s)
            q_len = hi - lo
            mask = layer.get_mask_sizes(torch.arange(q_len)) if s else (0, 0)
            K, V = layer.update(kt[:, :, lo:hi].clone(), vt[:, :, lo:hi].clone())
            shape = list(K.shape) + [0] * (4 - K.dim())
            out[f"{name}_step{s}_shape"] = np.array([K.dim()] + shape + list(V.shape) + [0] * (4 - V.dim()))
            out[f"{name}_step{s}_sha256"] = digest(np.concatenate([f16(K).ravel(), f16(V).ravel()]))
            out[f"{name}_step{s}_state"] = np.array([layer.keys_recent.shape[-2], layer.values_recent.shape[-2],
                                                     layer.cumulative_length, mask[0], mask[1]])
    return out


PRESETS = {
    "innerq_base": dict(k_bits=3, v_bits=3, key_flush_size=1, value_flush_size=32, key_group_size=32,
                        value_group_size=32, key_w_recent=96, value_w_recent=96, key_w_sink=32,
                        value_w_sink=32, key_normalize=True, key_quantize_over_token=False,
                        value_quantize_over_token=True, key_quantize_mode="symmetric",
                        value_quantize_mode="symmetric"),
    "asym4_nosink": dict(k_bits=4, v_bits=4, key_flush_size=1, value_flush_size=32, key_group_size=32,
                         value_group_size=32, key_w_recent=32, value_w_recent=64, key_w_sink=0,
                         value_w_sink=0, key_normalize=False, key_quantize_over_token=False,
                         value_quantize_over_token=True, key_quantize_mode="asymmetric",
                         value_quantize_mode="asymmetric"),
    "mixed_k2v4_flush32": dict(k_bits=2, v_bits=4, key_flush_size=32, value_flush_size=64,
                               key_group_size=32, value_group_size=32, key_w_recent=40, value_w_recent=70,
                               key_w_sink=4, value_w_sink=0, key_normalize=False,
                               key_quantize_over_token=False, value_quantize_over_token=True,
                               key_quantize_mode="asymmetric", value_quantize_mode="symmetric"),
    "hybrid_v": dict(k_bits=3, v_bits=2, key_flush_size=1, value_flush_size=32, key_group_size=32,
                     value_group_size=32, key_w_recent=96, value_w_recent=96, key_w_sink=32,
                     value_w_sink=32, key_normalize=True, key_quantize_over_token=False,
                     value_quantize_over_token=True, key_quantize_mode="symmetric",
                     value_quantize_mode="hybrid"),
    "k_only": dict(k_bits=4, v_bits=16, key_flush_size=1, key_group_size=64, key_w_recent=16,
                   key_w_sink=2, key_normalize=False, key_quantize_mode="asymmetric"),
}


def bf16(a):
    """bf16 tensor -> its uint16 bit patterns."""
    return a.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


BF16_PRESETS = ("innerq_base", "hybrid_v")


def bf16_fixtures(quant, cache, presets):
    """quant.py and cache.py on bf16 tensors."""
    out = {}
    xt = torch.from_numpy(quant_input()).to(torch.bfloat16)
    out["x"] = bf16(xt)
    for axis in ("channel", "token"):
        qa = getattr(quant, f"quantize_{axis}dim_asym")
        qs = getattr(quant, f"quantize_{axis}dim_sym")
        da = getattr(quant, f"dequantize_{axis}dim_asym")
        ds = getattr(quant, f"dequantize_{axis}dim_sym")
        for bits in (2, 3, 4):
            for G in (32, 64):
                c, s, z = qa(xt.clone(), G, bits)
                key = f"{axis}_asym_b{bits}_g{G}"
                out[key + "_codes"], out[key + "_scale"], out[key + "_zero"] = codes8(c), bf16(s), bf16(z)
                c, s, sg = qs(xt.clone(), G, bits)
                key = f"{axis}_sym_b{bits}_g{G}"
                out[key + "_codes"], out[key + "_scale"], out[key + "_signs"] = codes8(c), bf16(s), bf16(sg)
        hq = quant.quantize_hybrid(qa, qs, da, ds)
        hd = quant.dequantize_hybrid(da, ds)
        for bits in (2, 3, 4):
            c, s, z = hq(xt.clone(), 32, bits)
            key = f"{axis}_hybrid_b{bits}_g32"
            out[key + "_mask"] = s["mask"].cpu().numpy()
            deq = hd(c, s, z, 32).cpu().numpy().astype(np.float32)
            out[key + "_deq_pz_sha256"] = digest(deq + np.float32(0.0))
        c, s, z = qa(xt.clone(), 32, 4)
        out[f"{axis}_asym_b4_g32_deq_sha256"] = digest(da(c, s, z, 32).cpu().numpy().astype(np.float32))
        c, s, z = qs(xt.clone(), 32, 3)
        out[f"{axis}_sym_b3_g32_deq_pz_sha256"] = digest(ds(c, s, z, 32).cpu().numpy().astype(np.float32)
                                                         + np.float32(0.0))

    class Layer(cache.InnerqDynamicLayer):
        def get_max_length(self):   # abstract in the installed transformers
            return -1

    class Cfg:
        pass

    B, H, D = 1, 2, 64
    prefill, steps = 150, 70
    for name in BF16_PRESETS:
        cfg = Cfg()
        for k, v in presets[name].items():
            setattr(cfg, k, v)
        layer = Layer(cfg, 0)
        seed = sum(map(ord, name)) + 16
        kx = synth.kv_tensor(B, H, prefill + steps, D, seed=seed, n_out=2, factor=8.0)
        vx = synth.kv_tensor(B, H, prefill + steps, D, seed=seed + 1, n_out=2, factor=8.0)
        out[f"{name}_seed"] = np.array([seed, B, H, D, prefill, steps])
        kt = torch.from_numpy(kx).to(torch.bfloat16)
        vt = torch.from_numpy(vx).to(torch.bfloat16)
        # digests of the values (fp32, -0.0 read as +0.0: a packed sym field
        # keeps no sign for a zero code)
        def pz(K, V):
            return digest(np.concatenate([K.float().numpy().ravel(), V.float().numpy().ravel()]) + np.float32(0.0))

        K, V = layer.update(kt[:, :, :prefill].clone(), vt[:, :, :prefill].clone())
        out[f"{name}_step0_pz_sha256"] = pz(K, V)
        for s in range(steps):
            K, V = layer.update(kt[:, :, prefill + s:prefill + s + 1].clone(),
                                vt[:, :, prefill + s:prefill + s + 1].clone())
            if s == steps - 1:
                out[f"{name}_step{s + 1}_k"], out[f"{name}_step{s + 1}_v"] = bf16(K), bf16(V)
            out[f"{name}_step{s + 1}_pz_sha256"] = pz(K, V)
            out[f"{name}_len{s + 1}"] = np.array([K.shape[-2], V.shape[-2], layer.keys_recent.shape[-2],
                                                  layer.values_recent.shape[-2]])
    return out


def hybrid_tie_fixtures(quant):
    """Groups whose two hybrid L1 errors tie exactly: values on a coarse grid
    (a few distinct quarter multiples), so every error term and both sums are
    exact in fp32 whatever the summation order; chosen by the reference's own
    quantize / dequantize functions (errors summed in float64 here, for the
    choice only), then the reference's quantize_hybrid mask recorded (the
    comparison is strict: a tie keeps the asym codes).  Both axes, bits 2-4,
    groups of 32; 16 tied groups each, in a [1, 1, 16, 32] (channel) or
    [1, 1, 32, 16] (token) fp16 tensor."""
    out = {}
    G, n = 32, 16
    for axis in ("channel", "token"):
        qa = getattr(quant, f"quantize_{axis}dim_asym")
        qs = getattr(quant, f"quantize_{axis}dim_sym")
        da = getattr(quant, f"dequantize_{axis}dim_asym")
        ds = getattr(quant, f"dequantize_{axis}dim_sym")
        hq = quant.quantize_hybrid(qa, qs, da, ds)
        for bits in (2, 3, 4):
            rng = np.random.default_rng(1000 + bits + (0 if axis == "channel" else 50))
            groups = []
            while len(groups) < n:
                lv = rng.integers(-8, 9, size=int(rng.integers(2, 5))) / 4.0
                g = rng.choice(lv, size=G).astype(np.float16)
                x = torch.from_numpy(g.reshape(1, 1, 1, G) if axis == "channel" else g.reshape(1, 1, G, 1))
                xa = da(*qa(x.clone(), G, bits - 1), G).double()
                xs = ds(*qs(x.clone(), G, bits), G).double()
                ea = (xa - x.double()).abs().sum().item()
                es = (xs - x.double()).abs().sum().item()
                if ea == es and ea > 0:
                    groups.append(g)
            x = np.stack(groups)                        # [n, G]
            x = x.reshape(1, 1, n, G) if axis == "channel" else x.T.reshape(1, 1, G, n)
            c, sc, z = hq(torch.from_numpy(np.ascontiguousarray(x)), G, bits)
            key = f"{axis}_b{bits}"
            out[key + "_x"] = np.ascontiguousarray(x).view(np.uint16)
            out[key + "_mask"] = sc["mask"].cpu().numpy()
    return out


def main(root, sliding_only=False, bf16_only=False, ties_only=False, axes_only=False):
    quant, cache = load_reference(root)
    if ties_only:
        np.savez_compressed(os.path.join(HERE, "hybrid_ties.npz"), **hybrid_tie_fixtures(quant))
        print("wrote", os.path.join(HERE, "hybrid_ties.npz"))
        return
    if axes_only:
        np.savez_compressed(os.path.join(HERE, "axes_golden.npz"), **cache_traces(cache, AXES_PRESETS))
        print("wrote", os.path.join(HERE, "axes_golden.npz"))
        return
    if bf16_only:
        np.savez_compressed(os.path.join(HERE, "bf16_golden.npz"), **bf16_fixtures(quant, cache, PRESETS))
        print("wrote", os.path.join(HERE, "bf16_golden.npz"))
        return
    np.savez_compressed(os.path.join(HERE, "sliding_golden.npz"), **sliding_traces(cache))
    print("wrote", os.path.join(HERE, "sliding_golden.npz"))
    if sliding_only:
        return
    out = {}
    x = quant_input()
    out["x"] = x.view(np.uint16)
    xt = torch.from_numpy(x)
    for axis, fa, fs in (("channel", quant.quantize_channeldim_asym, quant.quantize_channeldim_sym),
                         ("token", quant.quantize_tokendim_asym, quant.quantize_tokendim_sym)):
        for bits in (2, 3, 4):
            for G in (32, 64):
                c, s, z = fa(xt.clone(), G, bits)
                key = f"{axis}_asym_b{bits}_g{G}"
                out[key + "_codes"] = codes8(c)
                out[key + "_scale"] = f16(s)
                out[key + "_zero"] = f16(z)
                c, s, sg = fs(xt.clone(), G, bits)
                key = f"{axis}_sym_b{bits}_g{G}"
                out[key + "_codes"] = codes8(c)
                out[key + "_scale"] = f16(s)
                out[key + "_signs"] = f16(sg)
                # dequantize outputs (fp32) for the asym/sym functions
    for axis in ("channel", "token"):
        qa = getattr(quant, f"quantize_{axis}dim_asym")
        qs = getattr(quant, f"quantize_{axis}dim_sym")
        da = getattr(quant, f"dequantize_{axis}dim_asym")
        ds = getattr(quant, f"dequantize_{axis}dim_sym")
        hq = quant.quantize_hybrid(qa, qs, da, ds)
        hd = quant.dequantize_hybrid(da, ds)
        for bits in (2, 3, 4):
            c, s, z = hq(xt.clone(), 32, bits)
            key = f"{axis}_hybrid_b{bits}_g32"
            out[key + "_mask"] = s["mask"].cpu().numpy()
            deq = hd(c, s, z, 32).cpu().numpy().astype(np.float32)
            out[key + "_deq_sha256"] = digest(deq)
            # the same values with -0.0 read as +0.0 (x + 0.0): a packed sym
            # field keeps no sign for a zero code
            out[key + "_deq_pz_sha256"] = digest(deq + np.float32(0.0))
        c, s, z = qa(xt.clone(), 32, 4)
        out[f"{axis}_asym_b4_g32_deq_sha256"] = digest(da(c, s, z, 32).cpu().numpy().astype(np.float32))
        c, s, z = qs(xt.clone(), 32, 3)
        out[f"{axis}_sym_b3_g32_deq_sha256"] = digest(ds(c, s, z, 32).cpu().numpy().astype(np.float32))

    # config 0: K,V fp16 [1,8,4096,128], 4 outlier channels/head x10, 4-bit asym G=32
    k0 = torch.from_numpy(synth.kv_tensor(1, 8, 4096, 128, seed=0, n_out=4, factor=10.0))
    v0 = torch.from_numpy(synth.kv_tensor(1, 8, 4096, 128, seed=1, n_out=4, factor=10.0))
    for name, t, fn in (("k", k0, quant.quantize_channeldim_asym), ("v", v0, quant.quantize_tokendim_asym)):
        c, s, z = fn(t.clone(), 32, 4)
        for part, arr in (("codes", c.numpy().astype(np.int32)), ("scale", f16(s)), ("zero", f16(z))):
            out[f"cfg0_{name}_{part}_sha256"] = digest(arr)
    np.savez_compressed(os.path.join(HERE, "quant_golden.npz"), **out)

    # ---------------- cache traces ----------------
    trace = cache_traces(cache, PRESETS)
    np.savez_compressed(os.path.join(HERE, "cache_golden.npz"), **trace)
    np.savez_compressed(os.path.join(HERE, "bf16_golden.npz"), **bf16_fixtures(quant, cache, PRESETS))
    np.savez_compressed(os.path.join(HERE, "axes_golden.npz"), **cache_traces(cache, AXES_PRESETS))
    print("wrote", os.path.join(HERE, "quant_golden.npz"), os.path.join(HERE, "cache_golden.npz"))


# The KIVI axis choices (scripts/run_lmeval.sh:54-93): keys grouped along
# tokens, values along head_dim, flushes of 32 keys and of single values.
AXES_PRESETS = {
    "kivi": dict(k_bits=2, v_bits=2, key_flush_size=32, value_flush_size=1, key_group_size=32,
                 value_group_size=32, key_w_recent=128, value_w_recent=128, key_w_sink=0, value_w_sink=0,
                 key_normalize=False, key_quantize_over_token=True, value_quantize_over_token=False,
                 key_quantize_mode="asymmetric", value_quantize_mode="asymmetric"),
    "kivi_sink": dict(k_bits=2, v_bits=2, key_flush_size=32, value_flush_size=1, key_group_size=32,
                      value_group_size=32, key_w_recent=96, value_w_recent=96, key_w_sink=32, value_w_sink=32,
                      key_normalize=False, key_quantize_over_token=True, value_quantize_over_token=False,
                      key_quantize_mode="asymmetric", value_quantize_mode="asymmetric"),
    # the same axes with sym keys and 3-bit hybrid values (every mode on both axes)
    "axes_sym_hybrid": dict(k_bits=4, v_bits=3, key_flush_size=32, value_flush_size=1, key_group_size=32,
                            value_group_size=32, key_w_recent=64, value_w_recent=48, key_w_sink=8,
                            value_w_sink=4, key_normalize=False, key_quantize_over_token=True,
                            value_quantize_over_token=False, key_quantize_mode="symmetric",
                            value_quantize_mode="hybrid"),
}


def cache_traces(cache, presets):
    """update() traces of the live reference's layer: per step the sha256 of
    the returned K and V, their lengths and the recent windows' lengths, and
    the last step's arrays."""
    class Layer(cache.InnerqDynamicLayer):
        def get_max_length(self):   # abstract in the installed transformers
            return -1

    class Cfg:
        pass

    trace = {}
    B, H, D = 1, 2, 64
    prefill, steps = 150, 70
    for name, kw in presets.items():
        cfg = Cfg()
        for k, v in kw.items():
            setattr(cfg, k, v)
        layer = Layer(cfg, 0)
        seed = sum(map(ord, name))
        kx = synth.kv_tensor(B, H, prefill + steps, D, seed=seed, n_out=2, factor=8.0)
        vx = synth.kv_tensor(B, H, prefill + steps, D, seed=seed + 1, n_out=2, factor=8.0)
        trace[f"{name}_seed"] = np.array([seed, B, H, D, prefill, steps])
        kt, vt = torch.from_numpy(kx), torch.from_numpy(vx)
        K, V = layer.update(kt[:, :, :prefill].clone(), vt[:, :, :prefill].clone())
        trace[f"{name}_step0_sha256"] = digest(np.concatenate([f16(K).ravel(), f16(V).ravel()]))
        for s in range(steps):
            K, V = layer.update(kt[:, :, prefill + s:prefill + s + 1].clone(),
                                vt[:, :, prefill + s:prefill + s + 1].clone())
            if s == steps - 1:
                trace[f"{name}_step{s + 1}_k"] = f16(K)
                trace[f"{name}_step{s + 1}_v"] = f16(V)
            trace[f"{name}_step{s + 1}_sha256"] = digest(np.concatenate([f16(K).ravel(), f16(V).ravel()]))
            trace[f"{name}_len{s + 1}"] = np.array([K.shape[-2], V.shape[-2],
                                                    layer.keys_recent.shape[-2], layer.values_recent.shape[-2]])
    return trace


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if not a.startswith("--")]
    main(args[0] if args else "/root/reference", sliding_only="--sliding-only" in sys.argv,
         bf16_only="--bf16-only" in sys.argv, ties_only="--ties-only" in sys.argv,
         axes_only="--axes-only" in sys.argv)
