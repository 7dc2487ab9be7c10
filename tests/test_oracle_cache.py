"""Pin the cache state-machine oracle (oracle/cache_ref.py) against traces of the
live reference InnerqDynamicLayer (tests/golden/cache_golden.npz)."""
import hashlib

import numpy as np
import pytest

from innerq_amd import synth
from oracle import cache_ref

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


class Cfg:
    def __init__(self, **kw):
        self.__dict__.update(kw)


def _sha(k, v):
    b = np.concatenate([k.view(np.uint16).ravel(), v.view(np.uint16).ravel()])
    return np.frombuffer(hashlib.sha256(b.tobytes()).digest(), dtype=np.uint8)


def golden_inputs(g, name):
    seed, B, H, D, prefill, steps = (int(x) for x in g[f"{name}_seed"])
    kx = synth.kv_tensor(B, H, prefill + steps, D, seed=seed, n_out=2, factor=8.0)
    vx = synth.kv_tensor(B, H, prefill + steps, D, seed=seed + 1, n_out=2, factor=8.0)
    return kx, vx, prefill, steps


# Keys grouped along tokens and values along head_dim: the KIVI presets
# (scripts/run_lmeval.sh:54-93) and sym keys with hybrid values on those axes
# (traces in axes_golden.npz).
AXES_PRESETS = {
    "kivi": dict(k_bits=2, v_bits=2, key_flush_size=32, value_flush_size=1, key_group_size=32,
                 value_group_size=32, key_w_recent=128, value_w_recent=128, key_w_sink=0, value_w_sink=0,
                 key_normalize=False, key_quantize_over_token=True, value_quantize_over_token=False,
                 key_quantize_mode="asymmetric", value_quantize_mode="asymmetric"),
    "kivi_sink": dict(k_bits=2, v_bits=2, key_flush_size=32, value_flush_size=1, key_group_size=32,
                      value_group_size=32, key_w_recent=96, value_w_recent=96, key_w_sink=32, value_w_sink=32,
                      key_normalize=False, key_quantize_over_token=True, value_quantize_over_token=False,
                      key_quantize_mode="asymmetric", value_quantize_mode="asymmetric"),
    "axes_sym_hybrid": dict(k_bits=4, v_bits=3, key_flush_size=32, value_flush_size=1, key_group_size=32,
                            value_group_size=32, key_w_recent=64, value_w_recent=48, key_w_sink=8,
                            value_w_sink=4, key_normalize=False, key_quantize_over_token=True,
                            value_quantize_over_token=False, key_quantize_mode="symmetric",
                            value_quantize_mode="hybrid"),
}


def test_kivi_presets_are_the_traced_configs():
    """innerq_amd.presets' KIVI entries are the configurations traced above"""
    from innerq_amd import presets
    for name in ("kivi", "kivi_sink"):
        assert presets.PRESETS[name] == AXES_PRESETS[name]


@pytest.mark.parametrize("name", list(AXES_PRESETS))
def test_cache_oracle_matches_axes_trace(axes_golden, name):
    """the oracle's layer with keys over tokens and values over channels
    (cache.py:93-119, the flush of 32 keys along the token axis) reproduces
    the live reference's traces step for step"""
    _check_oracle_trace(axes_golden, name, AXES_PRESETS[name])


@pytest.mark.parametrize("name", list(PRESETS))
def test_cache_oracle_matches_reference_trace(cache_golden, name):
    _check_oracle_trace(cache_golden, name, PRESETS[name])


def _check_oracle_trace(g, name, cfg):
    kx, vx, prefill, steps = golden_inputs(g, name)
    layer = cache_ref.CacheLayerRef(Cfg(**cfg))
    K, V = layer.update(kx[:, :, :prefill], vx[:, :, :prefill])
    np.testing.assert_array_equal(_sha(K, V), g[f"{name}_step0_sha256"])
    for s in range(steps):
        K, V = layer.update(kx[:, :, prefill + s:prefill + s + 1], vx[:, :, prefill + s:prefill + s + 1])
        if s == steps - 1:
            np.testing.assert_array_equal(K.view(np.uint16), g[f"{name}_step{s + 1}_k"])
            np.testing.assert_array_equal(V.view(np.uint16), g[f"{name}_step{s + 1}_v"])
        np.testing.assert_array_equal(_sha(K, V), g[f"{name}_step{s + 1}_sha256"], err_msg=f"step {s + 1}")
        lens = g[f"{name}_len{s + 1}"]
        assert (K.shape[-2], V.shape[-2], layer.keys_recent.shape[-2], layer.values_recent.shape[-2]) == tuple(lens)


@pytest.mark.parametrize("name", list(PRESETS))
def test_length_schedule_matches_reference_trace(cache_golden, name):
    """the length-only simulator reproduces the reference's recent-window lengths (incl. the V drain)"""
    p = PRESETS[name]
    g = cache_golden
    _, _, prefill, steps = golden_inputs(g, name)
    ks = cache_cache = cache_ref.schedule(prefill, steps, p.get("key_w_sink", 0), p.get("key_w_recent", 32),
                                          p.get("key_flush_size", 32), p.get("k_bits", 16) < 16,
                                          p.get("key_quantize_over_token", False))
    vs = cache_ref.schedule(prefill, steps, p.get("value_w_sink", 0), p.get("value_w_recent", 32),
                            p.get("value_flush_size", 32), p.get("v_bits", 16) < 16,
                            p.get("value_quantize_over_token", True))
    for s in range(1, steps + 1):
        lens = g[f"{name}_len{s}"]
        assert ks[s][2] == lens[2] and vs[s][2] == lens[3]
        assert sum(ks[s]) == lens[0] and sum(vs[s]) == lens[1]


def test_value_recent_window_drains():
    """V with flush 32 drains its recent window 96 -> 65 -> 34 -> 3 (cache.py:296-307)"""
    sched = cache_ref.schedule(500, 100, 32, 96, 32, True, True)
    nr = [x[2] for x in sched]
    assert nr[0] == 84  # (468 - r) % 32 == 0 -> r = 84
    assert min(nr[1:]) < 32 and max(nr[1:]) <= 96


# ------------------------------------------------------------------------------------------
# sliding-window layer (cache.py:421-461) against the live reference's traces
SLIDING = {
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


def sliding_inputs(g, name):
    seed, B, H, D, w, prefill, steps = (int(x) for x in g[f"{name}_seed"])
    kx = synth.kv_tensor(B, H, prefill + steps, D, seed=seed, n_out=2, factor=8.0)
    vx = synth.kv_tensor(B, H, prefill + steps, D, seed=seed + 1, n_out=2, factor=8.0)
    return kx, vx, w, prefill, steps


def _shape_row(K, V):
    return np.array([K.ndim] + list(K.shape) + [0] * (4 - K.ndim) + list(V.shape) + [0] * (4 - V.ndim))


@pytest.fixture(scope="module")
def sliding_golden():
    import os
    from tests.conftest import GOLDEN
    return np.load(os.path.join(GOLDEN, "sliding_golden.npz"))


@pytest.mark.parametrize("name", list(SLIDING))
def test_sliding_oracle_matches_reference_trace(sliding_golden, name):
    """The reference's sliding layer, bug included: per call the shapes and
    SHA-256 of K/V, the recent-window lengths, the cumulative length and the
    mask sizes announced before the call."""
    g = sliding_golden
    kx, vx, w, prefill, steps = sliding_inputs(g, name)
    layer = cache_ref.SlidingLayerRef(Cfg(**SLIDING[name]), w)
    for s in range(steps + 1):
        lo, hi = (0, prefill) if s == 0 else (prefill + s - 1, prefill + s)
        mask = layer.get_mask_sizes(hi - lo) if s else (0, 0)
        K, V = layer.update(kx[:, :, lo:hi], vx[:, :, lo:hi])
        np.testing.assert_array_equal(_shape_row(K, V), g[f"{name}_step{s}_shape"], err_msg=f"step {s}")
        np.testing.assert_array_equal(_sha(K, V), g[f"{name}_step{s}_sha256"], err_msg=f"step {s}")
        state = [layer.keys_recent.shape[-2], layer.values_recent.shape[-2], layer.cumulative_length, *mask]
        np.testing.assert_array_equal(state, g[f"{name}_step{s}_state"], err_msg=f"step {s}")
    # the reference hands back one token, rank 3, once the past exceeds the window
    assert K.ndim == 3


@pytest.mark.parametrize("name", list(SLIDING))
def test_sliding_fix_returns_the_announced_window(name):
    """fix=True: every call returns the last kv_length tokens of the full layer's
    K/V, kv_length as get_mask_sizes() announced it before the call."""
    cfg = Cfg(**SLIDING[name])
    kx = synth.kv_tensor(1, 2, 140, 64, seed=9, n_out=2, factor=8.0)
    vx = synth.kv_tensor(1, 2, 140, 64, seed=10, n_out=2, factor=8.0)
    w = 96
    fixed = cache_ref.SlidingLayerRef(cfg, w, fix=True)
    full = cache_ref.CacheLayerRef(cfg)
    for s in range(61):
        lo, hi = (0, 80) if s == 0 else (79 + s, 80 + s)
        kv_len, _ = fixed.get_mask_sizes(hi - lo)
        K, V = fixed.update(kx[:, :, lo:hi], vx[:, :, lo:hi])
        Kf, Vf = full.update(kx[:, :, lo:hi], vx[:, :, lo:hi])
        assert K.shape[-2] == kv_len, (s, K.shape, kv_len)
        np.testing.assert_array_equal(K, Kf[:, :, -kv_len:])
        np.testing.assert_array_equal(V, Vf[:, :, -kv_len:])
