"""The drop-in API surface (innerq_amd.quant / innerq_amd.cache) without a GPU:
names, configuration parsing, error behaviour and the no-CPU-path rule."""
import pytest
import torch

from innerq_amd import cache as C
from innerq_amd import quant as IQ


class Cfg:
    def __init__(self, **kw):
        self.__dict__.update(kw)


def test_qmode_matches_reference():
    assert IQ.QMode.from_str(" Asymmetric ") is IQ.QMode.ASYM
    assert IQ.QMode.from_str("symmetric") is IQ.QMode.SYM
    assert IQ.QMode.from_str("HYBRID") is IQ.QMode.HYBRID
    with pytest.raises(ValueError):
        IQ.QMode.from_str("int4")


def test_quant_api_names():
    for axis in ("channeldim", "tokendim"):
        for mode in ("asym", "sym"):
            assert callable(getattr(IQ, f"quantize_{axis}_{mode}"))
            assert callable(getattr(IQ, f"dequantize_{axis}_{mode}"))
    assert callable(IQ.quantize_hybrid(IQ.quantize_channeldim_asym, IQ.quantize_channeldim_sym,
                                       IQ.dequantize_channeldim_asym, IQ.dequantize_channeldim_sym))
    assert callable(IQ.dequantize_hybrid(IQ.dequantize_tokendim_asym, IQ.dequantize_tokendim_sym))


def test_no_cpu_path():
    x = torch.zeros(1, 2, 64, 64, dtype=torch.float16)
    with pytest.raises(TypeError):
        IQ.quantize_channeldim_asym(x, 32, 4)
    layer = C.InnerqDynamicLayer(Cfg(k_bits=4, v_bits=4), 0)
    with pytest.raises(TypeError):
        layer.update(x, x)


def test_config_defaults_match_reference():
    l = C.InnerqDynamicLayer(Cfg(), 3)
    assert (l.key_bits, l.value_bits, l.key_quantize, l.value_quantize) == (16, 16, False, False)
    assert (l.key_group_size, l.value_group_size, l.key_w_recent, l.value_w_recent) == (32, 32, 32, 32)
    assert (l.key_w_sink, l.value_w_sink, l.key_flush_size, l.value_flush_size) == (0, 0, 32, 32)
    assert (l.key_normalize, l.key_normalization_factor) == (False, None)
    assert (l.key_quantize_over_token, l.value_quantize_over_token) == (False, True)
    assert l.key_quantize_mode is IQ.QMode.SYM and l.value_quantize_mode is IQ.QMode.SYM
    assert (l.layer_idx, l.cumulative_length, l.is_initialized) == (3, 0, False)
    assert l.keys_q is None and l.values_scale_factor is None


def test_layer_queries_and_errors():
    l = C.InnerqDynamicLayer(Cfg(k_bits=2, v_bits=2), 0)
    l.cumulative_length = 10
    assert l.get_mask_sizes(torch.arange(3)) == (13, 0)   # cache_position (cache.py:398-402)
    assert l.get_mask_sizes(3) == (13, 0)                  # query_length (transformers 5.15)
    assert l.get_seq_length() == 10 and l.get_max_cache_shape() == -1 and l.get_max_length() == -1
    with pytest.raises(ValueError):
        l.crop(4)
    with pytest.raises(Exception):
        l.batch_repeat_interleave(2)
    with pytest.raises(Exception):
        l.batch_select_indices(torch.tensor([0]))


def test_sliding_window_layer_queries():
    l = C.InnerqDynamicSlidingWindowLayer(Cfg(k_bits=4), 0, sliding_window=8)
    assert l.is_sliding and l.get_max_cache_shape() == 8
    l.cumulative_length = 5
    assert l.get_mask_sizes(1) == (6, 0)
    l.cumulative_length = 20
    assert l.get_mask_sizes(torch.arange(1)) == (8, 13)


def test_dynamic_cache_layer_types():
    from transformers import LlamaConfig, MistralConfig
    cfg = LlamaConfig(num_hidden_layers=4, num_attention_heads=4, num_key_value_heads=2, hidden_size=64,
                      intermediate_size=32, vocab_size=16)
    cfg.k_bits = 3
    cache = C.DynamicCache(config=cfg)
    assert len(cache.layers) == 4 and not any(l.is_sliding for l in cache.layers)
    assert all(l.key_bits == 3 for l in cache.layers)
    mcfg = MistralConfig(num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, hidden_size=64,
                         intermediate_size=32, vocab_size=16, sliding_window=16)
    cache = C.DynamicCache(config=mcfg)
    assert all(isinstance(l, C.InnerqDynamicSlidingWindowLayer) and l.sliding_window == 16 for l in cache.layers)


def test_model_hooks_install_the_drop_in_cache():
    from transformers import LlamaConfig
    from innerq_amd.models import InnerqLlamaForCausalLM
    cfg = LlamaConfig(num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, hidden_size=64,
                      intermediate_size=32, vocab_size=16)
    cfg.k_bits, cfg.v_bits = 4, 2
    model = InnerqLlamaForCausalLM(cfg)
    kw = {}
    model._prepare_cache_for_generation(None, kw, None, 1, 0)
    cache = kw["past_key_values"]
    assert isinstance(cache, C.DynamicCache) and len(cache.layers) == 2
    assert cache.layers[0].key_bits == 4 and cache.layers[1].value_bits == 2


def test_fused_attention_registered():
    """Importing innerq_amd.models registers the "innerq_fused" attention (and
    sdpa's mask construction for it); a cache built from a config that selects
    it decodes in fused mode."""
    from transformers import AttentionInterface, LlamaConfig
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS
    import innerq_amd.models  # noqa: F401
    from innerq_amd.attention import innerq_fused_attention
    assert AttentionInterface._global_mapping[C.FUSED_ATTENTION] is innerq_fused_attention
    assert C.FUSED_ATTENTION in ALL_MASK_ATTENTION_FUNCTIONS._global_mapping
    cfg = LlamaConfig(num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, hidden_size=256,
                      intermediate_size=32, vocab_size=16)
    cfg._attn_implementation = C.FUSED_ATTENTION
    assert C.DynamicCache(config=cfg).fused_decode
    cfg._attn_implementation = "sdpa"
    assert not C.DynamicCache(config=cfg).fused_decode
    assert not C.DynamicCache().fused_decode


def test_fused_attention_untagged_keys_take_sdpa():
    """Keys that no fused-mode cache tagged (prefill, other caches) go to sdpa."""
    import torch
    from transformers.integrations.sdpa_attention import sdpa_attention_forward
    from innerq_amd.attention import innerq_fused_attention

    class M(torch.nn.Module):
        is_causal = True
        num_key_value_groups = 2

    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, 4, 5, 16, generator=g)
    k = torch.randn(1, 2, 5, 16, generator=g)
    v = torch.randn(1, 2, 5, 16, generator=g)
    a, _ = innerq_fused_attention(M(), q, k, v, None, scaling=0.25)
    b, _ = sdpa_attention_forward(M(), q, k, v, None, scaling=0.25)
    assert torch.equal(a, b)


def test_mask_answer_follows_in_place_edits():
    """The padding answer is cached per mask object and version: a mask reused and
    edited in place between passes (padding added) is read again, so a padded
    batch never reaches the fused kernels on a stale "no padding" answer; the
    cache holds no reference that keeps a mask alive."""
    import gc
    import weakref

    import torch
    from innerq_amd import attention as att
    m = torch.zeros(2, 1, 1, 8)  # additive mask: 0 = attend
    assert att._hidden_prefix(m) is None
    assert att._hidden_prefix(m) is None  # cached
    m[1, 0, 0, :3] = float("-inf")        # padding added in place
    assert att._hidden_prefix(m) == [0, 3]
    m.zero_()
    assert att._hidden_prefix(m) is None
    b = torch.ones(1, 1, 1, 8, dtype=torch.bool)
    assert att._hidden_prefix(b) is None
    b[0, 0, 0, 0] = False
    assert att._hidden_prefix(b) == [1]
    r = weakref.ref(b)
    del b
    gc.collect()
    assert r() is None
    assert att._hidden_prefix(None) is None


def test_mask_hidden_prefix_patterns():
    """Left padding (a hidden prefix per sequence, nothing else) gives the
    per-sequence start tokens the fused kernels take; a hole after the first
    attended token, a fully hidden row, or head rows that differ give False
    (the dense path).  The last query row decides (a decode step's mask)."""
    import torch
    from innerq_amd import attention as att
    b = torch.ones(3, 1, 2, 10, dtype=torch.bool)
    b[0, :, :, :4] = False
    b[2, :, :, :1] = False
    b[:, :, 0, :] = False                  # earlier query rows do not matter
    assert att._hidden_prefix(b) == [4, 0, 1]
    hole = b.clone()
    hole[1, :, -1, 6] = False              # a hidden token after attended ones
    assert att._hidden_prefix(hole) is False
    full = b.clone()
    full[1, :, -1, :] = False              # every token hidden
    assert att._hidden_prefix(full) is False
    f = torch.zeros(2, 4, 1, 6)
    f[0, :, :, :2] = torch.finfo(torch.float32).min
    assert att._hidden_prefix(f) == [2, 0]
    f[0, 3, :, 2] = torch.finfo(torch.float32).min  # one head row differs
    assert att._hidden_prefix(f) is False
