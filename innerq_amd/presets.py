"""The reference's InnerQ cache presets as configurations of the drop-in cache.

The reference sets these from its evaluation script (scripts/run_lmeval.sh:
innerq_base 94-113, innerq_small 114-133, innerq_hybrid 134-153, and the KIVI
comparators kivi 54-73, kivi_sink 74-93; the script's
K_* / V_* variables become the model-config attributes cache.py:71-91 reads).
The three InnerQ presets keep 32 fp16 sink tokens and a 96-token fp16 recent window per
role, quantize keys in 3-bit sym groups of 32 along head_dim with key
normalization and a flush of 1 token, and values in groups of 32 along tokens
with a flush of 32; they differ in the values' width and mode.

The script hands the key-normalization switch to lm-eval as
``normalize_key=$K_NORMALIZE`` (run_lmeval.sh:18), while the wrapper's
argument is ``key_normalize`` (src/innerq/lm_eval_innerq_wrapper.py:41, 111),
so whether the script's runs normalize keys depends on how lm-eval passes an
argument the wrapper does not name (lm-eval is not installed here).  These
presets follow the preset definitions (K_NORMALIZE=True); pass
``key_normalize=False`` to preset_config for the other reading.

    layer = InnerqDynamicLayer(preset_config("innerq_base"), 0)
"""
from __future__ import annotations

from types import SimpleNamespace

_COMMON = dict(k_bits=3, key_flush_size=1, value_flush_size=32, key_group_size=32, value_group_size=32,
               key_w_recent=96, value_w_recent=96, key_w_sink=32, value_w_sink=32, key_normalize=True,
               key_quantize_over_token=False, value_quantize_over_token=True, key_quantize_mode="symmetric")

_KIVI = dict(k_bits=2, v_bits=2, key_flush_size=32, value_flush_size=1, key_group_size=32, value_group_size=32,
             key_normalize=False, key_quantize_over_token=True, value_quantize_over_token=False,
             key_quantize_mode="asymmetric", value_quantize_mode="asymmetric")

PRESETS = {
    "innerq_base": dict(_COMMON, v_bits=3, value_quantize_mode="symmetric"),
    "innerq_small": dict(_COMMON, v_bits=2, value_quantize_mode="symmetric"),
    "innerq_hybrid": dict(_COMMON, v_bits=2, value_quantize_mode="hybrid"),
    # the script's KIVI comparators (run_lmeval.sh:54-73 and 74-93): 2-bit asym
    # keys grouped along tokens, flushed 32 at a time, and 2-bit asym values
    # grouped along head_dim, flushed one token at a time; fp16 windows of 128
    # recent tokens, or of 32 sinks and 96 recent tokens.  These layers decode
    # through update()'s dense K/V: attend() reads keys grouped along head_dim
    # and values along tokens only.
    "kivi": dict(_KIVI, key_w_recent=128, value_w_recent=128, key_w_sink=0, value_w_sink=0),
    "kivi_sink": dict(_KIVI, key_w_recent=96, value_w_recent=96, key_w_sink=32, value_w_sink=32),
}


def preset_config(name: str, **overrides) -> SimpleNamespace:
    """A config object carrying preset ``name``'s cache attributes (plus overrides)."""
    if name not in PRESETS:
        raise KeyError(f"unknown preset {name!r}; one of {sorted(PRESETS)}")
    return SimpleNamespace(**{**PRESETS[name], **overrides})
