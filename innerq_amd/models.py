"""The reference's model hooks (src/innerq/models/llama_innerq.py:7-18,
mistral_innerq.py) on the drop-in cache: ``generate`` builds an
``innerq_amd.cache.DynamicCache`` from the model config (k_bits, v_bits,
group sizes, windows, modes as config attributes).  Loaded with
``attn_implementation="innerq_fused"`` (registered by importing this module),
decode steps attend over the packed cache directly (innerq_amd.attention)."""
from transformers.models.llama.modeling_llama import LlamaForCausalLM
from transformers.models.mistral.modeling_mistral import MistralForCausalLM

from . import attention  # noqa: F401  (registers the "innerq_fused" attention)
from .cache import DynamicCache


class InnerqLlamaForCausalLM(LlamaForCausalLM):
    def _prepare_cache_for_generation(self, generation_config, model_kwargs, generation_mode, batch_size,
                                      max_cache_length):
        model_kwargs["past_key_values"] = DynamicCache(config=self.config.get_text_config(decoder=True))


class InnerqMistralForCausalLM(MistralForCausalLM):
    def _prepare_cache_for_generation(self, generation_config, model_kwargs, generation_mode, batch_size,
                                      max_cache_length):
        model_kwargs["past_key_values"] = DynamicCache(config=self.config.get_text_config(decoder=True))
