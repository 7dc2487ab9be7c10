"""The fused decode step inside transformers' models.

Registers the attention implementation ``"innerq_fused"``
(``AttentionInterface``, with sdpa's mask construction).  A model loaded with
``attn_implementation="innerq_fused"`` whose generation cache is the drop-in
``DynamicCache`` (``InnerqLlamaForCausalLM`` builds it) decodes each new token
with ``InnerqDynamicLayer.attend()``: QK^T, softmax and attn.V over the packed
K and V (``iq_decode_attention``), with no dense K/V in between.  A padding
mask that hides a prefix of each sequence (left padding, as generate() pads a
batch) becomes per-sequence start tokens of that call.  The reference instead
dequantizes the whole cache in ``update()`` and runs the model's attention
over it (src/innerq/cache.py:242-270, TF/models/llama/modeling_llama.py:201-210);
prefill, other mask patterns and layouts the fused kernels do not take keep
that path.
"""
from __future__ import annotations

import weakref

import torch
from transformers import AttentionInterface
from transformers.integrations.sdpa_attention import sdpa_attention_forward
from transformers.masking_utils import AttentionMaskInterface, sdpa_mask

from .cache import FUSED_ATTENTION


# (weak reference to the mask, its version counter, answer) of the last mask
# inspected: every layer of one forward pass receives the same mask object,
# so the device-to-host read that the answer needs happens once per decode
# step, not once per layer.  The version counter changes with every in-place
# edit, so a mask object reused and edited between passes is read again; the
# weak reference keeps no mask alive, and a different mask (another model's,
# another pass's) is a different object.
_last_mask: list = [None, -1, None]


def _hidden_prefix(attention_mask):
    """What the mask hides of the cache tokens its last query row covers: None
    (nothing), the per-sequence counts of leading tokens it hides when each row
    hides a prefix and nothing else (left padding; the fused kernels start each
    sequence there), or False (any other pattern: the dense path)."""
    if attention_mask is None:
        return None
    ref, ver, ans = _last_mask
    if ref is not None and ref() is attention_mask and ver == attention_mask._version:
        return ans
    m = attention_mask
    hide = ~m if m.dtype == torch.bool else m < 0
    ans = False
    if hide.dim() == 4:
        last = hide[:, :, -1, :]                       # [B, heads or 1, kv]
        n = last.shape[-1]
        same = (last == last[:, :1]).all()             # every head row alike
        row = last[:, 0]
        count = row.sum(-1)
        lead = row.to(torch.int32).cumprod(-1).sum(-1)  # leading hidden tokens
        ok = same & (count == lead).all() & (count < n).all()
        vals = torch.cat([ok.reshape(1).to(torch.int64), count.to(torch.int64)]).tolist()  # one read
        if vals[0]:
            pads = vals[1:]
            ans = pads if any(pads) else None
    _last_mask[:] = [weakref.ref(attention_mask), attention_mask._version, ans]
    return ans


def innerq_fused_attention(module, query, key, value, attention_mask, dropout: float = 0.0, scaling=None,
                           **kwargs):
    """transformers attention function: query [B, Hq, q_len, D]; returns
    ([B, q_len, Hq, D], None).  A key tensor tagged by DynamicCache.update
    (fused-decode mode, one new token) is served by its layer's attend();
    anything else by sdpa over the given (or, for a tagged step that attend()
    cannot take, the layer's dequantized) K and V."""
    layer = getattr(key, "_innerq_layer", None)
    if layer is None:
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout, scaling=scaling,
                                      **kwargs)
    if scaling is None:
        scaling = query.shape[-1] ** -0.5
    nrep = query.shape[1] // key.shape[1]
    pads = _hidden_prefix(attention_mask)
    if pads is not None and (pads is False or attention_mask.shape[-1] != layer.attend_length()
                             or len(pads) != query.shape[0]):
        pads = False  # a mask over other columns than the tokens attend() reads
    if (pads is False or dropout or query.dtype != layer.dtype or query.shape[-1] not in (64, 128)
            or nrep not in (1, 2, 4, 8) or query.shape[1] != nrep * key.shape[1]):
        k, v = layer.get_deq_tensors()
        return sdpa_attention_forward(module, query, k, v, attention_mask, dropout=dropout, scaling=scaling,
                                      **kwargs)
    out = layer.attend(query, scaling, pads)  # [B, Hq, 1, D]
    return out.transpose(1, 2).contiguous(), None


AttentionInterface.register(FUSED_ATTENTION, innerq_fused_attention)
AttentionMaskInterface.register(FUSED_ATTENTION, sdpa_mask)
