"""Drop-in for the reference's ``innerq.cache`` (src/innerq/cache.py) on MI355X.

``InnerqDynamicLayer``, ``InnerqDynamicSlidingWindowLayer`` and
``DynamicCache`` keep the reference's configuration attributes, state machine
(sinks, recent windows, flush of the oldest tokens, key normalization) and
``update()`` contract: the first call returns its inputs, later calls return
the dense fp16 K and V of [sink | dequantized | recent] (cache.py:235-281,
382-396), bit-identical to the reference's.

What differs is the storage: quantized tokens are kept packed (2/3/4-bit
codes + fp16 scale/zero) in ``ops.PackedStore`` and quantized on append by the
gfx950 kernels, instead of int32 code tensors grown with torch.cat.  The
reference's state attributes ``keys_q`` / ``keys_scale_factor`` /
``keys_zp_sign`` (and ``values_*``) are read-only views unpacked on access.

Two methods serve the fused decode path, which the reference does not have:
``append(k, v)`` advances the state without materializing K and V, and
``attend(q, scaling)`` runs softmax(q K^T * scaling) V over [sink | packed |
recent] in one gfx950 decode kernel chain (ops.decode_attention).
"""
from __future__ import annotations

from collections.abc import Iterable
import copy
from typing import Any, Optional, Sequence

import torch
from transformers.cache_utils import Cache, CacheLayerMixin

from . import ops
from .quant import QMode

# attn_implementation name of the fused decode path (innerq_amd.attention)
FUSED_ATTENTION = "innerq_fused"


class _Quantized:
    """The packed tokens of one role (K or V) of a layer.

    axis 'channel' groups along head_dim (quant.py:75-77), 'token' along tokens
    (quant.py:79-81).  Hybrid (quant.py:133-176) is one packed store that keeps,
    per group, the representation the reference's mask selects: (bits-1)-bit
    asym or bits-bit sym codes, marked by a flag bit in the group's scale.
    """

    def __init__(self, axis: str, like: torch.Tensor, group: int, bits: int, mode: QMode):
        B, H, _, D = like.shape
        self.axis, self.group, self.bits, self.mode = axis, group, bits, mode
        self.store = ops.PackedStore(axis, B, H, D, group, bits, mode.value, like.device, dtype=like.dtype)

    @property
    def length(self) -> int:
        return self.store.length

    def append(self, x: torch.Tensor, norm: Optional[torch.Tensor]) -> None:
        """Quantize x [B,H,n,D] (divided by norm in fp16 first, keys only) and append it."""
        if norm is not None and self.axis != "channel":
            raise NotImplementedError("key normalization is supported for keys grouped along head_dim")
        self.store.append(x, norm=norm)

    def dequant_into(self, out: torch.Tensor, norm: Optional[torch.Tensor]) -> None:
        """Dense values (times norm) of every packed token, written into the view ``out`` (the
        activation dtype or fp32)."""
        self.store.dequant(0, self.length, out=out, norm=norm)

    def reference_tensors(self):
        """(codes, scale, zero|signs) as quant.py returns them (dicts for hybrid)."""
        return ops.unpack_store(self.store)


class InnerqDynamicLayer(CacheLayerMixin):
    """cache.py:60-419 with packed quantized storage."""
    is_sliding = False

    def __init__(self, config, layer_idx):
        self.parse_config(config)
        self.layer_idx = layer_idx
        self.cumulative_length = 0
        super().__init__()

    def parse_config(self, config):
        """The reference's 15 configuration attributes and defaults (cache.py:71-91)."""
        self.key_bits = getattr(config, 'k_bits', 16)
        self.value_bits = getattr(config, 'v_bits', 16)
        self.key_quantize = False if self.key_bits >= 16 else True
        self.value_quantize = False if self.value_bits >= 16 else True

        self.key_group_size = getattr(config, 'key_group_size', 32)
        self.value_group_size = getattr(config, 'value_group_size', 32)
        self.key_w_recent = getattr(config, 'key_w_recent', 32)
        self.value_w_recent = getattr(config, 'value_w_recent', 32)
        self.key_w_sink = getattr(config, 'key_w_sink', 0)
        self.value_w_sink = getattr(config, 'value_w_sink', 0)
        self.key_flush_size = getattr(config, 'key_flush_size', 32)
        self.value_flush_size = getattr(config, 'value_flush_size', 32)
        self.key_normalize = getattr(config, 'key_normalize', False)
        self.key_normalization_factor = None

        self.key_quantize_over_token = getattr(config, 'key_quantize_over_token', False)
        self.value_quantize_over_token = getattr(config, 'value_quantize_over_token', True)

        self.key_quantize_mode = QMode.from_str(getattr(config, 'key_quantize_mode', 'symmetric'))
        self.value_quantize_mode = QMode.from_str(getattr(config, 'value_quantize_mode', 'symmetric'))
        self._kq: Optional[_Quantized] = None
        self._vq: Optional[_Quantized] = None
        self._kwin: Optional[ops.RecentWindow] = None
        self._vwin: Optional[ops.RecentWindow] = None

    # ---- recent windows (cache.py keys_recent / values_recent): views of
    # RecentWindow buffers that a decode step appends to in place ----
    @property
    def keys_recent(self):
        return None if self._kwin is None else self._kwin.tensor

    @keys_recent.setter
    def keys_recent(self, x):
        self._kwin = None if x is None else ops.RecentWindow(x)

    @property
    def values_recent(self):
        return None if self._vwin is None else self._vwin.tensor

    @values_recent.setter
    def values_recent(self, x):
        self._vwin = None if x is None else ops.RecentWindow(x)

    # ---- reference state attributes (read-only views of the packed stores) ----
    def _ref(self, q: Optional[_Quantized], i: int):
        return None if q is None or q.length == 0 else q.reference_tensors()[i]

    @property
    def keys_q(self):
        return self._ref(self._kq, 0)

    @property
    def keys_scale_factor(self):
        return self._ref(self._kq, 1)

    @property
    def keys_zp_sign(self):
        return self._ref(self._kq, 2)

    @property
    def values_q(self):
        return self._ref(self._vq, 0)

    @property
    def values_scale_factor(self):
        return self._ref(self._vq, 1)

    @property
    def values_zp_sign(self):
        return self._ref(self._vq, 2)

    # ---- prefill (cache.py:121-233) ----
    def _key_norm(self, key_states: torch.Tensor) -> Optional[torch.Tensor]:
        """The key normalization factor, computed once from the first keys that are
        quantized (cache.py:121-126); the quantize kernels divide by it."""
        if not self.key_normalize:
            return None
        if self.key_normalization_factor is None:
            self.key_normalization_factor = ops.key_norm_factor(key_states)
        return self.key_normalization_factor

    def normalize_keys(self, key_states: torch.Tensor) -> torch.Tensor:
        """cache.py:121-126: the keys divided by the normalization factor (set from
        these keys if unset), as the reference's method returns them."""
        norm = self._key_norm(key_states)
        return key_states if norm is None else key_states / norm

    def unnormalize_keys(self, key_states: torch.Tensor) -> torch.Tensor:
        """cache.py:128-133."""
        if self.key_normalize:
            if self.key_normalization_factor is None:
                raise Exception('key_normalize is set to True but key_normalization_factor is not set')
            key_states = key_states * self.key_normalization_factor
        return key_states

    def initialize_keys_sink(self, key_states: torch.Tensor) -> torch.Tensor:
        viable_w_sink_key = min(self.key_w_sink, key_states.shape[-2])
        if self.key_quantize:
            self.keys_sink = key_states[:, :, :viable_w_sink_key]
            key_states = key_states[:, :, viable_w_sink_key:]
        else:
            shape = list(key_states.shape)
            shape[-2] = 0
            self.keys_sink = torch.zeros(shape, dtype=self.dtype, device=self.device)
        return key_states

    def initialize_values_sink(self, value_states: torch.Tensor) -> torch.Tensor:
        viable_w_sink_value = min(self.value_w_sink, value_states.shape[-2])
        if self.value_quantize:
            self.values_sink = value_states[:, :, :viable_w_sink_value]
            value_states = value_states[:, :, viable_w_sink_value:]
        else:
            shape = list(value_states.shape)
            shape[-2] = 0
            self.values_sink = torch.zeros(shape, dtype=self.dtype, device=self.device)
        return value_states

    def initialize_keys_recent(self, key_states: torch.Tensor) -> torch.Tensor:
        if self.key_quantize:
            viable_recent_size_key = min(self.key_w_recent, key_states.shape[-2])
            if self.key_quantize_over_token:
                while (key_states.shape[-2] - viable_recent_size_key) % self.key_flush_size != 0:
                    viable_recent_size_key -= 1
        else:
            viable_recent_size_key = key_states.shape[-2]
        nq = key_states.shape[-2] - viable_recent_size_key
        self.keys_recent = key_states[:, :, nq:, :].contiguous()
        return key_states[:, :, :nq, :].contiguous()

    def initialize_values_recent(self, value_states: torch.Tensor) -> torch.Tensor:
        if self.value_quantize:
            viable_recent_size_value = min(self.value_w_recent, value_states.shape[-2])
            if self.value_quantize_over_token:
                while (value_states.shape[-2] - viable_recent_size_value) % self.value_flush_size != 0:
                    viable_recent_size_value -= 1
        else:
            viable_recent_size_value = value_states.shape[-2]
        nq = value_states.shape[-2] - viable_recent_size_value
        self.values_recent = value_states[:, :, nq:, :].contiguous()
        return value_states[:, :, :nq, :].contiguous()

    def _kq_for(self, like: torch.Tensor) -> _Quantized:
        if self._kq is None:
            axis = "token" if self.key_quantize_over_token else "channel"
            self._kq = _Quantized(axis, like, self.key_group_size, self.key_bits, self.key_quantize_mode)
        return self._kq

    def _vq_for(self, like: torch.Tensor) -> _Quantized:
        if self._vq is None:
            axis = "token" if self.value_quantize_over_token else "channel"
            self._vq = _Quantized(axis, like, self.value_group_size, self.value_bits, self.value_quantize_mode)
        return self._vq

    def _quantize_keys(self, key_states: torch.Tensor) -> None:
        if key_states.numel() == 0:
            return
        norm = self._key_norm(key_states)
        self._kq_for(key_states).append(key_states, norm)

    def _quantize_values(self, value_states: torch.Tensor) -> None:
        if value_states.numel() == 0:
            return
        self._vq_for(value_states).append(value_states, None)

    def initialize_keys_q(self, key_states: torch.Tensor) -> None:
        if self.key_quantize:
            self._quantize_keys(key_states)

    def initialize_values_q(self, value_states: torch.Tensor) -> None:
        if self.value_quantize:
            self._quantize_values(value_states)

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        ops.require_act(key_states, "key_states")
        ops.require_act(value_states, "value_states", key_states.dtype)
        self.dtype, self.device = key_states.dtype, key_states.device
        key_states = self.initialize_keys_sink(key_states)
        value_states = self.initialize_values_sink(value_states)
        key_states = self.initialize_keys_recent(key_states)
        value_states = self.initialize_values_recent(value_states)
        self.initialize_keys_q(key_states)
        self.initialize_values_q(value_states)
        self._keep_dequantized_rows()
        self.is_initialized = True

    # the reference's prefill and decode helpers (cache.py:212-224, 309-365), kept
    # for callers and subclasses that drive them; update() / append() run the same
    # state changes through the fused launches above and below
    def initialize_sinks(self, key_states: torch.Tensor, value_states: torch.Tensor):
        return self.initialize_keys_sink(key_states), self.initialize_values_sink(value_states)

    def initialize_recents(self, key_states: torch.Tensor, value_states: torch.Tensor):
        return self.initialize_keys_recent(key_states), self.initialize_values_recent(value_states)

    def initial_quantization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        self.initialize_keys_q(key_states)
        self.initialize_values_q(value_states)

    def update_recents(self, key_states: torch.Tensor, value_states: torch.Tensor):
        return self.update_keys_recent(key_states), self.update_values_recent(value_states)

    def quantize_new_keys(self, key_states: torch.Tensor) -> None:
        """cache.py:314-339: quantize these keys (normalized) and append them."""
        self._quantize_keys(key_states)

    def quantize_new_values(self, value_states: torch.Tensor) -> None:
        """cache.py:341-365: quantize these values and append them."""
        self._quantize_values(value_states)

    def _keep_dequantized_rows(self) -> None:
        """Tokens packed in one role while the other role still holds them in its
        window (K flushes token by token, V by groups of tokens) are attended as
        dense rows: each window's buffer keeps its flushed tokens' rows with their
        dequantized values (keys times the normalization factor; in the
        activation dtype: what update() returns for them), so a decode's packed
        segments of both roles can end at one V group boundary and the window
        kernel reads no packed rows.  Set up after the prefill with the rows past
        that boundary packed so far (window flushes keep them up).  fp16 layers:
        a bf16 row would hold the values 8 bits short of the fp32 dequantization
        that the packed reads give."""
        if not (self.key_quantize and not self.key_quantize_over_token and self.value_quantize
                and self.value_quantize_over_token and self.dtype == torch.float16):
            return
        kq = self._kq.length if self._kq is not None else 0
        vq = self._vq.length if self._vq is not None else 0
        e = self._packed_end()
        kend, vend = self.keys_sink.shape[-2] + kq, self.values_sink.shape[-2] + vq
        if self._kwin is not None and self.key_group_size <= 64:
            keep = self.value_w_recent + self.value_flush_size + 64
            p = min(kend - e, keep) if e is not None else 0
            pre = self._kq.store.dequant(kq - p, p, norm=self.key_normalization_factor) if p > 0 else None
            self._kwin = ops.RecentWindow(self._kwin.tensor, pre=pre, deq_rows=True, keep=keep)
        if self._vwin is not None and self.value_group_size <= 64:
            keep = self.key_w_recent + self.key_flush_size + self.value_group_size + 64
            p = min(vend - e, keep) if e is not None else 0
            pre = None
            if p > 0:  # dequantized by whole groups, the last p rows kept
                t0 = (vq - p) // self.value_group_size * self.value_group_size
                pre = self._vq.store.dequant(t0, vq - t0)[:, :, vq - t0 - p:]
            self._vwin = ops.RecentWindow(self._vwin.tensor, pre=pre, deq_rows=True, keep=keep)

    def _packed_end(self) -> Optional[int]:
        """The token where a decode's packed segments of both roles end: the end of
        the shorter store, rounded down to a V group boundary (None: no store)."""
        if self._kq is None or self._vq is None:
            return None
        nks, nvs = self.keys_sink.shape[-2], self.values_sink.shape[-2]
        e = min(nks + self._kq.length, nvs + self._vq.length)
        e = nvs + (e - nvs) // self.value_group_size * self.value_group_size
        return e if e >= max(nks, nvs) else None

    # ---- decode (cache.py:283-396) ----
    def _flush_sizes(self, m: int) -> tuple[int, int]:
        """Tokens flushed from [window | m new tokens] into the stores (cache.py:283-306)."""
        kf = self.key_flush_size if self.key_quantize and self._kwin.n + m >= self.key_flush_size else 0
        vf = self.value_flush_size if self.value_quantize and self._vwin.n + m >= self.value_flush_size else 0
        return kf, vf

    def update_keys_recent(self, key_states: torch.Tensor) -> torch.Tensor:
        """cache.py:283-294: append to the window, return (and drop) the tokens to flush."""
        kf = self._flush_sizes(key_states.shape[-2])[0]
        full = torch.cat([self.keys_recent, key_states], dim=-2)
        self.keys_recent = full[:, :, kf:]
        return full[:, :, :kf]

    def update_values_recent(self, value_states: torch.Tensor) -> torch.Tensor:
        """cache.py:296-307: append to the window, return (and drop) the tokens to flush."""
        vf = self._flush_sizes(value_states.shape[-2])[1]
        full = torch.cat([self.values_recent, value_states], dim=-2)
        self.values_recent = full[:, :, vf:]
        return full[:, :, :vf]

    def add_to_cache(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        """cache.py:309-365 in one launch (ops.window_append): the new tokens join the
        recent windows, the oldest flush into the packed stores."""
        kf, vf = self._flush_sizes(key_states.shape[-2])
        norm = None
        if kf:
            kq = self._kq_for(key_states)
            if self.key_normalize:
                if self.key_normalization_factor is None:  # the first flushed keys set it (cache.py:121-126)
                    self._key_norm(torch.cat([self.keys_recent, key_states], dim=-2)[:, :, :kf])
                norm = self.key_normalization_factor
        if vf:
            self._vq_for(value_states)
        ops.window_append(self._kwin, key_states, kf, self._kq.store if kf else None, norm,
                          self._vwin, value_states, vf, self._vq.store if vf else None)

    def _dense(self, sink, q: Optional[_Quantized], recent, norm, dtype) -> torch.Tensor:
        """[sink | dequantized (times norm) | recent] in dtype: one rounding of the
        fp32 dequantized values, as the reference's cat + .to(dtype)."""
        ns, nq, nr = sink.shape[-2], (q.length if q is not None else 0), recent.shape[-2]
        B, H, _, D = recent.shape
        out = torch.empty(B, H, ns + nq + nr, D, dtype=dtype, device=self.device)
        if ns:
            out[:, :, :ns].copy_(sink)
        if nq:
            q.dequant_into(out[:, :, ns:ns + nq], norm)
        if nr:
            out[:, :, ns + nq:].copy_(recent)
        return out

    def _deq_dtype(self, q: Optional[_Quantized]):
        # cache.py:235-281: fp32 once a dequantized segment joins the cat
        return torch.float32 if q is not None and q.length else self.dtype

    def get_keys_deq(self) -> torch.Tensor:
        return self._dense(self.keys_sink, self._kq, self.keys_recent, self.key_normalization_factor,
                           self._deq_dtype(self._kq))

    def get_values_deq(self) -> torch.Tensor:
        return self._dense(self.values_sink, self._vq, self.values_recent, None, self._deq_dtype(self._vq))

    def get_deq_tensors(self) -> tuple[torch.Tensor, torch.Tensor]:
        # written in self.dtype directly: the same values as get_*_deq().to(self.dtype)
        return (self._dense(self.keys_sink, self._kq, self.keys_recent, self.key_normalization_factor, self.dtype),
                self._dense(self.values_sink, self._vq, self.values_recent, None, self.dtype))

    def update(
        self,
        key_states: torch.Tensor,
        value_states: torch.Tensor,
        cache_kwargs: dict[str, Any] | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        self.cumulative_length += key_states.shape[-2]
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
            return key_states, value_states
        self.add_to_cache(key_states, value_states)
        return self.get_deq_tensors()

    def append(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        """update() without materializing K and V (for attend())."""
        self.cumulative_length += key_states.shape[-2]
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        else:
            self.add_to_cache(key_states, value_states)

    def _fused_refusal(self) -> Optional[str]:
        """Why attend() cannot read this layer's stores (None if it can): K must be
        grouped along head_dim, V along tokens (each asym, sym or hybrid), and a bf16
        layer's or a hybrid-K layer's K and V of one group size."""
        if (self.dtype == torch.bfloat16 and self._kq is not None and self._vq is not None
                and self._kq.group != self._vq.group):
            return "fused decode of a bf16 layer needs K and V of one group size"
        if self._kq is not None and self._kq.axis != "channel":
            return "fused decode reads keys grouped along the head_dim axis"
        if (self._kq is not None and self._kq.mode == QMode.HYBRID and self._vq is not None
                and self._kq.group != self._vq.group):
            return "fused decode of hybrid keys needs K and V of one group size"
        if self._vq is not None and self._vq.axis != "token":
            return "fused decode reads values grouped along the token axis"
        return None

    def fused_decode_ready(self, key_states: torch.Tensor) -> bool:
        """Whether attend() can serve this step: one new token per sequence, a
        prefilled layer, K grouped along head_dim and V along tokens (asym, sym or
        hybrid; hybrid K and bf16 layers with K and V of one group size)."""
        if not self.is_initialized or key_states.shape[-2] != 1:
            return False
        return self._fused_refusal() is None

    def attend(self, query_states: torch.Tensor, scaling: float, pads: Optional[Sequence[int]] = None
               ) -> torch.Tensor:
        """Decode attention of one new token per sequence over this layer's cache:
        softmax(q K^T * scaling, fp32) -> @ V (TF/models/llama/modeling_llama.py:201-210), with
        K and V read packed.  query_states [B, Hq, 1, D] in the layer's dtype (fp16 or bf16)
        -> [B, Hq, 1, D] of that dtype.  pads: per sequence, how many of its first
        tokens a padding mask hides (left padding; None: none)."""
        self._check_attend(query_states)
        return self._attend_rows(query_states[:, :, 0], scaling, self._attend_start(), pads)[:, :, None]

    def _attend_start(self) -> int:
        """The first token attend() reads (0: all of them)."""
        return 0

    def attend_length(self) -> int:
        """How many tokens attend() reads: the columns of a decode step's mask."""
        return self._n_tokens() - self._attend_start()

    def _check_attend(self, query_states: torch.Tensor) -> None:
        if query_states.dim() != 4 or query_states.shape[2] != 1:
            raise ValueError("attend() takes one query token per sequence: [B, Hq, 1, D]")
        if not self.is_initialized:
            raise RuntimeError("attend() needs a prefilled cache")
        why = self._fused_refusal()
        if why is not None:
            raise NotImplementedError(why)

    def _n_tokens(self) -> int:
        return self.keys_sink.shape[-2] + (self._kq.length if self._kq is not None else 0) + \
            self.keys_recent.shape[-2]

    def _attend_rows(self, q: torch.Tensor, scaling: float, s0: int,
                     pads: Optional[Sequence[int]]) -> torch.Tensor:
        """Sequence b attends to tokens [s0 + pads[b], T): one decode call over the
        whole batch without padding, else one per run of consecutive sequences of
        the same start, over batch views of the layer."""
        if pads is None or not any(pads):
            return self._attend_from(q, scaling, s0)
        B, n = q.shape[0], self._n_tokens() - s0
        pads = [int(p) for p in pads]
        if len(pads) != B or min(pads) < 0 or max(pads) >= n:
            raise ValueError(f"attend(): pads must give 0 <= pad < {n} for each of the {B} sequences, got {pads}")
        out = torch.empty_like(q)
        b0 = 0
        while b0 < B:
            b1 = b0 + 1
            while b1 < B and pads[b1] == pads[b0]:
                b1 += 1
            out[b0:b1] = self._attend_from(q[b0:b1], scaling, s0 + pads[b0], (b0, b1))
            b0 = b1
        return out

    def _attend_from(self, q: torch.Tensor, scaling: float, s0: int,
                     rows: Optional[tuple] = None) -> torch.Tensor:
        """decode_attention over this layer's tokens [s0, cumulative_length): the
        parts of [sink | packed | recent] of K and of V from token s0 on (of the
        sequences [rows[0], rows[1]) when rows is given, q holding theirs)."""
        def part_rows(x):
            return x if rows is None or x is None else x[rows[0]:rows[1]]

        def parts(sink, quant, nq, recent):
            # nq: the store's first nq tokens are read packed, then recent's rows
            ns = sink.shape[-2]
            dense_sink = part_rows(sink[:, :, s0:]) if s0 < ns else None
            t0 = min(max(s0 - ns, 0), nq)
            r0 = max(s0 - ns - nq, 0)
            dense_recent = part_rows(recent[:, :, r0:]) if recent.shape[-2] > r0 else None
            store = None
            if quant is not None:
                store = quant.store if rows is None else quant.store.batch_view(*rows)
                if nq < quant.length:
                    store = copy.copy(store)
                    store.length = nq
            return dense_sink, store, t0, dense_recent

        kq = self._kq.length if self._kq is not None else 0
        vq = self._vq.length if self._vq is not None else 0
        krecent, vrecent = self.keys_recent, self.values_recent
        e = self._packed_end()
        if e is not None and self._kwin is not None and self._vwin is not None:
            nk = self.keys_sink.shape[-2] + kq - e  # packed tokens past e, read as the rows kept
            nv = self.values_sink.shape[-2] + vq - e
            if nk <= self._kwin.shadow and nv <= self._vwin.shadow and (nk or nv):
                kq, krecent = kq - nk, self._kwin.rows_before(nk)
                vq, vrecent = vq - nv, self._vwin.rows_before(nv)
        ks, kst, kt0, kr = parts(self.keys_sink, self._kq, kq, krecent)
        vs, vst, vt0, vr = parts(self.values_sink, self._vq, vq, vrecent)
        norm = part_rows(self.key_normalization_factor) if self._kq is not None else None
        return ops.decode_attention(q, ks, kst, kr, vs, vst, vr, scaling, norm=norm, k_t0=kt0, v_t0=vt0)

    def get_mask_sizes(self, query_length) -> tuple[int, int]:
        """(kv_length, kv_offset); takes the query length (transformers >= 5.15) or
        the cache_position tensor (cache.py:398-402)."""
        if isinstance(query_length, torch.Tensor):
            query_length = query_length.shape[0]
        return self.get_seq_length() + query_length, 0

    def get_seq_length(self) -> int:
        return self.cumulative_length

    def get_max_length(self) -> int:
        return -1

    def get_max_cache_shape(self) -> int:
        return -1

    def crop(self, max_length: int) -> None:
        raise ValueError('This function is not implementable for quantized cache. '
                         'It leads to the loss of accuracy on the recent tokens')

    def batch_repeat_interleave(self, repeats: int) -> None:
        raise Exception('This function is not implemented yet.')

    def batch_select_indices(self, indices: torch.Tensor) -> None:
        raise Exception('This function is not implemented yet.')


class InnerqDynamicSlidingWindowLayer(InnerqDynamicLayer):
    """cache.py:421-461.

    By default update() behaves as the reference's: once the past exceeds the
    window it indexes ``[:, :, -w, :]``, a single token with the token axis
    dropped (cache.py:443-444), and one call earlier it returns one token more
    than get_mask_sizes() announces, so a model cannot decode past the window.
    The configuration attribute ``fix_sliding_window = True`` (not in the
    reference) returns instead the last w - 1 + q tokens of a q-token call once
    the past reaches the window: the kv_length that get_mask_sizes() announces.
    """
    is_sliding = True

    def __init__(self, config, layer_idx: int, sliding_window: int):
        super().__init__(config, layer_idx)
        self.sliding_window = sliding_window
        self.cumulative_length = 0
        self._sliding_window_tensor = torch.tensor(self.sliding_window, dtype=torch.long)
        self.fix_sliding_window = bool(getattr(config, "fix_sliding_window", False))

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        super().lazy_initialization(key_states, value_states)
        self._sliding_window_tensor = self._sliding_window_tensor.to(self.device)

    def update(self, key_states, value_states, cache_kwargs=None):
        full_key_states, full_value_states = super().update(key_states, value_states, cache_kwargs)
        q = key_states.shape[-2]
        past = self.cumulative_length - q
        w = self.sliding_window
        if not self.fix_sliding_window:
            if past > w:
                full_key_states = full_key_states[:, :, -w, :]
                full_value_states = full_value_states[:, :, -w, :]
        elif past >= w:
            full_key_states = full_key_states[:, :, -(w - 1 + q):]
            full_value_states = full_value_states[:, :, -(w - 1 + q):]
        return full_key_states, full_value_states

    def fused_decode_ready(self, key_states: torch.Tensor) -> bool:
        """With fix_sliding_window on, a one-token step attends to the last min(T, w)
        tokens, which attend() reads packed; without it the reference's update()
        (one token once the past exceeds the window) stays on the dense path."""
        if not self.fix_sliding_window or not self.is_initialized or key_states.shape[-2] != 1:
            return False
        return self._fused_refusal() is None

    def attend(self, query_states: torch.Tensor, scaling: float, pads: Optional[Sequence[int]] = None
               ) -> torch.Tensor:
        """Decode attention over the last min(T, w) tokens of the layer (T the tokens
        so far, this step's included): the window update() returns with
        fix_sliding_window on (w - 1 + q tokens of a q = 1 call once the past
        reaches w), read packed; pads count from the window's first token."""
        if not self.fix_sliding_window:
            raise NotImplementedError("attend() of a sliding-window layer needs fix_sliding_window = True")
        self._check_attend(query_states)
        return self._attend_rows(query_states[:, :, 0], scaling, self._attend_start(), pads)[:, :, None]

    def _attend_start(self) -> int:
        return max(self.cumulative_length - self.sliding_window, 0)

    def get_mask_sizes(self, query_length) -> tuple[int, int]:
        if isinstance(query_length, torch.Tensor):
            query_length = query_length.shape[0]
        is_full = self.cumulative_length >= self.sliding_window
        kv_offset = max(self.cumulative_length - self.sliding_window + 1, 0)
        if is_full:
            kv_length = self.sliding_window - 1 + query_length
        else:
            kv_length = self.cumulative_length + query_length
        return kv_length, kv_offset

    def get_max_length(self) -> int:
        return self.sliding_window

    def get_max_cache_shape(self) -> int:
        return self.sliding_window


class DynamicCache(Cache):
    """cache.py:463-496: one InnerqDynamic(SlidingWindow)Layer per decoder layer."""

    def __init__(
        self,
        ddp_cache_data: Iterable[tuple[torch.Tensor | None, ...]] | None = None,
        config=None,
        offloading: bool = False,
        offload_only_non_sliding: bool = False,
    ):
        layers = []
        if config is not None:
            decoder_config = config.get_text_config(decoder=True)
            sliding_window = getattr(decoder_config, "sliding_window", None) or getattr(
                decoder_config, "attention_chunk_size", None)
            layer_types = getattr(decoder_config, "layer_types", None)
            if layer_types is None:
                layer_types = ["sliding_attention" if sliding_window is not None else "full_attention"
                               for _ in range(decoder_config.num_hidden_layers)]
            if hasattr(decoder_config, "num_kv_shared_layers"):
                layer_types = layer_types[: -decoder_config.num_kv_shared_layers]
            for layer_idx, layer_type in enumerate(layer_types):
                if layer_type in ("sliding_attention", "chunked_attention"):
                    layers.append(InnerqDynamicSlidingWindowLayer(config=config, layer_idx=layer_idx,
                                                                  sliding_window=sliding_window))
                else:
                    layers.append(InnerqDynamicLayer(config=config, layer_idx=layer_idx))
        super().__init__(layers=layers, offloading=offloading, offload_only_non_sliding=offload_only_non_sliding)
        # the model's config, read again on every update(): the model may switch
        # its attention implementation while this cache lives
        self._config = config

    @property
    def fused_decode(self) -> bool:
        """Whether the model currently runs the fused attention (attn_implementation
        "innerq_fused"), which decodes over the packed stores without
        materializing K and V."""
        return self._config is not None and getattr(self._config, "_attn_implementation", None) == FUSED_ATTENTION

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int, *args, **kwargs):
        """Cache.update.  While the model runs the fused attention, a one-token
        step that the layer's attend() can serve is appended without
        materializing K and V; the returned key tensor carries the layer
        (``_innerq_layer``) for the fused attention function, which reads the
        packed cache through it.  Under any other attention implementation,
        checked on every call, update() returns the dense K and V as the
        reference does: append() and update() advance the same state, so the
        two kinds of step can follow each other in either order."""
        if layer_idx < len(self.layers) and self.fused_decode:
            layer = self.layers[layer_idx]
            if layer.fused_decode_ready(key_states):
                layer.append(key_states, value_states)
                key_states._innerq_layer = layer
                return key_states, value_states
        return super().update(key_states, value_states, layer_idx, *args, **kwargs)

    def __iter__(self):
        for layer in self.layers:
            yield layer.keys, layer.values, getattr(layer, "_sliding_window_tensor", None)
