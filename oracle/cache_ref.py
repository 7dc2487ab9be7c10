"""numpy restatement of the reference's InnerqDynamicLayer (TEST ORACLE ONLY).

Follows ``src/innerq/cache.py`` of mthcom/innerq:

* config parse                      cache.py:70-119
* key normalization                 cache.py:121-133
* sinks / recent window at prefill  cache.py:135-185
* prefill quantization              cache.py:187-233
* dense read path (get_*_deq)       cache.py:235-281
* recent-window flush               cache.py:283-312
* append quantization + concat      cache.py:314-380
* update()                          cache.py:382-396
* sliding-window layer              cache.py:421-461 (SlidingLayerRef)

State is held as numpy arrays ([B,H,T,D] fp16 for sinks / recents, the
quant_ref triples for the quantized middle).  ``update`` returns the dense
fp16 K and V the reference returns.
"""
from __future__ import annotations

import numpy as np

from . import quant_ref as Q

_QF = {
    ("asymmetric", False): (Q.quantize_channeldim_asym, Q.dequantize_channeldim_asym),
    ("asymmetric", True): (Q.quantize_tokendim_asym, Q.dequantize_tokendim_asym),
    ("symmetric", False): (Q.quantize_channeldim_sym, Q.dequantize_channeldim_sym),
    ("symmetric", True): (Q.quantize_tokendim_sym, Q.dequantize_tokendim_sym),
    ("hybrid", False): (Q.quantize_channeldim_hybrid, Q.dequantize_channeldim_hybrid),
    ("hybrid", True): (Q.quantize_tokendim_hybrid, Q.dequantize_tokendim_hybrid),
}


def _cat_triple(old, new, hybrid):
    if not hybrid:
        return np.concatenate([old, new], axis=2)
    return {k: np.concatenate([old[k], new[k]], axis=2) for k in old}


class CacheLayerRef:
    def __init__(self, config):
        g = lambda k, d: getattr(config, k, d)  # noqa: E731
        self.key_bits, self.value_bits = g("k_bits", 16), g("v_bits", 16)
        self.key_quantize = self.key_bits < 16
        self.value_quantize = self.value_bits < 16
        self.key_group_size = g("key_group_size", 32)
        self.value_group_size = g("value_group_size", 32)
        self.key_w_recent = g("key_w_recent", 32)
        self.value_w_recent = g("value_w_recent", 32)
        self.key_w_sink = g("key_w_sink", 0)
        self.value_w_sink = g("value_w_sink", 0)
        self.key_flush_size = g("key_flush_size", 32)
        self.value_flush_size = g("value_flush_size", 32)
        self.key_normalize = g("key_normalize", False)
        self.key_over_token = g("key_quantize_over_token", False)
        self.value_over_token = g("value_quantize_over_token", True)
        self.key_mode = Q.qmode_from_str(g("key_quantize_mode", "symmetric"))
        self.value_mode = Q.qmode_from_str(g("value_quantize_mode", "symmetric"))
        self.kq, self.kdq = _QF[(self.key_mode, self.key_over_token)]
        self.vq, self.vdq = _QF[(self.value_mode, self.value_over_token)]
        self.norm = None
        self.initialized = False
        self.cumulative_length = 0
        self.keys_q = self.values_q = None

    # cache.py:121-133
    def _normalize(self, k):
        if self.key_normalize:
            if self.norm is None:
                self.norm = np.sqrt(np.abs(k).max(axis=-2, keepdims=True).astype(np.float32)).astype(np.float16)
            k = (k.astype(np.float32) / self.norm.astype(np.float32)).astype(np.float16)
        return k

    def _recent_split(self, x, quantize, w_recent, over_token, flush):
        n = x.shape[-2]
        if quantize:
            r = min(w_recent, n)
            if over_token:
                while (n - r) % flush != 0:
                    r -= 1
        else:
            r = n
        return x[:, :, n - r:], x[:, :, :n - r]

    def _prefill(self, k, v):
        self.dtype = k.dtype
        ks = min(self.key_w_sink, k.shape[-2]) if self.key_quantize else 0
        vs = min(self.value_w_sink, v.shape[-2]) if self.value_quantize else 0
        self.keys_sink, k = k[:, :, :ks], k[:, :, ks:]
        self.values_sink, v = v[:, :, :vs], v[:, :, vs:]
        self.keys_recent, k = self._recent_split(k, self.key_quantize, self.key_w_recent,
                                                 self.key_over_token, self.key_flush_size)
        self.values_recent, v = self._recent_split(v, self.value_quantize, self.value_w_recent,
                                                   self.value_over_token, self.value_flush_size)
        if self.key_quantize and k.size:
            self.keys_q = self.kq(self._normalize(k), self.key_group_size, self.key_bits)
        if self.value_quantize and v.size:
            self.values_q = self.vq(v, self.value_group_size, self.value_bits)
        self.initialized = True

    def _flush(self, recent, new, quantize, flush):
        recent = np.concatenate([recent, new], axis=2)
        n = flush if (quantize and recent.shape[-2] >= flush) else 0
        return recent[:, :, n:], recent[:, :, :n]

    def _append(self, k, v):
        self.keys_recent, k = self._flush(self.keys_recent, k, self.key_quantize, self.key_flush_size)
        self.values_recent, v = self._flush(self.values_recent, v, self.value_quantize, self.value_flush_size)
        if k.size:
            new = self.kq(self._normalize(k), self.key_group_size, self.key_bits)
            self.keys_q = new if self.keys_q is None else tuple(
                _cat_triple(a, b, self.key_mode == "hybrid") for a, b in zip(self.keys_q, new))
        if v.size:
            new = self.vq(v, self.value_group_size, self.value_bits)
            self.values_q = new if self.values_q is None else tuple(
                _cat_triple(a, b, self.value_mode == "hybrid") for a, b in zip(self.values_q, new))

    def dense(self):
        """cache.py:235-281: cat(sink, deq(middle) [* norm], recent) -> fp16."""
        parts_k = [self.keys_sink.astype(np.float32)]
        if self.keys_q is not None:
            d = self.kdq(*self.keys_q, self.key_group_size)
            if self.key_normalize:
                d = d * self.norm.astype(np.float32)
            parts_k.append(d)
        parts_k.append(self.keys_recent.astype(np.float32))
        parts_v = [self.values_sink.astype(np.float32)]
        if self.values_q is not None:
            parts_v.append(self.vdq(*self.values_q, self.value_group_size))
        parts_v.append(self.values_recent.astype(np.float32))
        return (np.concatenate(parts_k, axis=2).astype(np.float16),
                np.concatenate(parts_v, axis=2).astype(np.float16))

    def update(self, k, v):
        """cache.py:382-396."""
        k = np.asarray(k, np.float16)
        v = np.asarray(v, np.float16)
        self.cumulative_length += k.shape[-2]
        if not self.initialized:
            self._prefill(k, v)
            return k, v
        self._append(k, v)
        return self.dense()

    def get_seq_length(self):
        return self.cumulative_length


class SlidingLayerRef(CacheLayerRef):
    """cache.py:421-461: the layer above behind a sliding window of w tokens.

    fix=False keeps the reference's indexing: once the past exceeds the window
    (cache.py:442), K and V become ``[:, :, -w, :]``, a single token with the
    token axis dropped (cache.py:443-444), and one call earlier they hold one
    token more than get_mask_sizes() announces.  fix=True returns the last
    w - 1 + q tokens of a q-token call once the past reaches the window, the
    kv_length get_mask_sizes() announces for it (cache.py:448-456)."""

    def __init__(self, config, sliding_window, fix=False):
        super().__init__(config)
        self.sliding_window = sliding_window
        self.fix = fix

    def update(self, k, v):
        K, V = super().update(k, v)
        q = np.asarray(k).shape[-2]
        past = self.cumulative_length - q
        w = self.sliding_window
        if not self.fix:
            if past > w:
                K, V = K[:, :, -w, :], V[:, :, -w, :]
        elif past >= w:
            K, V = K[:, :, -(w - 1 + q):], V[:, :, -(w - 1 + q):]
        return K, V

    def get_mask_sizes(self, query_length):
        """cache.py:448-456 (kv_length, kv_offset), before the call's update."""
        w = self.sliding_window
        kv_offset = max(self.cumulative_length - w + 1, 0)
        if self.cumulative_length >= w:
            return w - 1 + query_length, kv_offset
        return self.cumulative_length + query_length, kv_offset


def schedule(n_prefill, n_steps, w_sink, w_recent, flush, quantize=True, over_token=False):
    """Length-only simulator of the sink/recent/flush bookkeeping.

    Returns, after the prefill and after every decode step, the tuple
    (n_sink, n_quantized, n_recent).  Written from the flush rule alone
    (cache.py:157-185 and 283-307), independent of ``CacheLayerRef``.
    """
    sink = min(w_sink, n_prefill) if quantize else 0
    rest = n_prefill - sink
    if quantize:
        r = min(w_recent, rest)
        if over_token:
            while (rest - r) % flush:
                r -= 1
    else:
        r = rest
    nq, nr = rest - r, r
    out = [(sink, nq, nr)]
    for _ in range(n_steps):
        nr += 1
        if quantize and nr >= flush:
            nr -= flush
            nq += flush
        out.append((sink, nq, nr))
    return out
