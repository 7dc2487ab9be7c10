"""CPU baseline: the reference's decode read path, timed on host cores (TEST/BENCH ONLY).

What the reference does per decode step and layer once its cache is warm
(src/innerq/cache.py:394-396 -> 235-281, then transformers' eager attention
TF/models/llama/modeling_llama.py:179-215), restated with the same torch CPU
ops on int32 codes:

  K_deq = (codes_k.view(..., D/G, G).float() * s_k + z_k)      quant.py:83-87
  V_deq = (codes_v.view(..., T/G, G, D).float() * s_v + z_v)   quant.py:89-93
  K, V  = K_deq.to(fp16), V_deq.to(fp16)                        cache.py:279-280
  K, V  = repeat_kv(K), repeat_kv(V)                            modeling_llama.py:179-188
  w     = matmul(q, K^T) * head_dim**-0.5                       :204
  p     = softmax(w, dim=-1, dtype=float32).to(fp16)            :208
  out   = matmul(p, V)                                          :210

Only bench.py's cpu_baseline leg calls this; it is never the measured product.
"""
from __future__ import annotations

import time

import torch


def make_state(B: int, Hq: int, Hkv: int, T: int, D: int, G: int, bits_k: int, bits_v: int, seed: int = 0):
    g = torch.Generator().manual_seed(seed)
    return {
        "q": torch.randn(B, Hq, 1, D, generator=g).to(torch.float16),
        "ck": torch.randint(0, 2 ** bits_k, (B, Hkv, T, D), generator=g, dtype=torch.int32),
        "sk": (torch.rand(B, Hkv, T, D // G, generator=g) * 0.1).to(torch.float16),
        "zk": torch.randn(B, Hkv, T, D // G, generator=g).to(torch.float16),
        "cv": torch.randint(0, 2 ** bits_v, (B, Hkv, T, D), generator=g, dtype=torch.int32),
        "sv": (torch.rand(B, Hkv, T // G, D, generator=g) * 0.1).to(torch.float16),
        "zv": torch.randn(B, Hkv, T // G, D, generator=g).to(torch.float16),
        "G": G, "n_rep": Hq // Hkv,
    }


def _repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    if n_rep == 1:
        return x
    b, h, t, d = x.shape
    return x[:, :, None, :, :].expand(b, h, n_rep, t, d).reshape(b, h * n_rep, t, d)


def reference_step(st) -> torch.Tensor:
    G = st["G"]
    ck, cv = st["ck"], st["cv"]
    kd = ck.view(ck.shape[:-1] + (st["sk"].shape[-1], G)).to(torch.float32) * st["sk"].unsqueeze(-1).to(torch.float32)
    kd = (kd + st["zk"].unsqueeze(-1).to(torch.float32)).view(ck.shape)
    vd = cv.view(cv.shape[:-2] + (st["sv"].shape[-2], G, cv.shape[-1])).to(torch.float32) \
        * st["sv"].unsqueeze(-2).to(torch.float32)
    vd = (vd + st["zv"].unsqueeze(-2).to(torch.float32)).view(cv.shape)
    k = _repeat_kv(kd.to(torch.float16), st["n_rep"])
    v = _repeat_kv(vd.to(torch.float16), st["n_rep"])
    q = st["q"]
    w = torch.matmul(q, k.transpose(2, 3)) * (q.shape[-1] ** -0.5)
    p = torch.softmax(w, dim=-1, dtype=torch.float32).to(q.dtype)
    return torch.matmul(p, v)


def time_reference(B: int, Hq: int, Hkv: int, T: int, D: int, G: int, bits_k: int, bits_v: int, threads: int,
                   min_seconds: float = 10.0, max_reps: int = 50):
    """Mean seconds per reference step for the given (sample) shape using ``threads`` host threads."""
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        st = make_state(B, Hq, Hkv, T, D, G, bits_k, bits_v)
        reference_step(st)  # warm-up
        reps, t0 = 0, time.perf_counter()
        while reps < max_reps and (time.perf_counter() - t0) < min_seconds:
            reference_step(st)
            reps += 1
        return (time.perf_counter() - t0) / reps, reps
    finally:
        torch.set_num_threads(prev)
