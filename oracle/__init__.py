"""CPU oracle for the InnerQ KV-cache hot path -- TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product path (``innerq_amd``) never imports, links or calls
anything in here and raises when its HIP library is missing.

Modules
-------
quant_ref   numpy restatement of the reference's ``src/innerq/quant.py``
            (group quantize / dequantize, asym / sym / hybrid) with the exact
            per-op fp16 rounding of torch, plus the bit-packing convention and
            the packed HBM store layouts the HIP kernels write.
attn_ref    dequantize-then-matmul references for the decode QK^T and attn.V
            GEMVs and the full decode-attention step (GQA, fp32 softmax), as
            computed by transformers' eager attention over the dense K/V that
            ``cache.py`` returns.
cache_ref   restatement of the ``InnerqDynamicLayer`` state machine
            (sinks / recent window / flush / key normalization) over numpy
            arrays, producing the dense K/V that ``update()`` returns.
timing      the CPU baseline: the reference's torch CPU path
            (dequantize-then-matmul on int32 codes) timed on host cores.

Pinning (what checks each function; see tests/test_oracle_*.py):
  * quantize_asym / quantize_sym: golden vectors written by the live reference
    ``quant.py`` (tests/golden/), closed-form known answers (ramp, the
    benchmark_quantization.cu host pattern, half-to-even ties, constant
    groups), and invariants (range, min->0 / max->L, |deq-x| <= s/2).
  * dequantize_*: brute force over all 2^b codes against the affine map, and
    the golden vectors.
  * pack / unpack: bijection brute-forced over every code value at every lane
    position, 3-bit word-straddling codes 10 and 21 checked explicitly.
  * quantize_hybrid / dequantize_hybrid: golden vectors from the live reference.
  * attn_ref (tests/test_oracle_attn.py): softmax(qk_logits), av_out and
    decode_attention against transformers' own eager attention (repeat_kv +
    eager_attention_forward) on KV heads with distinct data; float64 index
    loops on tiny shapes with the GQA map kv = h // n_rep written out; the
    factored group sums (qk_factored / av_factored) over quantized codes
    against dequantize-then-matmul; each check rejects a planted mistake
    (h % Hkv head map, missing 1/sqrt(D), softmax over the wrong axis,
    dropped zero-point term).
  * cache_ref: golden traces of the live reference cache (token-index
    bookkeeping) and a length-only schedule simulator.
"""
