"""numpy restatement of the reference's group quantization (TEST ORACLE ONLY).

Follows ``src/innerq/quant.py`` of mthcom/innerq op by op:

* ``quantize_asym``      quant.py:58-73  (``quantize_channeldim_asym`` :75-77,
                                           ``quantize_tokendim_asym``  :79-81)
* ``dequantize_*_asym``  quant.py:83-93
* ``quantize_sym``       quant.py:95-111 (wrappers :113-119)
* ``dequantize_*_sym``   quant.py:121-131
* ``quantize_hybrid``    quant.py:133-151
* ``dequantize_hybrid``  quant.py:153-176
* ``QMODES``             quant.py:43-56

Rounding semantics.  The reference runs these ops on fp16 tensors.  Every
torch fp16 op used there (sub, true division by a tensor, division by the
Python int ``2**bit-1``) is computed in fp32 and rounded to fp16 with
round-to-nearest-even.  For +,-,*,/ fp32 carries more than 2*11+2 bits, so this
equals the correctly rounded fp16 result; numpy's float16 ufuncs produce the
same bits.  ``x / L`` also equals ``x * (1/L)`` for every fp16 x and
L in {1,3,7,15} (checked exhaustively in tests), so the CUDA reciprocal-multiply
path and the CPU divide path of torch agree.  ``round_`` is half-to-even
(``np.rint``).  A constant group gives scale 0, 0/0 = NaN survives ``clamp_``
and ``.to(int32)`` turns NaN into INT32_MIN on x86.

Bit packing (the convention of the reference's speedtest kernels,
speedtest/benchmark_quantization.cu:25-84 pack, benchmark_qkt.cu:239-270
unpack): within one quantization group, code i occupies bits [b*i, b*i+b) of
a little-endian bit string split into 32-bit words, LSB first.  A group of G
codes is G*b/32 words; 3-bit groups of 32 codes are 3 words and codes 10 and
21 straddle word boundaries.  Asym codes are stored as their low b bits
(INT32_MIN -> 0); sym codes are stored as offset binary,
``sign * magnitude + 2^(b-1)`` (the speedtest's sym packing,
benchmark_quantization.cu:128 and 161).

Packed HBM store layouts (this build's, written by the HIP kernels):

  K (groups along head_dim, one row per token):
      codes  u32 [B, H, Tcap/64, D/G, 64, W]     W = G*b/32
      meta   u16 [B, H, Tcap/64, D/G, 64, M]     M = 2 {scale, zero} asym, 1 sym
  V (groups along tokens):
      codes  u32 [B, H, Tcap/G, D, W]
      meta   u16 [B, H, Tcap/G, D, M]
"""
from __future__ import annotations

import numpy as np

INT32_MIN = np.int32(-2147483648)
QMODES = ("symmetric", "asymmetric", "hybrid")
TOKEN_BLOCK = 64  # tokens per K-store block (one wave64 column)


def qmode_from_str(value: str) -> str:
    """quant.py:48-56: strip + lower-case, must be one of the three modes."""
    normalized = value.strip().lower()
    if normalized in QMODES:
        return normalized
    raise ValueError("Value of Enum should be form the choices 'symmetric', "
                     "'asymmetric', and 'hybrid'.")


def _f16(a):
    return np.asarray(a, dtype=np.float16)


def round_bf16(a):
    """float32 -> nearest bf16 (ties to even), kept as float32; NaN -> 0x7fc0
    (torch's c10::BFloat16 conversion).  bf16 arrays here are float32 arrays
    holding bf16 values."""
    a = np.asarray(a, np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16) & 0xFFFF0000
    r = np.where(np.isnan(a), 0x7FC00000, r).astype(np.uint32)
    return r.view(np.float32)


def bf16_bits(a):
    return (round_bf16(a).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(u16):
    return (np.asarray(u16, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _cast(a, act):
    """a in the activation dtype: fp16 ('f16') or bf16 values in float32 ('bf16')."""
    return _f16(a) if act == "f16" else round_bf16(a)


def _div16(a, b, act="f16"):
    """a / b (or a / python int) computed in fp32 and rounded to the activation dtype."""
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        return _cast(np.asarray(a, np.float32) / np.asarray(b, np.float32), act)


def _sub16(a, b, act="f16"):
    with np.errstate(invalid="ignore", over="ignore"):
        return _cast(np.asarray(a, np.float32) - np.asarray(b, np.float32), act)


def _to_int32_like_torch(y16):
    """``.clamp_().round_().to(torch.int32)`` tail: NaN -> INT32_MIN (x86)."""
    y = np.rint(y16.astype(np.float32))
    out = np.where(np.isnan(y), 0, y).astype(np.int32)
    return np.where(np.isnan(y), INT32_MIN, out).astype(np.int32)


def _split(x, group, axis):
    shape = x.shape
    n = shape[axis]
    assert n % group == 0
    ng = n // group
    new_shape = shape[:axis] + (ng, group) + shape[axis + 1:]
    red_shape = shape[:axis] + (ng,) + shape[axis + 1:]
    return x.reshape(new_shape), red_shape


def quantize_asym(x, group_size, bit, expanded_dim, act="f16"):
    """quant.py:58-73 (asymmetric min/max quantization over groups of ``expanded_dim``).
    act: 'f16' (fp16 tensors) or 'bf16' (bf16 tensors, every op rounded to bf16)."""
    x = _cast(x, act)
    shape = x.shape
    xr, red_shape = _split(x, group_size, expanded_dim)
    mn = xr.min(axis=expanded_dim + 1, keepdims=True)      # exact; NaN propagates
    mx = xr.max(axis=expanded_dim + 1, keepdims=True)
    L = 2 ** bit - 1
    scale = _div16(_sub16(mx, mn, act), L, act)             # quant.py:68
    y = _div16(_sub16(xr, mn, act), scale, act)             # quant.py:69-70
    y = np.clip(y, 0, L)                                    # clamp keeps NaN
    codes = _to_int32_like_torch(y).reshape(shape)          # quant.py:71
    return codes, scale.reshape(red_shape), mn.reshape(red_shape)


def quantize_channeldim_asym(x, group_size, bit, act="f16"):
    return quantize_asym(x, group_size, bit, np.ndim(x) - 1, act)


def quantize_tokendim_asym(x, group_size, bit, act="f16"):
    return quantize_asym(x, group_size, bit, np.ndim(x) - 2, act)


def quantize_sym(x, group_size, bit, expanded_dim, act="f16"):
    """quant.py:95-111 (magnitude codes with b-1 bits + a separate sign tensor)."""
    x = _cast(x, act)
    bit = bit - 1
    shape = x.shape
    signs = ((x > 0).astype(x.dtype) - (x < 0).astype(x.dtype))  # torch.sign: +-0, NaN -> 0
    xr, red_shape = _split(x, group_size, expanded_dim)
    a = np.abs(xr)
    mx = a.max(axis=expanded_dim + 1, keepdims=True)
    L = 2 ** bit - 1
    scale = _div16(mx, L, act)                              # quant.py:107
    y = _div16(a, scale, act)                               # quant.py:108
    y = np.clip(y, 0, L)
    codes = _to_int32_like_torch(y).reshape(shape)          # quant.py:109
    return codes, scale.reshape(red_shape), signs


def quantize_channeldim_sym(x, group_size, bit, act="f16"):
    return quantize_sym(x, group_size, bit, np.ndim(x) - 1, act)


def quantize_tokendim_sym(x, group_size, bit, act="f16"):
    return quantize_sym(x, group_size, bit, np.ndim(x) - 2, act)


def dequantize_channeldim_asym(codes, scale, zero, group_size):
    """quant.py:83-87: fp32 ``c*s`` then ``+ z`` (c*s is exact, one rounding)."""
    c = codes.reshape(codes.shape[:-1] + (scale.shape[-1], group_size)).astype(np.float32)
    r = c * scale[..., None].astype(np.float32)
    r = r + zero[..., None].astype(np.float32)
    return r.reshape(codes.shape)


def dequantize_tokendim_asym(codes, scale, zero, group_size):
    """quant.py:89-93."""
    c = codes.reshape(codes.shape[:-2] + (scale.shape[-2], group_size, codes.shape[-1])).astype(np.float32)
    r = c * scale[..., None, :].astype(np.float32)
    r = r + zero[..., None, :].astype(np.float32)
    return r.reshape(codes.shape)


def dequantize_channeldim_sym(codes, scale, signs, group_size):
    """quant.py:121-125."""
    c = codes.reshape(codes.shape[:-1] + (scale.shape[-1], group_size)).astype(np.float32)
    r = (c * scale[..., None].astype(np.float32)).reshape(codes.shape)
    return r * signs.astype(np.float32)


def dequantize_tokendim_sym(codes, scale, signs, group_size):
    """quant.py:127-131."""
    c = codes.reshape(codes.shape[:-2] + (scale.shape[-2], group_size, codes.shape[-1])).astype(np.float32)
    r = (c * scale[..., None, :].astype(np.float32)).reshape(codes.shape)
    return r * signs.astype(np.float32)


def quantize_hybrid(zp_func, nozp_func, zp_deq_func, nozp_deq_func):
    """quant.py:133-151: (b-1)-bit asym and b-bit sym per group; mask=True picks sym.

    The per-group L1 errors are summed in float64 here; the reference sums in
    fp32, so the choice can differ only when the two errors agree to fp32
    precision.  Exact ties keep the asym codes (the strict comparison), as the
    reference's masks in tests/golden/hybrid_ties.npz pin; near-ties that fp32
    rounding in some summation order would split stay unpinned.
    """
    def hybrid_func(x, group_size, bit, act="f16"):
        x = _cast(x, act)
        q_zp = zp_func(x, group_size, bit - 1, act)
        q_nozp = nozp_func(x, group_size, bit, act)
        d_zp = zp_deq_func(*q_zp, group_size)
        d_nozp = nozp_deq_func(*q_nozp, group_size)
        q_dim = [i for i, (a, b) in enumerate(zip(q_zp[1].shape, x.shape)) if a != b]
        assert len(q_dim) == 1
        q_dim = q_dim[0]
        rs = q_zp[1].shape[:q_dim] + (q_zp[1].shape[q_dim], group_size) + q_zp[1].shape[q_dim + 1:]
        xf = x.astype(np.float32)
        e_zp = np.abs((d_zp - xf).astype(np.float64)).reshape(rs).sum(q_dim + 1)
        e_nozp = np.abs((d_nozp - xf).astype(np.float64)).reshape(rs).sum(q_dim + 1)
        mask = e_zp > e_nozp
        return ({"zp": q_zp[0], "nozp": q_nozp[0]},
                {"zp": q_zp[1], "nozp": q_nozp[1], "mask": mask},
                {"zp": q_zp[2], "nozp": q_nozp[2]})
    return hybrid_func


def dequantize_hybrid(zp_func, nozp_func):
    """quant.py:153-176: ``where(mask, sym_deq, asym_deq)`` per group."""
    def hybrid_func(codes, scale, sign_or_zp, group_size):
        zp_deq = zp_func(codes["zp"], scale["zp"], sign_or_zp["zp"], group_size)
        nozp_deq = nozp_func(codes["nozp"], scale["nozp"], sign_or_zp["nozp"], group_size)
        shape = codes["zp"].shape
        q_dim = [i for i, (a, b) in enumerate(zip(scale["zp"].shape, shape)) if a != b][0]
        rs = scale["zp"].shape[:q_dim] + (scale["zp"].shape[q_dim], group_size) + scale["zp"].shape[q_dim + 1:]
        mask = np.expand_dims(scale["mask"], q_dim + 1)
        out = np.where(mask, nozp_deq.reshape(rs), zp_deq.reshape(rs))
        return out.reshape(shape)
    return hybrid_func


quantize_channeldim_hybrid = quantize_hybrid(quantize_channeldim_asym, quantize_channeldim_sym,
                                             dequantize_channeldim_asym, dequantize_channeldim_sym)
quantize_tokendim_hybrid = quantize_hybrid(quantize_tokendim_asym, quantize_tokendim_sym,
                                           dequantize_tokendim_asym, dequantize_tokendim_sym)
dequantize_channeldim_hybrid = dequantize_hybrid(dequantize_channeldim_asym, dequantize_channeldim_sym)
dequantize_tokendim_hybrid = dequantize_hybrid(dequantize_tokendim_asym, dequantize_tokendim_sym)


# ----------------------------------------------------------------------------
# bit packing
# ----------------------------------------------------------------------------

def stored_codes(codes, bits, signs=None):
    """Value written into the b-bit field: asym -> low b bits; sym (signs
    given) -> sign*magnitude + 2^(b-1), offset binary."""
    c = np.asarray(codes).astype(np.int64)
    if signs is not None:
        c = c * np.asarray(signs).astype(np.int64) + (1 << (bits - 1))
    return (c & ((1 << bits) - 1)).astype(np.uint32)


def pack_groups(fields, bits):
    """fields u32 [..., G] (values < 2^bits) -> words u32 [..., G*bits/32], LSB first."""
    fields = np.asarray(fields, dtype=np.uint64)
    G = fields.shape[-1]
    assert (G * bits) % 32 == 0
    nw = G * bits // 32
    out = np.zeros(fields.shape[:-1] + (nw,), dtype=np.uint64)
    for i in range(G):
        bit = bits * i
        w, o = divmod(bit, 32)
        v = fields[..., i]
        out[..., w] |= (v << np.uint64(o)) & np.uint64(0xFFFFFFFF)
        if o + bits > 32:
            out[..., w + 1] |= v >> np.uint64(32 - o)
    return out.astype(np.uint32)


def unpack_groups(words, bits, G, signed=False):
    """Inverse of ``pack_groups``; ``signed`` decodes offset-binary fields (u - 2^(b-1))."""
    words = np.asarray(words, dtype=np.uint64)
    out = np.zeros(words.shape[:-1] + (G,), dtype=np.int64)
    mask = (1 << bits) - 1
    for i in range(G):
        bit = bits * i
        w, o = divmod(bit, 32)
        v = words[..., w] >> np.uint64(o)
        if o + bits > 32:
            v = v | (words[..., w + 1] << np.uint64(32 - o))
        v = (v & np.uint64(mask)).astype(np.int64)
        if signed:
            v = v - (1 << (bits - 1))
        out[..., i] = v
    return out.astype(np.int32)


# ----------------------------------------------------------------------------
# packed store layouts
# ----------------------------------------------------------------------------

def f16_bits(a):
    return np.asarray(a, dtype=np.float16).view(np.uint16)


def build_k_store(codes, scale, zero_or_signs, bits, group, mode, tcap=None):
    """Channel-dim quantized K [B,H,T,D] -> (codes u32, meta u16) in the K-store layout.

    ``mode`` 'asymmetric': zero_or_signs is the fp16 zero point [B,H,T,D/G];
    'symmetric': it is the sign tensor [B,H,T,D].
    """
    B, H, T, D = codes.shape
    ng = D // group
    W = group * bits // 32
    tcap = tcap or -(-T // TOKEN_BLOCK) * TOKEN_BLOCK
    assert tcap % TOKEN_BLOCK == 0 and tcap >= T
    if mode == "symmetric":
        fields = stored_codes(codes, bits, zero_or_signs)
        M = 1
    else:
        fields = stored_codes(codes, bits)
        M = 2
    words = pack_groups(fields.reshape(B, H, T, ng, group), bits)       # [B,H,T,ng,W]
    cw = np.zeros((B, H, tcap, ng, W), np.uint32)
    cw[:, :, :T] = words
    cw = cw.reshape(B, H, tcap // TOKEN_BLOCK, TOKEN_BLOCK, ng, W).transpose(0, 1, 2, 4, 3, 5)
    meta = np.zeros((B, H, tcap, ng, M), np.uint16)
    meta[:, :, :T, :, 0] = f16_bits(scale)
    if M == 2:
        meta[:, :, :T, :, 1] = f16_bits(zero_or_signs)
    meta = meta.reshape(B, H, tcap // TOKEN_BLOCK, TOKEN_BLOCK, ng, M).transpose(0, 1, 2, 4, 3, 5)
    return np.ascontiguousarray(cw), np.ascontiguousarray(meta)


def build_v_store(codes, scale, zero_or_signs, bits, group, mode, tcap=None):
    """Token-dim quantized V [B,H,T,D] -> (codes u32 [B,H,Tcap/G,D,W], meta u16 [B,H,Tcap/G,D,M])."""
    B, H, T, D = codes.shape
    assert T % group == 0
    tcap = tcap or T
    assert tcap % group == 0 and tcap >= T
    W = group * bits // 32
    if mode == "symmetric":
        fields = stored_codes(codes, bits, zero_or_signs)
        M = 1
    else:
        fields = stored_codes(codes, bits)
        M = 2
    f = fields.reshape(B, H, T // group, group, D).transpose(0, 1, 2, 4, 3)  # [B,H,ng,D,G]
    cw = np.zeros((B, H, tcap // group, D, W), np.uint32)
    cw[:, :, :T // group] = pack_groups(f, bits)
    meta = np.zeros((B, H, tcap // group, D, M), np.uint16)
    meta[:, :, :T // group, :, 0] = f16_bits(scale)
    if M == 2:
        meta[:, :, :T // group, :, 1] = f16_bits(zero_or_signs)
    return cw, meta


def k_store_to_codes(cw, meta, T, bits, group, mode):
    """Inverse view of ``build_k_store``: (field codes int32 [B,H,T,D], scale, zero|None).

    Sym fields come back as signed values sign*magnitude."""
    B, H, nblk, ng, TB, W = cw.shape
    w = cw.transpose(0, 1, 2, 4, 3, 5).reshape(B, H, nblk * TB, ng, W)[:, :, :T]
    codes = unpack_groups(w, bits, group, signed=(mode == "symmetric")).reshape(B, H, T, ng * group)
    m = meta.transpose(0, 1, 2, 4, 3, 5).reshape(B, H, nblk * TB, ng, -1)[:, :, :T]
    scale = m[..., 0].view(np.float16)
    zero = m[..., 1].view(np.float16) if m.shape[-1] == 2 else None
    return codes, scale, zero


def v_store_to_codes(cw, meta, T, bits, group, mode):
    B, H, ngcap, D, W = cw.shape
    ng = T // group
    f = unpack_groups(cw[:, :, :ng], bits, group, signed=(mode == "symmetric"))  # [B,H,ng,D,G]
    codes = f.transpose(0, 1, 2, 4, 3).reshape(B, H, T, D)
    m = meta[:, :, :ng]
    scale = m[..., 0].view(np.float16)
    zero = m[..., 1].view(np.float16) if m.shape[-1] == 2 else None
    return codes, scale, zero
