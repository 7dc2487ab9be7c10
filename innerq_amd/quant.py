"""Drop-in for the reference's ``innerq.quant`` (src/innerq/quant.py) on MI355X.

Same names, arguments and return values as the reference; the arithmetic runs
in the gfx950 kernels of libinnerq_hip.so with the reference's fp16 semantics
(every op rounded to fp16, round half to even, 0/0 groups -> INT32_MIN codes),
so codes are bit-exact and scales/zeros equal.  Tensors must be fp16 HIP
device tensors; there is no CPU path (a CPU tensor raises TypeError).

Supported: bits 2/3/4 (asym also 1, which the asym half of 2-bit hybrid
quantization uses), group sizes 32/64/128.  Unsupported arguments raise ValueError; a group size that does
not divide the grouped axis raises AssertionError, as in the reference
(quant.py:61, 99).
"""
from __future__ import annotations

from enum import Enum

import torch

from . import ops


class QMode(Enum):
    """quant.py:43-56."""
    SYM = 'symmetric'
    ASYM = 'asymmetric'
    HYBRID = 'hybrid'

    @classmethod
    def from_str(cls, value: str):
        normalized = value.strip().lower()
        for member in cls:
            if member.value == normalized:
                return member
        raise ValueError('Value of Enum should be form the choices \'symmetric\', \'asymmetric\', and \'hybrid\'.')


def _check(tensor, group_size, bit, dim, bits=(2, 3, 4)):
    if not isinstance(tensor, torch.Tensor) or not tensor.is_cuda:
        raise TypeError("innerq_amd.quant works on HIP device tensors (there is no CPU path)")
    if tensor.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"innerq_amd.quant quantizes fp16 or bf16 tensors, got {tensor.dtype}")
    assert tensor.shape[dim] % group_size == 0
    if group_size not in (32, 64, 128):
        raise ValueError(f"group_size must be 32, 64 or 128, got {group_size}")
    if bit not in bits:
        raise ValueError(f"bit must be one of {bits}, got {bit}")


ASYM_BITS = (1, 2, 3, 4)  # 1: the asym half of 2-bit hybrid quantization (quant.py:136)


def quantize_channeldim_asym(tensor, group_size, bit):
    """(codes int32, scale, min) with groups along the last dim (quant.py:58-77)."""
    _check(tensor, group_size, bit, tensor.dim() - 1, ASYM_BITS)
    return ops.quantize_dense(tensor, group_size, bit, "asymmetric", "channel")


def quantize_tokendim_asym(tensor, group_size, bit):
    """(codes int32, scale, min) with groups along dim -2 (quant.py:58-73, 79-81)."""
    _check(tensor, group_size, bit, tensor.dim() - 2, ASYM_BITS)
    return ops.quantize_dense(tensor, group_size, bit, "asymmetric", "token")


def quantize_channeldim_sym(tensor, group_size, bit):
    """(magnitude codes int32, scale, signs) with groups along the last dim (quant.py:95-115)."""
    _check(tensor, group_size, bit, tensor.dim() - 1)
    return ops.quantize_dense(tensor, group_size, bit, "symmetric", "channel")


def quantize_tokendim_sym(tensor, group_size, bit):
    """(magnitude codes int32, scale, signs) with groups along dim -2 (quant.py:95-111, 117-119)."""
    _check(tensor, group_size, bit, tensor.dim() - 2)
    return ops.quantize_dense(tensor, group_size, bit, "symmetric", "token")


def _deq(tensor, scale, zs, group_size, op_dtype, mode, axis):
    return ops.dequantize_dense(tensor, scale, zs, group_size, mode, axis, dtype=op_dtype)


def dequantize_channeldim_asym(tensor, scale, zero_points, group_size, op_dtype=torch.float32):
    """float(c) * float(s) + float(z) in op_dtype (quant.py:83-87)."""
    return _deq(tensor, scale, zero_points, group_size, op_dtype, "asymmetric", "channel")


def dequantize_tokendim_asym(tensor, scale, zero_points, group_size, op_dtype=torch.float32):
    """quant.py:89-93."""
    return _deq(tensor, scale, zero_points, group_size, op_dtype, "asymmetric", "token")


def dequantize_channeldim_sym(tensor, scale, signs, group_size, op_dtype=torch.float32):
    """float(c) * float(s) * sign (quant.py:121-125)."""
    return _deq(tensor, scale, signs, group_size, op_dtype, "symmetric", "channel")


def dequantize_tokendim_sym(tensor, scale, signs, group_size, op_dtype=torch.float32):
    """quant.py:127-131."""
    return _deq(tensor, scale, signs, group_size, op_dtype, "symmetric", "token")


def _axis(tensor_shape, scale_shape):
    """The grouped axis, found as the reference finds it (the dim where the scale is smaller)."""
    q_dim = [i for i, (a, b) in enumerate(zip(tensor_shape, scale_shape)) if a != b]
    assert len(q_dim) == 1
    nd = len(tensor_shape)
    if q_dim[0] == nd - 1:
        return "channel"
    if q_dim[0] == nd - 2:
        return "token"
    raise ValueError("hybrid quantization groups along one of the last two dims")


def quantize_hybrid(zp_func, nozp_func, zp_deq_func, nozp_deq_func):
    """Factory of the hybrid quantizer (quant.py:133-151): asym with bit-1 bits
    and sym with bit bits, and per group a mask that picks the sym codes when
    their L1 error is smaller."""
    def hybrid_func(tensor, group_size, bit):
        if bit not in (2, 3, 4):
            raise ValueError(f"hybrid quantization needs bit in (2, 3, 4), got {bit}")
        tensor_q_zp = zp_func(tensor, group_size, bit - 1)  # NOTE: the asym function has no sign bit
        tensor_q_nozp = nozp_func(tensor, group_size, bit)
        tensor_deq_zp = zp_deq_func(*tensor_q_zp, group_size)
        tensor_deq_nozp = nozp_deq_func(*tensor_q_nozp, group_size)
        axis = _axis(tuple(tensor.shape), tuple(tensor_q_zp[1].shape))
        mask = ops.hybrid_mask(tensor, tensor_deq_zp, tensor_deq_nozp, group_size, axis)
        q_tensor_combined = {'zp': tensor_q_zp[0], 'nozp': tensor_q_nozp[0]}
        scale_combined = {'zp': tensor_q_zp[1], 'nozp': tensor_q_nozp[1], 'mask': mask}
        zp_combined = {'zp': tensor_q_zp[2], 'nozp': tensor_q_nozp[2]}
        return q_tensor_combined, scale_combined, zp_combined
    return hybrid_func


def dequantize_hybrid(zp_func, nozp_func):
    """Factory of the hybrid dequantizer (quant.py:153-176): the mask selects
    the sym or the asym dequantization per group."""
    def hybrid_func(tensor, scale, sign_or_zp, group_size, op_dtype=torch.float32):
        zp_deq = zp_func(tensor['zp'], scale['zp'], sign_or_zp['zp'], group_size, op_dtype)
        nozp_deq = nozp_func(tensor['nozp'], scale['nozp'], sign_or_zp['nozp'], group_size, op_dtype)
        axis = _axis(tuple(tensor['zp'].shape), tuple(scale['zp'].shape))
        # fp16 / bf16 -> fp32 is exact, so selecting in fp32 and writing op_dtype is the same selection
        return ops.hybrid_select(zp_deq.float(), nozp_deq.float(), scale['mask'], group_size, axis, dtype=op_dtype)
    return hybrid_func
