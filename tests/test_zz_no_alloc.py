"""The no-allocation decode entry point (iq_decode_attention_noalloc) against
iq_decode_attention on the GPU, through the C ABI.

The two entry points share every kernel; only the workspace differs (the
library's per-GPU scratch array against a caller-allocated buffer).  The
fused kernel's waves claim token blocks dynamically, so the fp32 summation
order, and with it the last bit of an output, can differ from call to call:
the outputs are compared within the decode tolerance (1e-3, max-normwise),
and both against fp32 attention over the library's dequantized K and V.  Two
calls in a row, the second on a smaller input, check that the scratch keeps no
state that a later call depends on.
"""
import ctypes

import pytest
import torch

from innerq_amd import _lib, ops

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _inputs(B, Hkv, nrep, D, Tq, R, kbits, vbits, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    k = torch.randn(B, Hkv, Tq + R, D, generator=gen, device=DEV).to(torch.float16)
    v = torch.randn(B, Hkv, Tq + R, D, generator=gen, device=DEV).to(torch.float16)
    q = torch.randn(B, Hkv * nrep, D, generator=gen, device=DEV).to(torch.float16)
    kst = ops.PackedStore("channel", B, Hkv, D, 32, kbits, "asymmetric", DEV, t_cap=Tq)
    vst = ops.PackedStore("token", B, Hkv, D, 32, vbits, "asymmetric", DEV, t_cap=Tq)
    kst.append(k[:, :, :Tq])
    vst.append(v[:, :, :Tq])
    kr = k[:, :, Tq:] if R else None
    vr = v[:, :, Tq:] if R else None
    kd = torch.cat([kst.dequant(dtype=torch.float32), k[:, :, Tq:].float()], dim=2)
    lg = torch.matmul(q.float().view(B, Hkv, nrep, D), kd.transpose(-1, -2).contiguous()) * D ** -0.5
    del kd
    vd = torch.cat([vst.dequant(dtype=torch.float32), v[:, :, Tq:].float()], dim=2)
    ref = torch.matmul(torch.softmax(lg, dim=-1), vd).view(B, Hkv * nrep, D)
    return q, kst, vst, kr, vr, ref


def _err(a, b):
    return ((a.float() - b.float()).abs().max() / b.float().abs().max()).item()


def _noalloc(q, kst, vst, kr, vr, scale, out=None, stream=None):
    B, Hq, D = q.shape
    kn = [0, kst.length, 0 if kr is None else kr.shape[2]]
    vn = [0, vst.length, 0 if vr is None else vr.shape[2]]
    ks = (_lib.iq_segment * 3)(ops._segment(None, None, 0), ops._segment(None, kst, kn[1]),
                               ops._segment(kr, None, kn[2]))
    vs = (_lib.iq_segment * 3)(ops._segment(None, None, 0), ops._segment(None, vst, vn[1]),
                               ops._segment(vr, None, vn[2]))
    if out is None:
        out = torch.full((B, Hq, D), float("nan"), dtype=torch.float16, device=DEV)
    stream = torch.cuda.current_stream() if stream is None else stream
    st = _lib.lib().iq_decode_attention_noalloc(
        ctypes.c_void_p(q.data_ptr()), q.stride(0), q.stride(1), None, ks, vs, B, Hq, kst.H, sum(kn), D,
        float(scale), ctypes.c_void_p(out.data_ptr()), out.stride(0), out.stride(1),
        ctypes.c_void_p(stream.cuda_stream))
    assert st == 0, _lib.strerror(st)
    return out


def test_noalloc_matches_decode_attention_twice():
    cases = [(8, 8, 4, 128, 32768 - 128, 128, 2, 4, 1),   # one config-4 layer: 2-bit K, 4-bit V, a window
             (2, 4, 4, 128, 4096, 40, 4, 4, 2)]           # then a smaller step on the same scratch
    for B, Hkv, nrep, D, Tq, R, kb, vb, seed in cases:
        print(f"no-alloc case B={B} Hkv={Hkv} nrep={nrep} D={D} Tq={Tq} R={R} kbits={kb} vbits={vb}", flush=True)
        q, kst, vst, kr, vr, ref32 = _inputs(B, Hkv, nrep, D, Tq, R, kb, vb, seed)
        need = _lib.lib().iq_decode_workspace_bytes(B, Hkv * nrep, Tq + R, D)
        assert need <= _lib.lib().iq_decode_noalloc_max_bytes()
        got = _noalloc(q, kst, vst, kr, vr, D ** -0.5)
        ref = ops.decode_attention(q, None, kst, kr, None, vst, vr, D ** -0.5)
        torch.cuda.synchronize()
        assert not torch.isnan(got).any()
        e_api, e_ref = _err(got, ref), _err(got, ref32)
        print(f"  vs iq_decode_attention {e_api:.2e}, vs fp32 attention {e_ref:.2e}", flush=True)
        assert e_api < 1e-3 and e_ref < 1e-3 and _err(ref, ref32) < 1e-3


def test_noalloc_under_graph_capture():
    """The no-allocation step captured in a HIP graph on a side stream and replayed
    several times, with eager decode calls between the replays: every replay
    equals eager decode_attention (decode tolerance).  As the header says, one
    eager call on the device comes first: it looks up the scratch array's
    address, which a capture must not be the first to do."""
    B, Hkv, nrep, D, Tq, R = 4, 8, 4, 128, 8192, 96
    q, kst, vst, kr, vr, ref32 = _inputs(B, Hkv, nrep, D, Tq, R, 4, 4, seed=3)
    side = torch.cuda.Stream()
    out = torch.empty(B, Hkv * nrep, D, dtype=torch.float16, device=DEV)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _noalloc(q, kst, vst, kr, vr, D ** -0.5, out=out, stream=side)  # the eager first call
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    eager = ops.decode_attention(q, None, kst, kr, None, vst, vr, D ** -0.5)
    torch.cuda.synchronize()
    assert _err(out, eager) < 1e-3 and _err(eager, ref32) < 1e-3
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        _noalloc(q, kst, vst, kr, vr, D ** -0.5, out=out, stream=side)
    for i in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        print(f"replay {i}: vs eager {_err(out, eager):.2e}", flush=True)
        assert not torch.isnan(out).any()
        assert _err(out, eager) < 1e-3
        ops.decode_attention(q, None, kst, kr, None, vst, vr, D ** -0.5)  # eager work between replays
        _noalloc(q, kst, vst, kr, vr, D ** -0.5)                            # and on the same scratch
        torch.cuda.synchronize()
