"""C-ABI checks that run without a GPU: the library loads, exports every
function include/innerq_abi.h declares, and rejects bad arguments on the host
before any launch (each case below has exactly one invalid argument, so no
call here ever reaches a kernel launch)."""
import ctypes
import os
import re

import pytest

from innerq_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "innerq_abi.h")
FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(iq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_functions()
    assert "iq_qk_gemv" in names and "iq_av_gemv" in names and "iq_quantize_k" in names
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) <= set(_lib.SIGNATURES), set(names) - set(_lib.SIGNATURES)


def test_version_and_strerror():
    lib = _lib.lib()
    assert lib.iq_abi_version() == 3
    assert lib.iq_strerror(0) == b"ok"
    assert b"bits" in lib.iq_strerror(-2)
    assert lib.iq_strerror(12345) == b"unknown status"


def _store_bytes(fn, *args):
    cb, mb = ctypes.c_int64(), ctypes.c_int64()
    st = getattr(_lib.lib(), fn)(*args, ctypes.byref(cb), ctypes.byref(mb))
    return st, cb.value, mb.value


def test_store_sizes():
    st, cb, mb = _store_bytes("iq_k_store_bytes", 8, 8, 32768, 128, 32, 4, 0)
    assert st == 0 and cb == 8 * 8 * 32768 * 64 and mb == 8 * 8 * 32768 * 4 * 4
    st, cb, mb = _store_bytes("iq_v_store_bytes", 8, 8, 32768, 128, 64, 2, 1)
    assert st == 0 and cb == 8 * 8 * 32768 * 32 and mb == 8 * 8 * 512 * 128 * 2
    assert _store_bytes("iq_k_store_bytes", 1, 1, 100, 128, 32, 4, 0)[0] == -5   # t_cap % 64
    assert _store_bytes("iq_k_store_bytes", 1, 1, 64, 128, 32, 5, 0)[0] == -2    # bits
    assert _store_bytes("iq_k_store_bytes", 1, 1, 64, 96, 64, 4, 0)[0] == -3     # D % G
    assert _store_bytes("iq_v_store_bytes", 1, 1, 48, 128, 32, 4, 0)[0] == -3    # t_cap % G
    assert _store_bytes("iq_v_store_bytes", 1, 1, 64, 128, 32, 4, 3)[0] == -7    # mode
    # hybrid: b-bit fields, an asym-sized {scale | flag, zero} meta word per unit
    st, cb, mb = _store_bytes("iq_v_store_bytes", 2, 4, 4096, 128, 32, 2, 2)
    assert st == 0 and cb == 2 * 4 * 4096 * 32 and mb == 2 * 4 * 128 * 128 * 4
    st, cb, mb = _store_bytes("iq_k_store_bytes", 2, 4, 4096, 128, 32, 3, 2)
    assert st == 0 and cb == 2 * 4 * 4096 * 48 and mb == 2 * 4 * 4096 * 4 * 4
    assert _store_bytes("iq_v_store_bytes", 1, 1, 64, 128, 32, 1, 2)[0] == -2    # hybrid needs bits >= 2


def qk_args(**kw):
    a = dict(q=FAKE, sqb=1024, sqh=128, norm=None, kc=FAKE, km=FAKE, t_cap=1024, B=1, Hq=32, Hkv=8, t0=0,
             T=512, D=128, G=32, bits=4, mode=0, scale=1.0, out=FAKE, sob=1, soh=1, ws=FAKE, wsb=1 << 20,
             stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize("kw,err", [
    (dict(q=None), -1), (dict(kc=None), -1), (dict(out=None), -1),
    (dict(bits=5), -2), (dict(bits=1), -2), (dict(G=48), -3), (dict(G=256), -3),
    (dict(mode=3), -7), (dict(mode=2), -7), (dict(D=96), -4), (dict(Hkv=5), -4), (dict(Hq=48), -4),
    (dict(T=-1), -4), (dict(t0=32), -5), (dict(t_cap=1000), -5), (dict(T=1100), -8),
    (dict(kc=ctypes.c_void_p(0x1004)), -5), (dict(ws=None), -6), (dict(wsb=64), -6),
    (dict(ws=ctypes.c_void_p(0x1008)), -5),
])
def test_qk_rejects(kw, err):
    assert _lib.lib().iq_qk_gemv(*qk_args(**kw)) == err


def av_args(**kw):
    a = dict(p=FAKE, spb=1, sph=1, vc=FAKE, vm=FAKE, t_cap=1024, B=1, Hq=32, Hkv=8, t0=0, T=512, D=128, G=32,
             bits=4, mode=0, out32=FAKE, out16=None, sob=1, soh=1, acc=0, ws=None, wsb=0, stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize("kw,err", [
    (dict(p=None), -1), (dict(vm=None), -1), (dict(out32=None), -1), (dict(out32=None, acc=1, out16=FAKE), -1),
    (dict(bits=0), -2), (dict(G=16), -3), (dict(T=500), -3), (dict(t0=16), -3), (dict(mode=-1), -7),
    (dict(mode=3), -7), (dict(mode=2, bits=1), -2),
    (dict(D=256), -4), (dict(Hq=12), -4), (dict(T=2048), -8), (dict(vc=ctypes.c_void_p(0x1008)), -5),
    (dict(ws=None, wsb=0), -6), (dict(ws=FAKE, wsb=16), -6),
])
def test_av_rejects(kw, err):
    assert _lib.lib().iq_av_gemv(*av_args(**kw)) == err


def test_workspace_queries():
    lib = _lib.lib()
    n = lib.iq_av_workspace_bytes(8, 32, 32768, 128, 32)
    assert n >= 8 * 32 * 32768 * 2 + 8 * 32 * 128 * 4
    # per query head: D/2 query pairs + one fp32 sum per group (4 groups at G=32)
    assert lib.iq_qk_workspace_bytes(8, 32, 128) >= 8 * 32 * (64 + 4) * 4
    assert lib.iq_av_workspace_bytes(8, 32, 32768, 96, 32) == 0
    assert lib.iq_decode_workspace_bytes(8, 32, 32768, 128) >= 8 * 32 * 32768 * 2  # fp16 probability records
    assert lib.iq_decode_workspace_bytes(0, 32, 32768, 128) == 0


def quant_k_args(**kw):
    a = dict(x=FAKE, sxb=0, sxh=0, sxt=128, norm=None, B=1, H=1, n=4, D=128, G=32, bits=4, mode=0, kc=FAKE,
             km=FAKE, t_cap=64, t_off=0, c32=None, s16=None, z16=None, sg16=None, stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize("kw,err", [
    (dict(x=None), -1), (dict(kc=None), -1), (dict(bits=8), -2), (dict(G=64, D=96), -3), (dict(G=33), -3),
    (dict(mode=3), -7), (dict(n=-1), -4), (dict(t_off=62), -8), (dict(t_cap=100), -5),
    (dict(mode=2, c32=FAKE), -7), (dict(mode=2, s16=FAKE), -7), (dict(mode=2, kc=None, km=None), -7),
    (dict(mode=2, bits=1), -2),
    (dict(x=ctypes.c_void_p(0x1002)), -5), (dict(sxt=100), -5), (dict(mode=1, z16=FAKE), -7),
    (dict(mode=0, sg16=FAKE), -7),
])
def test_quantize_k_rejects(kw, err):
    assert _lib.lib().iq_quantize_k(*quant_k_args(**kw)) == err


def quant_v_args(**kw):
    a = dict(x=FAKE, sxb=0, sxh=0, sxt=128, B=1, H=1, n=64, D=128, G=32, bits=4, mode=0, vc=FAKE, vm=FAKE,
             t_cap=64, t_off=0, c32=None, s16=None, z16=None, sg16=None, stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize("kw,err", [
    (dict(x=None), -1), (dict(vm=None), -1), (dict(bits=1, mode=1), -2), (dict(n=48), -3), (dict(t_off=32), -8),
    (dict(t_off=16), -5), (dict(t_cap=48), -5), (dict(mode=7), -7), (dict(mode=2, sg16=FAKE), -7),
    (dict(mode=2, vc=None, vm=None), -7),
])
def test_quantize_v_rejects(kw, err):
    assert _lib.lib().iq_quantize_v(*quant_v_args(**kw)) == err


def test_decode_rejects():
    lib = _lib.lib()
    seg = (_lib.iq_segment * 3)()
    seg[0].n, seg[1].n, seg[2].n = 10, 0, 0
    vseg = (_lib.iq_segment * 3)()
    vseg[0].n = 10
    # dense segments without pointers
    assert lib.iq_decode_attention(FAKE, 1, 1, None, seg, vseg, 1, 32, 8, 10, 128, 1.0, FAKE, 1, 1, None, 0,
                                   None) == -1
    seg[0].dense = 0x1000
    vseg[0].dense = 0x1000
    # token counts disagree
    assert lib.iq_decode_attention(FAKE, 1, 1, None, seg, vseg, 1, 32, 8, 11, 128, 1.0, FAKE, 1, 1, None, 0,
                                   None) == -4
    # no workspace
    assert lib.iq_decode_attention(FAKE, 1, 1, None, seg, vseg, 1, 32, 8, 10, 128, 1.0, FAKE, 1, 1, None, 0,
                                   None) == -6
    # quantized K segment with bad bits
    seg[1].n, seg[0].n = 5, 5
    seg[1].codes, seg[1].meta, seg[1].t_cap, seg[1].bits, seg[1].group, seg[1].mode = 0x1000, 0x1000, 64, 7, 32, 0
    assert lib.iq_decode_attention(FAKE, 1, 1, None, seg, vseg, 1, 32, 8, 10, 128, 1.0, FAKE, 1, 1, FAKE, 1 << 30,
                                   None) == -2
    # a hybrid K store is read by the fused kernel only (K and V of one group
    # size): with V groups of 64 it is refused before any launch
    seg[0].n, seg[1].n = 0, 64
    seg[1].bits, seg[1].mode = 4, 2
    vseg[0].n, vseg[1].n = 0, 64
    vseg[1].codes, vseg[1].meta, vseg[1].t_cap, vseg[1].bits, vseg[1].group, vseg[1].mode = 0x1000, 0x1000, 64, 4, 64, 1
    assert lib.iq_decode_attention(FAKE, 1, 1, None, seg, vseg, 1, 32, 8, 64, 128, 1.0, FAKE, 1, 1, FAKE, 1 << 30,
                                   None) == -7


def test_dequant_rejects():
    lib = _lib.lib()
    assert lib.iq_dequant_k(FAKE, FAKE, 64, None, 1, 1, 0, 65, 128, 32, 4, 0, FAKE, None, 1, 1, 1, None) == -8
    assert lib.iq_dequant_k(FAKE, FAKE, 64, None, 1, 1, 0, 64, 128, 32, 4, 0, None, None, 1, 1, 1, None) == -1
    assert lib.iq_dequant_v(FAKE, FAKE, 64, 1, 1, 0, 40, 128, 32, 4, 0, FAKE, None, 1, 1, 1, None) == -3
    assert lib.iq_dequant_dense(FAKE, FAKE, FAKE, 1, 40, 1, 32, 0, 0, FAKE, None) == -3
    assert lib.iq_dequant_dense(FAKE, FAKE, FAKE, 1, 64, 1, 32, 0, 2, FAKE, None) == -4


def test_cpu_tensor_raises_no_fallback():
    import torch
    from innerq_amd import ops
    with pytest.raises(TypeError, match="no CPU path"):
        ops.quantize_dense(torch.zeros(2, 64, dtype=torch.float16), 32, 4, "asymmetric", "channel")


def test_decode_stage_rejects():
    lib = _lib.lib()
    ns = ctypes.c_int(-7)
    seg = (_lib.iq_segment * 3)()
    seg[2].n = 64
    seg[2].dense = FAKE
    # a NULL split-count pointer, then a bad shape: rejected before any launch
    assert lib.iq_decode_attention_splits(FAKE, 1024, 128, None, seg, seg, 1, 32, 8, 64, 128, 1.0, FAKE, 1 << 30,
                                          None, None) == -1
    assert lib.iq_decode_attention_splits(FAKE, 1024, 128, None, seg, seg, 1, 32, 8, 64, 96, 1.0, FAKE, 1 << 30,
                                          ctypes.byref(ns), None) == -4
    assert ns.value == -7
    assert lib.iq_decode_attention_combine(0, 1, 32, 64, 128, FAKE, 4096, 128, FAKE, 1 << 30, None) == -4
    # T = 64: one 256-token split of packed tokens + at most four slices of dense tokens
    assert lib.iq_decode_attention_combine(6, 1, 32, 64, 128, FAKE, 4096, 128, FAKE, 1 << 30, None) == -4
    assert lib.iq_decode_attention_combine(1, 1, 32, 64, 128, None, 4096, 128, FAKE, 1 << 30, None) == -1
    assert lib.iq_decode_attention_combine(1, 1, 32, 64, 128, FAKE, 4096, 128, FAKE, 64, None) == -6


def test_decode_live_stages_reject():
    """iq_decode_attention_splits_live / _combine_live: bad arguments and plans are
    refused before any launch, and a refused split call leaves the plan as it was."""
    lib = _lib.lib()
    seg = (_lib.iq_segment * 3)()
    seg[2].n = 64
    seg[2].dense = FAKE
    plan = _lib.iq_split_plan(nsplit=-7)
    assert lib.iq_decode_attention_splits_live(FAKE, 1024, 128, None, seg, seg, 1, 32, 8, 64, 128, 1.0, FAKE,
                                               1 << 30, None, None) == -1
    assert lib.iq_decode_attention_splits_live(FAKE, 1024, 128, None, seg, seg, 1, 32, 8, 64, 96, 1.0, FAKE,
                                               1 << 30, ctypes.byref(plan), None) == -4
    assert lib.iq_decode_attention_splits_live(FAKE, 1024, 128, None, seg, seg, 1, 32, 8, 64, 128, 1.0, FAKE,
                                               64, ctypes.byref(plan), None) == -6
    assert plan.nsplit == -7

    def combine(p, B=8, Hq=32, T=32768, D=128, out=FAKE, ws_bytes=1 << 40):
        return lib.iq_decode_attention_combine_live(ctypes.byref(p), B, Hq, T, D, out, 4096, 128, FAKE, ws_bytes,
                                                    None)

    ok = dict(nsplit=128, nsf=128, grid=256, nrep=4, pair_e0=68)
    assert lib.iq_decode_attention_combine_live(None, 8, 32, 32768, 128, FAKE, 4096, 128, FAKE, 1 << 40, None) == -1
    assert combine(_lib.iq_split_plan(**ok), out=None) == -1
    assert combine(_lib.iq_split_plan(**ok), ws_bytes=64) == -6
    for bad in (dict(nrep=3), dict(nsplit=0, nsf=0), dict(nsf=129), dict(nsplit=133), dict(pair_e0=128),
                dict(pair_e0=-1), dict(grid=-1), dict(grid=1021), dict(nsf=1, nsplit=1, grid=65),
                dict(nsplit=128, nsf=120)):
        assert combine(_lib.iq_split_plan(**dict(ok, **bad))) == -4, bad
    assert combine(_lib.iq_split_plan(**ok), D=96) == -4


def test_decode_activation_dtype_must_agree():
    """The activation dtype of a decode call is the IQ_MODE_BF16 bit of its
    segments' modes: segments holding tokens that disagree, or a dense segment
    whose mode carries any other bit, are refused before any launch."""
    lib = _lib.lib()
    BF = _lib.IQ_MODE_BF16
    k = (_lib.iq_segment * 3)()
    v = (_lib.iq_segment * 3)()
    for seg in (k, v):
        seg[2].n, seg[2].dense, seg[2].s_b, seg[2].s_h, seg[2].s_t = 64, FAKE, 64 * 128, 64 * 128, 128
    k[2].mode = BF  # bf16 keys, fp16 values
    assert lib.iq_decode_attention(FAKE, 4096, 128, None, k, v, 1, 32, 8, 64, 128, 1.0, FAKE, 4096, 128, FAKE,
                                   1 << 30, None) == -7
    k[2].mode, v[2].mode = 1, 1  # a dense segment with a store mode
    assert lib.iq_decode_attention(FAKE, 4096, 128, None, k, v, 1, 32, 8, 64, 128, 1.0, FAKE, 4096, 128, FAKE,
                                   1 << 30, None) == -7
    k[2].mode, v[2].mode = BF, BF  # bf16 throughout: the split stage alone refuses it (fp16 combine)
    ns = ctypes.c_int(-7)
    assert lib.iq_decode_attention_splits(FAKE, 4096, 128, None, k, v, 1, 32, 8, 64, 128, 1.0, FAKE, 1 << 30,
                                          ctypes.byref(ns), None) == -7


def test_decode_slot_limit_where_every_slot_is_read():
    """Past 1020 splits of 256 tokens (261,120 tokens), a combine that reads every
    split slot cannot hold them: the split stage alone and the unfused kernels (K
    and V of different group sizes) return IQ_ERR_SHAPE before any launch.  A full
    call on the fused path reads only its live slots and takes any length (GPU
    test)."""
    lib = _lib.lib()
    T = 300032
    k = (_lib.iq_segment * 3)()
    v = (_lib.iq_segment * 3)()
    for seg, group in ((k, 32), (v, 64)):
        seg[1].n, seg[1].t_cap, seg[1].t0 = T, T, 0
        seg[1].codes, seg[1].meta, seg[1].bits, seg[1].group, seg[1].mode = 0x1000, 0x1000, 4, group, 0
    big = 1 << 40
    assert lib.iq_decode_attention(FAKE, 4096, 128, None, k, v, 1, 32, 8, T, 128, 1.0, FAKE, 4096, 128, FAKE, big,
                                   None) == -4
    ns = ctypes.c_int(-7)
    v[1].group = 32
    assert lib.iq_decode_attention_splits(FAKE, 4096, 128, None, k, v, 1, 32, 8, T, 128, 1.0, FAKE, big,
                                          ctypes.byref(ns), None) == -4
    assert ns.value == -7


def test_decode_noalloc_limits():
    """The no-allocation decode entry point: its scratch size, and a call whose
    workspace would exceed it refused with IQ_ERR_WORKSPACE before any HIP call
    (the FAKE pointers are never dereferenced); a bad shape is refused first."""
    lib = _lib.lib()
    assert lib.iq_decode_noalloc_max_bytes() == 64 << 20
    k = (_lib.iq_segment * 3)()
    v = (_lib.iq_segment * 3)()
    T = 131072
    for s, grp in ((k, 32), (v, 32)):
        s[1].n, s[1].codes, s[1].meta, s[1].t_cap, s[1].t0 = T, 0x1000, 0x1000, T, 0
        s[1].bits, s[1].group, s[1].mode = 4, grp, 0
    need = lib.iq_decode_workspace_bytes(64, 32, T, 128)
    assert need > 64 << 20
    assert lib.iq_decode_attention_noalloc(FAKE, 4096, 128, None, k, v, 64, 32, 8, T, 128, 1.0, FAKE, 4096, 128,
                                           None) == -6
    assert lib.iq_decode_attention_noalloc(FAKE, 4096, 128, None, k, v, 64, 32, 8, T, 96, 1.0, FAKE, 4096, 128,
                                           None) == -4
    assert lib.iq_decode_attention_noalloc(FAKE, 4096, 128, None, k, v, 64, 32, 8, T, 128, 1.0, None, 4096, 128,
                                           None) == -1


def _window(**kw):
    w = _lib.iq_window()
    d = dict(buf=0x1000, s_b=0, s_h=0, s_t=128, cap=64, start=0, n=8, x=0x2000, sx_b=0, sx_h=0, sx_t=128, m=1,
             flush=0, codes=None, meta=None, t_cap=0, t_off=0, bits=4, group=32, mode=0, axis=0, norm=None)
    d.update(kw)
    for k, v in d.items():
        setattr(w, k, v)
    return w


@pytest.mark.parametrize("kw,err", [
    (dict(start=60, n=4, m=1), -8),                         # no room after the window
    (dict(m=-1), -4), (dict(flush=10, n=8, m=1), -4),        # flush beyond [window | new]
    (dict(x=None), -1), (dict(buf=None), -1),
    (dict(flush=1), -1),                                     # flushing without a store
    (dict(flush=1, codes=0x3000, meta=0x4000, t_cap=64, bits=5), -2),
    (dict(flush=1, codes=0x3000, meta=0x4000, t_cap=64, mode=3), -7),
    (dict(flush=1, codes=0x3000, meta=0x4000, t_cap=64, t_off=64), -8),
    (dict(flush=1, codes=0x3000, meta=0x4000, t_cap=100), -5),              # K layout: t_cap % 64
    (dict(flush=8, n=8, m=1, codes=0x3000, meta=0x4000, t_cap=64, axis=1), -3),  # V layout: whole groups
    (dict(flush=1, codes=0x3000, meta=0x4000, t_cap=64, axis=1, norm=0x5000), -4),
])
def test_window_append_rejects(kw, err):
    """Every bad argument is refused on the host before any launch."""
    w = _window(**kw)
    assert _lib.lib().iq_window_append(ctypes.byref(w), None, 1, 1, 128, None) == err
    assert _lib.lib().iq_window_append(None, ctypes.byref(w), 1, 1, 128, None) == err
