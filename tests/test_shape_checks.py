"""Host-side shape validation of the ops wrappers (innerq_amd/ops.py).

The C ABI receives device pointers, t_cap and sizes but not the shapes of the
caller's tensors, so a q, p, segment or output that disagrees with a store
would make a kernel read or write past an allocation.  The wrappers check
every shape in Python first and raise ValueError before any launch; these
tests drive those checks with shape tuples and store descriptors only (no
tensor reaches a kernel)."""
from types import SimpleNamespace

import pytest
import torch

from innerq_amd import ops


def store(axis, B=2, H=4, D=128, length=256, group=32):
    return SimpleNamespace(axis=axis, B=B, H=H, D=D, length=length, group=group, t_cap=512)


K = store("channel")
V = store("token")


def test_qk_good():
    ops.check_qk_shapes((2, 16, 128), K, 0, 256, (2, 16, 256), 2 * 4 * 128)
    ops.check_qk_shapes((2, 4, 128), K, 64, 100)


@pytest.mark.parametrize("q,st,t0,T,out,norm", [
    ((2, 16), K, 0, 256, None, None),                       # q rank
    ((3, 16, 128), K, 0, 256, None, None),                  # batch
    ((2, 16, 64), K, 0, 256, None, None),                   # head_dim
    ((2, 6, 128), K, 0, 256, None, None),                   # GQA: 6 over 4
    ((2, 16, 128), V, 0, 256, None, None),                  # a V store
    ((2, 16, 128), K, 200, 100, None, None),                # past length
    ((2, 16, 128), K, -1, 10, None, None),                  # negative t0
    ((2, 16, 128), K, 0, 256, (2, 16, 255), None),          # out tokens
    ((2, 16, 128), K, 0, 256, (2, 8, 256), None),           # out heads
    ((2, 16, 128), K, 0, 256, None, 4 * 128),               # norm size
])
def test_qk_bad(q, st, t0, T, out, norm):
    with pytest.raises(ValueError):
        ops.check_qk_shapes(q, st, t0, T, out, norm)


def test_av_good():
    ops.check_av_shapes((2, 16, 256), V, 0, 256, [(2, 16, 128)])
    ops.check_av_shapes((2, 16, 300), V, 32, 192, [(2, 16, 128), (2, 16, 128)])


@pytest.mark.parametrize("p,st,t0,T,outs", [
    ((2, 16), V, 0, 256, []),                               # p rank
    ((3, 16, 256), V, 0, 256, []),                          # batch
    ((2, 16, 255), V, 0, 256, []),                          # p shorter than T
    ((2, 10, 256), V, 0, 256, []),                          # GQA
    ((2, 16, 256), K, 0, 256, []),                          # a K store
    ((2, 16, 256), V, 64, 256, []),                         # past length
    ((2, 16, 256), V, 0, 256, [(2, 16, 64)]),               # out head_dim
    ((2, 16, 256), V, 0, 256, [(2, 16, 128), (1, 16, 128)]),
])
def test_av_bad(p, st, t0, T, outs):
    with pytest.raises(ValueError):
        ops.check_av_shapes(p, st, t0, T, outs)


def test_decode_good():
    seg = (2, 4, 32, 128)
    r = ops.check_decode_shapes((2, 16, 128), seg, K, seg, seg, V, seg, 2 * 4 * 128, (2, 16, 128))
    assert r == (2, 16, 4, 256 + 64, 128)
    # dense only
    assert ops.check_decode_shapes((2, 8, 128), None, None, seg, None, None, seg)[3] == 32
    # K packed one token further than V, the window takes up the difference
    k1 = store("channel", length=257)
    assert ops.check_decode_shapes((2, 16, 128), None, k1, (2, 4, 31, 128), None, V, (2, 4, 32, 128))[3] == 288


SEG = (2, 4, 32, 128)


@pytest.mark.parametrize("q,ks,kst,kr,vs,vst,vr,norm,out", [
    ((2, 16, 128), None, None, None, None, None, None, None, None),           # no segment at all
    ((2, 16), None, K, None, None, V, None, None, None),                       # q rank
    ((3, 16, 128), None, K, None, None, V, None, None, None),                  # batch vs stores
    ((2, 16, 128), (2, 4, 32, 64), K, None, SEG, V, None, None, None),        # sink head_dim
    ((2, 16, 128), None, K, (2, 2, 32, 128), None, V, SEG, None, None),       # recent KV heads
    ((2, 16, 128), None, K, (2, 4, 32), None, V, SEG, None, None),            # segment rank
    ((2, 16, 128), None, store("channel", H=2), None, None, V, None, None, None),  # store heads differ
    ((2, 16, 128), None, V, None, None, V, None, None, None),                  # K from a token-grouped store
    ((2, 16, 128), None, K, None, None, K, None, None, None),                  # V from a channel-grouped store
    ((2, 12, 128), None, K, None, None, V, None, None, None),                  # 12 over 4 is fine ...
    ((2, 16, 128), None, K, SEG, None, V, None, None, None),                   # token counts differ
    ((2, 16, 128), None, K, None, None, V, None, 3, None),                     # norm size
    ((2, 16, 128), None, K, None, None, V, None, None, (2, 16, 64)),           # out shape
])
def test_decode_bad(q, ks, kst, kr, vs, vst, vr, norm, out):
    if q == (2, 12, 128):  # ... 12 query heads over 4 KV heads is GQA 3: valid shapes; the
        ops.check_decode_shapes(q, ks, kst, kr, vs, vst, vr, norm, out)  # kernel-side limit is the ABI's
        return
    with pytest.raises(ValueError):
        ops.check_decode_shapes(q, ks, kst, kr, vs, vst, vr, norm, out)


def test_reserve_zeroes_new_capacity():
    """Rows of a K store's last block past ``length`` are never written by a
    quantize; new capacity starts zeroed so they carry no stale memory and
    to_bytes() of equal stores is byte-identical."""
    blobs = []
    for seed in (1, 2):
        # dirty the allocator with different garbage first
        junk = torch.full((1 << 16,), seed, dtype=torch.int32)
        del junk
        st = ops.PackedStore("channel", 2, 3, 128, 32, 4, "asymmetric", "cpu", t_cap=64)
        assert int(st.codes.abs().sum()) == 0 and int(st.meta.abs().sum()) == 0
        # K layout [B*H, blocks, D/G, 64 tokens, words]
        cv = st.codes.view(6, st.t_cap // 64, 4, 64, -1)
        cv[:, 0, :, :10].fill_(7)  # "append" 10 tokens of codes
        st.length = 10
        st.reserve(st.t_cap + 64)  # grow: old units copied, the rest zero
        cv = st.codes.view(6, st.t_cap // 64, 4, 64, -1)
        assert int(cv[:, 0, :, :10].ne(7).sum()) == 0 and int(cv[:, 0, :, 10:].abs().sum()) == 0
        assert int(cv[:, 1:].abs().sum()) == 0
        blobs.append(st.to_bytes())
    assert blobs[0] == blobs[1]
