"""iq_window_append (one decode step of a layer's recent windows, both roles in
one launch) against the separate path it replaces: the new tokens land after
the window, and the flushed tokens' packed bytes equal those of
PackedStore.append (iq_quantize_k / iq_quantize_v) on the same tokens, for both
store layouts, every mode (hybrid included), key normalization, flushes that
reach into the new tokens, and a buffer that has to grow."""
import numpy as np
import pytest
import torch

from innerq_amd import ops, synth

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _mixed(B, H, T, D, seed):
    x = synth.kv_tensor(B, H, T, D, seed=seed, n_out=3, factor=8.0).astype(np.float32)
    x[..., :40] += 5.0  # offset columns: hybrid groups of both kinds
    x[0, 0, 70, :] = 0.0         # an all-zero key token (constant channel groups)
    x[0, 1, 2 * 32:3 * 32, 5] = -2.0  # a constant token group of a value column
    return x.astype(np.float16)


def _bytes(st):
    u = st.unit
    n = -(-st.length // u)
    bh = st.B * st.H
    c = st.codes.view(bh, st.t_cap // u, -1)[:, :n].cpu().numpy()
    m = st.meta.view(bh, st.t_cap // u, -1)[:, :n].cpu().numpy()
    return c, m


@pytest.mark.parametrize("kmode,vmode", [("asymmetric", "symmetric"), ("symmetric", "hybrid"), ("hybrid", "asymmetric")])
@pytest.mark.parametrize("bits,G", [(2, 32), (3, 64), (4, 128)])
@pytest.mark.parametrize("norm", [False, True])
def test_window_append_matches_separate_path(kmode, vmode, bits, G, norm):
    B, H, D = 2, 3, 128
    T = 4 * G + 50
    kx, vx = _mixed(B, H, T, D, seed=bits + G), _mixed(B, H, T, D, seed=bits * G + 1)
    kt, vt = _t(kx), _t(vx)
    knorm = ops.key_norm_factor(kt[:, :, :64]) if norm else None
    # windows of 20 (K) and G + 5 (V) tokens after a first store part
    k0, v0 = 64, 2 * G
    ks = ops.PackedStore("channel", B, H, D, G, bits, kmode, DEV)
    vs = ops.PackedStore("token", B, H, D, G, bits, vmode, DEV)
    ks.append(kt[:, :, :k0], norm=knorm)
    vs.append(vt[:, :, :v0])
    kw, vw = ops.RecentWindow(kt[:, :, k0:k0 + 20]), ops.RecentWindow(vt[:, :, v0:v0 + G + 5])
    kref = ops.PackedStore("channel", B, H, D, G, bits, kmode, DEV)
    vref = ops.PackedStore("token", B, H, D, G, bits, vmode, DEV)
    kref.append(kt[:, :, :k0], norm=knorm)
    vref.append(vt[:, :, :v0])
    kpos, vpos = k0 + 20, v0 + G + 5   # next new token of each role
    kdone, vdone = k0, v0          # tokens in the stores
    # the last step flushes the whole K window and two of its three new tokens
    steps = [(1, 1, 0), (1, 3, 0), (2, 0, G), (1, 1, 0), (3, 22, 0)]
    for m, kf, vf in steps:
        # m new tokens (a key-value pair each), kf keys and vf values flushed
        knew, vnew = kt[:, :, kpos:kpos + m], vt[:, :, vpos:vpos + m]
        ops.window_append(kw, knew, kf, ks if kf else None, knorm if kf else None, vw, vnew, vf, vs if vf else None)
        if kf:
            kref.append(kt[:, :, kdone:kdone + kf], norm=knorm)
        if vf:
            vref.append(vt[:, :, vdone:vdone + vf])
        kpos, vpos, kdone, vdone = kpos + m, vpos + m, kdone + kf, vdone + vf
        torch.cuda.synchronize()
        assert torch.equal(kw.tensor, kt[:, :, kdone:kpos]) and torch.equal(vw.tensor, vt[:, :, vdone:vpos])
        assert ks.length == kref.length and vs.length == vref.length
        for a, b in ((ks, kref), (vs, vref)):
            ca, ma = _bytes(a)
            cb, mb = _bytes(b)
            np.testing.assert_array_equal(ca, cb)
            np.testing.assert_array_equal(ma, mb)


def test_window_grows_and_keeps_old_views():
    """Appending past the buffer's end moves the window to a larger buffer; a
    view taken before keeps its values."""
    B, H, D = 1, 2, 64
    x = _t(synth.kv_tensor(B, H, 400, D, seed=5))
    w = ops.RecentWindow(x[:, :, :10])
    views = []
    for i in range(10, 400, 7):
        ops.window_append(w, x[:, :, i:i + 7], 0, None, None, None, None, 0, None)
        views.append((w.tensor, min(i + 7, 400)))
    torch.cuda.synchronize()
    assert w.n == 400 and torch.equal(w.tensor, x)
    for v, end in views:
        assert torch.equal(v, x[:, :, :end])


@pytest.mark.parametrize("bits,G", [(2, 32), (4, 64)])
def test_window_append_hybrid_special_groups(bits, G):
    """Hybrid flushes (one lane per element, the error sums in element order)
    against the one-thread-per-group quantize on groups that test the choice's
    edges: a NaN, an all-zero group, constant groups (both errors zero: asym
    kept), a group of one large and many tiny values (error terms far apart in
    magnitude), and an fp16 subnormal group."""
    B, H, D = 1, 2, 128
    T = 3 * G
    kx = synth.kv_tensor(B, H, T, D, seed=71, n_out=3, factor=8.0).astype(np.float32)
    vx = synth.kv_tensor(B, H, T, D, seed=72, n_out=3, factor=8.0).astype(np.float32)
    for x in (kx, vx):
        x[0, 0, 3, 7] = np.nan                 # a K group and a V group with a NaN
        x[0, 1, 5, :] = 0.0                    # an all-zero token (K groups)
        x[0, 1, :, 9] = 0.25                   # a constant column (V groups)
        x[0, 0, 9, :G] = 1e-4                  # tiny values ...
        x[0, 0, 9, 3] = 3000.0                 # ... and one large one in a K group
        x[0, 1, 11, G:2 * G] = 3e-6            # fp16 subnormals
    kx, vx = kx.astype(np.float16), vx.astype(np.float16)
    kt, vt = _t(kx), _t(vx)
    ks = ops.PackedStore("channel", B, H, D, G, bits, "hybrid", DEV)
    vs = ops.PackedStore("token", B, H, D, G, bits, "hybrid", DEV)
    kref = ops.PackedStore("channel", B, H, D, G, bits, "hybrid", DEV)
    vref = ops.PackedStore("token", B, H, D, G, bits, "hybrid", DEV)
    kw, vw = ops.RecentWindow(kt[:, :, :1]), ops.RecentWindow(vt[:, :, :1])
    # every token through the window: T - 1 new tokens, then all T flushed at once
    ops.window_append(kw, kt[:, :, 1:], T, ks, None, vw, vt[:, :, 1:], T, vs)
    kref.append(kt)
    vref.append(vt)
    torch.cuda.synchronize()
    for a, b in ((ks, kref), (vs, vref)):
        ca, ma = _bytes(a)
        cb, mb = _bytes(b)
        np.testing.assert_array_equal(ca, cb)
        np.testing.assert_array_equal(ma, mb)
    # both kinds of group occur
    for st in (ks, vs):
        mw = st.meta.view(torch.int32).cpu().numpy().astype(np.uint32)
        assert ((mw & 0x8000) != 0).any() and ((mw & 0x8000) == 0).any()


@pytest.mark.parametrize("kmode", ["asymmetric", "symmetric", "hybrid"])
@pytest.mark.parametrize("bits,G", [(2, 32), (3, 64)])
@pytest.mark.parametrize("norm", [False, True])
def test_window_append_keeps_dequantized_rows(kmode, bits, G, norm):
    """deq_rows: each flushed key's buffer row holds its dequantized values
    (times the normalization factor, rounded once to fp16), bit-exact to the
    store's dequant of those tokens, including flushes that reach into the new
    tokens and a move to a larger buffer (the last `keep` rows survive)."""
    B, H, D = 2, 3, 128
    kx = _mixed(B, H, 260, D, seed=bits * 11 + G)
    kt = _t(kx)
    knorm = ops.key_norm_factor(kt[:, :, :64]) if norm else None
    ks = ops.PackedStore("channel", B, H, D, G, bits, kmode, DEV)
    ks.append(kt[:, :, :64], norm=knorm)
    kw = ops.RecentWindow(kt[:, :, 64:84], deq_rows=True, keep=48)
    pos, done = 84, 64
    steps = [(1, 1), (1, 3), (2, 0), (3, 22)] + [(1, 1)] * 90  # the single-token steps move the buffer
    for m, kf in steps:
        ops.window_append(kw, kt[:, :, pos:pos + m], kf, ks if kf else None, knorm if kf else None,
                          None, None, 0, None)
        pos, done = pos + m, done + kf
    torch.cuda.synchronize()
    assert torch.equal(kw.tensor, kt[:, :, done:pos])
    p = kw.shadow
    assert 0 < p <= done - 64 and p >= 48  # a move kept 48, the steps after it added theirs
    ref = ks.dequant(done - p, p, norm=knorm)
    np.testing.assert_array_equal(kw.rows_before(p)[:, :, :p].cpu().numpy(), ref.cpu().numpy())


@pytest.mark.parametrize("vmode", ["asymmetric", "symmetric", "hybrid"])
@pytest.mark.parametrize("bits,G", [(2, 32), (4, 64)])
def test_window_append_keeps_dequantized_value_rows(vmode, bits, G):
    """deq_rows on a V window (groups along tokens): each flushed group's buffer
    rows hold its dequantized values, bit-exact to the store's dequant, through
    flushes that reach into the new tokens and a move to a larger buffer."""
    B, H, D = 2, 3, 128
    vx = _mixed(B, H, 40 * G, D, seed=bits * 13 + G)
    vt = _t(vx)
    vs = ops.PackedStore("token", B, H, D, G, bits, vmode, DEV)
    vs.append(vt[:, :, :2 * G])
    vw = ops.RecentWindow(vt[:, :, 2 * G:2 * G + 5], deq_rows=True, keep=2 * G)
    pos, done = 2 * G + 5, 2 * G
    steps = [(G - 5, 0), (3, G), (1, 0), (2 * G, 2 * G)] + [(G // 2, 0), (G // 2, G)] * 30
    for m, vf in steps:
        ops.window_append(None, None, 0, None, None, vw, vt[:, :, pos:pos + m], vf, vs if vf else None)
        pos, done = pos + m, done + vf
    torch.cuda.synchronize()
    assert torch.equal(vw.tensor, vt[:, :, done:pos])
    p = vw.shadow
    assert p >= 2 * G and p % G == 0
    ref = vs.dequant(done - p, p)
    np.testing.assert_array_equal(vw.rows_before(p)[:, :, :p].cpu().numpy(), ref.cpu().numpy())


def test_recent_window_keeps_rows_before_it_when_it_moves():
    """RecentWindow: the rows kept before the window (deq_rows) survive a move
    to a larger buffer up to `keep` of them, right before the window;
    rows_before(p) refuses more rows than are held."""
    x = torch.arange(2 * 3 * 10 * 4, dtype=torch.float16, device=DEV).reshape(2, 3, 10, 4)
    pre = -torch.arange(2 * 3 * 6 * 4, dtype=torch.float16, device=DEV).reshape(2, 3, 6, 4) - 1
    w = ops.RecentWindow(x, pre=pre, deq_rows=True, keep=4)
    assert (w.start, w.n, w.shadow) == (6, 10, 6)
    assert torch.equal(w.tensor, x) and torch.equal(w.rows_before(6)[:, :, :6], pre)
    cap = w.buf.shape[2]
    w.reserve(cap)  # forces a move
    assert w.buf.shape[2] >= 4 + 10 + cap and (w.start, w.shadow) == (4, 4)
    assert torch.equal(w.tensor, x) and torch.equal(w.rows_before(4)[:, :, :4], pre[:, :, 2:])
    with pytest.raises(ValueError):
        w.rows_before(5)
    plain = ops.RecentWindow(x)
    assert (plain.shadow, plain.deq_rows) == (0, False)
