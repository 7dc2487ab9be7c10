"""The packed store's wire / on-disk format (PackedStore.to_bytes / from_bytes,
save / load) on the host: a round trip keeps every valid unit bit for bit,
foreign or inconsistent blobs are refused.  No kernel runs here; the GPU
tests check that a loaded store decodes and keeps appending like the
original."""
import json
import struct

import pytest
import torch

from innerq_amd import ops


def _filled(axis, bits, mode, length, t_cap, seed, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    st = ops.PackedStore(axis, 2, 3, 128, 32, bits, mode, "cpu", t_cap=t_cap, dtype=dtype)
    st.codes.copy_(torch.randint(-2**31, 2**31 - 1, st.codes.shape, dtype=torch.int32, generator=g))
    st.meta.copy_(torch.randint(-2**15, 2**15 - 1, st.meta.shape, dtype=torch.int16, generator=g))
    st.length = length
    return st


def _units(st):
    u = st.unit
    used = -(-st.length // u)
    nu = st.t_cap // u
    bh = st.B * st.H
    return st.codes.view(bh, nu, -1)[:, :used], st.meta.view(bh, nu, -1)[:, :used]


@pytest.mark.parametrize("axis,bits,mode,length", [("channel", 4, "asymmetric", 150), ("channel", 3, "symmetric", 64),
                                                   ("token", 2, "asymmetric", 96), ("token", 4, "symmetric", 0)])
def test_round_trip(axis, bits, mode, length, tmp_path):
    st = _filled(axis, bits, mode, length, 200, seed=bits + length)
    p = tmp_path / "store.safetensors"
    st.save(str(p))
    back = ops.PackedStore.load(str(p), "cpu", t_cap=500)
    assert (back.axis, back.B, back.H, back.D, back.group, back.bits, back.mode, back.length) == \
        (st.axis, st.B, st.H, st.D, st.group, st.bits, st.mode, st.length)
    assert back.t_cap >= 500
    for a, b in zip(_units(st), _units(back)):
        assert torch.equal(a, b)
    # only the valid units travel: the blob is the packed bytes plus a small header
    hdr = struct.unpack("<Q", st.to_bytes()[:8])[0]
    used = -(-length // st.unit)
    body = st.B * st.H * used * (st.codes.numel() // (st.B * st.H * (st.t_cap // st.unit)) * 4 +
                                 st.meta.numel() // (st.B * st.H * (st.t_cap // st.unit)) * 2)
    assert len(st.to_bytes()) == 8 + hdr + body


def test_header_fields():
    st = _filled("channel", 4, "asymmetric", 70, 128, seed=1)
    blob = st.to_bytes()
    n = struct.unpack("<Q", blob[:8])[0]
    md = json.loads(blob[8:8 + n])["__metadata__"]
    assert md == {"format": "innerq-packed-store", "version": "1", "axis": "channel", "B": "2", "H": "3",
                  "D": "128", "group": "32", "bits": "4", "mode": "asymmetric", "length": "70", "unit": "64",
                  "dtype": "float16"}


def test_bf16_store_keeps_its_dtype(tmp_path):
    st = _filled("token", 3, "hybrid", 96, 128, seed=3, dtype=torch.bfloat16)
    back = ops.PackedStore.from_bytes(st.to_bytes(), "cpu")
    assert back.dtype == torch.bfloat16 and back.mode_arg == st.mode_arg
    for a, b in zip(_units(st), _units(back)):
        assert torch.equal(a, b)


def test_blob_without_dtype_reads_as_fp16():
    # blobs written before the dtype key existed are fp16 stores
    st = _filled("channel", 4, "asymmetric", 70, 128, seed=1)
    blob = st.to_bytes()
    n = struct.unpack("<Q", blob[:8])[0]
    hdr = json.loads(blob[8:8 + n])
    del hdr["__metadata__"]["dtype"]
    h = json.dumps(hdr, sort_keys=True, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)
    back = ops.PackedStore.from_bytes(struct.pack("<Q", len(h)) + h + blob[8 + n:], "cpu")
    assert back.dtype == torch.float16


def test_foreign_and_inconsistent_blobs_are_refused():
    from safetensors.torch import save
    st = _filled("token", 4, "asymmetric", 64, 64, seed=2)
    blob = st.to_bytes()
    with pytest.raises(ValueError):
        ops.PackedStore.from_bytes(save({"x": torch.zeros(1)}, metadata={"format": "other"}), "cpu")
    n = struct.unpack("<Q", blob[:8])[0]
    md = json.loads(blob[8:8 + n])["__metadata__"]
    from safetensors.torch import load
    t = load(blob)
    bad = dict(md, length="96")  # more tokens than the units hold
    with pytest.raises(ValueError):
        ops.PackedStore.from_bytes(save(t, metadata=bad), "cpu")
    bad = dict(md, version="3")
    with pytest.raises(ValueError):
        ops.PackedStore.from_bytes(save(t, metadata=bad), "cpu")


def _version(blob):
    n = struct.unpack("<Q", blob[:8])[0]
    return json.loads(blob[8:8 + n])["__metadata__"]["version"]


@pytest.mark.parametrize("mode,dtype,want", [("asymmetric", torch.float16, "1"), ("symmetric", torch.float16, "1"),
                                             ("hybrid", torch.float16, "2"), ("asymmetric", torch.bfloat16, "2"),
                                             ("hybrid", torch.bfloat16, "2")])
def test_version_marks_what_a_version_1_reader_cannot_read(mode, dtype, want):
    """fp16 asym / sym stores stay version 1 blobs; a bf16 or hybrid store is written
    as version 2, which a strict version-1 reader (the earlier from_bytes, which
    checked version == "1" and knew neither the dtype key nor the hybrid flag)
    refuses instead of decoding its metadata halves as fp16 or its flags as signs.
    This reader reads both."""
    st = _filled("token", 3, mode, 96, 128, seed=5, dtype=dtype)
    blob = st.to_bytes()
    assert _version(blob) == want
    strict_v1_accepts = _version(blob) == "1"
    assert strict_v1_accepts == (mode != "hybrid" and dtype == torch.float16)
    back = ops.PackedStore.from_bytes(blob, "cpu")
    assert back.dtype == dtype and back.mode_arg == st.mode_arg


def test_version_1_blob_claiming_bf16_is_refused():
    from safetensors.torch import load, save
    st = _filled("token", 3, "asymmetric", 96, 128, seed=6, dtype=torch.bfloat16)
    blob = st.to_bytes()
    n = struct.unpack("<Q", blob[:8])[0]
    md = json.loads(blob[8:8 + n])["__metadata__"]
    with pytest.raises(ValueError):
        ops.PackedStore.from_bytes(save(load(blob), metadata=dict(md, version="1")), "cpu")


@pytest.mark.parametrize("axis", ["channel", "token"])
def test_batch_view_shares_the_sequences_memory(axis):
    """batch_view(b0, b1): the stores of sequences [b0, b1) as a B = b1 - b0 store
    over the same memory (what a padded batch's per-start decode calls read)."""
    st = ops.PackedStore(axis, 3, 2, 128, 32, 4, "asymmetric", "cpu", t_cap=128)
    st.codes.copy_(torch.arange(st.codes.numel(), dtype=torch.int32))
    st.meta.copy_(torch.arange(st.meta.numel(), dtype=torch.int32).to(torch.int16))
    st.length = 96
    v = st.batch_view(1, 3)
    assert (v.B, v.H, v.t_cap, v.length, v.mode) == (2, 2, st.t_cap, 96, st.mode)
    assert torch.equal(v.codes, st.codes.view(3, -1)[1:].reshape(-1))
    assert torch.equal(v.meta, st.meta.view(3, -1)[1:].reshape(-1))
    assert v.codes.data_ptr() == st.codes.data_ptr() + st.codes.numel() // 3 * 4
    assert v.nbytes() == st.nbytes() * 2 // 3
    with pytest.raises(ValueError):
        st.batch_view(2, 2)
    empty = ops.PackedStore(axis, 3, 2, 128, 32, 4, "symmetric", "cpu")
    assert empty.batch_view(0, 1).B == 1

