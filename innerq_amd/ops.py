"""torch-facing wrappers of the C ABI (device memory and streams only).

Every function here checks that its tensors live on a HIP device and calls one
entry point of libinnerq_hip.so on the current torch stream.  There is no CPU
path: a CPU tensor or a missing library raises.
"""
from __future__ import annotations

import copy
import ctypes
from typing import Optional, Sequence

import torch

from . import _lib
from ._lib import IQ_MODE_ASYM, IQ_MODE_HYBRID, IQ_MODE_SYM, TOKEN_BLOCK, call

MODES = {"asymmetric": IQ_MODE_ASYM, "symmetric": IQ_MODE_SYM, "hybrid": IQ_MODE_HYBRID}
MODE_NAMES = {v: k for k, v in MODES.items()}


def _p(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_device(t: torch.Tensor, name: str, dtype=torch.float16) -> None:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a HIP device tensor (innerq_amd has no CPU path)")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")


def act_flag(dtype) -> int:
    """The mode bit of an activation dtype: IQ_MODE_BF16 for bf16, 0 for fp16."""
    if dtype == torch.bfloat16:
        return _lib.IQ_MODE_BF16
    if dtype == torch.float16:
        return 0
    raise TypeError(f"activations must be torch.float16 or torch.bfloat16, got {dtype}")


def require_act(t: torch.Tensor, name: str, dtype=None) -> None:
    """A HIP device tensor of an activation dtype (fp16 or bf16; exactly ``dtype`` when given)."""
    require_device(t, name, dtype)
    act_flag(t.dtype)


def require_f16_store(store, role: str) -> None:
    if store is not None and store.dtype != torch.float16:
        raise TypeError(f"{role}: the decode kernels take fp16 stores; a {store.dtype} store is read through "
                        "dequant() (the reference's dequantize-then-attend path)")


def mode_id(mode) -> int:
    if isinstance(mode, int):
        return mode
    m = getattr(mode, "value", mode)
    if m not in MODES:
        raise ValueError(f"packed kernels support 'asymmetric', 'symmetric' and 'hybrid', not {m!r}")
    return MODES[m]


def _shape_error(msg: str):
    raise ValueError(msg)


def check_store(store, role: str, axis: str, B: int, H: Optional[int], D: int) -> None:
    """``store`` (a PackedStore, or anything with its attributes) holds [B, H, *, D]
    grouped along ``axis``; H = None accepts any head count."""
    if store.axis != axis:
        _shape_error(f"{role}: store grouped along the {store.axis} axis, this call reads a "
                     f"{'head_dim' if axis == 'channel' else 'token'}-grouped store")
    if store.B != B or store.D != D or (H is not None and store.H != H):
        _shape_error(f"{role}: store holds [B={store.B}, H={store.H}, D={store.D}], the call has "
                     f"[B={B}, H={H if H is not None else store.H}, D={D}]")


def check_range(store, role: str, t0: int, T: int) -> None:
    if t0 < 0 or T < 0 or t0 + T > store.length:
        _shape_error(f"{role}: tokens [{t0}, {t0 + T}) are not inside the store's {store.length} tokens")


def check_gqa(Hq: int, Hkv: int) -> None:
    if Hkv <= 0 or Hq % Hkv:
        _shape_error(f"{Hq} query heads do not divide over {Hkv} KV heads")


def check_out(shape, want, role: str = "out") -> None:
    if tuple(shape) != tuple(want):
        _shape_error(f"{role} has shape {tuple(shape)}, expected {tuple(want)}")


def check_norm(norm_numel: Optional[int], B: int, Hkv: int, D: int) -> None:
    if norm_numel is not None and norm_numel != B * Hkv * D:
        _shape_error(f"key normalization factor has {norm_numel} values, expected B*Hkv*D = {B * Hkv * D}")


def check_qk_shapes(q_shape, store, t0: int, T: int, out_shape=None, norm_numel=None) -> None:
    """Shapes of a QK^T GEMV call (host only): q [B,Hq,D] over store tokens
    [t0, t0+T) of a head_dim-grouped store [B,Hkv,*,D]; out [B,Hq,T]."""
    if len(q_shape) != 3:
        _shape_error(f"q must be [B, Hq, D], got {tuple(q_shape)}")
    B, Hq, D = q_shape
    check_store(store, "K", "channel", B, None, D)
    check_gqa(Hq, store.H)
    check_range(store, "K", t0, T)
    check_norm(norm_numel, B, store.H, D)
    if out_shape is not None:
        check_out(out_shape, (B, Hq, T))


def check_av_shapes(p_shape, store, t0: int, T: int, out_shapes=()) -> None:
    """Shapes of an attn.V GEMV call (host only): p [B,Hq,>=T] (p[..., i] weighs
    store token t0+i) over a token-grouped store [B,Hkv,*,D]; outputs [B,Hq,D]."""
    if len(p_shape) != 3:
        _shape_error(f"p must be [B, Hq, T], got {tuple(p_shape)}")
    B, Hq, Tp = p_shape
    check_store(store, "V", "token", B, None, store.D)
    check_gqa(Hq, store.H)
    check_range(store, "V", t0, T)
    if Tp < T:
        _shape_error(f"p holds {Tp} tokens, the call reads {T}")
    for s in out_shapes:
        check_out(s, (B, Hq, store.D))


def check_decode_shapes(q_shape, k_sink, k_store, k_recent, v_sink, v_store, v_recent, norm_numel=None,
                        out_shape=None, k_t0: int = 0, v_t0: int = 0) -> tuple:
    """Shapes of a decode-attention call (host only).  Dense segments are shapes
    [B,Hkv,n,D] or None; stores are PackedStores (or anything with their
    attributes) or None, read from store token k_t0 / v_t0 on.  Returns
    (B, Hq, Hkv, T, D)."""
    if len(q_shape) != 3:
        _shape_error(f"q must be [B, Hq, D], got {tuple(q_shape)}")
    B, Hq, D = q_shape
    Hkv = None
    for st in (k_store, v_store):
        if st is not None:
            Hkv = st.H
            break
    for name, seg in (("k_sink", k_sink), ("k_recent", k_recent), ("v_sink", v_sink), ("v_recent", v_recent)):
        if seg is None:
            continue
        if len(seg) != 4:
            _shape_error(f"{name} must be [B, Hkv, n, D], got {tuple(seg)}")
        Hkv = seg[1] if Hkv is None else Hkv
        if (seg[0], seg[1], seg[3]) != (B, Hkv, D):
            _shape_error(f"{name} has shape {tuple(seg)}, expected [B={B}, Hkv={Hkv}, n, D={D}]")
    if Hkv is None:
        _shape_error("decode attention needs at least one K/V segment")
    if k_store is not None:
        check_store(k_store, "K", "channel", B, Hkv, D)
    if v_store is not None:
        check_store(v_store, "V", "token", B, Hkv, D)
    check_gqa(Hq, Hkv)
    check_norm(norm_numel, B, Hkv, D)

    def n_of(seg):
        return 0 if seg is None else seg[2]

    for role, st, t0 in (("K", k_store, k_t0), ("V", v_store, v_t0)):
        if t0 < 0 or (st is None and t0) or (st is not None and t0 > st.length):
            _shape_error(f"{role} store offset {t0} outside the store")
    T = n_of(k_sink) + (k_store.length - k_t0 if k_store is not None else 0) + n_of(k_recent)
    Tv = n_of(v_sink) + (v_store.length - v_t0 if v_store is not None else 0) + n_of(v_recent)
    if T != Tv:
        _shape_error(f"K has {T} tokens but V has {Tv}")
    if out_shape is not None:
        check_out(out_shape, (B, Hq, D))
    return B, Hq, Hkv, T, D


class PackedStore:
    """Packed codes + fp16 metadata of one quantized K or V segment.

    axis='channel': groups along head_dim, K-store layout (what QK^T reads);
    axis='token':   groups along tokens, V-store layout (what attn.V reads).
    Capacity grows geometrically; ``length`` tokens are valid.
    """

    def __init__(self, axis: str, B: int, H: int, D: int, group: int, bits: int, mode, device,
                 t_cap: int = 0, dtype=torch.float16):
        if axis not in ("channel", "token"):
            raise ValueError(axis)
        self.axis, self.B, self.H, self.D = axis, B, H, D
        self.group, self.bits, self.mode = group, bits, mode_id(mode)
        act_flag(dtype)
        self.dtype = dtype  # activation dtype: of the appended tokens, the scales / zero points and dequant()
        self.device = torch.device(device)
        self.length = 0
        self.t_cap = 0
        self.codes = torch.empty(0, dtype=torch.int32, device=self.device)
        self.meta = torch.empty(0, dtype=torch.int16, device=self.device)
        self.reserve(t_cap)

    @property
    def mode_arg(self) -> int:
        """The mode as the C ABI takes it: the quantizer mode plus the activation dtype's flag."""
        return self.mode | act_flag(self.dtype)

    @property
    def unit(self) -> int:
        return TOKEN_BLOCK if self.axis == "channel" else self.group

    def _bytes(self, t_cap: int):
        cb, mb = ctypes.c_int64(), ctypes.c_int64()
        fn = "iq_k_store_bytes" if self.axis == "channel" else "iq_v_store_bytes"
        call(fn, self.B, self.H, t_cap, self.D, self.group, self.bits, self.mode, ctypes.byref(cb), ctypes.byref(mb))
        return cb.value, mb.value

    def reserve(self, n_tokens: int) -> None:
        """Ensure capacity for ``n_tokens`` tokens (amortized doubling; old data is kept)."""
        u = self.unit
        need = -(-max(n_tokens, 0) // u) * u
        if need <= self.t_cap:
            return
        new_cap = max(need, 2 * self.t_cap, 4 * u)
        new_cap = -(-new_cap // u) * u
        cb, mb = self._bytes(new_cap)
        codes = torch.empty(cb // 4, dtype=torch.int32, device=self.device)
        meta = torch.empty(mb // 2, dtype=torch.int16, device=self.device)
        # new capacity starts zeroed: the rows of a partly filled 64-token K block
        # past ``length`` are never written by a quantize, and to_bytes() ships the
        # whole block, so they must not carry stale device memory
        ou, nu, bh = self.t_cap // u, new_cap // u, self.B * self.H
        cv, mv = codes.view(bh, nu, -1), meta.view(bh, nu, -1)
        if ou:
            cv[:, :ou].copy_(self.codes.view(bh, ou, -1))
            mv[:, :ou].copy_(self.meta.view(bh, ou, -1))
        cv[:, ou:].zero_()
        mv[:, ou:].zero_()
        self.codes, self.meta, self.t_cap = codes, meta, new_cap

    def batch_view(self, b0: int, b1: int) -> "PackedStore":
        """Sequences [b0, b1) of this store as a store of B = b1 - b0 that shares its
        memory (a read view: a reserve() or append() through either reaches only
        that object's own tensors)."""
        if not 0 <= b0 < b1 <= self.B:
            raise ValueError(f"batch_view: [{b0}, {b1}) is not a range of the store's {self.B} sequences")
        v = copy.copy(self)
        v.B = b1 - b0
        if self.t_cap:
            v.codes = self.codes.view(self.B, -1)[b0:b1].reshape(-1)
            v.meta = self.meta.view(self.B, -1)[b0:b1].reshape(-1)
        return v

    def nbytes(self, n_tokens: Optional[int] = None) -> int:
        """Packed code + metadata bytes of ``n_tokens`` (default: length) tokens."""
        n = self.length if n_tokens is None else n_tokens
        m = 2 if self.mode == IQ_MODE_SYM else 4
        groups = n * (self.D // self.group) if self.axis == "channel" else (n // self.group) * self.D
        return self.B * self.H * (n * self.D * self.bits // 8 + groups * m)

    # --- wire / on-disk format ------------------------------------------------
    # A safetensors blob: tensors "codes" int32 [B*H, U, words per unit] and
    # "meta" int16 [B*H, U, halves per unit] holding the first U = ceil(length /
    # unit) units of every (batch, head) exactly as they lie in HBM (unit = a
    # 64-token block for axis 'channel', a G-token group for 'token'; the word
    # and half order inside a unit is the store layout), plus string metadata:
    # format "innerq-packed-store", version, axis, B, H, D, group, bits, mode
    # ("asymmetric" | "symmetric" | "hybrid"), length, unit, dtype ("float16" |
    # "bfloat16").  Codes are LSB-first fields of little-endian u32 words; sym
    # fields are offset binary; a hybrid unit's meta is {scale | flag << 15,
    # zero} (flag set: the group holds sym fields).  Version "1" blobs hold
    # fp16 asym or sym stores only (a reader of version 1 knows no dtype and no
    # hybrid flag); a bf16 or hybrid store is written as version "2", which
    # such a reader refuses instead of misreading its metadata.  Both are read.
    WIRE_FORMAT = "innerq-packed-store"
    WIRE_VERSION = "2"             # the newest version written
    WIRE_VERSIONS = ("1", "2")     # versions read

    @staticmethod
    def _safetensors(tensors: dict, metadata: dict) -> bytes:
        """A safetensors container (8-byte little-endian header size, JSON header,
        raw little-endian data) with its JSON keys sorted, so equal stores give
        byte-identical blobs (safetensors' own writer orders the metadata map
        differently from call to call)."""
        import json
        import struct
        dt = {torch.int32: "I32", torch.int16: "I16"}
        header, off, bufs = {"__metadata__": dict(sorted(metadata.items()))}, 0, []
        for name in sorted(tensors):
            t = tensors[name].contiguous()
            b = t.numpy().tobytes()
            header[name] = {"dtype": dt[t.dtype], "shape": list(t.shape), "data_offsets": [off, off + len(b)]}
            off += len(b)
            bufs.append(b)
        h = json.dumps(header, sort_keys=True, separators=(",", ":")).encode()
        h += b" " * (-len(h) % 8)
        return struct.pack("<Q", len(h)) + h + b"".join(bufs)

    def to_bytes(self) -> bytes:
        """The store's valid units in the wire format (see above)."""
        bh, u = self.B * self.H, self.unit
        used = -(-self.length // u)
        nu = self.t_cap // u
        codes = self.codes.view(bh, nu, -1)[:, :used].contiguous().cpu() if nu else \
            torch.empty(bh, 0, 0, dtype=torch.int32)
        meta = self.meta.view(bh, nu, -1)[:, :used].contiguous().cpu() if nu else \
            torch.empty(bh, 0, 0, dtype=torch.int16)
        v2 = self.dtype == torch.bfloat16 or self.mode == IQ_MODE_HYBRID
        md = {"format": self.WIRE_FORMAT, "version": "2" if v2 else "1", "axis": self.axis, "B": self.B,
              "H": self.H, "D": self.D, "group": self.group, "bits": self.bits,
              "mode": MODE_NAMES[self.mode], "length": self.length, "unit": u,
              "dtype": "bfloat16" if self.dtype == torch.bfloat16 else "float16"}
        return self._safetensors({"codes": codes, "meta": meta}, {k: str(v) for k, v in md.items()})

    @classmethod
    def from_bytes(cls, blob: bytes, device, t_cap: int = 0) -> "PackedStore":
        """A store on ``device`` holding what to_bytes() wrote (capacity at least
        ``t_cap`` tokens).  Raises ValueError on a foreign or inconsistent blob."""
        import json
        import struct
        from safetensors.torch import load
        n = struct.unpack("<Q", blob[:8])[0]
        md = json.loads(blob[8:8 + n].decode("utf-8")).get("__metadata__", {})
        if md.get("format") != cls.WIRE_FORMAT or md.get("version") not in cls.WIRE_VERSIONS:
            raise ValueError(f"not an {cls.WIRE_FORMAT} blob of version {' or '.join(cls.WIRE_VERSIONS)}: "
                             f"{md.get('format')!r} v{md.get('version')!r}")
        t = load(blob)
        B, H, D, group, bits, length = (int(md[k]) for k in ("B", "H", "D", "group", "bits", "length"))
        dtype = {"float16": torch.float16, "bfloat16": torch.bfloat16}.get(md.get("dtype", "float16"))
        if dtype is None:
            raise ValueError(f"unknown activation dtype {md.get('dtype')!r}")
        if md["version"] == "1" and dtype != torch.float16 and md.get("dtype") is not None:
            raise ValueError("a version 1 blob holds an fp16 store")
        st = cls(md["axis"], B, H, D, group, bits, md["mode"], device, t_cap=max(t_cap, length), dtype=dtype)
        u = st.unit
        used, nu = -(-length // u), st.t_cap // u
        if int(md["unit"]) != u:
            raise ValueError("unit does not match the axis and group")
        cv, mv = st.codes.view(B * H, nu, -1), st.meta.view(B * H, nu, -1)
        if tuple(t["codes"].shape) != (B * H, used, cv.shape[2]) or tuple(t["meta"].shape) != (B * H, used, mv.shape[2]):
            raise ValueError("codes / meta shapes do not match the store header")
        cv[:, :used].copy_(t["codes"])
        mv[:, :used].copy_(t["meta"])
        st.length = length
        return st

    def save(self, path: str) -> None:
        with open(path, "wb") as f:
            f.write(self.to_bytes())

    @classmethod
    def load(cls, path: str, device, t_cap: int = 0) -> "PackedStore":
        with open(path, "rb") as f:
            return cls.from_bytes(f.read(), device, t_cap)

    # --- writes -------------------------------------------------------------
    def append(self, x: torch.Tensor, norm: Optional[torch.Tensor] = None) -> None:
        """Quantize x [B,H,n,D] (the store's dtype) and append it (quantize-on-append)."""
        require_device(x, "x", self.dtype)
        if x.dim() != 4 or (x.shape[0], x.shape[1], x.shape[3]) != (self.B, self.H, self.D):
            _shape_error(f"append: x has shape {tuple(x.shape)}, the store holds [B={self.B}, H={self.H}, n, "
                         f"D={self.D}]")
        B, H, n, D = x.shape
        if self.axis == "token" and n % self.group:
            _shape_error(f"append: a token-grouped store takes whole groups of {self.group} tokens, got {n}")
        if n == 0:
            return
        self.reserve(self.length + n)
        if self.axis == "channel":
            if x.stride(-1) != 1 or x.data_ptr() % 16 or any(s % 8 for s in x.stride()[:3]):
                x = x.contiguous()
            if norm is not None:
                require_device(norm, "norm", self.dtype)
                norm = norm.reshape(B, H, D).contiguous()
            call("iq_quantize_k", _p(x), x.stride(0), x.stride(1), x.stride(2), _p(norm), B, H, n, D, self.group,
                 self.bits, self.mode_arg, _p(self.codes), _p(self.meta), self.t_cap, self.length, None, None, None,
                 None, _stream(x.device))
        else:
            if x.stride(-1) != 1:
                x = x.contiguous()
            call("iq_quantize_v", _p(x), x.stride(0), x.stride(1), x.stride(2), B, H, n, D, self.group, self.bits,
                 self.mode_arg, _p(self.codes), _p(self.meta), self.t_cap, self.length, None, None, None, None,
                 _stream(x.device))
        self.length += n

    # --- reads --------------------------------------------------------------
    def dequant(self, t0: int = 0, T: Optional[int] = None, out: Optional[torch.Tensor] = None,
                norm: Optional[torch.Tensor] = None, dtype=None) -> torch.Tensor:
        """Dense [B,H,T,D] values of tokens [t0, t0+T) (the store's dtype, or fp32); ``out`` may be a
        strided view."""
        T = self.length - t0 if T is None else T
        check_range(self, "dequant", t0, T)
        if out is None:
            out = torch.empty(self.B, self.H, T, self.D, dtype=dtype or self.dtype, device=self.device)
        check_out(out.shape, (self.B, self.H, T, self.D))
        if out.stride(-1) != 1:
            _shape_error("dequant output must have a contiguous last dimension")
        o16 = _p(out) if out.dtype == self.dtype else None
        o32 = _p(out) if out.dtype == torch.float32 else None
        if o16 is None and o32 is None:
            raise TypeError(f"dequant output must be {self.dtype} or fp32")
        st = out.stride()
        if self.axis == "channel":
            if norm is not None:
                norm = norm.reshape(self.B, self.H, self.D).contiguous()
            call("iq_dequant_k", _p(self.codes), _p(self.meta), self.t_cap, _p(norm), self.B, self.H, t0, T, self.D,
                 self.group, self.bits, self.mode_arg, o16, o32, st[0], st[1], st[2], _stream(out.device))
        else:
            if norm is not None:
                raise ValueError("a key normalization factor applies to head_dim-grouped (K) stores only")
            call("iq_dequant_v", _p(self.codes), _p(self.meta), self.t_cap, self.B, self.H, t0, T, self.D,
                 self.group, self.bits, self.mode_arg, o16, o32, st[0], st[1], st[2], _stream(out.device))
        return out


class RecentWindow:
    """An fp16 recent window [B,H,n,D] (cache.py's keys_recent / values_recent)
    kept in a buffer with room to grow: tokens [start, start + n) of ``buf``.
    A decode step writes its new tokens after the window and advances
    ``start`` past the flushed ones (window_append), so no step copies the
    window.  When the buffer is full the window moves to the front of a new,
    larger buffer; a view returned earlier keeps its old buffer and values.

    With ``deq_rows`` (a K window), each flushed token's row keeps, in place,
    its dequantized values (times the key normalization factor, in the
    activation dtype): the ``shadow`` rows before ``start`` are the tokens
    just before the window, as update() returns them (at most ``keep`` of them
    survive a move to a larger buffer).  A view taken earlier then sees its
    flushed rows change to those values."""

    def __init__(self, x: torch.Tensor, pre: Optional[torch.Tensor] = None, deq_rows: bool = False,
                 keep: int = 0):
        require_act(x, "recent window")
        B, H, n, D = x.shape
        p = 0 if pre is None else pre.shape[2]
        self.buf = torch.empty(B, H, max(2 * (n + p), n + p + 64), D, dtype=x.dtype, device=x.device)
        if p:
            self.buf[:, :, :p].copy_(pre)
        self.buf[:, :, p:p + n].copy_(x)
        self.start, self.n = p, n
        self.deq_rows, self.keep, self.shadow = deq_rows, keep, p

    @property
    def tensor(self) -> torch.Tensor:
        return self.buf[:, :, self.start:self.start + self.n]

    def rows_before(self, p: int) -> torch.Tensor:
        """The p shadow rows before the window and the window: [B,H,p+n,D]."""
        if not 0 <= p <= self.shadow:
            raise ValueError(f"rows_before: {p} rows asked, {self.shadow} held")
        return self.buf[:, :, self.start - p:self.start + self.n]

    def reserve(self, m: int) -> None:
        """Room for m more tokens after the window."""
        B, H, cap, D = self.buf.shape
        if self.start + self.n + m <= cap:
            return
        p = min(self.shadow, self.keep)
        buf = torch.empty(B, H, max(2 * (p + self.n + m), p + self.n + m + 64), D, dtype=self.buf.dtype,
                          device=self.buf.device)
        buf[:, :, :p + self.n].copy_(self.buf[:, :, self.start - p:self.start + self.n])
        self.buf, self.start, self.shadow = buf, p, p


def window_append(kwin: Optional[RecentWindow], knew: Optional[torch.Tensor], kflush: int,
                  kstore: Optional[PackedStore], knorm: Optional[torch.Tensor],
                  vwin: Optional[RecentWindow], vnew: Optional[torch.Tensor], vflush: int,
                  vstore: Optional[PackedStore]) -> None:
    """One decode step of a layer's recent windows in one launch: the new tokens
    [B,H,m,D] go after each window, the first ``flush`` tokens of [window | new]
    are quantized into the store (cache.py:283-365), the windows advance past
    them and the stores grow by them."""
    roles, keep, shape = [], [], None
    for win, x, fl, st, norm in ((kwin, knew, kflush, kstore, knorm), (vwin, vnew, vflush, vstore, None)):
        if win is None:
            roles.append(None)
            continue
        require_device(x, "new tokens", win.buf.dtype)
        if x.stride(-1) != 1:
            x = x.contiguous()
        B, H, m, D = x.shape
        if win.buf.shape[0] != B or win.buf.shape[1] != H or win.buf.shape[3] != D:
            _shape_error(f"window_append: new tokens {tuple(x.shape)} do not fit a window of "
                         f"[{win.buf.shape[0]}, {win.buf.shape[1]}, n, {win.buf.shape[3]}]")
        shape = (B, H, D)
        win.reserve(m)
        w = _lib.iq_window()
        w.buf = win.buf.data_ptr()
        w.s_b, w.s_h, w.s_t = win.buf.stride()[:3]
        w.cap, w.start, w.n = win.buf.shape[2], win.start, win.n
        w.x = x.data_ptr()
        w.sx_b, w.sx_h, w.sx_t = x.stride()[:3]
        w.m, w.flush = m, fl
        if fl:
            if st is None:
                raise ValueError("window_append: flushing tokens needs a store")
            if st.axis == "token" and fl % st.group:
                _shape_error(f"window_append: a token-grouped store takes whole groups of {st.group} tokens, "
                             f"got {fl}")
            st.reserve(st.length + fl)
            w.codes, w.meta = st.codes.data_ptr(), st.meta.data_ptr()
            w.t_cap, w.t_off = st.t_cap, st.length
            if st.dtype != x.dtype:
                raise TypeError(f"window_append: {x.dtype} tokens into a {st.dtype} store")
            w.bits, w.group, w.mode = st.bits, st.group, st.mode_arg
            w.axis = 0 if st.axis == "channel" else 1
            w.deq_rows = 1 if win.deq_rows else 0
            if norm is not None:
                if st.axis != "channel":
                    raise NotImplementedError("key normalization is supported for keys grouped along head_dim")
                norm = norm.reshape(B, H, D).contiguous()
                w.norm = norm.data_ptr()
        keep.append((x, norm))
        roles.append(w)
    if shape is None:
        return
    call("iq_window_append", ctypes.byref(roles[0]) if roles[0] is not None else None,
         ctypes.byref(roles[1]) if roles[1] is not None else None, *shape, _stream(knew.device if knew is not None
                                                                                   else vnew.device))
    for win, x, fl, st in ((kwin, knew, kflush, kstore), (vwin, vnew, vflush, vstore)):
        if win is not None:
            win.start += fl
            win.n += x.shape[-2] - fl
            if fl:
                st.length += fl
                # the flushed rows now hold their dequantized values (deq_rows), right
                # after the shadow rows before them; else no row before the window does
                win.shadow = win.shadow + fl if win.deq_rows else 0


def quantize_dense(x: torch.Tensor, group: int, bits: int, mode, axis: str):
    """Reference-format quantization of a [rows, n, inner]-viewable fp16 or bf16 tensor.

    Returns (codes int32 like x, scale, zero | signs in x's dtype) exactly as
    quant.py's quantize_{channeldim,tokendim}_{asym,sym}.
    """
    require_act(x, "tensor")
    m = mode_id(mode)
    dt = x.dtype
    if m == IQ_MODE_HYBRID:
        raise ValueError("quantize_dense takes 'asymmetric' or 'symmetric'; hybrid quantization is "
                         "quant.quantize_hybrid (both halves) or a hybrid PackedStore")
    shape = tuple(x.shape)
    x = x.contiguous()
    dev = x.device
    codes = torch.empty(shape, dtype=torch.int32, device=dev)
    if axis == "channel":
        n = shape[-1]
        rows = x.numel() // max(n, 1)
        red = shape[:-1] + (n // group,)
        scale = torch.empty(red, dtype=dt, device=dev)
        zs = torch.empty(red if m == IQ_MODE_ASYM else shape, dtype=dt, device=dev)
        call("iq_quantize_k", _p(x), 0, 0, n, None, 1, 1, rows, n, group, bits, m | act_flag(dt), None, None, 0, 0,
             _p(codes), _p(scale), _p(zs) if m == IQ_MODE_ASYM else None, _p(zs) if m == IQ_MODE_SYM else None,
             _stream(dev))
    else:
        n, inner = shape[-2], shape[-1]
        outer = x.numel() // max(n * inner, 1)
        red = shape[:-2] + (n // group, inner)
        scale = torch.empty(red, dtype=dt, device=dev)
        zs = torch.empty(red if m == IQ_MODE_ASYM else shape, dtype=dt, device=dev)
        call("iq_quantize_v", _p(x), 0, n * inner, inner, 1, outer, n, inner, group, bits, m | act_flag(dt), None,
             None, 0, 0,
             _p(codes), _p(scale), _p(zs) if m == IQ_MODE_ASYM else None, _p(zs) if m == IQ_MODE_SYM else None,
             _stream(dev))
    return codes, scale, zs


def dequantize_dense(codes: torch.Tensor, scale: torch.Tensor, zs: torch.Tensor, group: int, mode, axis: str,
                     dtype=torch.float32) -> torch.Tensor:
    require_device(codes, "tensor", torch.int32)
    require_act(scale, "scale")
    require_device(zs, "zero_points/signs", scale.dtype)
    shape = tuple(codes.shape)
    if axis == "channel":
        outer, n, inner = codes.numel() // max(shape[-1], 1), shape[-1], 1
    else:
        n, inner = shape[-2], shape[-1]
        outer = codes.numel() // max(n * inner, 1)
    if dtype not in (torch.float32, scale.dtype):
        raise TypeError(f"op_dtype must be torch.float32 or the scales' {scale.dtype}")
    out = torch.empty(shape, dtype=dtype, device=codes.device)
    call("iq_dequant_dense", _p(codes.contiguous()), _p(scale.contiguous()), _p(zs.contiguous()), outer, n, inner,
         group, mode_id(mode) | act_flag(scale.dtype), 0 if dtype == torch.float32 else 1, _p(out),
         _stream(codes.device))
    return out


_WS = {}


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        _WS[key] = ws
    return ws


def qk_gemv(q: torch.Tensor, k: PackedStore, scale: float, norm: Optional[torch.Tensor] = None, t0: int = 0,
            T: Optional[int] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """logits [B,Hq,T] fp32 = scale * q . K[t0:t0+T] over a channel-grouped store."""
    require_f16_store(k, "qk_gemv")
    require_device(q, "q")
    T = k.length - t0 if T is None else T
    check_qk_shapes(q.shape, k, t0, T, None if out is None else out.shape,
                    None if norm is None else norm.numel())
    B, Hq, D = q.shape
    if q.stride(-1) != 1:
        q = q.contiguous()
    if out is None:
        out = torch.empty(B, Hq, T, dtype=torch.float32, device=q.device)
    require_device(out, "out", torch.float32)
    if out.stride(-1) != 1:
        _shape_error("logits output must have a contiguous token dimension")
    if norm is not None:
        norm = norm.reshape(k.B, k.H, D).contiguous()
    ws = _workspace(q.device, _lib.lib().iq_qk_workspace_bytes(B, Hq, D))
    call("iq_qk_gemv", _p(q), q.stride(0), q.stride(1), _p(norm), _p(k.codes), _p(k.meta), k.t_cap, B, Hq, k.H, t0,
         T, D, k.group, k.bits, k.mode, float(scale), _p(out), out.stride(0), out.stride(1), _p(ws), ws.numel(),
         _stream(q.device))
    return out


def av_gemv(p: torch.Tensor, v: PackedStore, t0: int = 0, T: Optional[int] = None,
            out: Optional[torch.Tensor] = None, out32: Optional[torch.Tensor] = None,
            accumulate: bool = False) -> torch.Tensor:
    """out [B,Hq,D] = p . V[t0:t0+T] over a token-grouped store (fp16 and/or fp32 outputs)."""
    require_f16_store(v, "av_gemv")
    require_device(p, "p")
    T = v.length - t0 if T is None else T
    check_av_shapes(p.shape, v, t0, T, [o.shape for o in (out, out32) if o is not None])
    B, Hq, Tp = p.shape
    if p.stride(-1) != 1:
        p = p.contiguous()
    if out is None and out32 is None:
        out = torch.empty(B, Hq, v.D, dtype=torch.float16, device=p.device)
    if out is not None:
        require_device(out, "out")
    if out32 is not None:
        require_device(out32, "out32", torch.float32)
    ref = out if out is not None else out32
    if out is not None and out32 is not None and out.stride() != out32.stride():
        _shape_error("out and out32 must have the same strides")
    if ref.stride(-1) != 1:
        _shape_error("attn.V output must have a contiguous head_dim")
    nbytes = _lib.lib().iq_av_workspace_bytes(B, Hq, T, v.D, v.group)
    ws = _workspace(p.device, nbytes)
    call("iq_av_gemv", _p(p), p.stride(0), p.stride(1), _p(v.codes), _p(v.meta), v.t_cap, B, Hq, v.H, t0, T, v.D,
         v.group, v.bits, v.mode, _p(out32), _p(out), ref.stride(0), ref.stride(1), 1 if accumulate else 0, _p(ws),
         ws.numel(), _stream(p.device))
    return out if out is not None else out32


def _segment(dense: Optional[torch.Tensor], store: Optional[PackedStore], n: int, t0: int = 0,
             dtype=torch.float16):
    """A decode segment (dtype: the call's activation dtype; a store's mode and a
    dense segment's mode carry its bf16 bit)."""
    s = _lib.iq_segment()
    s.n = n
    if n == 0:
        return s
    if store is not None:
        s.codes, s.meta, s.t_cap, s.t0 = store.codes.data_ptr(), store.meta.data_ptr(), store.t_cap, t0
        s.bits, s.group, s.mode = store.bits, store.group, store.mode_arg
    else:
        require_device(dense, "segment", dtype)
        s.mode = act_flag(dtype)
        if dense.stride(-1) != 1:
            _shape_error("a dense K/V segment must have a contiguous head_dim")
        s.dense = dense.data_ptr()
        s.s_b, s.s_h, s.s_t = dense.stride(0), dense.stride(1), dense.stride(2)
    return s


def _decode_args(q, k_sink, k_store, k_recent, v_sink, v_store, v_recent, norm, out=None, k_t0=0, v_t0=0):
    """Checks and C-ABI segments of a decode call; the activation dtype (fp16 or
    bf16) is the query's, and every store, dense segment, factor and output has it."""
    require_act(q, "q")
    act = q.dtype
    for role, st in (("K", k_store), ("V", v_store)):
        if st is not None and st.dtype != act:
            raise TypeError(f"decode attention {role}: a {st.dtype} store with a {act} query")

    def shp(t):
        return None if t is None else tuple(t.shape)

    B, Hq, Hkv, T, D = check_decode_shapes(shp(q), shp(k_sink), k_store, shp(k_recent), shp(v_sink), v_store,
                                           shp(v_recent), None if norm is None else norm.numel(),
                                           None if out is None else tuple(out.shape), k_t0, v_t0)
    if out is not None:
        require_device(out, "out", act)
        if out.stride(-1) != 1:
            _shape_error("decode output must have a contiguous head_dim")
    if q.stride(-1) != 1:
        q = q.contiguous()

    def n_of(t):
        return 0 if t is None else t.shape[2]

    kn = [n_of(k_sink), k_store.length - k_t0 if k_store is not None else 0, n_of(k_recent)]
    vn = [n_of(v_sink), v_store.length - v_t0 if v_store is not None else 0, n_of(v_recent)]
    ks = (_lib.iq_segment * 3)(_segment(k_sink, None, kn[0], dtype=act), _segment(None, k_store, kn[1], k_t0),
                               _segment(k_recent, None, kn[2], dtype=act))
    vs = (_lib.iq_segment * 3)(_segment(v_sink, None, vn[0], dtype=act), _segment(None, v_store, vn[1], v_t0),
                               _segment(v_recent, None, vn[2], dtype=act))
    if norm is not None:
        require_device(norm, "norm", act)
        norm = norm.reshape(B, Hkv, D).contiguous()
    ws = _workspace(q.device, _lib.lib().iq_decode_workspace_bytes(B, Hq, T, D))
    return q, B, Hq, Hkv, T, D, ks, vs, norm, ws


def decode_attention(q: torch.Tensor, k_sink: Optional[torch.Tensor], k_store: Optional[PackedStore],
                     k_recent: Optional[torch.Tensor], v_sink: Optional[torch.Tensor],
                     v_store: Optional[PackedStore], v_recent: Optional[torch.Tensor], scale: float,
                     norm: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                     k_t0: int = 0, v_t0: int = 0) -> torch.Tensor:
    """One decode step of attention for q [B,Hq,D] over [sink | packed | recent] K and V
    (fp16 or bf16: the query's dtype, which every segment and the output share); the
    stores are read from token k_t0 / v_t0 on (a sliding window's start)."""
    q, B, Hq, Hkv, T, D, ks, vs, norm, ws = _decode_args(q, k_sink, k_store, k_recent, v_sink, v_store, v_recent,
                                                         norm, out, k_t0, v_t0)
    if out is None:
        out = torch.empty(B, Hq, D, dtype=q.dtype, device=q.device)
    call("iq_decode_attention", _p(q), q.stride(0), q.stride(1), _p(norm), ks, vs, B, Hq, Hkv, T, D, float(scale),
         _p(out), out.stride(0), out.stride(1), _p(ws), ws.numel(), _stream(q.device))
    return out


def decode_attention_splits(q, k_sink, k_store, k_recent, v_sink, v_store, v_recent, scale, norm=None) -> int:
    """The split stage of decode_attention (statistics + partials in the device's
    decode workspace); returns the split count for decode_attention_combine."""
    q, B, Hq, Hkv, T, D, ks, vs, norm, ws = _decode_args(q, k_sink, k_store, k_recent, v_sink, v_store, v_recent,
                                                         norm)
    ns = ctypes.c_int(0)
    call("iq_decode_attention_splits", _p(q), q.stride(0), q.stride(1), _p(norm), ks, vs, B, Hq, Hkv, T, D,
         float(scale), _p(ws), ws.numel(), ctypes.byref(ns), _stream(q.device))
    return ns.value


def decode_attention_combine(nsplit: int, B: int, Hq: int, T: int, D: int, device,
                             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The combine stage: merges the splits left in the device's decode workspace."""
    device = torch.device(device)
    if out is None:
        out = torch.empty(B, Hq, D, dtype=torch.float16, device=device)
    require_device(out, "out")
    check_out(out.shape, (B, Hq, D))
    ws = _workspace(device, _lib.lib().iq_decode_workspace_bytes(B, Hq, T, D))
    call("iq_decode_attention_combine", nsplit, B, Hq, T, D, _p(out), out.stride(0), out.stride(1), _p(ws),
         ws.numel(), _stream(device))
    return out


def decode_attention_splits_live(q, k_sink, k_store, k_recent, v_sink, v_store, v_recent, scale,
                                 norm=None) -> "_lib.iq_split_plan":
    """The split stage exactly as decode_attention launches it (live split slots,
    the same fused-kernel grid); returns the plan for decode_attention_combine_live."""
    q, B, Hq, Hkv, T, D, ks, vs, norm, ws = _decode_args(q, k_sink, k_store, k_recent, v_sink, v_store, v_recent,
                                                         norm)
    plan = _lib.iq_split_plan()
    call("iq_decode_attention_splits_live", _p(q), q.stride(0), q.stride(1), _p(norm), ks, vs, B, Hq, Hkv, T, D,
         float(scale), _p(ws), ws.numel(), ctypes.byref(plan), _stream(q.device))
    return plan


def decode_attention_combine_live(plan, B: int, Hq: int, T: int, D: int, device,
                                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The combine of a decode_attention_splits_live stage (the same workspace)."""
    device = torch.device(device)
    dtype = torch.bfloat16 if plan.bf16 else torch.float16
    if out is None:
        out = torch.empty(B, Hq, D, dtype=dtype, device=device)
    require_device(out, "out", dtype)
    check_out(out.shape, (B, Hq, D))
    ws = _workspace(device, _lib.lib().iq_decode_workspace_bytes(B, Hq, T, D))
    call("iq_decode_attention_combine_live", ctypes.byref(plan), B, Hq, T, D, _p(out), out.stride(0), out.stride(1),
         _p(ws), ws.numel(), _stream(device))
    return out


# --- cache-side helpers --------------------------------------------------------
def unpack_store(store: PackedStore, t0: int = 0, T: Optional[int] = None):
    """Reference-format (codes int32, scale fp16, zero | signs fp16) of store tokens [t0, t0+T);
    for a hybrid store the dicts of quant.py:146-149 (see split_hybrid)."""
    T = store.length - t0 if T is None else T
    check_range(store, "unpack", t0, T)
    B, H, D, G = store.B, store.H, store.D, store.group
    dev = store.device
    codes = torch.empty(B, H, T, D, dtype=torch.int32, device=dev)
    red = (B, H, T, D // G) if store.axis == "channel" else (B, H, T // G, D)
    scale = torch.empty(red, dtype=store.dtype, device=dev)
    zs = torch.empty(red if store.mode != IQ_MODE_SYM else (B, H, T, D), dtype=store.dtype, device=dev)
    fn = "iq_unpack_k" if store.axis == "channel" else "iq_unpack_v"
    call(fn, _p(store.codes), _p(store.meta), store.t_cap, B, H, t0, T, D, G, store.bits, store.mode_arg, _p(codes),
         _p(scale), _p(zs), _stream(dev))
    if store.mode == IQ_MODE_HYBRID:
        return split_hybrid(codes, scale, zs, store.bits, store.group, store.axis)
    return codes, scale, zs


def split_hybrid(fields: torch.Tensor, scale_raw: torch.Tensor, zero: torch.Tensor, bits: int, group: int,
                 axis: str):
    """quant.py's hybrid dicts (quant.py:146-149) from the raw unpack of a hybrid store:
    ``fields`` int32 [B,H,T,D] (the stored b-bit fields), ``scale_raw`` the meta's scale half
    with the flag in bit 15, ``zero`` the meta's zero half.  mask = the flag bit (a bit test,
    so a -0.0 scale counts as flagged).  The store keeps only the representation the mask
    selects; the other half of each group reads as zeros (codes, scale, zero point, sign),
    which dequantize_hybrid (quant.py:153-176) never selects."""
    raw = scale_raw.view(torch.int16)
    mask = torch.bitwise_and(raw, -0x8000) != 0
    el = torch.repeat_interleave(mask, group, dim=-1 if axis == "channel" else 2)
    signed = fields - (1 << (bits - 1))
    dt = scale_raw.dtype
    zero_i, zero_h = torch.zeros((), dtype=torch.int32, device=fields.device), \
        torch.zeros((), dtype=dt, device=fields.device)
    s_abs = torch.bitwise_and(raw, 0x7fff).view(dt)
    codes = {"zp": torch.where(el, zero_i, fields), "nozp": torch.where(el, signed.abs(), zero_i)}
    scale = {"zp": torch.where(mask, zero_h, s_abs), "nozp": torch.where(mask, s_abs, zero_h), "mask": mask}
    zs = {"zp": torch.where(mask, zero_h, zero), "nozp": torch.where(el, torch.sign(signed).to(dt), zero_h)}
    return codes, scale, zs


def key_norm_factor(k: torch.Tensor) -> torch.Tensor:
    """sqrt(max_t |k|) of k [B,H,T,D] as [B,H,1,D] in k's dtype (cache.py:121-126)."""
    require_act(k, "key_states")
    if k.stride(-1) != 1:
        k = k.contiguous()
    B, H, T, D = k.shape
    out = torch.empty(B, H, 1, D, dtype=k.dtype, device=k.device)
    call("iq_key_norm_factor", _p(k), k.stride(0), k.stride(1), k.stride(2), B, H, T, D, act_flag(k.dtype), _p(out),
         _stream(k.device))
    return out


def hybrid_mask(x: torch.Tensor, deq_a: torch.Tensor, deq_s: torch.Tensor, group: int, axis: str,
                norm: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Per-group choice of the sym quantization (quant.py:133-151) over [BH,T,D]-viewable tensors."""
    require_act(x, "tensor")
    require_device(deq_a, "deq_zp", torch.float32)
    require_device(deq_s, "deq_nozp", torch.float32)
    *lead, T, D = x.shape
    BH = int(torch.tensor(lead).prod()) if lead else 1
    ax = 0 if axis == "channel" else 1
    shape = tuple(lead) + ((T, D // group) if ax == 0 else (T // group, D))
    mask = torch.empty(shape, dtype=torch.bool, device=x.device)
    if norm is not None:
        require_device(norm, "norm", x.dtype)
        norm = norm.reshape(BH, D).contiguous()
    call("iq_hybrid_mask", _p(x.contiguous()), _p(norm), _p(deq_a.contiguous()), _p(deq_s.contiguous()), BH, T, D,
         group, ax, act_flag(x.dtype), _p(mask), _stream(x.device))
    return mask


def hybrid_select(deq_a: torch.Tensor, deq_s: torch.Tensor, mask: torch.Tensor, group: int, axis: str,
                  dtype=torch.float32) -> torch.Tensor:
    """mask ? deq_s : deq_a over [BH,T,D]-viewable fp32 tensors (quant.py:153-176)."""
    require_device(deq_a, "deq_zp", torch.float32)
    require_device(deq_s, "deq_nozp", torch.float32)
    require_device(mask, "mask", torch.bool)
    *lead, T, D = deq_a.shape
    BH = int(torch.tensor(lead).prod()) if lead else 1
    codes = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
    if dtype not in codes:
        raise TypeError("op_dtype must be torch.float32, torch.float16 or torch.bfloat16")
    out = torch.empty(deq_a.shape, dtype=dtype, device=deq_a.device)
    call("iq_hybrid_select", _p(deq_a.contiguous()), _p(deq_s.contiguous()), _p(mask.contiguous()), BH, T, D, group,
         0 if axis == "channel" else 1, codes[dtype], _p(out), _stream(deq_a.device))
    return out
