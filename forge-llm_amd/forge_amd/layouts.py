"""Packed-weight formats of the quantized-linear path.

The formats are Forge's artifact format and stay byte-identical to it (the reference defines them in
``forge/kernels/layouts/w4.py:1-30,83-172``, ``w8.py:1-30``, ``layout.py:124-190`` and ``bits.py:18-35``): a stored
model packed by Forge loads here unchanged, and the other way round.  The code that produces and reads those bytes
is this module's own.

Logical weight (what a quantiser hands over):  codes ``q uint8 [N, K]`` in 0..15, ``scales [N, G]``,
zero-points ``uint8 [N, G]`` or None (symmetric: zero-point 8), optionally ``g_idx int32 [K]`` (act order); the
dense weight is ``W[n, k] = (q[n, k] - zero[n, g(k)]) * scale[n, g(k)]``.

Physical W4 layouts, each a :class:`Layout` with a deterministic id (blake2b of the storage description):

``portable_row`` (``w4.portable_row.v1-73e10e``)
    ``qweight int32 [N, ceil(K/8)]``, code ``k`` of row ``n`` in word ``k // 8`` at bits ``4 * (k % 8)``.  What the
    gfx950 GEMV, prefill and generic kernels read.
``mma_fragment`` (``w4.mma_fragment_k16n64.v1-445296``)
    The reference's NVIDIA ``m16n8k16`` B-fragment order over 16 x 64 tiles.  Accepted from artifacts and repacked
    to portable_row at prepare time; no gfx950 kernel reads it.
``cdna4_mfma`` (``w4.cdna4_mfma_k128n16.v1-…``, this build's own)
    The B-operand order of gfx950's ``v_mfma_f32_16x16x32_{bf16,f16}`` over tiles of 16 channels x 128 columns:
    ``qweight int32 [ceil(N/16), ceil(K/128) * 256]``, one 1 KiB tile per 256 words, tile ``(nt, kt)`` at row ``nt``,
    words ``256 kt ..``.  Lane ``l = 16 j + r`` of a wavefront owns words ``4 l .. 4 l + 3`` of a tile (one 16-byte
    load); word ``s`` holds channel ``16 nt + r``, columns ``128 kt + 32 s + 8 j + t`` (t = 0..7) -- the eight B
    values lane ``l`` feeds k-step ``s`` -- with column ``t`` in nibble slot ``t / 2`` (even t) or ``4 + t / 2`` (odd
    t), so ``(word >> 4 p) & 0x000F000F`` is the pair ``(t, t + 1) = (2p, 2p + 1)`` as two 16-bit lanes: one
    ``v_and_or_b32`` with the magic exponent turns it into an exact bf16 / fp16 pair, in MFMA order, with no
    shuffle of weights or activations.  Padding columns carry their group's zero-point (they dequantise to 0),
    padding channels code 8.  Scales and zero-points are stored as in portable_row.

These are load-time data-movement utilities (torch tensor ops, on whatever device the tensors live); the
arithmetic of the path -- dequantisation and every GEMM -- runs in the HIP library only (``PackedW4.dequantize``
calls ``fg_w4_dequant``).
"""
from __future__ import annotations

import hashlib
import json
import threading
from dataclasses import asdict, dataclass, field
from typing import Any, Callable

import torch

from .errors import ConfigError, HardwareUnsupported, NotFound

KIND_PORTABLE = KIND_PORTABLE_ROW = "portable_row"
KIND_FRAGMENT = "mma_fragment"
KIND_CDNA4 = "cdna4_mfma"
IDENTITY_INTERLEAVE: tuple[int, ...] = (0, 1, 2, 3, 4, 5, 6, 7)
# slot i of a word holds element MARLIN_INTERLEAVE[i]: even elements in the low half-word, odd ones in the high
MARLIN_INTERLEAVE: tuple[int, ...] = (0, 2, 4, 6, 1, 3, 5, 7)
TILE_K, TILE_N = 16, 64  # mma_fragment storage tile
CDNA4_TILE_K, CDNA4_TILE_N = 128, 16  # cdna4_mfma storage tile


# ================================================================================================ integer helpers
def roundup(x: int, m: int) -> int:
    return ceil_div(x, m) * int(m)


def ceil_div(a: int, b: int) -> int:
    return (int(a) + int(b) - 1) // int(b)


def effective_group(group_size: int | None, k: int) -> int:
    """Columns per group; ``group_size <= 0`` (or None) means one group spanning the row."""
    return int(k) if group_size is None or int(group_size) <= 0 else int(group_size)


def num_groups(k: int, group_size: int | None) -> int:
    return ceil_div(k, effective_group(group_size, k))


# ================================================================================================ nibble codec
# Codes are packed two per byte (even position in the low nibble) and four bytes per little-endian int32, so nibble j
# of a word sits at bits 4j: the int32 view of the packed bytes is the word array (x86 hosts and gfx950 are both
# little-endian).
def pack_nibbles_int32(nib: torch.Tensor) -> torch.Tensor:
    """``nib [..., 8]`` (values 0..15) -> ``int32 [...]`` with nibble ``j`` at bits ``4j``."""
    if nib.shape[-1] != 8:
        raise ValueError("last dim must be 8")
    b = nib.to(torch.uint8) & 0xF
    pairs = (b[..., 0::2] | (b[..., 1::2] << 4)).contiguous()
    return pairs.view(torch.int32).squeeze(-1)


def unpack_nibbles_int32(words: torch.Tensor) -> torch.Tensor:
    """``int32 [...]`` -> ``uint8 [..., 8]`` (inverse of :func:`pack_nibbles_int32`)."""
    b = words.contiguous().unsqueeze(-1).view(torch.uint8)  # [..., 4]
    return torch.stack((b & 0xF, b >> 4), dim=-1).flatten(-2)


def _codes_to_words(codes: torch.Tensor) -> torch.Tensor:
    """``uint8 [..., 8w]`` codes in storage order -> ``int32 [..., w]``."""
    return pack_nibbles_int32(codes.reshape(*codes.shape[:-1], -1, 8))


def _words_to_codes(words: torch.Tensor) -> torch.Tensor:
    """``int32 [..., w]`` -> ``uint8 [..., 8w]`` codes in storage order."""
    return unpack_nibbles_int32(words).flatten(-2)


# ================================================================================================ layouts
@dataclass(frozen=True)
class Layout:
    """Storage layout descriptor.  Its fields, ``to_dict`` / ``from_dict`` and id scheme are the artifact interface
    of ``forge/kernels/layouts/layout.py:41-90``; ``id`` covers only what changes the stored bytes."""

    id: str
    kind: str
    bits: int
    atom: str = ""
    tile_k: int = 1
    tile_n: int = 1
    vec_bytes: int = 16
    interleave: tuple[int, ...] = IDENTITY_INTERLEAVE
    scales: dict = field(default_factory=dict, hash=False, compare=False)
    swizzle: dict = field(default_factory=dict, hash=False, compare=False)
    partition: dict = field(default_factory=dict, hash=False, compare=False)
    schedule: dict = field(default_factory=dict, hash=False, compare=False)
    executor: str = "hip"
    chip_family: str = "generic"

    def to_dict(self) -> dict[str, Any]:
        out = asdict(self)
        out["interleave"] = list(self.interleave)
        return out

    @classmethod
    def from_dict(cls, d: dict[str, Any]) -> Layout:
        known = {f for f in cls.__dataclass_fields__}
        kw = {k: v for k, v in d.items() if k in known}
        kw["interleave"] = tuple(kw.get("interleave", IDENTITY_INTERLEAVE))
        return cls(**kw)


def _storage_id(base: str, storage: dict[str, Any]) -> str:
    text = json.dumps(storage, sort_keys=True, separators=(",", ":"))
    return base + "-" + hashlib.blake2b(text.encode(), digest_size=3).hexdigest()


class _Registry:
    """Layouts by id, so an artifact that carries only ``layout_id`` can be read back."""

    def __init__(self) -> None:
        self._by_id: dict[str, Layout] = {}
        self._lock = threading.RLock()

    def add(self, lay: Layout) -> Layout:
        with self._lock:
            self._by_id[lay.id] = lay
        return lay

    def find(self, layout_id: str) -> Layout | None:
        with self._lock:
            return self._by_id.get(layout_id)

    def all(self) -> list[Layout]:
        with self._lock:
            return [self._by_id[k] for k in sorted(self._by_id)]


_LAYOUTS = _Registry()


def register_layout(lay: Layout) -> Layout:
    return _LAYOUTS.add(lay)


def get_layout(layout_id: str) -> Layout:
    lay = _LAYOUTS.find(layout_id)
    if lay is None:
        raise NotFound(f"unknown layout id {layout_id!r}", details={"known": [x.id for x in _LAYOUTS.all()]})
    return lay


def known_layouts() -> list[Layout]:
    return _LAYOUTS.all()


def _as_layout(layout: Layout | str | None, default: Layout) -> Layout:
    if layout is None:
        return default
    return get_layout(layout) if isinstance(layout, str) else layout


def portable_layout(bits: int) -> Layout:
    """Row-sequential codes (4-bit: 8 per int32 word; 8-bit: one int8 per element), scales ``[G, N]``."""
    if bits not in (4, 8):
        raise ConfigError(f"portable layout supports 4 or 8 bits, got {bits}")
    scales = {"orientation": "col_contig_GxN", "pad_n_to": 1}
    swizzle = {"kind": "none"}
    tile_k = 8 if bits == 4 else 1
    storage = {"kind": KIND_PORTABLE, "bits": bits, "atom": "", "tile_k": tile_k, "tile_n": 1,
               "interleave": list(IDENTITY_INTERLEAVE), "scales": scales, "swizzle": swizzle}
    return register_layout(Layout(_storage_id(f"w{bits}.portable_row.v1", storage), KIND_PORTABLE, bits,
                                  tile_k=tile_k, scales=scales, swizzle=swizzle, chip_family="any"))


def fragment_layout(interleave: tuple[int, ...] = MARLIN_INTERLEAVE) -> Layout:
    """The reference's NVIDIA m16n8k16 B-fragment layout (16 x 64 tiles), read from artifacts only."""
    scales = {"orientation": "col_contig_GxN", "pad_n_to": TILE_N}
    swizzle = {"kind": "xor", "vec_bytes": 16, "rule": "vec_col ^= row % 8"}
    storage = {"kind": KIND_FRAGMENT, "bits": 4, "atom": "mma_b_k2x2", "tile_k": TILE_K, "tile_n": TILE_N,
               "interleave": list(interleave), "scales": scales, "swizzle": swizzle}
    return register_layout(Layout(_storage_id("w4.mma_fragment_k16n64.v1", storage), KIND_FRAGMENT, 4,
                                  atom="m16n8k16", tile_k=TILE_K, tile_n=TILE_N, interleave=tuple(interleave),
                                  scales=scales, swizzle=swizzle, executor="native"))


def cdna4_layout() -> Layout:
    """gfx950 MFMA B-operand order over 16-channel x 128-column tiles (module docstring)."""
    scales = {"orientation": "col_contig_GxN", "pad_n_to": 1}
    swizzle = {"kind": "none"}
    storage = {"kind": KIND_CDNA4, "bits": 4, "atom": "mfma_f32_16x16x32_b", "tile_k": CDNA4_TILE_K,
               "tile_n": CDNA4_TILE_N, "interleave": list(MARLIN_INTERLEAVE), "scales": scales, "swizzle": swizzle}
    return register_layout(Layout(_storage_id("w4.cdna4_mfma_k128n16.v1", storage), KIND_CDNA4, 4,
                                  atom="v_mfma_f32_16x16x32", tile_k=CDNA4_TILE_K, tile_n=CDNA4_TILE_N,
                                  interleave=MARLIN_INTERLEAVE, scales=scales, swizzle=swizzle, executor="hip",
                                  chip_family="gfx950"))


PORTABLE_W4 = portable_layout(4)
PORTABLE_W8 = portable_layout(8)
FRAGMENT_W4 = fragment_layout()
CDNA4_W4 = cdna4_layout()


# ================================================================================================ W4 storage codecs
# A codec maps the padded code matrix ``uint8 [n_pad, k_pad]`` to the stored ``qweight`` and back.  Each layout kind
# has one; pack / unpack / repack only go through this table.
@dataclass(frozen=True)
class _W4Codec:
    pad_n: int
    pad_k: int
    scale_pad_n: bool  # scales / zero-points padded to n_pad (mma_fragment) or kept at N
    encode: Callable[[torch.Tensor, Layout], torch.Tensor]
    decode: Callable[[torch.Tensor, int, int, Layout], torch.Tensor]


def _portable_encode(codes: torch.Tensor, lay: Layout) -> torch.Tensor:
    return _codes_to_words(codes)


def _portable_decode(qweight: torch.Tensor, n_pad: int, k_pad: int, lay: Layout) -> torch.Tensor:
    return _words_to_codes(qweight)[:n_pad, :k_pad]


_FRAG_CACHE: dict[tuple, torch.Tensor] = {}


def fragment_tile_perm(interleave: tuple[int, ...] = MARLIN_INTERLEAVE) -> tuple[torch.Tensor, torch.Tensor]:
    """Storage position of every element of one 16 x 64 mma_fragment tile: returns ``(idx, inv)`` with ``idx[pos]``
    the flat ``k * 64 + n`` coordinate stored at nibble position ``pos`` (word ``pos // 8``, slot ``pos % 8``) and
    ``inv`` its inverse.

    Built forward from the m16n8k16 B-operand ownership (``forge/kernels/layouts/w4.py:56-80``): element ``(k, n)``
    belongs to lane ``4 (n % 8) + (k % 8) // 2``, N block ``n // 8`` and pair ``r = k % 2 + 2 (k // 8)``; the lane's
    natural element ``32 lane + 4 block + r`` sits at slot ``interleave^-1`` of that index inside its word.
    """
    key = tuple(int(i) for i in interleave)
    hit = _FRAG_CACHE.get(key)
    if hit is None:
        k = torch.arange(TILE_K).view(-1, 1).expand(TILE_K, TILE_N)
        n = torch.arange(TILE_N).view(1, -1).expand(TILE_K, TILE_N)
        lane = 4 * (n % 8) + (k % 8) // 2
        natural = 32 * lane + 4 * (n // 8) + (k % 2) + 2 * (k // 8)
        slot_of = torch.empty(8, dtype=torch.int64)
        slot_of[torch.tensor(key)] = torch.arange(8)
        pos = 8 * (natural // 8) + slot_of[natural % 8]  # [16, 64] -> storage position
        if torch.unique(pos).numel() != TILE_K * TILE_N:
            raise AssertionError("fragment permutation is not bijective")
        inv = pos.reshape(-1)  # coordinate -> position
        idx = torch.empty_like(inv)
        idx[inv] = torch.arange(inv.numel())
        hit = _FRAG_CACHE[key] = torch.stack((idx, inv))
    return hit[0], hit[1]


def _fragment_encode(codes: torch.Tensor, lay: Layout) -> torch.Tensor:
    n_pad, k_pad = codes.shape
    kt, nt = k_pad // TILE_K, n_pad // TILE_N
    idx, _ = fragment_tile_perm(lay.interleave)
    tiles = codes.t().reshape(kt, TILE_K, nt, TILE_N).permute(0, 2, 1, 3).reshape(kt, nt, TILE_K * TILE_N)
    return _codes_to_words(tiles[..., idx.to(codes.device)]).reshape(kt, nt * (TILE_K * TILE_N // 8))


def _fragment_decode(qweight: torch.Tensor, n_pad: int, k_pad: int, lay: Layout) -> torch.Tensor:
    kt, nt = k_pad // TILE_K, n_pad // TILE_N
    _, inv = fragment_tile_perm(lay.interleave)
    seq = _words_to_codes(qweight.reshape(kt, nt, -1))
    tiles = seq[..., inv.to(seq.device)].reshape(kt, nt, TILE_K, TILE_N)
    return tiles.permute(0, 2, 1, 3).reshape(k_pad, n_pad).t()


def _cdna4_encode(codes: torch.Tensor, lay: Layout) -> torch.Tensor:
    # codes [NT*16 (r), KT*128 (s, j, t)] -> [NT, KT, j, r, s, slot] with slot i holding column t = interleave[i]
    n_pad, k_pad = codes.shape
    nt, kt = n_pad // CDNA4_TILE_N, k_pad // CDNA4_TILE_K
    v = codes.reshape(nt, CDNA4_TILE_N, kt, 4, 4, 8)[..., list(lay.interleave)]
    v = v.permute(0, 2, 4, 1, 3, 5).reshape(nt, kt * CDNA4_TILE_N * CDNA4_TILE_K)
    return _codes_to_words(v)


def _cdna4_decode(qweight: torch.Tensor, n_pad: int, k_pad: int, lay: Layout) -> torch.Tensor:
    nt, kt = n_pad // CDNA4_TILE_N, k_pad // CDNA4_TILE_K
    v = _words_to_codes(qweight).reshape(nt, kt, 4, CDNA4_TILE_N, 4, 8)  # [NT, KT, j, r, s, slot]
    inverse = [0] * 8
    for slot, t in enumerate(lay.interleave):
        inverse[t] = slot
    v = v[..., inverse].permute(0, 3, 1, 4, 2, 5)  # [NT, r, KT, s, j, t]
    return v.reshape(n_pad, k_pad)


_W4_CODECS = {
    KIND_PORTABLE: _W4Codec(1, 8, False, _portable_encode, _portable_decode),
    KIND_FRAGMENT: _W4Codec(TILE_N, TILE_K, True, _fragment_encode, _fragment_decode),
    KIND_CDNA4: _W4Codec(CDNA4_TILE_N, CDNA4_TILE_K, False, _cdna4_encode, _cdna4_decode),
}


def _codec(lay: Layout) -> _W4Codec:
    c = _W4_CODECS.get(lay.kind)
    if c is None or lay.bits != 4:
        raise ConfigError(f"layout {lay.id} ({lay.kind}, {lay.bits}-bit) is not a W4 storage layout")
    return c


def w4_storage_shapes(lay: Layout, n: int, k: int, n_groups: int, has_zeros: bool) -> dict[str, tuple[int, int]]:
    """Shapes of the stored tensors of an ``N x K`` weight in ``lay`` (what a module registers as buffers)."""
    c = _codec(lay)
    n_pad, k_pad = roundup(n, c.pad_n), roundup(k, c.pad_k)
    if lay.kind == KIND_PORTABLE:
        q = (n, k_pad // 8)
    elif lay.kind == KIND_FRAGMENT:
        q = (k_pad // TILE_K, n_pad * TILE_K // 8)
    else:
        q = (n_pad // CDNA4_TILE_N, k_pad * CDNA4_TILE_N // 8)
    sn = n_pad if c.scale_pad_n else n
    out = {"qweight": q, "scales": (n_groups, sn)}
    if has_zeros:
        out["zeros"] = (n_groups, ceil_div(sn, 8))
    return out


# ================================================================================================ PackedW4
@dataclass
class PackedW4:
    """A packed 4-bit weight with scales, optional zero-points and act-order ``g_idx`` in some :class:`Layout`.
    Field names, ``tensors()`` keys, ``tensor_roles()`` and ``state()`` are the artifact interface
    (``forge/kernels/layouts/w4.py:83-172``)."""

    qweight: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor | None
    layout: Layout
    n: int
    k: int
    group_size: int
    g_idx: torch.Tensor | None = None
    meta: dict[str, Any] = field(default_factory=dict)

    layout_id = property(lambda self: self.layout.id)
    shape = property(lambda self: (self.n, self.k))
    num_groups = property(lambda self: int(self.scales.shape[0]))
    device = property(lambda self: self.qweight.device)

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.tensors().values())

    @property
    def bits_per_weight(self) -> float:
        return 8.0 * self.nbytes / max(1, self.n * self.k)

    def to(self, device: Any = None, dtype: torch.dtype | None = None) -> PackedW4:
        """A copy on ``device`` (``dtype`` converts the scales only)."""
        def move(t: torch.Tensor | None, dt: torch.dtype | None = None) -> torch.Tensor | None:
            if t is None:
                return None
            return t.to(device=t.device if device is None else device, dtype=dt or t.dtype)

        return PackedW4(move(self.qweight), move(self.scales, dtype), move(self.zeros), self.layout, self.n, self.k,
                        self.group_size, move(self.g_idx), dict(self.meta))

    def unpack(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
        return unpack_w4(self)

    def dequantize(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Dense ``[N, K]`` weight: ``(q - z) * s`` in fp32, rounded once to ``dtype`` -- by the HIP kernel."""
        from .ops_gemm import w4_dequant

        return w4_dequant(self, dtype)

    def tensors(self) -> dict[str, torch.Tensor]:
        named = {"qweight": self.qweight, "scales": self.scales, "zeros": self.zeros, "g_idx": self.g_idx}
        return {k: v for k, v in named.items() if v is not None}

    @staticmethod
    def tensor_roles() -> dict[str, str]:
        return {"qweight": "payload", "scales": "scale", "zeros": "zero", "g_idx": "perm"}

    def state(self) -> dict[str, Any]:
        return {"layout_id": self.layout.id, "layout": self.layout.to_dict(), "n": self.n, "k": self.k,
                "group_size": self.group_size, "scale_dtype": str(self.scales.dtype).split(".")[-1]}

    @classmethod
    def from_tensors(cls, tensors: dict[str, torch.Tensor], state: dict[str, Any]) -> PackedW4:
        lay = _LAYOUTS.find(state.get("layout_id", "")) or Layout.from_dict(state["layout"])
        return cls(tensors["qweight"], tensors["scales"], tensors.get("zeros"), lay, int(state["n"]), int(state["k"]),
                   int(state["group_size"]), tensors.get("g_idx"))


def _column_groups(k: int, k_pad: int, gs: int, n_groups: int, g_idx: torch.Tensor | None,
                   device: torch.device) -> torch.Tensor:
    """Group of every padded column: ``min(k // gs, G - 1)``, or ``g_idx`` with padding columns in the last
    column's group."""
    if g_idx is None:
        return (torch.arange(k_pad, device=device) // gs).clamp(max=n_groups - 1)
    gi = g_idx.to(device=device, dtype=torch.int64)
    return torch.cat((gi, gi[-1:].expand(k_pad - k)))


def _validate_w4(q: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor | None, group_size: int,
                 g_idx: torch.Tensor | None) -> int:
    """Check the logical parts; returns the number of groups."""
    if q.dim() != 2:
        raise ConfigError(f"codes must be a 2-D [N, K] tensor, got shape {tuple(q.shape)}")
    if q.dtype != torch.uint8:
        raise ConfigError(f"codes must be uint8 in 0..15, got {q.dtype}")
    n, k = q.shape
    if n * k == 0:
        raise ConfigError(f"cannot pack an empty weight [N={n}, K={k}]")
    if group_size is not None and group_size > 0 and group_size % 8:
        raise ConfigError(f"group_size must be <= 0 (per channel) or a multiple of 8, got {group_size}")
    if g_idx is not None:
        if g_idx.dim() != 1 or g_idx.shape[0] != k:
            raise ConfigError(f"g_idx must be [K={k}], got {tuple(g_idx.shape)}")
        g = int(scales.shape[-1]) if scales.dim() == 2 else 0
        lo, hi = int(g_idx.min()), int(g_idx.max())
        if lo < 0 or hi >= g:
            raise ConfigError(f"g_idx values {lo}..{hi} do not index the {g} scale groups")
    else:
        g = num_groups(k, group_size)
    for name, t in (("scales", scales), ("zeros", zeros)):
        if t is not None and tuple(t.shape) != (n, g):
            raise ConfigError(f"{name} must be [N={n}, G={g}], got {tuple(t.shape)}")
    if int(q.max()) > 15:
        raise ConfigError("codes above 15 do not fit 4 bits")
    if zeros is not None:
        zi = zeros.to(torch.int16)
        if int(zi.min()) < 0 or int(zi.max()) > 15:
            raise ConfigError("zero-points must lie in 0..15")
    return g


def pack_w4(q: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor | None = None, group_size: int = 128,
            layout: Layout | str | None = None, g_idx: torch.Tensor | None = None) -> PackedW4:
    """Pack the logical parts (module docstring) into ``layout`` (default portable_row).  Signature and stored
    bytes as ``forge/kernels/layouts/w4.py:203-257``."""
    lay = _as_layout(layout, PORTABLE_W4)
    if lay.bits != 4:
        raise ConfigError(f"layout {lay.id} is not a 4-bit layout")
    c = _codec(lay)
    g = _validate_w4(q, scales, zeros, group_size, g_idx)
    n, k = q.shape
    gs = effective_group(group_size, k)
    if lay.kind == KIND_FRAGMENT and group_size > 0 and gs % TILE_K:
        raise ConfigError(f"the mma_fragment layout needs group_size % 16 == 0, got {group_size}")
    dev = q.device
    n_pad, k_pad = roundup(n, c.pad_n), roundup(k, c.pad_k)
    zp = torch.full((n, g), 8, dtype=torch.uint8, device=dev) if zeros is None else zeros.to(torch.uint8)
    codes = torch.full((n_pad, k_pad), 8, dtype=torch.uint8, device=dev)
    if lay.kind == KIND_FRAGMENT:
        codes.zero_()
    codes[:n, :k] = q
    if k_pad > k:  # padding columns dequantise to exactly 0: code = the column's zero-point
        codes[:n, k:] = zp[:, _column_groups(k, k_pad, gs, g, g_idx, dev)[k:]]
    qweight = c.encode(codes, lay).contiguous()
    sn = n_pad if c.scale_pad_n else n
    sc = torch.zeros((g, sn), dtype=scales.dtype, device=dev)
    sc[:, :n] = scales.t()
    zq = None
    if zeros is not None:
        zt = torch.zeros((g, roundup(sn, 8)), dtype=torch.uint8, device=dev)
        zt[:, :n] = zp.t()
        zq = _codes_to_words(zt)
    gi = None if g_idx is None else g_idx.to(torch.int32).contiguous()
    return PackedW4(qweight, sc.contiguous(), zq, lay, n, k, int(group_size), gi, {"n_pad": n_pad, "k_pad": k_pad})


def unpack_w4(p: PackedW4) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """Exact inverse of :func:`pack_w4`: ``(q uint8 [N, K], scales [N, G], zeros uint8 [N, G] | None)``."""
    c = _codec(p.layout)
    n_pad, k_pad = roundup(p.n, c.pad_n), roundup(p.k, c.pad_k)
    codes = c.decode(p.qweight, n_pad, k_pad, p.layout)
    q = codes[:p.n, :p.k].contiguous()
    scales = p.scales[:, :p.n].t().contiguous()
    zeros = None if p.zeros is None else _words_to_codes(p.zeros)[:, :p.n].t().contiguous()
    return q, scales, zeros


def repack(p: PackedW4, new_layout: Layout | str) -> PackedW4:
    """The same logical weight in another layout: a permutation of the stored codes, never a re-quantisation."""
    lay = _as_layout(new_layout, PORTABLE_W4)
    if lay.id == p.layout.id:
        return p
    q, s, z = unpack_w4(p)
    return pack_w4(q, s, z, p.group_size, lay, p.g_idx)


def sz8_blocks(scales: torch.Tensor, zeros: torch.Tensor | None, n: int) -> tuple[torch.Tensor, torch.Tensor | None]:
    """A portable_row weight's scales ``[G, >= N]`` and zero words ``[G, >= N / 8]`` re-blocked by 8 channels for the
    decode GEMV's contiguous reads (``fg_w4a16_gemv_sz8``): ``scales8 [N / 8, G, 8]`` with scale ``(g, n)`` at
    ``[n // 8, g, n % 8]``, ``zeros8 [N / 8, G]`` with the zero word of group ``g`` and channels ``8 b .. 8 b + 7`` at
    ``[b, g]``.  A permutation of the stored values on their device (no arithmetic); ``zeros`` None stays None."""
    if n % 8:
        raise ConfigError(f"8-channel scale blocks need N % 8 == 0, got N={n}")
    if scales.dim() != 2 or scales.shape[1] < n or (zeros is not None and zeros.shape[1] < n // 8):
        raise ConfigError(f"scales {tuple(scales.shape)} / zeros {None if zeros is None else tuple(zeros.shape)} do "
                          f"not cover N={n}")
    g = scales.shape[0]
    s8 = scales[:, :n].reshape(g, n // 8, 8).permute(1, 0, 2).contiguous()
    z8 = None if zeros is None else zeros[:, :n // 8].t().contiguous()
    return s8, z8


def require_portable(p: PackedW4) -> None:
    if p.layout.kind != KIND_PORTABLE:
        raise ConfigError(f"this kernel reads the portable_row layout, got {p.layout_id}; repack() first")


# ================================================================================================ act order
class _Missing:
    """Marker of a cold or stale act-order cache when computing is not allowed (e.g. during graph capture)."""

    def __repr__(self) -> str:
        return "MISSING_SORT"

    def __bool__(self) -> bool:
        return False


MISSING_SORT = _Missing()
_ACT_ORDER_KEY = "hip.act_order"  # p.meta entry: (tensor versions, result or None)


def sort_columns_by_group(p: PackedW4) -> tuple[PackedW4, torch.Tensor] | None:
    """Act-order weight made regular: K columns stably sorted by group id so each group is one contiguous run
    (``forge/kernels/layouts/w4.py:308-337``).  Returns ``(weight in portable_row, perm int32 [K])`` with
    ``x @ W^T == x[:, perm] @ W_sorted^T``, or None when there is no ``g_idx`` or the group sizes are not those of
    ``group_size`` (each group exactly that many columns, the last the remainder).  Reads ``g_idx`` on the host:
    prepare time only."""
    if p.g_idx is None:
        return None
    gs, g = effective_group(p.group_size, p.k), int(p.scales.shape[0])
    gi = p.g_idx.detach().to("cpu", torch.int64)
    if gi.numel() != p.k or int(gi.min()) < 0 or int(gi.max()) >= g:
        return None
    sizes = torch.bincount(gi, minlength=g)
    expect = torch.tensor([min(gs, p.k - i * gs) for i in range(g)])
    if (expect <= 0).any() or not torch.equal(sizes, expect):
        return None
    perm = torch.sort(gi, stable=True).indices
    q, s, z = unpack_w4(p)
    perm_dev = perm.to(q.device)
    return pack_w4(q.index_select(1, perm_dev), s, z, p.group_size, PORTABLE_W4), perm_dev.to(torch.int32)


def _versions(p: PackedW4) -> tuple:
    return tuple((t.data_ptr(), t._version, tuple(t.shape), str(t.device)) for t in p.tensors().values())


def cached_group_sort(p: PackedW4, *, compute: bool = True) -> Any:
    """:func:`sort_columns_by_group`, memoised in ``p.meta`` and invalidated when any of ``p``'s tensors changes.
    Returns None (no g_idx or irregular groups), the ``(weight, perm)`` pair, or :data:`MISSING_SORT` when the
    cache is cold and ``compute`` is false."""
    if p.g_idx is None:
        return None
    key = _versions(p)
    entry = p.meta.get(_ACT_ORDER_KEY)
    if entry is None or entry[0] != key:
        if not compute:
            return MISSING_SORT
        entry = p.meta[_ACT_ORDER_KEY] = (key, sort_columns_by_group(p))
    return entry[1]


# ================================================================================================ RTN quantisers
def _groups_of(w: torch.Tensor, group_size: int) -> tuple[torch.Tensor, int, int]:
    """``w [N, K]`` as fp32 ``[N, G, gs]``; a ragged last group is filled with zeros.  Zeros never change the
    quantities below: the absolute max is >= 0 and the asymmetric range always includes 0."""
    n, k = w.shape
    gs = effective_group(group_size, k)
    g = ceil_div(k, gs)
    wf = torch.zeros((n, g * gs), dtype=torch.float32, device=w.device)
    wf[:, :k] = w
    return wf.view(n, g, gs), g, gs


def _rounded_scale(raw: torch.Tensor, scale_dtype: torch.dtype) -> torch.Tensor:
    """The stored scale: floored at 1e-12, rounded to ``scale_dtype``, and floored again in fp32 (a tiny scale can
    round to 0 in fp16) -- the value the codes are computed with."""
    return raw.clamp_min(1e-12).to(scale_dtype).float().clamp_min(1e-12)


def quantize_w4_rtn(w: torch.Tensor, group_size: int = 128, sym: bool = True,
                    scale_dtype: torch.dtype = torch.float16) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """Round-to-nearest int4 (``forge/kernels/layouts/rtn.py:27-57``) -> ``(q uint8 [N, K], scales [N, G],
    zeros uint8 [N, G] | None)``.  Symmetric: ``scale = amax / 7``, ``q = clamp(round(w / scale), -8, 7) + 8``
    (zero-point 8, ``zeros`` None).  Asymmetric: ``scale = (max(w, 0) - min(w, 0)) / 15``,
    ``zero = clamp(round(-min / scale), 0, 15)``, ``q = clamp(round(w / scale + zero), 0, 15)``."""
    if w.dim() != 2:
        raise ConfigError("w must be [N, K]")
    n, k = w.shape
    wg, g, gs = _groups_of(w, group_size)
    if sym:
        s = _rounded_scale(wg.abs().amax(-1) / 7.0, scale_dtype)
        codes = torch.round(wg / s[..., None]).clamp(-8, 7) + 8
        zeros = None
    else:
        lo, hi = wg.amin(-1).clamp(max=0), wg.amax(-1).clamp(min=0)
        s = _rounded_scale((hi - lo) / 15.0, scale_dtype)
        zf = torch.round(-lo / s).clamp(0, 15)
        codes = torch.round(wg / s[..., None] + zf[..., None]).clamp(0, 15)
        zeros = zf.to(torch.uint8)
    q = codes.reshape(n, g * gs)[:, :k].to(torch.uint8).contiguous()
    return q, s.to(scale_dtype), zeros


def quantize_w8_rtn(w: torch.Tensor, group_size: int = -1,
                    scale_dtype: torch.dtype = torch.float16) -> tuple[torch.Tensor, torch.Tensor]:
    """Round-to-nearest symmetric int8 (``forge/kernels/layouts/rtn.py:60-72``): ``scale = amax / 127`` (stored in
    ``scale_dtype``), ``q = clamp(round(w / scale), -128, 127)``; returns ``(q int8 [N, K], scales [N, G])``."""
    if w.dim() != 2:
        raise ConfigError("w must be [N, K]")
    n, k = w.shape
    wg, g, gs = _groups_of(w, group_size)
    s = _rounded_scale(wg.abs().amax(-1) / 127.0, scale_dtype)
    q = torch.round(wg / s[..., None]).clamp(-128, 127).reshape(n, g * gs)[:, :k]
    return q.to(torch.int8).contiguous(), s.to(scale_dtype)


# ================================================================================================ W8A8 weights (host)
# Host-side producers of the W8A8 weight formats, for checkpoints quantised on the CPU before they reach the GPU
# (the reference builds both packed kinds from a dense CPU nn.Linear, forge/kernels/ops_gemm.py:391-393,945).  Every
# step is an IEEE fp32 operation done the way the device quantisers do it (fg_quant.hip): scale = amax / fmax by true
# division with a tensor divisor, 1 where `amax > 0` is false (all-zero groups and NaN-poisoned ones), codes from
# x / scale by true division, so a weight quantised here or on the GPU has the same codes and scales bit for bit.
_E4M3_MAX = 448.0


def _amax_scale(amax: torch.Tensor, fmax: float) -> torch.Tensor:
    return torch.where(amax > 0, amax / torch.full_like(amax, fmax), torch.ones_like(amax))


def quantize_fp8_weight(w: torch.Tensor, granularity: str = "per_channel",
                        block: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """OCP e4m3fn weight codes ``[N, K]`` and fp32 scales: ``per_tensor`` ``[1]``, ``per_channel`` ``[N]``, or
    ``block2d`` ``[ceil(N/block), ceil(K/block)]`` (``forge/kernels/ref/gemm_fp8.py:43-85``); codes are
    ``e4m3fn(clamp(w / s, -448, 448))``, rounded to nearest even."""
    if w.dim() != 2:
        raise ConfigError("w must be [N, K]")
    if granularity not in ("per_tensor", "per_channel", "block2d"):
        raise ConfigError(f"unknown fp8 weight granularity {granularity!r}")
    wf = w.detach().float()
    n, k = wf.shape
    if granularity == "per_channel":
        s = _amax_scale(wf.abs().amax(dim=1) if k else wf.new_zeros(n), _E4M3_MAX)
        full = s[:, None]
    elif granularity == "per_tensor":
        s = _amax_scale(wf.abs().amax().reshape(1) if wf.numel() else wf.new_zeros(1), _E4M3_MAX)
        full = s.reshape(1, 1)
    else:
        if block <= 0:
            raise ConfigError(f"block must be positive, got {block}")
        nb, kb = ceil_div(n, block), ceil_div(k, block)
        tiles = wf.new_zeros((nb * block, kb * block))
        tiles[:n, :k] = wf  # zero padding changes no tile's absolute max
        s = _amax_scale(tiles.view(nb, block, kb, block).abs().amax(dim=(1, 3)), _E4M3_MAX)
        full = s.repeat_interleave(block, 0).repeat_interleave(block, 1)[:n, :k]
    q = (wf / full).clamp(-_E4M3_MAX, _E4M3_MAX).to(torch.float8_e4m3fn)
    return q.contiguous(), s.contiguous()


def quantize_int8_weight(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-channel int8 weight codes ``[N, K]`` and fp32 scales ``[N]`` (``forge/kernels/ref/gemm_int8.py
    :17-35`` with ``per_channel``): ``s = amax / 127``, ``q = clamp(round_half_even(w / s), -127, 127)``."""
    if w.dim() != 2:
        raise ConfigError("w must be [N, K]")
    wf = w.detach().float()
    s = _amax_scale(wf.abs().amax(dim=1) if wf.shape[1] else wf.new_zeros(wf.shape[0]), 127.0)
    q = torch.round(wf / s[:, None]).clamp(-127, 127)
    return torch.nan_to_num(q, nan=0.0).to(torch.int8).contiguous(), s.contiguous()


# ================================================================================================ simple int4
SIMPLE_LAYOUT_ID = "forge.simple.v1"


def pack_simple_int4(codes: torch.Tensor) -> torch.Tensor:
    """Codes ``[N, K]`` (< 16) in the compress pipeline's "simple" layout (``forge/formats/packing.py:1-5``):
    ``uint8 [N, ceil(K/2)]``, code ``k`` in byte ``k // 2``, even ``k`` in the low nibble."""
    c = codes.to(torch.uint8)
    if c.shape[1] % 2:
        c = torch.cat((c, torch.zeros_like(c[:, :1])), dim=1)
    return (c[:, 0::2] | (c[:, 1::2] << 4)).contiguous()


def unpack_simple_int4(q8: torch.Tensor, k: int) -> torch.Tensor:
    """Inverse of :func:`pack_simple_int4`."""
    return torch.stack((q8 & 0xF, q8 >> 4), dim=-1).reshape(q8.shape[0], -1)[:, :k].contiguous()


def pack_w4_from_simple(qweight: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor | None, group_size: int,
                        k: int) -> PackedW4:
    """A ``forge.simple.v1`` int4 weight (``forge/compress/packed.py:9-12,265-274``: ``qweight uint8 [N, K/2]``,
    ``scales [N, G]``, ``zeros uint8 [N, G]`` or None) as a portable_row :class:`PackedW4`, bit-identical to
    ``pack_w4(codes, scales, zeros, group_size)``.  Both formats put code ``k`` at bit ``4 (k % 8)`` of the
    little-endian word ``k // 8``: for ``K % 8 == 0`` the packed bytes are reused as an int32 view (no copy)."""
    if qweight.dtype != torch.uint8 or qweight.dim() != 2 or qweight.shape[1] != (k + 1) // 2:
        raise ConfigError(f"simple int4 qweight must be uint8 [N, ceil(K/2)={(k + 1) // 2}], got "
                          f"{tuple(qweight.shape)} {qweight.dtype}")
    if k % 8:  # portable_row pads K to 8 with zero-point codes: go through the codes
        return pack_w4(unpack_simple_int4(qweight, k), scales, zeros, group_size)
    n = qweight.shape[0]
    if group_size is not None and group_size > 0 and group_size % 8:
        raise ConfigError(f"group_size must be <= 0 or a multiple of 8, got {group_size}")
    g = num_groups(k, group_size)
    if tuple(scales.shape) != (n, g) or (zeros is not None and tuple(zeros.shape) != (n, g)):
        raise ConfigError(f"scales / zeros must be [N={n}, G={g}]")
    if zeros is not None and int(zeros.to(torch.int16).max()) > 15:
        raise ConfigError("zero-points must lie in 0..15")
    zq = None
    if zeros is not None:
        zt = torch.zeros((g, roundup(n, 8)), dtype=torch.uint8, device=qweight.device)
        zt[:, :n] = zeros.to(torch.uint8).t()
        zq = _codes_to_words(zt)
    return PackedW4(qweight.contiguous().view(torch.int32), scales.t().contiguous(), zq, PORTABLE_W4, n, k,
                    int(group_size), None, {"n_pad": n, "k_pad": k})


# ================================================================================================ PackedW8
@dataclass
class PackedW8:
    """Symmetric int8 weight in the portable_row W8 layout (``forge/kernels/layouts/w8.py:18-80``):
    ``qweight int8 [N, K]``, ``scales [G, N]``, per channel (``group_size <= 0``) or grouped along K."""

    qweight: torch.Tensor
    scales: torch.Tensor
    layout: Layout
    n: int
    k: int
    group_size: int
    meta: dict[str, Any] = field(default_factory=dict)

    layout_id = property(lambda self: self.layout.id)
    shape = property(lambda self: (self.n, self.k))
    num_groups = property(lambda self: int(self.scales.shape[0]))
    device = property(lambda self: self.qweight.device)

    @property
    def nbytes(self) -> int:
        return self.qweight.numel() * self.qweight.element_size() + self.scales.numel() * self.scales.element_size()

    @property
    def bits_per_weight(self) -> float:
        return 8.0 * self.nbytes / max(1, self.n * self.k)

    def to(self, device: Any = None, dtype: torch.dtype | None = None) -> PackedW8:
        dev = self.qweight.device if device is None else device
        return PackedW8(self.qweight.to(dev), self.scales.to(device=dev, dtype=dtype or self.scales.dtype),
                        self.layout, self.n, self.k, self.group_size, dict(self.meta))

    def unpack(self) -> tuple[torch.Tensor, torch.Tensor]:
        return unpack_w8(self)

    def dequantize(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Dense ``[N, K]`` weight ``q * s`` (exact in fp32), cast to ``dtype``."""
        q, s = unpack_w8(self)
        return dequantize_w8_parts(q, s, self.group_size).to(dtype)

    def tensors(self) -> dict[str, torch.Tensor]:
        return {"qweight": self.qweight, "scales": self.scales}

    @staticmethod
    def tensor_roles() -> dict[str, str]:
        return {"qweight": "payload", "scales": "scale"}

    def state(self) -> dict[str, Any]:
        return {"layout_id": self.layout.id, "layout": self.layout.to_dict(), "n": self.n, "k": self.k,
                "group_size": self.group_size, "scale_dtype": str(self.scales.dtype).split(".")[-1]}

    @classmethod
    def from_tensors(cls, tensors: dict[str, torch.Tensor], state: dict[str, Any]) -> PackedW8:
        lay = _LAYOUTS.find(state.get("layout_id", "")) or Layout.from_dict(state["layout"])
        return cls(tensors["qweight"], tensors["scales"], lay, int(state["n"]), int(state["k"]),
                   int(state["group_size"]))


def pack_w8(q: torch.Tensor, scales: torch.Tensor, group_size: int = -1, layout: Layout | str | None = None) -> PackedW8:
    """``q int8 [N, K]`` and ``scales [N, G]`` as a :class:`PackedW8` (scales stored transposed, ``[G, N]``)."""
    lay = _as_layout(layout, PORTABLE_W8)
    if lay.bits != 8:
        raise ConfigError(f"layout {lay.id} is not an 8-bit layout")
    if q.dim() != 2 or q.dtype != torch.int8:
        raise ConfigError(f"codes must be an int8 [N, K] tensor, got {q.dtype} {tuple(q.shape)}")
    n, k = q.shape
    g = num_groups(k, group_size)
    if tuple(scales.shape) != (n, g):
        raise ConfigError(f"scales must be [N={n}, G={g}], got {tuple(scales.shape)}")
    return PackedW8(q.contiguous(), scales.t().contiguous(), lay, n, k, int(group_size))


def unpack_w8(p: PackedW8) -> tuple[torch.Tensor, torch.Tensor]:
    """``(q int8 [N, K], scales [N, G])``."""
    return p.qweight, p.scales.t().contiguous()


def dequantize_w8_parts(q: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """``W[n, k] = q[n, k] * scales[n, k // gs]`` in fp32 (exact: int8 times a 16-bit float fits fp32)."""
    k = q.shape[1]
    cols = torch.arange(k, device=q.device) // effective_group(group_size, k)
    return q.float() * scales.float().index_select(1, cols)


__all__ = [
    "CDNA4_W4", "FRAGMENT_W4", "HardwareUnsupported", "IDENTITY_INTERLEAVE", "KIND_CDNA4", "KIND_FRAGMENT",
    "KIND_PORTABLE", "KIND_PORTABLE_ROW", "Layout", "MARLIN_INTERLEAVE", "MISSING_SORT", "PORTABLE_W4", "PORTABLE_W8",
    "PackedW4", "PackedW8", "SIMPLE_LAYOUT_ID", "cached_group_sort", "cdna4_layout", "ceil_div", "dequantize_w8_parts",
    "effective_group", "fragment_layout", "fragment_tile_perm", "get_layout", "known_layouts", "num_groups",
    "pack_nibbles_int32", "pack_simple_int4", "pack_w4", "pack_w4_from_simple", "pack_w8", "portable_layout",
    "quantize_fp8_weight", "quantize_int8_weight", "quantize_w4_rtn", "quantize_w8_rtn", "register_layout", "repack", "require_portable", "roundup",
    "sort_columns_by_group", "sz8_blocks", "unpack_nibbles_int32", "unpack_simple_int4", "unpack_w4", "unpack_w8",
    "w4_storage_shapes",
]
