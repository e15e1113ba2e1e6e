"""Packed-weight formats of the quantized-linear path (the artifact format Forge writes; kept byte-identical).

Mirrors the public surface of ``forge/kernels/layouts`` (``w4.py:83-365``, ``layout.py:85-233``, ``bits.py:18-43``,
``rtn.py:27-72``): :class:`Layout` descriptors with deterministic ids, :class:`PackedW4` (+ ``pack_w4`` /
``unpack_w4`` / ``repack``), the act-order column sort, and the RTN int4 quantiser used by ``from_dense``.

W4 ``portable_row`` (what the gfx950 kernels read): ``qweight int32 [N, ceil(K/8)]`` with nibble ``j`` of word ``w``
holding ``q[n, 8w + j]``; ``scales [G, N]``; ``zeros int32 [G, ceil(N/8)]`` with 8 channels per word, or ``None`` for
the symmetric zero-point 8.  K padding columns carry their group's zero-point so they dequantise to exactly 0.

The reference's ``mma_fragment`` layout (an NVIDIA m16n8k16 B-fragment order, ``w4.py:56-80``) is accepted as input
and repacked to portable_row once at prepare time; it is never produced for the GPU path.

These are load-time data-movement utilities (torch tensor ops on whatever device the tensors live on); the
arithmetic of the path -- dequantisation and every GEMM -- runs only in the HIP library (``PackedW4.dequantize``
calls ``fg_w4_dequant``).
"""
from __future__ import annotations

import hashlib
import json
import threading
from dataclasses import asdict, dataclass, field
from typing import Any

import torch

from .errors import ConfigError, HardwareUnsupported, NotFound

KIND_PORTABLE = KIND_PORTABLE_ROW = "portable_row"
KIND_FRAGMENT = "mma_fragment"
IDENTITY_INTERLEAVE: tuple[int, ...] = (0, 1, 2, 3, 4, 5, 6, 7)
MARLIN_INTERLEAVE: tuple[int, ...] = (0, 2, 4, 6, 1, 3, 5, 7)
TILE_K, TILE_N = 16, 64


# ------------------------------------------------------------------------------------------------ bit helpers
def roundup(x: int, m: int) -> int:
    return -(-int(x) // int(m)) * int(m)


def ceil_div(a: int, b: int) -> int:
    return -(-int(a) // int(b))


def pack_nibbles_int32(nib: torch.Tensor) -> torch.Tensor:
    """``nib[..., 8]`` (0..15) -> int32 with nibble ``j`` at bits ``4j`` (two's-complement wrap of bit 31)."""
    if nib.shape[-1] != 8:
        raise ValueError("last dim must be 8")
    shifts = torch.arange(0, 32, 4, dtype=torch.int64, device=nib.device)
    w = ((nib.to(torch.int64) & 0xF) << shifts).sum(dim=-1)
    return torch.where(w >= 2 ** 31, w - 2 ** 32, w).to(torch.int32)


def unpack_nibbles_int32(words: torch.Tensor) -> torch.Tensor:
    """int32 ``[...]`` -> uint8 ``[..., 8]``."""
    shifts = torch.arange(0, 32, 4, dtype=torch.int64, device=words.device)
    return ((words.to(torch.int64).unsqueeze(-1) & 0xFFFFFFFF) >> shifts & 0xF).to(torch.uint8)


# ------------------------------------------------------------------------------------------------ layouts
@dataclass(frozen=True)
class Layout:
    """Storage layout descriptor; ``id`` hashes only what changes the stored bytes (``layout.py:85-137``)."""

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
        d = asdict(self)
        d["interleave"] = list(self.interleave)
        return d

    @classmethod
    def from_dict(cls, d: dict[str, Any]) -> Layout:
        d = dict(d)
        d["interleave"] = tuple(d.get("interleave", IDENTITY_INTERLEAVE))
        return cls(**d)


def _layout_id(base: str, sig: dict[str, Any]) -> str:
    blob = json.dumps(sig, sort_keys=True, separators=(",", ":")).encode()
    return f"{base}-{hashlib.blake2b(blob, digest_size=3).hexdigest()}"


_REG: dict[str, Layout] = {}
_REG_LOCK = threading.RLock()


def register_layout(lay: Layout) -> Layout:
    with _REG_LOCK:
        _REG[lay.id] = lay
    return lay


def get_layout(layout_id: str) -> Layout:
    with _REG_LOCK:
        lay = _REG.get(layout_id)
    if lay is None:
        raise NotFound(f"unknown layout id {layout_id!r}", details={"known": sorted(_REG)})
    return lay


def known_layouts() -> list[Layout]:
    with _REG_LOCK:
        return [_REG[k] for k in sorted(_REG)]


def portable_layout(bits: int) -> Layout:
    if bits not in (4, 8):
        raise ConfigError(f"portable layout supports 4 or 8 bits, got {bits}")
    sig = {"kind": KIND_PORTABLE, "bits": bits, "atom": "", "tile_k": 8 if bits == 4 else 1, "tile_n": 1,
           "interleave": list(IDENTITY_INTERLEAVE), "scales": {"orientation": "col_contig_GxN", "pad_n_to": 1},
           "swizzle": {"kind": "none"}}
    return register_layout(Layout(id=_layout_id(f"w{bits}.portable_row.v1", sig), kind=KIND_PORTABLE, bits=bits,
                                  tile_k=sig["tile_k"], scales=sig["scales"], swizzle=sig["swizzle"], chip_family="any"))


def fragment_layout(interleave: tuple[int, ...] = MARLIN_INTERLEAVE) -> Layout:
    sig = {"kind": KIND_FRAGMENT, "bits": 4, "atom": "mma_b_k2x2", "tile_k": TILE_K, "tile_n": TILE_N,
           "interleave": list(interleave), "scales": {"orientation": "col_contig_GxN", "pad_n_to": TILE_N},
           "swizzle": {"kind": "xor", "vec_bytes": 16, "rule": "vec_col ^= row % 8"}}
    return register_layout(Layout(id=_layout_id("w4.mma_fragment_k16n64.v1", sig), kind=KIND_FRAGMENT, bits=4,
                                  atom="m16n8k16", tile_k=TILE_K, tile_n=TILE_N, interleave=tuple(interleave),
                                  scales=sig["scales"], swizzle=sig["swizzle"], executor="native"))


PORTABLE_W4 = portable_layout(4)
PORTABLE_W8 = portable_layout(8)
FRAGMENT_W4 = fragment_layout()


def fragment_tile_perm(interleave: tuple[int, ...] = MARLIN_INTERLEAVE) -> tuple[torch.Tensor, torch.Tensor]:
    """Nibble position -> flat ``k*64 + n`` coordinate inside one 16x64 fragment tile, and its inverse.

    Position ``p`` (word ``p // 8``, slot ``p % 8``) stores natural element ``e = 8*(p//8) + interleave[p%8]``;
    natural element ``e`` belongs to lane ``e // 32``, N block ``(e % 32) // 4`` and pair ``r = e % 4``, i.e.
    ``k = 2*(lane % 4) + r % 2 + 8*(r // 2)``, ``n = 8*block + lane // 4`` (``forge/kernels/layouts/w4.py:56-80``).
    """
    pos = torch.arange(TILE_K * TILE_N)
    il = torch.tensor(interleave, dtype=torch.int64)
    natural = (pos // 8) * 8 + il[pos % 8]
    lane, e = natural // 32, natural % 32
    block, r = e // 4, e % 4
    k = (lane % 4) * 2 + (r % 2) + 8 * (r // 2)
    n = block * 8 + lane // 4
    idx = k * TILE_N + n
    inv = torch.empty_like(idx)
    inv[idx] = pos
    if torch.unique(idx).numel() != idx.numel():
        raise AssertionError("fragment permutation is not bijective")
    return idx, inv


def effective_group(group_size: int, k: int) -> int:
    return int(k) if group_size is None or group_size <= 0 else int(group_size)


def num_groups(k: int, group_size: int) -> int:
    return ceil_div(k, effective_group(group_size, k))


# ------------------------------------------------------------------------------------------------ PackedW4
@dataclass
class PackedW4:
    """A packed 4-bit weight + scales (+ zeros, g_idx) in some :class:`Layout` (``w4.py:83-172``)."""

    qweight: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor | None
    layout: Layout
    n: int
    k: int
    group_size: int
    g_idx: torch.Tensor | None = None
    meta: dict[str, Any] = field(default_factory=dict)

    @property
    def layout_id(self) -> str:
        return self.layout.id

    @property
    def shape(self) -> tuple[int, int]:
        return (self.n, self.k)

    @property
    def num_groups(self) -> int:
        return int(self.scales.shape[0])

    @property
    def device(self) -> torch.device:
        return self.qweight.device

    @property
    def nbytes(self) -> int:
        ts = [self.qweight, self.scales] + [t for t in (self.zeros, self.g_idx) if t is not None]
        return sum(t.numel() * t.element_size() for t in ts)

    @property
    def bits_per_weight(self) -> float:
        return 8.0 * self.nbytes / max(1, self.n * self.k)

    def to(self, device: Any = None, dtype: torch.dtype | None = None) -> PackedW4:
        def mv(t, dt=None):
            return None if t is None else t.to(device=device or t.device, dtype=dt or t.dtype)

        return PackedW4(mv(self.qweight), mv(self.scales, dtype), mv(self.zeros), self.layout, self.n, self.k,
                        self.group_size, mv(self.g_idx), dict(self.meta))

    def unpack(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
        return unpack_w4(self)

    def dequantize(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Dense ``[N, K]`` weight: ``(q - z) * s`` in fp32, rounded once to ``dtype`` -- by the HIP kernel."""
        from .ops_gemm import w4_dequant

        return w4_dequant(self, dtype)

    def tensors(self) -> dict[str, torch.Tensor]:
        out = {"qweight": self.qweight, "scales": self.scales}
        if self.zeros is not None:
            out["zeros"] = self.zeros
        if self.g_idx is not None:
            out["g_idx"] = self.g_idx
        return out

    @staticmethod
    def tensor_roles() -> dict[str, str]:
        return {"qweight": "payload", "scales": "scale", "zeros": "zero", "g_idx": "perm"}

    def state(self) -> dict[str, Any]:
        return {"layout_id": self.layout.id, "layout": self.layout.to_dict(), "n": self.n, "k": self.k,
                "group_size": self.group_size, "scale_dtype": str(self.scales.dtype).replace("torch.", "")}

    @classmethod
    def from_tensors(cls, tensors: dict[str, torch.Tensor], state: dict[str, Any]) -> PackedW4:
        lay = get_layout(state["layout_id"]) if state.get("layout_id") in _REG else Layout.from_dict(state["layout"])
        return cls(tensors["qweight"], tensors["scales"], tensors.get("zeros"), lay, int(state["n"]), int(state["k"]),
                   int(state["group_size"]), tensors.get("g_idx"))


def _check_inputs(q, scales, zeros, group_size, g_idx):
    if q.dim() != 2:
        raise ConfigError(f"q must be [N, K], got {tuple(q.shape)}")
    n, k = q.shape
    if n == 0 or k == 0:
        raise ConfigError("empty weight")
    if group_size is not None and group_size > 0 and group_size % 8 != 0:
        raise ConfigError(f"group_size must be -1 or a multiple of 8, got {group_size}")
    if g_idx is None:
        g = num_groups(k, group_size)
    else:
        if tuple(g_idx.shape) != (k,):
            raise ConfigError("g_idx must have shape [K]")
        g = int(scales.shape[1])
        if int(g_idx.max()) >= g or int(g_idx.min()) < 0:
            raise ConfigError("g_idx out of range for scales")
    if tuple(scales.shape) != (n, g):
        raise ConfigError(f"scales must be [N={n}, G={g}], got {tuple(scales.shape)}")
    if zeros is not None and tuple(zeros.shape) != (n, g):
        raise ConfigError(f"zeros must be [N={n}, G={g}], got {tuple(zeros.shape)}")
    if q.dtype != torch.uint8:
        raise ConfigError("q must be uint8 (values 0..15)")
    if int(q.max()) > 15:
        raise ConfigError("q contains values > 15")
    if zeros is not None and (int(zeros.max()) > 15 or int(zeros.min()) < 0):
        raise ConfigError("zeros must be in 0..15")


def pack_w4(q: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor | None = None, group_size: int = 128,
            layout: Layout | str | None = None, g_idx: torch.Tensor | None = None) -> PackedW4:
    """Pack logical ``(q uint8 [N,K], scales [N,G], zeros uint8 [N,G] | None)`` (``w4.py:203-257``)."""
    lay = PORTABLE_W4 if layout is None else (get_layout(layout) if isinstance(layout, str) else layout)
    if lay.bits != 4:
        raise ConfigError(f"layout {lay.id} is not a 4-bit layout")
    _check_inputs(q, scales, zeros, group_size, g_idx)
    n, k = q.shape
    g = scales.shape[1]
    gs = effective_group(group_size, k)
    if lay.kind == KIND_FRAGMENT and group_size > 0 and gs % TILE_K != 0:
        raise ConfigError(f"fragment layout needs group_size multiple of 16 (got {group_size})")
    if lay.kind == KIND_PORTABLE:
        k_pad, n_pad = roundup(k, 8), n
    elif lay.kind == KIND_FRAGMENT:
        k_pad, n_pad = roundup(k, TILE_K), roundup(n, TILE_N)
    else:
        raise ConfigError(f"cannot pack W4 into layout kind {lay.kind}")
    dev = q.device
    zp = zeros.to(torch.uint8) if zeros is not None else torch.full((n, g), 8, dtype=torch.uint8, device=dev)
    qp = torch.zeros((n_pad, k_pad), dtype=torch.uint8, device=dev)
    qp[:n, :k] = q
    if k_pad > k:  # padding columns take their group's zero-point -> dequantise to 0
        gk = (torch.clamp(torch.arange(k, k_pad, device=dev) // gs, max=g - 1) if g_idx is None
              else g_idx[-1].long().repeat(k_pad - k).to(dev))
        qp[:n, k:] = zp[:, gk]
    if lay.kind == KIND_PORTABLE:
        qweight = pack_nibbles_int32(qp.view(n_pad, k_pad // 8, 8))
    else:
        idx, _ = fragment_tile_perm(lay.interleave)
        kt, nt = k_pad // TILE_K, n_pad // TILE_N
        tiles = qp.t().contiguous().view(kt, TILE_K, nt, TILE_N).permute(0, 2, 1, 3).reshape(kt, nt, TILE_K * TILE_N)
        qweight = pack_nibbles_int32(tiles[..., idx.to(dev)].reshape(kt, nt, 128, 8)).reshape(kt, nt * 128)
    sc = torch.zeros((g, n_pad), dtype=scales.dtype, device=dev)
    sc[:, :n] = scales.t()
    zq = None
    if zeros is not None:
        zt = torch.zeros((g, roundup(n_pad, 8)), dtype=torch.uint8, device=dev)
        zt[:, :n] = zp.t()
        zq = pack_nibbles_int32(zt.view(g, -1, 8))
    gi = None if g_idx is None else g_idx.to(torch.int32).contiguous()
    return PackedW4(qweight.contiguous(), sc.contiguous(), zq, lay, n, k, int(group_size), gi,
                    {"n_pad": n_pad, "k_pad": k_pad})


def unpack_w4(p: PackedW4) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """Exact inverse of :func:`pack_w4` -> ``(q uint8 [N,K], scales [N,G], zeros uint8 [N,G] | None)``."""
    lay, n, k = p.layout, p.n, p.k
    if lay.kind == KIND_PORTABLE:
        nib = unpack_nibbles_int32(p.qweight)
        q = nib.reshape(nib.shape[0], -1)[:n, :k]
    elif lay.kind == KIND_FRAGMENT:
        k_pad, n_pad = roundup(k, TILE_K), roundup(n, TILE_N)
        kt, nt = k_pad // TILE_K, n_pad // TILE_N
        _, inv = fragment_tile_perm(lay.interleave)
        seq = unpack_nibbles_int32(p.qweight.view(kt, nt, 128)).reshape(kt, nt, TILE_K * TILE_N)
        full = seq[..., inv.to(seq.device)].view(kt, nt, TILE_K, TILE_N).permute(0, 2, 1, 3).reshape(k_pad, n_pad)
        q = full.t()[:n, :k]
    else:
        raise ConfigError(f"cannot unpack layout kind {lay.kind}")
    scales = p.scales[:, :n].t().contiguous()
    zeros = None
    if p.zeros is not None:
        zeros = unpack_nibbles_int32(p.zeros).reshape(p.zeros.shape[0], -1)[:, :n].t().contiguous()
    return q.contiguous(), scales, zeros


def repack(p: PackedW4, new_layout: Layout | str) -> PackedW4:
    """Re-pack into another layout (pure permutation of the stored nibbles; no re-quantisation)."""
    lay = get_layout(new_layout) if isinstance(new_layout, str) else new_layout
    if lay.id == p.layout.id:
        return p
    q, s, z = unpack_w4(p)
    return pack_w4(q, s, z, p.group_size, lay, p.g_idx)


def sort_columns_by_group(p: PackedW4) -> tuple[PackedW4, torch.Tensor] | None:
    """Act-order weights (``g_idx``) made regular by a stable sort of the K columns by group (``w4.py:308-337``).

    Returns ``(sorted portable weight, perm int32 [K])`` with ``x @ W^T == x[:, perm] @ W_sorted^T``, or None when
    there is no ``g_idx`` or the groups are irregular.  Synchronises the device: prepare time only.
    """
    if p.g_idx is None:
        return None
    gs, g = effective_group(p.group_size, p.k), int(p.scales.shape[0])
    gi = p.g_idx.long().cpu()
    if gi.numel() != p.k or int(gi.min()) < 0 or int(gi.max()) >= g:
        return None
    want = torch.full((g,), gs, dtype=torch.int64)
    want[-1] = p.k - gs * (g - 1)
    if int(want[-1]) <= 0 or not torch.equal(torch.bincount(gi, minlength=g), want):
        return None
    perm = torch.argsort(gi, stable=True)
    q, s, z = unpack_w4(p)
    dev = q.device
    return pack_w4(q[:, perm.to(dev)], s, z, p.group_size, PORTABLE_W4, None), perm.to(torch.int32).to(dev)


class _Missing:
    def __repr__(self) -> str:
        return "MISSING_SORT"

    def __bool__(self) -> bool:
        return False


MISSING_SORT = _Missing()
_NO_SORT = object()
GROUP_SORT_KEY = "_gsorted"


def _stamp(*ts: torch.Tensor | None) -> tuple:
    return tuple((t.data_ptr(), t._version, tuple(t.shape), str(t.device)) for t in ts if t is not None)


def cached_group_sort(p: PackedW4, *, compute: bool = True) -> Any:
    """``(sorted weight, perm)`` cached in ``p.meta`` and stamped with the source tensors' identity/version
    (``w4.py:348-365``); ``MISSING_SORT`` when cold and ``compute`` is false (e.g. under graph capture)."""
    if p.g_idx is None:
        return None
    stamp = _stamp(p.qweight, p.scales, p.zeros, p.g_idx)
    hit = p.meta.get(GROUP_SORT_KEY)
    if hit is None or hit[0] != stamp:
        if not compute:
            return MISSING_SORT
        res = sort_columns_by_group(p)
        hit = p.meta[GROUP_SORT_KEY] = (stamp, _NO_SORT if res is None else res)
    return None if hit[1] is _NO_SORT else hit[1]


# ------------------------------------------------------------------------------------------------ RTN quantiser
def _grouped(w: torch.Tensor, group_size: int) -> tuple[torch.Tensor, int, int]:
    n, k = w.shape
    gs = effective_group(group_size, k)
    g = ceil_div(k, gs)
    wf = w.float()
    if g * gs > k:
        wf = torch.nn.functional.pad(wf, (0, g * gs - k), value=float("nan"))
    return wf.view(n, g, gs), g, gs


def quantize_w4_rtn(w: torch.Tensor, group_size: int = 128, sym: bool = True,
                    scale_dtype: torch.dtype = torch.float16) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """Round-to-nearest int4 (``rtn.py:27-57``): symmetric ``scale = amax/7`` (zero-point 8 implied), asymmetric
    ``scale = (max - min)/15``, ``zero = round(-min/scale)``; the scale is rounded to ``scale_dtype`` before use."""
    if w.dim() != 2:
        raise ConfigError("w must be [N, K]")
    n, k = w.shape
    wg, g, gs = _grouped(w, group_size)
    valid = ~torch.isnan(wg)
    wz = torch.where(valid, wg, torch.zeros_like(wg))
    if sym:
        scale = (wz.abs().amax(dim=-1) / 7.0).clamp_min(1e-12)
        scale = scale.to(scale_dtype).float().clamp_min(1e-12)
        q = torch.round(wz / scale.unsqueeze(-1)).clamp(-8, 7) + 8
        zeros = None
    else:
        big = torch.finfo(torch.float32).max
        wmin = torch.where(valid, wg, torch.full_like(wg, big)).amin(dim=-1).clamp(max=0)
        wmax = torch.where(valid, wg, torch.full_like(wg, -big)).amax(dim=-1).clamp(min=0)
        scale = ((wmax - wmin) / 15.0).clamp_min(1e-12)
        scale = scale.to(scale_dtype).float().clamp_min(1e-12)
        zf = torch.round(-wmin / scale).clamp(0, 15)
        q = torch.round(wz / scale.unsqueeze(-1) + zf.unsqueeze(-1)).clamp(0, 15)
        zeros = zf.to(torch.uint8)
    q = q.reshape(n, g * gs)[:, :k].to(torch.uint8)
    return q.contiguous(), scale.to(scale_dtype), zeros


# ------------------------------------------------------------------------------------------------ simple int4
SIMPLE_LAYOUT_ID = "forge.simple.v1"


def pack_simple_int4(codes: torch.Tensor) -> torch.Tensor:
    """Codes ``[N, K]`` (values < 16) in the compress pipeline's "simple" layout (``forge/formats/packing.py:1-5``):
    ``uint8 [N, ceil(K/2)]``, element ``k`` in byte ``k // 2`` at bit offset ``4 * (k % 2)`` (even = low nibble)."""
    c = codes.to(torch.uint8)
    n, k = c.shape
    if k % 2:
        c = torch.nn.functional.pad(c, (0, 1))
    return (c[:, 0::2] | (c[:, 1::2] << 4)).contiguous()


def unpack_simple_int4(q8: torch.Tensor, k: int) -> torch.Tensor:
    """Inverse of :func:`pack_simple_int4`: ``uint8 [N, ceil(K/2)]`` -> codes ``uint8 [N, K]``."""
    lo, hi = q8 & 0xF, q8 >> 4
    return torch.stack((lo, hi), dim=-1).reshape(q8.shape[0], -1)[:, :k].contiguous()


def pack_w4_from_simple(qweight: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor | None, group_size: int,
                        k: int) -> PackedW4:
    """A ``forge.simple.v1`` int4 weight (``forge/compress/packed.py:9-12,265-274``: ``qweight uint8 [N, K/2]``,
    ``scales [N, G]``, ``zeros uint8 [N, G]`` or None) as a portable_row :class:`PackedW4`, bit-identical to
    ``pack_w4(codes, scales, zeros, group_size)``.  Both formats put code ``k`` at bit ``4 * (k % 8)`` of the
    little-endian 32-bit word ``k // 8``, so for ``K % 8 == 0`` the packed weights are the same bytes and are reused
    as an int32 view (no copy); scales are transposed and zero-points packed eight channels per word."""
    if qweight.dtype != torch.uint8 or qweight.dim() != 2 or qweight.shape[1] != (k + 1) // 2:
        raise ConfigError(f"simple int4 qweight must be uint8 [N, ceil(K/2)={(k + 1) // 2}], got "
                          f"{tuple(qweight.shape)} {qweight.dtype}")
    if k % 8 != 0:  # the portable layout pads K to 8 with the zero-point code: go through the codes
        return pack_w4(unpack_simple_int4(qweight, k), scales, zeros, group_size)
    n = qweight.shape[0]
    if group_size is not None and group_size > 0 and group_size % 8 != 0:
        raise ConfigError(f"group_size must be -1 or a multiple of 8, got {group_size}")
    g = num_groups(k, group_size)
    if tuple(scales.shape) != (n, g) or (zeros is not None and tuple(zeros.shape) != (n, g)):
        raise ConfigError(f"scales / zeros must be [N={n}, G={g}]")
    if zeros is not None and int(zeros.to(torch.int16).max()) > 15:
        raise ConfigError("zeros must be in 0..15")
    qw = qweight.contiguous().view(torch.int32)
    zq = None
    if zeros is not None:  # channels past N in the last word are 0, as pack_w4 writes them
        zt = torch.zeros((g, roundup(n, 8)), dtype=torch.uint8, device=qweight.device)
        zt[:, :n] = zeros.to(torch.uint8).t()
        zq = pack_nibbles_int32(zt.view(g, -1, 8))
    return PackedW4(qw, scales.t().contiguous(), zq, PORTABLE_W4, n, k, int(group_size), None,
                    {"n_pad": n, "k_pad": k})


# ------------------------------------------------------------------------------------------------ PackedW8
@dataclass
class PackedW8:
    """Symmetric int8 weight + scales in the portable_row W8 layout (``w8.py:18-80``): ``qweight int8 [N, K]``,
    ``scales [G, N]`` (column-contiguous per group), per-channel (``group_size <= 0``) or grouped along K."""

    qweight: torch.Tensor
    scales: torch.Tensor
    layout: Layout
    n: int
    k: int
    group_size: int
    meta: dict[str, Any] = field(default_factory=dict)

    @property
    def layout_id(self) -> str:
        return self.layout.id

    @property
    def shape(self) -> tuple[int, int]:
        return (self.n, self.k)

    @property
    def num_groups(self) -> int:
        return int(self.scales.shape[0])

    @property
    def device(self) -> torch.device:
        return self.qweight.device

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.qweight, self.scales))

    @property
    def bits_per_weight(self) -> float:
        return 8.0 * self.nbytes / max(1, self.n * self.k)

    def to(self, device: Any = None, dtype: torch.dtype | None = None) -> PackedW8:
        return PackedW8(self.qweight.to(device or self.qweight.device),
                        self.scales.to(device=device or self.scales.device, dtype=dtype or self.scales.dtype),
                        self.layout, self.n, self.k, self.group_size, dict(self.meta))

    def unpack(self) -> tuple[torch.Tensor, torch.Tensor]:
        return unpack_w8(self)

    def dequantize(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Dense ``[N, K]`` weight ``q * s`` in fp32 (exact), cast to ``dtype`` (``w8.py:54-56,101-104``)."""
        q, s = unpack_w8(self)
        return dequantize_w8_parts(q, s, self.group_size).to(dtype)

    def tensors(self) -> dict[str, torch.Tensor]:
        return {"qweight": self.qweight, "scales": self.scales}

    @staticmethod
    def tensor_roles() -> dict[str, str]:
        return {"qweight": "payload", "scales": "scale"}

    def state(self) -> dict[str, Any]:
        return {"layout_id": self.layout.id, "layout": self.layout.to_dict(), "n": self.n, "k": self.k,
                "group_size": self.group_size, "scale_dtype": str(self.scales.dtype).replace("torch.", "")}

    @classmethod
    def from_tensors(cls, tensors: dict[str, torch.Tensor], state: dict[str, Any]) -> PackedW8:
        lay = get_layout(state["layout_id"]) if state.get("layout_id") in _REG else Layout.from_dict(state["layout"])
        return cls(tensors["qweight"], tensors["scales"], lay, int(state["n"]), int(state["k"]), int(state["group_size"]))


def pack_w8(q: torch.Tensor, scales: torch.Tensor, group_size: int = -1, layout: Layout | str | None = None) -> PackedW8:
    """``q int8 [N, K]``, ``scales [N, G]`` -> :class:`PackedW8` (``w8.py:83-94``: scales stored transposed)."""
    lay = PORTABLE_W8 if layout is None else (get_layout(layout) if isinstance(layout, str) else layout)
    if lay.bits != 8:
        raise ConfigError(f"layout {lay.id} is not an 8-bit layout")
    if q.dim() != 2 or q.dtype != torch.int8:
        raise ConfigError("q must be int8 [N, K]")
    n, k = q.shape
    g = num_groups(k, group_size)
    if tuple(scales.shape) != (n, g):
        raise ConfigError(f"scales must be [N={n}, G={g}], got {tuple(scales.shape)}")
    return PackedW8(q.contiguous(), scales.t().contiguous(), lay, n, k, int(group_size))


def unpack_w8(p: PackedW8) -> tuple[torch.Tensor, torch.Tensor]:
    """``(q int8 [N, K], scales [N, G])`` (``w8.py:97-98``)."""
    return p.qweight, p.scales.t().contiguous()


def dequantize_w8_parts(q: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """``W[n, k] = q[n, k] * scales[n, k // gs]`` in fp32 (``w8.py:101-104``); exact, as int8 x fp16 fits fp32."""
    n, k = q.shape
    gi = torch.arange(k, device=q.device) // effective_group(group_size, k)
    return q.float() * scales.float()[:, gi]


def quantize_w8_rtn(w: torch.Tensor, group_size: int = -1,
                    scale_dtype: torch.dtype = torch.float16) -> tuple[torch.Tensor, torch.Tensor]:
    """Round-to-nearest symmetric int8 (``rtn.py:60-72``): ``scale = amax / 127`` rounded to ``scale_dtype``,
    ``q = clamp(round(w / scale), -128, 127)``; returns ``(q int8 [N, K], scales [N, G])``."""
    if w.dim() != 2:
        raise ConfigError("w must be [N, K]")
    n, k = w.shape
    wg, g, gs = _grouped(w, group_size)
    wz = torch.where(torch.isnan(wg), torch.zeros_like(wg), wg)
    scale = (wz.abs().amax(dim=-1) / 127.0).clamp_min(1e-12)
    scale = scale.to(scale_dtype).float().clamp_min(1e-12)
    q = torch.round(wz / scale.unsqueeze(-1)).clamp(-128, 127)
    return q.reshape(n, g * gs)[:, :k].to(torch.int8).contiguous(), scale.to(scale_dtype)


def require_portable(p: PackedW4) -> None:
    if p.layout.kind != KIND_PORTABLE:
        raise ConfigError(f"the gfx950 W4A16 kernels need the portable_row layout, got {p.layout_id}; repack() first")


__all__ = [
    "FRAGMENT_W4", "GROUP_SORT_KEY", "HardwareUnsupported", "IDENTITY_INTERLEAVE", "KIND_FRAGMENT", "KIND_PORTABLE",
    "KIND_PORTABLE_ROW", "Layout", "MARLIN_INTERLEAVE", "MISSING_SORT", "PORTABLE_W4", "PORTABLE_W8", "PackedW4",
    "PackedW8", "SIMPLE_LAYOUT_ID", "cached_group_sort", "ceil_div", "dequantize_w8_parts", "effective_group", "fragment_layout",
    "fragment_tile_perm", "get_layout", "known_layouts", "num_groups", "pack_nibbles_int32", "pack_simple_int4", "pack_w4", "pack_w4_from_simple", "pack_w8",
    "portable_layout", "quantize_w4_rtn", "quantize_w8_rtn", "register_layout", "repack", "roundup",
    "sort_columns_by_group", "unpack_nibbles_int32", "unpack_simple_int4", "unpack_w4", "unpack_w8",
]
