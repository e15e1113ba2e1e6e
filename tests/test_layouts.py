"""CPU tests of the product's packed formats (forge_amd.layouts) against the oracle's independent packer."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from forge_amd import layouts as L
from forge_amd.errors import ConfigError, NotFound
from oracle import w4 as ow
from tests._util import w4_parts


@pytest.mark.parametrize("n", [1, 7, 64, 65, 130])
@pytest.mark.parametrize("k", [8, 33, 100, 257])
@pytest.mark.parametrize("gs", [-1, 16, 64])
@pytest.mark.parametrize("sym", [True, False])
def test_product_pack_equals_oracle_pack(n, k, gs, sym):
    q, s, z = w4_parts(n, k, gs, sym, seed=n * 7 + k)
    p = L.pack_w4(q, s, z, gs)
    o = ow.pack_w4(q.numpy(), s.numpy(), None if z is None else z.numpy(), gs)
    assert np.array_equal(p.qweight.numpy(), o["qweight"])
    assert np.array_equal(p.scales.numpy(), o["scales"])
    assert (z is None and p.zeros is None) or np.array_equal(p.zeros.numpy(), o["zeros"])
    q2, s2, z2 = L.unpack_w4(p)
    assert torch.equal(q, q2) and torch.equal(s, s2) and ((z is None and z2 is None) or torch.equal(z, z2))
    assert p.layout_id == ow.layout_id(4) == "w4.portable_row.v1-73e10e"


@pytest.mark.parametrize("n,k,gs", [(33, 100, 32), (64, 128, 64), (7, 50, -1), (130, 257, 16)])
def test_fragment_artifact_repacks_to_identical_portable_bytes(n, k, gs):
    q, s, z = w4_parts(n, k, gs, False, seed=3)
    a = L.pack_w4(q, s, z, gs, L.PORTABLE_W4)
    b = L.repack(a, L.FRAGMENT_W4)
    assert b.layout_id == "w4.mma_fragment_k16n64.v1-445296"
    assert b.qweight.shape == ((k + 15) // 16, ((n + 63) // 64) * 128)
    for x, y in zip(L.unpack_w4(a), L.unpack_w4(b)):
        assert (x is None and y is None) or torch.equal(x, y)
    back = L.repack(b, L.PORTABLE_W4)
    assert torch.equal(back.qweight, a.qweight) and torch.equal(back.scales, a.scales) and torch.equal(back.zeros, a.zeros)
    assert L.repack(a, L.PORTABLE_W4) is a


def test_fragment_permutation_lane_ownership():
    """Lane l owns k = 2(l%4)+{0,1}(+8), n = 8 nb + l//4 (tests/test_kernels_gemm_layouts.py:185-195)."""
    idx, inv = L.fragment_tile_perm((0, 1, 2, 3, 4, 5, 6, 7))
    assert sorted(idx.tolist()) == list(range(1024)) and torch.equal(inv[idx], torch.arange(1024))
    lane = 5
    mine = idx[lane * 32:(lane + 1) * 32]
    ks, ns = mine // 64, mine % 64
    assert set((ns % 8).tolist()) == {lane // 4}
    assert ks.tolist()[:4] == [2 * (lane % 4), 2 * (lane % 4) + 1, 2 * (lane % 4) + 8, 2 * (lane % 4) + 9]


def test_packer_validation_errors():
    q, s, z = w4_parts(8, 32, 16, True)
    with pytest.raises(ConfigError):
        L.pack_w4(q + 16, s, z, 16)
    with pytest.raises(ConfigError):
        L.pack_w4(q, s[:, :1], z, 16)
    with pytest.raises(ConfigError):
        L.pack_w4(q, s, z, 12)
    with pytest.raises(ConfigError):
        L.pack_w4(q.float(), s, z, 16)
    with pytest.raises(ConfigError):
        L.pack_w4(q, s, z, 8, L.FRAGMENT_W4)
    with pytest.raises(ConfigError):
        L.pack_w4(q, s, z, 16, L.PORTABLE_W8)
    with pytest.raises(NotFound):
        L.get_layout("nope")


def test_state_roundtrip_and_size():
    q, s, z = w4_parts(64, 256, 128, False)
    p = L.pack_w4(q, s, z, 128)
    p2 = L.PackedW4.from_tensors(p.tensors(), p.state())
    assert p2.layout_id == p.layout_id and torch.equal(p2.qweight, p.qweight)
    assert abs(p.bits_per_weight - (4 + 20 / 128)) < 0.2
    assert L.PackedW4.tensor_roles()["qweight"] == "payload"


def test_act_order_sort_matches_oracle():
    n, k, gs = 24, 96, 32
    q, s, _ = w4_parts(n, k, gs, True, seed=4)
    g = torch.Generator().manual_seed(5)
    g_idx = (torch.arange(k) // gs)[torch.randperm(k, generator=g)].to(torch.int32)
    p = L.pack_w4(q, s, None, gs, g_idx=g_idx)
    sp, perm = L.sort_columns_by_group(p)
    osp, operm = ow.sort_columns_by_group(ow.pack_w4(q.numpy(), s.numpy(), None, gs, g_idx.numpy()))
    assert np.array_equal(perm.numpy(), operm) and np.array_equal(sp.qweight.numpy(), osp["qweight"])
    assert L.cached_group_sort(p)[1] is L.cached_group_sort(p)[1]  # cached
    assert L.cached_group_sort(L.pack_w4(q, s, None, gs)) is None


def test_rtn_quantiser_bounds():
    w = torch.randn(16, 100, generator=torch.Generator().manual_seed(0))
    for sym in (True, False):
        q, s, z = L.quantize_w4_rtn(w, 32, sym=sym, scale_dtype=torch.float32)
        gi = torch.arange(100) // 32
        zz = 8.0 if z is None else z.float()[:, gi]
        deq = (q.float() - zz) * s[:, gi]
        assert q.max() <= 15 and (z is None) == sym
        assert (deq - w).abs().max() <= s.max() * 0.51 + 1e-6


@pytest.mark.parametrize("n,k,gs,sym", [(37, 96, 32, False), (16, 256, 128, True), (9, 100, 8, False), (40, 64, -1, True)])
def test_simple_int4_to_portable_is_bit_identical(n, k, gs, sym):
    """forge.simple.v1 int4 (forge/formats/packing.py:1-5: element k in byte k // 2, even k = low nibble) converted to
    portable_row equals pack_w4 of the same codes bit for bit; for K % 8 == 0 the weights are the same bytes."""
    g = torch.Generator().manual_seed(n * k)
    q = torch.randint(0, 16, (n, k), generator=g, dtype=torch.uint8)
    ng = L.num_groups(k, gs)
    s = (torch.rand(n, ng, generator=g) * 0.02 + 0.001).half()
    z = None if sym else torch.randint(0, 16, (n, ng), generator=g, dtype=torch.uint8)
    simple = L.pack_simple_int4(q)
    # the simple layout restated element by element
    for (r, c) in [(0, 0), (0, 1), (n - 1, k - 1), (n // 2, 7)]:
        assert (int(simple[r, c // 2]) >> (4 * (c % 2))) & 15 == int(q[r, c])
    assert torch.equal(L.unpack_simple_int4(simple, k), q)
    a = L.pack_w4_from_simple(simple, s, z, gs, k)
    b = L.pack_w4(q, s, z, gs)
    assert torch.equal(a.qweight, b.qweight) and torch.equal(a.scales, b.scales) and a.layout_id == b.layout_id
    assert (a.zeros is None) == (b.zeros is None) and (a.zeros is None or torch.equal(a.zeros, b.zeros))
    if k % 8 == 0:
        assert a.qweight.data_ptr() == simple.data_ptr()  # a view, no copy
    qq, ss, zz = L.unpack_w4(a)
    assert torch.equal(qq, q) and torch.equal(ss, s) and (zz is None or torch.equal(zz, z))


def _cdna4_brute_force(q: torch.Tensor, zeros: torch.Tensor | None, gs: int) -> torch.Tensor:
    """The cdna4_mfma words placed one code at a time from the layout's definition: tile (nt, kt) at words
    [nt, 256 kt ..]; lane l = 16 j + r owns words 4 l .. 4 l + 3; word s holds channel 16 nt + r, columns
    128 kt + 32 s + 8 j + t, column t in nibble slot t // 2 (t even) or 4 + t // 2 (t odd); padding columns hold the
    group's zero-point (8 when symmetric), padding channels 8."""
    n, k = q.shape
    nt, kt = -(-n // 16), -(-k // 128)
    g = -(-k // gs)
    words = [[0] * (kt * 256) for _ in range(nt)]
    for tn in range(nt):
        for tk in range(kt):
            for j in range(4):
                for r in range(16):
                    for s in range(4):
                        w = 0
                        for t in range(8):
                            ch, col = 16 * tn + r, 128 * tk + 32 * s + 8 * j + t
                            if ch >= n:
                                code = 8
                            elif col >= k:
                                code = 8 if zeros is None else int(zeros[ch, min(col // gs, g - 1)])
                            else:
                                code = int(q[ch, col])
                            slot = t // 2 if t % 2 == 0 else 4 + t // 2
                            w |= code << (4 * slot)
                        words[tn][tk * 256 + 4 * (16 * j + r) + s] = w - (1 << 32) if w >= 1 << 31 else w
    return torch.tensor(words, dtype=torch.int32)


@pytest.mark.parametrize("n,k,gs,sym", [(16, 128, 128, False), (21, 200, 64, False), (40, 384, 128, True),
                                        (5, 96, -1, False)])
def test_cdna4_layout_matches_its_definition_and_round_trips(n, k, gs, sym):
    q, s, z = w4_parts(n, k, gs, sym, seed=n + k)
    p = L.pack_w4(q, s, z, gs, L.CDNA4_W4)
    assert p.layout.kind == L.KIND_CDNA4 and p.layout_id.startswith("w4.cdna4_mfma_k128n16.v1-")
    assert p.qweight.shape == (-(-n // 16), -(-k // 128) * 256)
    assert torch.equal(p.qweight, _cdna4_brute_force(q, z, L.effective_group(gs, k)))
    # scales and zero-points are stored exactly as in portable_row; codes survive both repack directions
    a = L.pack_w4(q, s, z, gs)
    assert torch.equal(p.scales, a.scales) and ((z is None and p.zeros is None) or torch.equal(p.zeros, a.zeros))
    for x, y in zip(L.unpack_w4(p), (q, s, z)):
        assert (x is None and y is None) or torch.equal(x, y)
    assert torch.equal(L.repack(p, L.PORTABLE_W4).qweight, a.qweight)
    assert torch.equal(L.repack(a, L.CDNA4_W4).qweight, p.qweight)
    shapes = L.w4_storage_shapes(L.CDNA4_W4, n, k, L.num_groups(k, gs), z is not None)
    assert shapes["qweight"] == tuple(p.qweight.shape) and shapes["scales"] == tuple(p.scales.shape)


def test_cdna4_unpack_pairs_are_mfma_b_operands():
    """(word >> 4p) & 0x000F000F is the pair of columns (2p, 2p + 1) of the lane's eight k-step columns."""
    n, k = 16, 128
    q = (torch.arange(n * k) % 16).to(torch.uint8).reshape(n, k)
    q = q[torch.randperm(n, generator=torch.Generator().manual_seed(1))]
    p = L.pack_w4(q, torch.ones(n, 1).half(), None, -1, L.CDNA4_W4)
    words = p.qweight[0].to(torch.int64) & 0xFFFFFFFF
    for lane in (0, 17, 38, 63):
        j, r = lane // 16, lane % 16
        for s in range(4):
            w = int(words[4 * lane + s])
            for pair in range(4):
                v = (w >> (4 * pair)) & 0x000F000F
                cols = 32 * s + 8 * j + 2 * pair
                assert (v & 0xF, v >> 16) == (int(q[r, cols]), int(q[r, cols + 1]))


@pytest.mark.parametrize("n,k,gs,sym", [(24, 256, 128, False), (4096, 512, 64, True), (40, 96, 32, False)])
def test_sz8_blocks_is_the_documented_permutation(n, k, gs, sym):
    """scales8[n // 8, g, n % 8] == scales[g, n] and zeros8[b, g] == zero word (g, b) for every element, checked
    element by element against the packed portable_row tensors (the nibble n % 8 of zeros8[n // 8, g] is channel n's
    zero-point); padding past N (scales stored wider) is dropped; N % 8 != 0 is refused."""
    q, s, z = w4_parts(n, k, gs, sym, seed=n + k)
    p = L.pack_w4(q, s, z, gs)
    s8, z8 = L.sz8_blocks(p.scales, p.zeros, n)
    G = p.scales.shape[0]
    assert s8.shape == (n // 8, G, 8) and s8.is_contiguous() and s8.dtype == p.scales.dtype
    for g in range(G):
        for c in range(n):
            assert s8[c // 8, g, c % 8].item() == p.scales[g, c].item()
            if z is not None:
                assert (int(z8[c // 8, g]) >> (4 * (c % 8))) & 0xF == int(z[c, g])
    assert (z8 is None) == sym
    # a wider stored scale row (ldz / lds padding) keeps the first N channels
    wide = torch.cat([p.scales, torch.zeros(G, 8, dtype=p.scales.dtype)], 1)
    assert torch.equal(L.sz8_blocks(wide, p.zeros, n)[0], s8)
    with pytest.raises(ConfigError):
        L.sz8_blocks(p.scales[:, :n - 4], None, n - 4)
