"""Host-side preparation of the one-launch decode step (engine/decode.py), on the CPU: the per-block work table
and the weight re-layouts the kernel indexes (tile lane order, down slices, packed scale / min words)."""
import pytest
import torch

import decode


@pytest.mark.parametrize("cfg_kw", [dict(), dict(inter=2048), dict(NKV=8), dict(NKV=2, inter=4096)])
def test_work_table_covers_every_tile_once(cfg_kw):
    cfg = decode.Config(**cfg_kw)
    nb, nsp = 256, min(32, 256 // cfg.NKV)
    t = decode.work_table(cfg, nb, nsp)
    qkv_tiles = (cfg.NH + 2 * cfg.NKV) * cfg.HD // 16
    n_tiles = qkv_tiles + 2 * cfg.inter // 16
    tiles = t[:, :8]
    assert (tiles >= 0).sum(1).max() <= decode.MAX_TILES
    # q / k / v tiles come first and fit the first pass
    for b in range(nb):
        row = [int(v) for v in tiles[b] if v >= 0]
        nq = sum(v < qkv_tiles for v in row)
        assert nq <= decode.FIRST_PASS and all(v < qkv_tiles for v in row[:nq])
    got = sorted(int(v) for v in tiles.flatten() if v >= 0)
    assert got == list(range(n_tiles))
    # slices are contiguous, cover all MLP channels, and each block owns the gate/up tiles of its slices
    sb, se = t[:, 8].tolist(), t[:, 9].tolist()
    assert sb[0] == 0 and se[-1] == cfg.inter // 16 and all(se[b] == sb[b + 1] for b in range(nb - 1))
    assert max(e - s for s, e in zip(sb, se)) <= decode.MAX_SLICES
    for b in range(nb):
        own = set(int(v) for v in tiles[b] if v >= qkv_tiles)
        assert own == {qkv_tiles + 2 * k + h for k in range(sb[b], se[b]) for h in (0, 1)}
    assert (t[:, 10:] == -1).all()


def test_o_layout_items():
    """item i of (head h, row group r) holds row 128r + i // 4, the codes of columns 128h + 32(i % 4) .. + 32"""
    g = torch.Generator().manual_seed(1)
    nh = 16
    q = torch.randint(0, 256, (2048, nh * 64), generator=g, dtype=torch.uint8)
    o = decode.o_layout(q, nh)
    assert o.shape == (nh, 16, 512, 16)
    for h, r, i in ((0, 0, 0), (3, 5, 7), (15, 15, 511), (9, 2, 130)):
        row, c = 128 * r + i // 4, i % 4
        assert torch.equal(o[h, r, i], q[row, 64 * h + 16 * c: 64 * h + 16 * c + 16])


def test_tile_layout_lane_order():
    g = torch.Generator().manual_seed(0)
    q = torch.randint(0, 256, (64, 1024), generator=g, dtype=torch.uint8)
    t = decode.tile_layout(q)
    assert t.shape == (4, 16, 64, 16)
    for T, grp, lane in ((0, 0, 0), (1, 3, 17), (3, 15, 63), (2, 7, 40)):
        j, s = lane % 16, lane // 16
        assert torch.equal(t[T, grp, lane], q[16 * T + j, 64 * grp + 16 * s: 64 * grp + 16 * s + 16])


def test_down_layout_slices():
    g = torch.Generator().manual_seed(1)
    q = torch.randint(0, 256, (2048, 1024), generator=g, dtype=torch.uint8)  # inter = 2048
    t = decode.down_layout(q)
    assert t.shape == (128, 2048, 8)
    for k, r in ((0, 0), (5, 777), (127, 2047)):
        assert torch.equal(t[k, r], q[r, 8 * k: 8 * k + 8])


def test_pack_scale_min_words():
    s = torch.tensor([[1.5, -2.0]], dtype=torch.float16)
    m = torch.tensor([[0.25, 65504.0]], dtype=torch.float16)
    w = decode.pack_scale_min(s, m)
    lo = (w & 0xFFFF).to(torch.int16).view(torch.float16)
    hi = (w >> 16).to(torch.int16).view(torch.float16)
    assert torch.equal(lo, s) and torch.equal(hi, m)


def test_interleave_gate_up_rows():
    cfg = decode.Config(NH=16, NKV=4, inter=32)
    a = (cfg.NH + 2 * cfg.NKV) * cfg.HD
    t = torch.arange(a + 2 * cfg.inter).reshape(-1, 1)
    r = decode.interleave_gate_up(t, cfg).flatten().tolist()
    assert r[:a] == list(range(a))
    # per 8 channels: 8 gate rows then the 8 matching up rows
    assert r[a:a + 16] == list(range(a, a + 8)) + list(range(a + cfg.inter, a + cfg.inter + 8))
