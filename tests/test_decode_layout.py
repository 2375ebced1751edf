"""Host-side preparation of the one-launch decode step (engine/decode.py), on the CPU: the per-block work table
and the weight re-layouts the kernel indexes (tile lane order, down slices, packed scale / min words)."""
import pytest
import torch

import decode


@pytest.mark.parametrize("cfg_kw", [dict(), dict(inter=2048), dict(NKV=8), dict(NKV=2, inter=4096)])
def test_work_table_covers_every_tile_once(cfg_kw):
    cfg = decode.Config(**cfg_kw)
    nb, nsp = 256, min(32, 256 // cfg.NKV)
    lim = decode.decode_limits()
    t = decode.work_table(cfg, nb, nsp)
    qkv_tiles = (cfg.NH + 2 * cfg.NKV) * cfg.HD // 16
    n_tiles = qkv_tiles + 2 * cfg.inter // 16
    tiles = t[:, :lim.max_tiles]
    assert (tiles >= 0).sum(1).max() <= lim.max_tiles
    # q / k / v tiles come first and fit the first pass
    for b in range(nb):
        row = [int(v) for v in tiles[b] if v >= 0]
        nq = sum(v < qkv_tiles for v in row)
        assert nq <= lim.first_pass and all(v < qkv_tiles for v in row[:nq])
    got = sorted(int(v) for v in tiles.flatten() if v >= 0)
    assert got == list(range(n_tiles))
    # slices are contiguous, cover all MLP channels, and each block owns the gate/up tiles of its slices
    sb, se = t[:, lim.slice_begin_col].tolist(), t[:, lim.slice_end_col].tolist()
    assert sb[0] == 0 and se[-1] == cfg.inter // 16 and all(se[b] == sb[b + 1] for b in range(nb - 1))
    assert max(e - s for s, e in zip(sb, se)) <= lim.max_slices
    for b in range(nb):
        own = set(int(v) for v in tiles[b] if v >= qkv_tiles)
        assert own == {qkv_tiles + 2 * k + h for k in range(sb[b], se[b]) for h in (0, 1)}
    assert (t[:, lim.slice_end_col + 1:] == -1).all()


def test_limits_match_the_kernel_contract():
    """The limits come from the library (rk_decode_get_limits), not from copies in Python."""
    lim = decode.decode_limits()
    assert 1 <= lim.first_pass <= lim.max_tiles < lim.slice_begin_col < lim.slice_end_col < lim.work_stride
    assert lim.max_slices >= 1 and lim.x_copies >= 1 and lim.max_splits >= 1
    # the default model fits: 2048-slot cache over 64 splits, 688 MLP slices over 256 blocks
    cfg = decode.Config()
    assert -(-cfg.S // 64) <= lim.max_slots_per_split and -(-cfg.inter // 16 // 256) <= lim.max_slices


def _table_and_cfg():
    cfg = decode.Config()
    return decode.work_table(cfg, 256, 64), cfg


def test_validation_rejects_a_qkv_tile_after_the_first_pass():
    """A q / k / v tile placed after the first pass would be published after the block's own q poll (which may wait
    for it): a circular wait. The host refuses such a table before any launch."""
    lim = decode.decode_limits()
    t, cfg = _table_and_cfg()
    qkv_tiles = (cfg.NH + 2 * cfg.NKV) * cfg.HD // 16
    b = next(i for i in range(256) if 0 <= int(t[i, 0]) < qkv_tiles and int(t[i, lim.first_pass]) >= 0)
    bad = t.clone()
    bad[b, 0], bad[b, lim.first_pass] = t[b, lim.first_pass], t[b, 0]  # move the q/k/v tile to the second pass
    with pytest.raises(ValueError, match="first"):
        decode.validate_work_table(bad, cfg)


@pytest.mark.parametrize("edit", ["drop_tile", "dup_tile", "gap", "slice_gap", "foreign_tile", "wide"])
def test_validation_rejects_malformed_tables(edit):
    lim = decode.decode_limits()
    t, cfg = _table_and_cfg()
    bad = t.clone()
    n0 = int((t[0, :lim.max_tiles] >= 0).sum())
    if edit == "drop_tile":
        bad[0, n0 - 1] = -1
    elif edit == "dup_tile":
        bad[0, n0 - 1] = t[1, 0]
    elif edit == "gap":
        bad[0, 0] = -1
    elif edit == "slice_gap":
        bad[5, lim.slice_end_col] += 1
    elif edit == "foreign_tile":  # swap one gate/up tile between two blocks: tiles stay unique, ownership breaks
        i, j = n0 - 1, int((t[100, :lim.max_tiles] >= 0).sum()) - 1
        bad[0, i], bad[100, j] = t[100, j], t[0, i]
    elif edit == "wide":
        bad = torch.cat([bad, bad[:, :1]], 1)
    with pytest.raises(ValueError):
        decode.validate_work_table(bad, cfg)


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


# ---------------------------------------------------------------------------------------------- role-split step
@pytest.mark.parametrize("inter,nkv", [(11008, 4), (2048, 4), (128, 4), (11008, 8)])
def test_role_table_partitions_the_work(inter, nkv):
    """64 latency blocks numbered 0..63 once each, latency group g (indices g * 64 / NKV .. + 64 / NKV - 1, the
    blocks that exchange KV head g's q / k / v and split partials) with one b % 8 (one XCD: a launch deals block b
    to XCD (b + c) % 8), no two groups with the same; 192 stream blocks numbered 0..191 once each, XCD by XCD,
    whose MLP slices form a contiguous partition of inter / 16 with at most max_slices each (stream blocks may hold
    none when the MLP is narrow)."""
    lim = decode.roles_limits()
    cfg = decode.Config(inter=inter, NKV=nkv)
    t = decode.role_table(cfg, lim)
    assert t.shape == (lim.blocks, 4)
    kind, idx, sb, se = (t[:, i].tolist() for i in range(4))
    lat = [b for b in range(lim.blocks) if kind[b] == 0]
    assert len(lat) == lim.latency_blocks
    assert sorted(idx[b] for b in lat) == list(range(lim.latency_blocks))
    per = lim.latency_blocks // nkv
    xcds = [{b % 8 for b in lat if idx[b] // per == g} for g in range(nkv)]
    assert all(len(x) == 1 for x in xcds) and len(set.union(*xcds)) == nkv
    assert [next(iter(x)) for x in xcds] == decode.latency_xcd(cfg)
    stream = sorted((b for b in range(lim.blocks) if kind[b] == 1), key=lambda b: idx[b])
    assert [idx[b] for b in stream] == list(range(lim.blocks - lim.latency_blocks))
    end = 0
    for b in stream:
        assert sb[b] == end and 0 <= se[b] - sb[b] <= lim.max_slices
        end = se[b]
    assert end == inter // 16
    # stream indices run XCD by XCD
    assert [b % 8 for b in stream] == sorted(b % 8 for b in stream)


def test_role_limits_match_the_kernel_contract():
    lim = decode.roles_limits()
    assert (lim.blocks, lim.latency_blocks, lim.max_slices, lim.x_copies) == (256, 64, 4, 16)
    assert lim.max_splits * lim.slots_per_wave * 0 == 0 and lim.waves * lim.slots_per_wave >= 2048 // 16


def test_group_scale_min_words():
    """win_sm of the role-split step: per (tile, group, row) the word of (row 16 tile + row, group)."""
    g = torch.Generator().manual_seed(3)
    sm = torch.randint(-2 ** 31, 2 ** 31 - 1, (64, 16), dtype=torch.int32, generator=g)
    out = decode.group_scale_min(sm)
    assert out.shape == (4, 16, 16)
    for T in range(4):
        for grp in range(16):
            for r in range(16):
                assert out[T, grp, r] == sm[16 * T + r, grp]


def test_role_head_rows_fit_the_waves():
    """stream block i, wave w takes head rows i + 192 (w + 16 k): every row once, at most 64 per wave."""
    for n in (16385, 257, 1):
        rows = sorted(i + 192 * (w + 16 * k) for i in range(192) for w in range(16) for k in range(64)
                      if i + 192 * (w + 16 * k) < n)
        assert rows == list(range(n))
        assert max(len([k for k in range(64) if i + 192 * (w + 16 * k) < n]) for i in range(192) for w in range(16)) <= 64
