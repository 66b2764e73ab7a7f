"""Pins the oracle's snapshot renderer, obs_v0/reward_v0 and masked reset.

Renderer: the reference's own known answers (all-zero tile -> shade 0,
all-0xFF tile with BGP 0xE4 -> shade 3, packed == pack(unpacked)), hand-built
scenes whose pixels follow from the DMG tile/window/sprite rules (signed tile
addressing, window origin at WX-7, sprite flips, OBJ-behind-BG priority,
lowest-x-then-lowest-index overlap, 10 sprites per line), and an independent
full-frame numpy renderer downsampled at even coordinates.

obs/reward: the known-answer slots of the reference's stage tests.
Reset: masked envs equal the snapshot, unmasked envs are untouched.
"""

from __future__ import annotations

import numpy as np
import pytest

from ._isa import flat_rom, oracle, run_frames, set_regs


def _idle(n):
    return oracle(flat_rom({0x150: bytes([0x18, 0xFE])}), n)


def unpack(packed: np.ndarray) -> np.ndarray:
    out = np.zeros(packed.shape[:-1] + (packed.shape[-1] * 4,), np.uint8)
    for k in range(4):
        out[..., k::4] = (packed >> (2 * k)) & 3
    return out


# ---------------------------------------------------------------------------
# independent full-frame renderer (160x144), one line at a time with that
# line's registers: from the IO page (snapshot renderer, then sampled at even
# x/y) or from the env-0 scanline latches (full-frame renderer)
# ---------------------------------------------------------------------------
def line_np(mem: np.ndarray, y: int, regs: dict) -> np.ndarray:
    lcdc, scy, scx, bgp = regs["lcdc"], regs["scy"], regs["scx"], regs["bgp"]
    obp = (regs["obp0"], regs["obp1"])
    wy, wx, win_row = regs["wy"], regs["wx"], regs["win_row"]
    xs = np.arange(160)
    color = np.zeros(160, np.int64)
    if lcdc & 1:
        win = bool(lcdc & 0x20) & (y >= wy) & (xs >= wx - 7)
        px = np.where(win, (xs - (wx - 7)) & 0xFF, (xs + scx) & 0xFF)
        py = np.where(win, win_row & 0xFF, (y + scy) & 0xFF)
        mapbase = np.where(win, 0x9C00 if lcdc & 0x40 else 0x9800, 0x9C00 if lcdc & 0x08 else 0x9800)
        tid = mem[mapbase + (py // 8) * 32 + px // 8].astype(np.int64)
        if lcdc & 0x10:
            taddr = 0x8000 + tid * 16
        else:
            taddr = 0x9000 + np.where(tid >= 128, tid - 256, tid) * 16
        lo = mem[taddr + (py % 8) * 2].astype(np.int64)
        hi = mem[taddr + (py % 8) * 2 + 1].astype(np.int64)
        sh = 7 - px % 8
        color = ((hi >> sh) & 1) * 2 + ((lo >> sh) & 1)
    shade = np.where(lcdc & 1, (bgp >> (2 * color)) & 3, 0)
    if lcdc & 2:
        h = 16 if lcdc & 4 else 8
        oam = mem[0xFE00:0xFEA0].reshape(40, 4).astype(np.int64)
        line = [
            k for k in range(40)
            if 0 < oam[k, 1] < 168 and 0 < oam[k, 0] < 160 and oam[k, 0] - 16 <= y < oam[k, 0] - 16 + h
        ][:10]  # fmt: skip
        best = {}
        for k in line:
            sy, sx, tile, attr = oam[k]
            row = y - (sy - 16)
            if attr & 0x40:
                row = h - 1 - row
            if h == 16:
                tile = (tile & 0xFE) + (1 if row >= 8 else 0)
                row %= 8
            lo = int(mem[0x8000 + tile * 16 + row * 2])
            hi = int(mem[0x8000 + tile * 16 + row * 2 + 1])
            for x in range(max(sx - 8, 0), min(sx, 160)):
                p = x - (sx - 8)
                b = p if attr & 0x20 else 7 - p
                c = ((hi >> b) & 1) * 2 + ((lo >> b) & 1)
                if c == 0:
                    continue
                if x not in best or sx - 8 < best[x][0]:
                    best[x] = (sx - 8, c, attr)
        for x, (_, c, attr) in best.items():
            if attr & 0x80 and lcdc & 1 and color[x] != 0:
                continue
            shade[x] = (obp[(attr >> 4) & 1] >> (2 * c)) & 3
    return shade.astype(np.uint8)


def frame_np(mem: np.ndarray) -> np.ndarray:
    r = {k: int(mem[a]) for k, a in (("lcdc", 0xFF40), ("scy", 0xFF42), ("scx", 0xFF43),
                                     ("bgp", 0xFF47), ("obp0", 0xFF48), ("obp1", 0xFF49),
                                     ("wy", 0xFF4A), ("wx", 0xFF4B))}  # fmt: skip
    return np.stack([line_np(mem, y, dict(r, win_row=y - r["wy"])) for y in range(144)])


LATCH_ROWS = ("lcdc", "scx", "scy", "bgp", "wx", "wy", "win_row", "obp0", "obp1")


def frame_latched_np(mem: np.ndarray, lat: np.ndarray) -> np.ndarray:
    rows = []
    for y in range(144):
        rows.append(line_np(mem, y, {k: int(lat[i, y]) for i, k in enumerate(LATCH_ROWS)}))
    return np.stack(rows)


def render_both(m):
    m.render(packed=False)
    m.render(packed=True)
    return m.pix.copy(), m.pix_packed.copy()


def test_reference_tile_known_answers():
    """BG_STATIC-style checks of the reference (test_ppu_downsampled_pixels.py
    :68-124): tile 0 all zero -> shade 0; all 0xFF with BGP 0xE4 -> shade 3."""
    m = _idle(2)
    try:
        for i in range(2):
            m.mem[i, 0xFF40], m.mem[i, 0xFF47] = 0x91, 0xE4
            m.mem[i, 0x9800:0x9C00] = 0
        m.mem[0, 0x8000:0x8010] = 0x00
        m.mem[1, 0x8000:0x8010] = 0xFF
        pix, packed = render_both(m)
        assert np.unique(pix[0]).tolist() == [0]
        assert np.unique(pix[1]).tolist() == [3]
        np.testing.assert_array_equal(unpack(packed), pix)
    finally:
        m.close()


def test_hand_built_scenes():
    m = _idle(4)
    mem = m.mem
    try:
        # env 0: signed tile data (LCDC.4 = 0): id 0x80 -> 0x8800, id 0x7F -> 0x97F0
        mem[0, 0xFF40], mem[0, 0xFF47] = 0x81, 0xE4
        mem[0, 0x9800], mem[0, 0x9801] = 0x80, 0x7F
        mem[0, 0x8800:0x8810] = [0xFF, 0x00] * 8  # colour 1
        mem[0, 0x97F0:0x9800] = [0x00, 0xFF] * 8  # colour 2
        # env 1: window at WX=7+32, WY=16 from the 9C00 map, tile 1 all colour 3
        mem[1, 0xFF40], mem[1, 0xFF47] = 0xF1, 0xE4
        mem[1, 0xFF4A], mem[1, 0xFF4B] = 16, 7 + 32
        mem[1, 0x9C00:0xA000] = 1
        mem[1, 0x8010:0x8020] = 0xFF
        # envs 2/3: one sprite at screen (20, 10) whose two leftmost pixels are
        # colour 1; env 3 has the x-flip bit, which moves them to x 26/27
        for i, attr in ((2, 0x00), (3, 0x20)):
            mem[i, 0xFF40], mem[i, 0xFF48] = 0x93, 0xE4
            mem[i, 0x8020:0x8030] = [0xC0, 0x00] * 8  # tile 2
            mem[i, 0xFE00:0xFE04] = [10 + 16, 20 + 8, 2, attr]
        pix, packed = render_both(m)
        np.testing.assert_array_equal(unpack(packed), pix)
        assert pix[0, 0, 0] == 1 and pix[0, 0, 4] == 2  # x=0 tile 0x80, x=8 tile 0x7F
        assert (pix[1, 8:, 16:] == 3).all() and (pix[1, :8, :] == 0).all()
        assert (pix[1, :, :16] == 0).all()
        assert pix[2, 5, 10] == 1 and pix[2, 5, 13] == 0  # unflipped: x 20 lit
        assert pix[3, 5, 13] == 1 and pix[3, 5, 10] == 0  # flipped: x 26 lit
    finally:
        m.close()


def test_sprite_rules_known_answers():
    m = _idle(1)
    mem = m.mem
    try:
        # BGP 0xE5: colour 0 -> shade 1, colour 1 -> shade 1
        mem[0, 0xFF40], mem[0, 0xFF47], mem[0, 0xFF48], mem[0, 0xFF49] = 0x93, 0xE5, 0xE4, 0x1B
        mem[0, 0x8040:0x8050] = 0xFF  # tile 4 colour 3
        mem[0, 0x8050:0x8060] = [0xFF, 0x00] * 8  # tile 5 colour 1
        mem[0, 0x9800 + 32 * 8 : 0x9800 + 32 * 9] = 5  # BG colour 1 on lines 64..71
        oam = [
            (64 + 16, 40 + 8, 4, 0x80),  # BG-priority sprite over BG colour 1 -> hidden
            (0 + 16, 50 + 8, 4, 0x00),  # x 50..57, OBP0 colour 3 -> shade 3
            (0 + 16, 48 + 8, 4, 0x10),  # x 48..55, OBP1 colour 3 -> shade 0, lower x wins
        ]
        oam += [(100 + 16, 8 * k + 8, 4, 0x00) for k in range(11)]  # 11 on line 100
        for k, s_ in enumerate(oam):
            mem[0, 0xFE00 + 4 * k : 0xFE04 + 4 * k] = s_
        m.render(packed=False)
        pix = m.pix[0]
        assert pix[32, 20] == 1  # (40, 64): BG colour 1 wins over the BG-priority sprite
        assert pix[0, 24] == 0 and pix[0, 27] == 0  # x 48..55: OBP1 sprite (lower x) wins
        assert pix[0, 28] == 3  # x 56: only the OBP0 sprite covers it
        assert pix[0, 30] == 1  # x 60: background
        assert (pix[50, 0:40] == 3).all()  # x 0..79 covered by the first 10 sprites
        assert pix[50, 40] == 1 and pix[50, 43] == 1  # the 11th sprite (x 80..87) dropped
    finally:
        m.close()


def test_renderer_matches_independent_full_frame_renderer():
    rng = np.random.default_rng(11)
    n = 24
    m = _idle(n)
    try:
        mem = m.mem
        mem[:, 0x8000:0xA000] = rng.integers(0, 256, (n, 0x2000))
        oam = rng.integers(0, 256, (n, 160))
        oam[:, 0::4] = rng.integers(0, 176, (n, 40))
        oam[:, 1::4] = rng.integers(0, 176, (n, 40))
        mem[:, 0xFE00:0xFEA0] = oam
        for reg in (0xFF42, 0xFF43, 0xFF47, 0xFF48, 0xFF49):
            mem[:, reg] = rng.integers(0, 256, n)
        mem[:, 0xFF4A] = rng.integers(0, 160, n)
        mem[:, 0xFF4B] = rng.integers(0, 175, n)
        mem[:, 0xFF40] = rng.integers(0, 256, n)
        pix, packed = render_both(m)
        np.testing.assert_array_equal(unpack(packed), pix)
        for i in range(n):
            want = frame_np(mem[i])[::2, ::2]
            np.testing.assert_array_equal(pix[i], want, err_msg=f"env {i} lcdc {mem[i, 0xFF40]:#x}")
    finally:
        m.close()


@pytest.mark.parametrize("stage", ["emulate_only", "reward_only", "obs_only", "full_step"])
def test_obs_reward_stage_known_answers(stage):
    """Reference test_warp_vec_ws2_stage.py:54-154 on a 0-frame launch."""
    m = _idle(1)
    try:
        m.obs[:] = 3.0
        m.reward[:] = -1.0
        set_regs(m, pc=0x2000, sp=0x1234, a=0x2A)
        m.mem[0, 0xC000:0xC010] = [0x10, 0x05] + list(range(14))
        m.step(None, frames=0, stage=stage)
        r_want = np.float32(((0x2A ^ ((0x10 + 0x05 * 3) & 0xFF)) & 0xFF) / 255.0)
        if stage in ("reward_only", "full_step"):
            assert m.reward[0] == r_want
        else:
            assert m.reward[0] == -1.0
        o = m.obs[0]
        if stage in ("obs_only", "full_step"):
            assert o[0] == np.float32(0x2000 / 65535.0)
            assert o[1] == np.float32(0x1234 / 65535.0)
            assert o[2] == np.float32(0x2A / 255.0)
            assert o[10] == np.float32(0x10 / 255.0) and o[11] == np.float32(0x05 / 255.0)
            assert o[26] == np.float32((0x10 ^ 0x05) / 255.0)
            assert o[27] == np.float32(((0x00 + 0x01 * 5) & 0xFF) / 255.0)
        else:
            assert (o == 3.0).all()
    finally:
        m.close()


def test_masked_reset_restores_only_masked_envs():
    """Reference test_reset_cache.py:32-101: masked envs equal the snapshot
    (memory, registers, cart state, pixels); unmasked envs are untouched."""
    from gbxcule_amd.carts.synth import cart_c3, seeded_actions
    from gbxcule_amd.carts.bootstub import build_bootstub
    from oracle.ref import RefMachine

    m = RefMachine(3, cart_c3(2), build_bootstub())
    try:
        m.step(seeded_actions(0, 0, 3), frames=2)
        m.render(packed=False)
        m.snapshot(0, with_pix=True)
        snap_mem = m.mem[0].copy()
        snap_pc = int(m.field("pc")[0])
        snap_cs = m.cart_state[0].copy()
        snap_pix = m.pix[0].copy()
        m.mem[1, 0xC000:0xC002] = (0xAA, 0xBB)
        m.mem[2, 0xC000:0xC002] = (0xCC, 0xDD)
        m.field("pc")[1:] = (0x1234, 0x5678)
        m.cart_state[1:, 2] = (5, 7)
        m.pix[1].fill(3)
        m.pix[2].fill(2)
        m.masked_reset(np.array([0, 1, 0], np.uint8))
        np.testing.assert_array_equal(m.mem[1], snap_mem)
        assert int(m.field("pc")[1]) == snap_pc
        np.testing.assert_array_equal(m.cart_state[1], snap_cs)
        np.testing.assert_array_equal(m.pix[1], snap_pix)
        assert tuple(m.mem[2, 0xC000:0xC002]) == (0xCC, 0xDD)
        assert int(m.field("pc")[2]) == 0x5678 and m.cart_state[2, 2] == 7
        assert (m.pix[2] == 2).all()
    finally:
        m.close()


def test_idle_run_keeps_frame_counter_consistent():
    """frames x 70224 cycles pass per step with the LCD off (no LCD toggles)."""
    m = _idle(2)
    try:
        run_frames(m, 3)
        cyc = m.field("cycle_count")
        assert (cyc >= 3 * 70224).all() and (cyc < 3 * 70224 + 12).all()
        np.testing.assert_array_equal(m.field("cycle_in_frame"), cyc - 3 * 70224)
    finally:
        m.close()


# ---------------------------------------------------------------------------
# env-0 full-frame renderer from the scanline latches (kernels/ppu_step.py)
# ---------------------------------------------------------------------------
def test_env0_frame_matches_independent_latched_renderer():
    """Random VRAM/OAM and random per-line latches (every register different
    on every line), against the line-by-line numpy renderer."""
    rng = np.random.default_rng(21)
    m = _idle(1)
    try:
        for trial in range(12):
            m.mem[0, 0x8000:0xA000] = rng.integers(0, 256, 0x2000)
            oam = rng.integers(0, 256, 160)
            oam[0::4] = rng.integers(0, 176, 40)
            oam[1::4] = rng.integers(0, 176, 40)
            m.mem[0, 0xFE00:0xFEA0] = oam
            lat = rng.integers(0, 256, (9, 144)).astype(np.uint8)
            lat[5] = rng.integers(0, 160, 144)  # WY mostly on screen
            lat[4] = rng.integers(0, 175, 144)
            if trial % 3 == 0:
                lat[0] = rng.integers(0, 256)  # one LCDC for the whole frame
            m.latches[:] = lat
            got = m.render_bg_env0()
            want = frame_latched_np(m.mem[0], lat)
            np.testing.assert_array_equal(got, want, err_msg=f"trial {trial}")
    finally:
        m.close()


def test_env0_frame_with_steady_latches_equals_snapshot_renderer():
    """Latches equal to the IO registers on every line (window line y - WY):
    the full frame sampled at even x/y is exactly the snapshot render."""
    rng = np.random.default_rng(22)
    m = _idle(1)
    try:
        for trial in range(8):
            mem = m.mem
            mem[0, 0x8000:0xA000] = rng.integers(0, 256, 0x2000)
            oam = rng.integers(0, 256, 160)
            oam[0::4] = rng.integers(0, 176, 40)
            oam[1::4] = rng.integers(0, 176, 40)
            mem[0, 0xFE00:0xFEA0] = oam
            for reg in (0xFF40, 0xFF42, 0xFF43, 0xFF47, 0xFF48, 0xFF49):
                mem[0, reg] = rng.integers(0, 256)
            mem[0, 0xFF4A], mem[0, 0xFF4B] = rng.integers(0, 144), rng.integers(0, 168)
            ys = np.arange(144)
            regs = [mem[0, a] for a in (0xFF40, 0xFF43, 0xFF42, 0xFF47, 0xFF4B, 0xFF4A)]
            lat = np.zeros((9, 144), np.uint8)
            lat[:6] = np.array(regs, np.uint8)[:, None]
            lat[6] = np.where(ys >= mem[0, 0xFF4A], (ys - int(mem[0, 0xFF4A])) & 0xFF, 0)
            lat[7], lat[8] = mem[0, 0xFF48], mem[0, 0xFF49]
            m.latches[:] = lat
            m.render(packed=False)
            np.testing.assert_array_equal(m.render_bg_env0()[::2, ::2], m.pix[0])
    finally:
        m.close()


def test_env0_frame_raster_scroll_known_answer():
    """A per-line SCX latch (a raster effect): tile 1 lights only its leftmost
    column, the map is all tile 1, and line y scrolls by y, so pixel (x, y) is
    shade 3 exactly when (x + y) % 8 == 0; line 7 also switches to the window
    (WX 7 + 40, window line 3) on the 9C00 map of tile 2 (all colour 2)."""
    m = _idle(1)
    mem = m.mem
    try:
        mem[0, 0x9800:0x9C00] = 1
        mem[0, 0x9C00:0xA000] = 2
        mem[0, 0x8010:0x8020] = [0x80, 0x80] * 8  # colour 3 at column 0
        mem[0, 0x8020:0x8030] = [0x00, 0xFF] * 8  # colour 2 everywhere
        lat = np.zeros((9, 144), np.uint8)
        lat[0] = 0x91  # BG on, unsigned tiles, window off
        lat[1] = np.arange(144) & 0xFF  # SCX = y
        lat[3] = 0xE4
        lat[0, 7] = 0xF1  # window on, map 9C00
        lat[4, 7], lat[5, 7], lat[6, 7] = 7 + 40, 0, 3
        m.latches[:] = lat
        f = m.render_bg_env0()
        ys, xs = np.mgrid[0:144, 0:160]
        want = np.where((xs + ys) % 8 == 0, 3, 0)
        want[7, 40:] = 2
        np.testing.assert_array_equal(f, want)
    finally:
        m.close()
