"""Parity at the configurations' full env counts (16,384 / 65,536 / 131,072).

The oracle cannot replay 131,072 envs in a test's time, so every env is tied
to it in two parts:

* Envs never interact, and every env starts from the same reset state, so two
  envs with the same history (the same action in every step, and for the
  masked-reset workload the same restore steps) must end in the same state.
  The device computes a per-env digest of everything the step touches (the
  64 KiB memory image, every scalar, both counters, the cart state, cart RAM,
  serial bytes, obs/reward and the rendered pixels) and every env must equal
  the representative of its history group.
* The oracle replays one representative per group (chosen at random inside
  the group, so the checked lanes spread over every block and lane position),
  plus env 0 and env N-1, on those envs' own action columns, and each must be
  bit-exact against it: full state, obs, reward, pixels, serial bytes and
  the env-0 scanline latches.

A wrong interleave index, block offset, lane mask or any cross-lane write at
full size breaks the first part; any semantic difference breaks the second.
"""

from __future__ import annotations

import numpy as np
import pytest

from gbxcule_amd.carts.synth import seeded_actions
from oracle.ref import RefMachine

from ._parity import ref_export_env
from .conftest import require_gpu

pytestmark = pytest.mark.gpu

CASES = [
    # cart, envs, frameskip, steps, action seed, render
    ("c2", 16384, 24, 3, 1, None),
    ("c3", 16384, 24, 3, 2, "packed"),
    ("c4", 131072, 24, 3, 3, None),
    ("c4", 131072, 1, 3, 13, None),
    ("c4m3", 65536, 24, 3, 4, None),
]


def _backend(rom, boot, n, fs, render):
    from gbxcule_amd.backend import HipVecBackend

    return HipVecBackend(
        rom,
        num_envs=n,
        frames_per_step=fs,
        release_after_frames=8,
        stage="full_step",
        render_pixels=render == "unpacked",
        render_pixels_packed=render == "packed",
        bootrom=boot,
    )


def _row_digest(x, seed: int):
    """int64 [N] weighted byte sums of the rows of a [N, L] device tensor."""
    import torch

    n = x.shape[0]
    x = x.reshape(n, -1)
    w = torch.from_numpy(
        np.random.default_rng(seed).integers(1, 2**62, x.shape[1], dtype=np.int64)
    ).cuda()
    out = torch.empty(n, dtype=torch.int64, device="cuda")
    step = max(1, (1 << 27) // max(1, x.shape[1]))
    for i in range(0, n, step):
        out[i : i + step] = (x[i : i + step].to(torch.int64) * w).sum(1)
    return out


def _cart_ram_digest(dut):
    """int64 [N] digest of each env's cart RAM (None for carts without RAM)."""
    import torch

    from gbxcule_amd import _lib
    from gbxcule_amd.abi import ENV_BLOCK

    ram = dut._info(_lib.INFO_RAM_BYTES)
    if ram == 0:
        return None
    stride = dut._info(_lib.INFO_CART_RAM_STRIDE)
    npad = dut._info(_lib.INFO_PADDED_ENVS)
    v = dut._view(_lib.BUF_CART_RAM, (npad // ENV_BLOCK, stride, ENV_BLOCK), "uint8")
    w = torch.from_numpy(np.random.default_rng(77).integers(1, 2**62, ram, dtype=np.int64)).cuda()
    out = torch.empty((npad // ENV_BLOCK, ENV_BLOCK), dtype=torch.int64, device="cuda")
    step = max(1, (1 << 27) // (stride * ENV_BLOCK))
    for b in range(0, npad // ENV_BLOCK, step):
        out[b : b + step] = (v[b : b + step, :ram].to(torch.int64) * w[None, :, None]).sum(1)
    return out.reshape(-1)[: dut.num_envs]


def _digests(dut, render) -> dict[str, np.ndarray]:
    import torch

    torch.cuda.synchronize()
    d = {
        "state_hash": dut.state_hash_torch(),
        "obs": _row_digest(dut.obs_torch().view(torch.int32), 11),
        "reward": dut.reward_torch().view(torch.int32).to(torch.int64),
    }
    cr = _cart_ram_digest(dut)
    if cr is not None:
        d["cart_ram"] = cr
    if render == "packed":
        d["pix_packed"] = _row_digest(dut.pixels_packed_torch(), 12)
    elif render == "unpacked":
        d["pix"] = _row_digest(dut.pixels_torch(), 13)
    out = {k: v.cpu().numpy() for k, v in d.items()}
    serial = dut.export_serial()
    out["serial"] = serial.astype(np.int64) @ np.random.default_rng(14).integers(
        1, 2**30, serial.shape[1], dtype=np.int64
    )
    return out


def _groups(keys: np.ndarray, seed: int) -> tuple[np.ndarray, np.ndarray]:
    """(rep_of[N], reps): a random representative env for each distinct key."""
    perm = np.random.default_rng(seed).permutation(keys.size)
    _, first, inv = np.unique(keys[perm], return_index=True, return_inverse=True)
    reps_perm = perm[first]  # representative of each unique key
    rep_of = np.empty(keys.size, dtype=np.int64)
    rep_of[perm] = reps_perm[inv.reshape(-1)]
    return rep_of, np.unique(reps_perm)


def _check_groups(dig: dict[str, np.ndarray], rep_of: np.ndarray, tag: str) -> None:
    for name, v in dig.items():
        bad = np.nonzero(v != v[rep_of])[0]
        if bad.size:
            e = int(bad[0])
            raise AssertionError(
                f"[{tag}] {name}: {bad.size} envs differ from the representative of their history "
                f"group; env {e} vs env {int(rep_of[e])}"
            )


def _check_sample(dut, ref, sample: np.ndarray, render, tag: str) -> None:
    """Full state of each sampled env against the oracle's replay of it."""
    import torch

    from gbxcule_amd.state_io import FIELDS

    for j, e in enumerate(sample.tolist()):
        got, want = dut.export_env(e), ref_export_env(ref, j)
        for i, name in enumerate(FIELDS):
            if got.scalars[i] != want.scalars[i]:
                raise AssertionError(
                    f"[{tag}] env {e} field {name}: hip={got.scalars[i]} oracle={want.scalars[i]}"
                )
        np.testing.assert_array_equal(got.cart_state, want.cart_state, err_msg=f"{tag} env {e} cart")
        if not np.array_equal(got.mem, want.mem):
            a = int(np.nonzero(got.mem != want.mem)[0][0])
            raise AssertionError(
                f"[{tag}] env {e} memory differs at {a:#06x}: hip={got.mem[a]:#04x} oracle={want.mem[a]:#04x}"
            )
        np.testing.assert_array_equal(got.cart_ram, want.cart_ram, err_msg=f"{tag} env {e} cart RAM")
    idx = torch.from_numpy(sample).cuda()
    obs = dut.obs_torch()[idx].cpu().numpy()
    np.testing.assert_array_equal(obs.view(np.uint32), ref.obs.view(np.uint32), err_msg=f"{tag} obs")
    rew = dut.reward_torch()[idx].cpu().numpy()
    np.testing.assert_array_equal(rew.view(np.uint32), ref.reward.view(np.uint32), err_msg=f"{tag} reward")
    np.testing.assert_array_equal(dut.export_serial()[sample], ref.serial_buf, err_msg=f"{tag} serial")
    assert sample[0] == 0
    np.testing.assert_array_equal(dut.export_latches(), ref.latches, err_msg=f"{tag} env-0 latches")
    if render == "packed":
        ref.render(packed=True, threads=8)
        got = dut.pixels_packed_torch()[idx].cpu().numpy()
        np.testing.assert_array_equal(got, ref.pix_packed, err_msg=f"{tag} packed pixels")
    elif render == "unpacked":
        ref.render(packed=False, threads=8)
        got = dut.pixels_torch()[idx].cpu().numpy()
        np.testing.assert_array_equal(got, ref.pix, err_msg=f"{tag} pixels")


def _sample(reps: np.ndarray, n: int) -> np.ndarray:
    return np.unique(np.concatenate([reps, [0, n - 1]])).astype(np.int64)


@pytest.mark.parametrize("cart,n,fs,steps,seed,render", CASES)
def test_full_size_parity(carts, bootstub, cart, n, fs, steps, seed, render):
    require_gpu()
    rom = carts[cart]
    tag = f"{cart} n={n} fs={fs}"
    print(f"full-size parity {tag}", flush=True)
    dut = _backend(rom, bootstub, n, fs, render)
    ref = None
    try:
        dut.reset(seed=seed)
        acts = [seeded_actions(seed, k, n) for k in range(steps)]
        keys = np.zeros(n, dtype=np.int64)
        for k in range(steps):
            dut.step(acts[k])
            keys = keys * 9 + acts[k].astype(np.int64) + 1
        rep_of, reps = _groups(keys, seed)
        dig = _digests(dut, render)
        _check_groups(dig, rep_of, tag)
        assert np.unique(dig["state_hash"]).size > 1 or cart == "c3"

        sample = _sample(reps, n)
        ref = RefMachine(sample.size, rom, bootstub)
        ref.step(None, 0, 0, "full_step")
        for k in range(steps):
            ref.step(acts[k][sample], fs, 8, "full_step", threads=8)
        _check_sample(dut, ref, sample, render, tag)
        assert int(ref.field("instr_count").min()) > 0
        assert int(ref.field("trap_flag").sum()) == 0
    finally:
        dut.close()
        if ref is not None:
            ref.close()


def test_full_size_rollout_with_masked_reset(carts, bootstub):
    """The RL rollout shape at 131,072 envs: snapshot of env 0 after step 0,
    a seeded ~1% mask restored before each later step, unpacked pixels and a
    32-byte RAM-sense gather every step."""
    require_gpu()
    import torch

    from gbxcule_amd.reset_cache import ResetCache

    n, fs, seed, steps = 131072, 24, 5, 3
    rom = carts["c5"]
    tag = f"c5 n={n}"
    print(f"full-size parity {tag} (masked reset)", flush=True)
    rng = np.random.default_rng(seed)
    addrs = np.sort(rng.choice(np.arange(0xC000, 0xE000), 32, replace=False)).astype(np.int32)
    addrs[:4] = (0xFF40, 0xFF44, 0xFF0F, 0xFFFF)
    dut = _backend(rom, bootstub, n, fs, "unpacked")
    ref = None
    try:
        dut.reset(seed=0)
        acts = [seeded_actions(seed, k, n) for k in range(steps)]
        masks = [None] + [rng.random(n) < 0.01 for _ in range(1, steps)]
        # history = (step of the last restore, actions since), base 9
        reset_at = np.zeros(n, dtype=np.int64)
        hist = np.zeros(n, dtype=np.int64)
        dut.step(acts[0])
        hist = hist * 9 + acts[0] + 1
        cache = ResetCache.from_backend(dut, env_idx=0)
        snap_hist = hist[0]
        senses = []
        for k in range(1, steps):
            cache.apply_mask_torch(torch.from_numpy(masks[k].astype(np.uint8)).cuda().bool())
            reset_at[masks[k]] = k
            hist[masks[k]] = snap_hist
            dut.step(acts[k])
            hist = hist * 9 + acts[k] + 1
            senses.append(dut.ram_senses_torch(addrs).cpu().numpy())
        assert all(m.sum() > 0 for m in masks[1:])
        keys = reset_at * 9 ** (steps + 2) + hist
        rep_of, reps = _groups(keys, seed)
        dig = _digests(dut, "unpacked")
        _check_groups(dig, rep_of, tag)
        # senses of the last step must be the raw bytes of each env's memory
        rows = torch.from_numpy(addrs.astype(np.int64)).cuda()
        want = dut.memory_blocks_torch()[:, rows, :].permute(0, 2, 1).reshape(-1, addrs.size)[:n].cpu().numpy()
        np.testing.assert_array_equal(senses[-1], want)

        sample = _sample(reps, n)
        ref = RefMachine(sample.size, rom, bootstub)
        ref.step(None, 0, 0, "full_step")
        ref.step(acts[0][sample], fs, 8, "full_step", threads=8)
        ref.render(packed=False)
        ref.snapshot(0, with_pix=True)
        for k in range(1, steps):
            ref.masked_reset(masks[k][sample].astype(np.uint8))
            ref.step(acts[k][sample], fs, 8, "full_step", threads=8)
        _check_sample(dut, ref, sample, "unpacked", tag)
        np.testing.assert_array_equal(senses[-1][sample], ref.mem[:, addrs])
    finally:
        dut.close()
        if ref is not None:
            ref.close()
